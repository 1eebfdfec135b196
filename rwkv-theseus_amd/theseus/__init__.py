"""MI355X-native drop-in for the hot path of RWKV-Theseus: the WKV7 state
recurrence operator (``theseus.wkv7``) and the TimeMix layer around it
(``theseus.timemix``)."""
