"""Token-by-token serving of a TimeMix layer with its state carried in place.

The reference serves a converted model through ``Runner`` -> ``AttentionAdapter`` ->
``TimeMix.forward`` one token per call, and every call returns a new
``{"shift", "wkv"}`` state (theseus/hf_model.py:96-108; the WKV forward allocates the
end state, kernels/wkv7_state.cpp:21).  ``TimeMix.step_`` is the opt-in alternative
that updates a caller-owned state in place through the single-step kernel; this module
adds what a serving loop needs around it:

* ``serving_state(state)``: an owned, contiguous copy of a state that ``forward``
  returned (its ``shift`` is a view of the input, which ``step_`` must not overwrite);
* ``CapturedStep``: one ``step_`` captured into a HIP graph (``torch.cuda.CUDAGraph``),
  so a token costs one graph launch instead of ~20 kernel launches from Python.  The
  state tensors and the input/output buffers keep fixed addresses, which is what makes
  the capture valid; every replay advances the captured state by one token.  The graph
  also reads float32 copies of the layer's small parameters (the stacked shift-lerp
  coefficients; bf16 vectors), which the CapturedStep owns (theseus.fused.param_cache):
  after an in-place weight update call ``refresh_params()`` before the next replay.
"""
from __future__ import annotations

import contextlib

import torch

from . import fused


def serving_state(state):
    """Owned contiguous copies of a ``{"shift", "wkv"}`` state (shift in its dtype, wkv
    float32), safe to update in place with ``TimeMix.step_``."""
    return {"shift": state["shift"].detach().clone(memory_format=torch.contiguous_format),
            "wkv": state["wkv"].detach().float().clone(memory_format=torch.contiguous_format)}


def _autocast(dtype):
    # autocast's weight-cast cache may not be used under graph capture
    if dtype is None:
        return contextlib.nullcontext()
    return torch.autocast("cuda", dtype=dtype, cache_enabled=False)


class CapturedStep:
    """``model.step_(x, state)`` for x [B,1,C], captured once into a HIP graph.

    ``step(x)`` copies x into the graph's input buffer, replays the graph (which
    advances ``state`` in place by one token) and returns the graph's output buffer
    (overwritten by the next call: copy it to keep it).  ``state`` is the caller's
    dict; its two tensors must stay alive and keep their storage while this object is
    used.  ``autocast`` is the dtype the step runs under (as the reference's Runner
    does, hf_model.py:205) or None for a model already in the activation dtype.

    Capture runs the step twice eagerly first (on a side stream, as torch's capture
    requires) and then restores ``state`` to its value at construction.

    The graph reads the parameters in place -- the projection weights directly, the
    small parameters through float32 copies held by this object (``self.params``,
    made during the eager steps, so none is allocated under capture and none can be
    freed while the graph may still replay).  Weights must be updated in place (same
    storage); after such an update, ``refresh_params()`` rewrites the copies, so the
    next replay computes with the new weights.
    """

    def __init__(self, model, state, x_example, autocast=torch.bfloat16):
        if x_example.dim() != 3 or x_example.shape[1] != 1 or not x_example.is_cuda:
            raise ValueError("CapturedStep takes a CUDA x of shape [B,1,C]")
        self.model, self.state, self.autocast = model, state, autocast
        self.x = x_example.detach().clone()
        self.params = {}  # derived parameter tensors the graph reads (fused.param_cache)
        saved = {k: v.clone() for k, v in state.items()}
        side = torch.cuda.Stream(device=self.x.device)
        side.wait_stream(torch.cuda.current_stream(self.x.device))
        with torch.cuda.stream(side), torch.no_grad(), _autocast(autocast), fused.param_cache(self.params):
            for _ in range(2):
                model.step_(self.x, state)
        torch.cuda.current_stream(self.x.device).wait_stream(side)
        with torch.no_grad():
            for k, v in state.items():
                v.copy_(saved[k])
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad(), _autocast(autocast), fused.param_cache(self.params):
            self.out = model.step_(self.x, state)
        torch.cuda.synchronize(self.x.device)

    def refresh_params(self):
        """Rewrite the graph's parameter copies from the model's current (in place
        updated) weights; the next replay uses them."""
        fused.refresh_param_cache(self.params)

    def __call__(self, x):
        with torch.no_grad():
            self.x.copy_(x)
        self.graph.replay()
        return self.out
