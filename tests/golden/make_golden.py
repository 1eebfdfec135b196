"""Writes the golden WKV7 vectors in this directory.

1. ``wkv7_hand_n2_t2.json`` -- a B=H=1, N=2, T=2 case whose outputs are
   evaluated from closed forms derived by hand from the recurrence of
   theseus/wkv7.py:16-28 (no loop, no oracle): with both steps at w = 0 every
   key decays by d = exp(-e^{-1/2}/2) and

       S1 = [[d+1, 2d+2], [3d-1, 4d+2]],            y1 = [d+1, 3d-1]
       S2 = [[d^2+3d+2, 2d^2+2d+4], [3d^2+3d+2, 4d^2+2d+2]]
       y2 = [3d^2+5d+6, 7d^2+5d+4]

   for s0 = [[1,2],[3,4]], (a1,b1,k1,v1,r1) = ([1,0],[0,1],[1,1],[1,-1],[1,0])
   and (a2,b2,k2,v2,r2) = ([0,1],[1,0],[0,2],[2,1],[1,1]).
   Gradients of L = sum(y*dy) + sum(sT*dsT) are added by central finite
   differences of the closed form (float64), so they do not come from the
   oracle's adjoint either.

2. ``wkv7_small_seeded.npz`` -- a seeded B=1, T=21 (a 16-step segment plus a
   5-step tail), H=2, N=8 float32 case with float64 outputs from the oracle,
   kept so that changes to the oracle itself show up as a diff.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parents[1] / "rwkv-theseus_amd"))


def hand_inputs():
    s0 = np.array([[1.0, 2.0], [3.0, 4.0]])
    steps = [dict(a=[1, 0], b=[0, 1], k=[1, 1], v=[1, -1], r=[1, 0], w=[0, 0]),
             dict(a=[0, 1], b=[1, 0], k=[0, 2], v=[2, 1], r=[1, 1], w=[0, 0])]
    x = {n: np.array([[[s[n]] for s in steps]], dtype=np.float64) for n in "rwkvab"}
    return x, s0[None, None]


def closed_form(x, s0):
    """Generic 2x2, 2-step closed form (expanded by hand, see module doc)."""
    d = [[math.exp(-0.6065306597126334 / (1.0 + math.exp(-x["w"][0, t, 0, j]))) for j in range(2)]
         for t in range(2)]
    S = s0[0, 0].copy()
    ys = []
    for t in range(2):
        a, b, k, v, r = (x[n][0, t, 0] for n in "abkvr")
        sa0 = S[0, 0] * a[0] + S[0, 1] * a[1]
        sa1 = S[1, 0] * a[0] + S[1, 1] * a[1]
        S = np.array([[S[0, 0] * d[t][0] + sa0 * b[0] + v[0] * k[0], S[0, 1] * d[t][1] + sa0 * b[1] + v[0] * k[1]],
                      [S[1, 0] * d[t][0] + sa1 * b[0] + v[1] * k[0], S[1, 1] * d[t][1] + sa1 * b[1] + v[1] * k[1]]])
        ys.append([S[0, 0] * r[0] + S[0, 1] * r[1], S[1, 0] * r[0] + S[1, 1] * r[1]])
    return np.array(ys)[None, :, None, :], S[None, None]


def main():
    x, s0 = hand_inputs()
    y, sT = closed_form(x, s0)
    d = math.exp(-0.6065306597126334 / 2)
    # the expanded polynomials of the module docstring must agree with the generic form
    assert np.allclose(y[0, :, 0], [[d + 1, 3 * d - 1], [3 * d * d + 5 * d + 6, 7 * d * d + 5 * d + 4]], atol=1e-13)
    assert np.allclose(sT[0, 0], [[d * d + 3 * d + 2, 2 * d * d + 2 * d + 4], [3 * d * d + 3 * d + 2, 4 * d * d + 2 * d + 2]], atol=1e-13)
    dy = np.array([[[[0.5, -1.0]], [[2.0, 0.25]]]])
    dsT = np.array([[[[1.0, -0.5], [0.75, 2.0]]]])

    def loss(xx, ss):
        yy, st = closed_form(xx, ss)
        return float((yy * dy).sum() + (st * dsT).sum())

    eps = 1e-6
    grads = {}
    for n in "rwkvab":
        g = np.zeros_like(x[n])
        for idx in np.ndindex(g.shape):
            xp = {m: v.copy() for m, v in x.items()}
            xm = {m: v.copy() for m, v in x.items()}
            xp[n][idx] += eps
            xm[n][idx] -= eps
            g[idx] = (loss(xp, s0) - loss(xm, s0)) / (2 * eps)
        grads["d" + n] = g.tolist()
    g = np.zeros_like(s0)
    for idx in np.ndindex(g.shape):
        sp, sm = s0.copy(), s0.copy()
        sp[idx] += eps
        sm[idx] -= eps
        g[idx] = (loss(x, sp) - loss(x, sm)) / (2 * eps)
    grads["ds0"] = g.tolist()
    out = {"doc": "B=H=1,N=2,T=2 WKV7 case; y/sT from closed forms, gradients by central differences",
           "inputs": {n: x[n].tolist() for n in "rwkvab"}, "s0": s0.tolist(),
           "dy": dy.tolist(), "dsT": dsT.tolist(), "y": y.tolist(), "sT": sT.tolist(), "grads": grads,
           "fd_eps": eps}
    (HERE / "wkv7_hand_n2_t2.json").write_text(json.dumps(out, indent=1))

    from oracle import wkv7_oracle as O
    from theseus.synthetic import wkv7_inputs
    inp = wkv7_inputs(1, 21, 2, 8, seed=777, dtype=__import__("torch").float32, s0_std=0.1, with_dsT=True)
    arr = {n: inp[n].numpy().astype(np.float64) for n in inp}
    yo, sTo = O.forward(*(arr[n] for n in "rwkvab"), arr["s0"])
    go = O.backward(*(arr[n] for n in "rwkvab"), arr["s0"], arr["dy"], arr["dsT"])
    np.savez_compressed(HERE / "wkv7_small_seeded.npz", seed=777, y=yo, sT=sTo,
                        **{"d" + n: gg for n, gg in zip("rwkvab", go[:6])}, ds0=go[6])


if __name__ == "__main__":
    main()
