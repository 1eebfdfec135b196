"""Pins the CPU oracle (oracle/wkv7_oracle.py, oracle/wkv7_oracle.c) before it
is trusted as the checker of the HIP kernels.

Each check is an independent formulation, chosen so that a plausible slip in
the restatement (a dropped term, a transposed state, a wrong sign in the
decay derivative, an off-by-one in the reverse loop) fails at least one:
closed forms worked by hand, a dense Kronecker transition, special cases with
textbook answers, finite differences, torch autograd, and numpy == C.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import wkv7_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _inputs(B, T, H, N, seed=0, s0_std=0.1):
    rng = np.random.default_rng(seed)
    r, w, k, v = (rng.standard_normal((B, T, H, N)) for _ in range(4))
    kk = rng.standard_normal((B, T, H, N))
    kk /= np.linalg.norm(kk, axis=-1, keepdims=True)
    alpha = 1 / (1 + np.exp(-rng.standard_normal((B, T, H, N))))
    s0 = rng.standard_normal((B, H, N, N)) * s0_std
    dy = rng.standard_normal((B, T, H, N))
    dsT = rng.standard_normal((B, H, N, N))
    return r, w, k, v, -kk, kk * alpha, s0, dy, dsT


def test_hand_computed_n2_t2_forward():
    g = json.loads((GOLDEN / "wkv7_hand_n2_t2.json").read_text())
    x = [np.array(g["inputs"][n]) for n in "rwkvab"]
    y, sT = O.forward(*x, np.array(g["s0"]))
    d = math.exp(-0.6065306597126334 / 2)
    np.testing.assert_allclose(y[0, :, 0], [[d + 1, 3 * d - 1], [3 * d * d + 5 * d + 6, 7 * d * d + 5 * d + 4]], atol=1e-13)
    np.testing.assert_allclose(y, np.array(g["y"]), atol=1e-13)
    np.testing.assert_allclose(sT, np.array(g["sT"]), atol=1e-13)


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_hand_computed_n2_t2_backward(impl):
    g = json.loads((GOLDEN / "wkv7_hand_n2_t2.json").read_text())
    x = [np.array(g["inputs"][n]) for n in "rwkvab"]
    args = (*x, np.array(g["s0"]), np.array(g["dy"]), np.array(g["dsT"]))
    grads = O.backward(*args) if impl == "numpy" else O.backward_c(*args)
    for name, got in zip(["dr", "dw", "dk", "dv", "da", "db", "ds0"], grads):
        np.testing.assert_allclose(got, np.array(g["grads"][name]), atol=1e-7, err_msg=name)


def test_dense_kronecker_transition():
    """vec(S_t) = kron(I, M_t^T) vec(S_{t-1}) + vec(v k^T), M_t = diag(d_t) + a_t b_t^T."""
    r, w, k, v, a, b, s0, _, _ = _inputs(1, 6, 2, 4, seed=3)
    y, sT = O.forward(r, w, k, v, a, b, s0)
    N = 4
    for h in range(2):
        s = s0[0, h].reshape(-1)
        for t in range(6):
            M = np.diag(O.decay(w[0, t, h])) + np.outer(a[0, t, h], b[0, t, h])
            s = np.kron(np.eye(N), M.T) @ s + np.outer(v[0, t, h], k[0, t, h]).reshape(-1)
            yk = np.kron(np.eye(N), r[0, t, h][None, :]) @ s
            np.testing.assert_allclose(y[0, t, h], yk, atol=1e-12)
        np.testing.assert_allclose(sT[0, h].reshape(-1), s, atol=1e-12)


def test_special_cases():
    r, w, k, v, a, b, s0, _, _ = _inputs(2, 9, 3, 5, seed=4)
    z = np.zeros_like(r)
    # r = 0 -> y = 0
    y, _ = O.forward(z, w, k, v, a, b, s0)
    assert np.abs(y).max() == 0.0
    # a = b = k = v = 0 -> each key column is scaled by the product of its decays
    _, sT = O.forward(r, w, z, z, z, z, s0)
    cum = np.prod(O.decay(w), axis=1)  # [B,H,N]
    np.testing.assert_allclose(sT, s0 * cum[:, :, None, :], rtol=1e-12)
    # sigmoid(w) -> 0 (d -> 1) and a = b = 0 -> linear attention, a cumulative sum of v k^T
    wneg = np.full_like(w, -60.0)
    y, sT = O.forward(r, wneg, k, v, z, z, s0)
    outer = np.einsum("bthi,bthj->bthij", v, k)
    S = s0[:, None] + np.cumsum(outer, axis=1).transpose(0, 1, 2, 3, 4)
    np.testing.assert_allclose(sT, S[:, -1], atol=1e-10)
    np.testing.assert_allclose(y, np.einsum("bthij,bthj->bthi", S, r), atol=1e-10)


def test_decay_range():
    w = np.linspace(-30, 30, 101)
    d = O.decay(w)
    assert np.all(d <= 1.0) and np.all(d >= math.exp(-0.6065306597126334) - 1e-15)
    assert abs(O.decay(0.0) - math.exp(-0.6065306597126334 / 2)) < 1e-15


def test_chunk_split_invariance():
    r, w, k, v, a, b, s0, _, _ = _inputs(1, 23, 2, 6, seed=5)
    y, sT = O.forward(r, w, k, v, a, b, s0)
    y1, s1 = O.forward(*(x[:, :10] for x in (r, w, k, v, a, b)), s0)
    y2, s2 = O.forward(*(x[:, 10:] for x in (r, w, k, v, a, b)), s1)
    np.testing.assert_allclose(np.concatenate([y1, y2], 1), y, atol=1e-13)
    np.testing.assert_allclose(s2, sT, atol=1e-13)


def test_backward_finite_differences():
    r, w, k, v, a, b, s0, dy, dsT = _inputs(1, 3, 1, 3, seed=6, s0_std=0.5)
    xs = [r, w, k, v, a, b, s0]
    grads = O.backward(r, w, k, v, a, b, s0, dy, dsT)

    def loss(vals):
        y, sT = O.forward(*vals)
        return float((y * dy).sum() + (sT * dsT).sum())

    eps = 1e-6
    for n, (x, g) in enumerate(zip(xs, grads)):
        fd = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            p = [z.copy() for z in xs]
            m = [z.copy() for z in xs]
            p[n][idx] += eps
            m[n][idx] -= eps
            fd[idx] = (loss(p) - loss(m)) / (2 * eps)
        np.testing.assert_allclose(g, fd, atol=1e-7, rtol=1e-6, err_msg=f"input {n}")


def test_backward_matches_torch_autograd():
    r, w, k, v, a, b, s0, dy, dsT = _inputs(2, 11, 2, 7, seed=7)
    grads = O.backward(r, w, k, v, a, b, s0, dy, dsT)
    ts = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (r, w, k, v, a, b, s0)]
    y, sT = O.reference_torch(*ts)
    y0, sT0 = O.forward(r, w, k, v, a, b, s0)
    np.testing.assert_allclose(y.detach().numpy(), y0, atol=1e-12)
    np.testing.assert_allclose(sT.detach().numpy(), sT0, atol=1e-12)
    torch.autograd.backward((y, sT), (torch.tensor(dy), torch.tensor(dsT)))
    for t, g in zip(ts, grads):
        np.testing.assert_allclose(t.grad.numpy(), g, atol=1e-11)


@pytest.mark.skipif(not O.c_available(), reason="C oracle not built (make -C oracle)")
def test_c_matches_numpy():
    args = _inputs(2, 37, 3, 16, seed=8)
    y, sT = O.forward(*args[:7])
    yc, sTc = O.forward_c(*args[:7])
    np.testing.assert_allclose(yc, y, atol=1e-11)
    np.testing.assert_allclose(sTc, sT, atol=1e-11)
    for g, gc in zip(O.backward(*args), O.backward_c(*args)):
        np.testing.assert_allclose(gc, g, atol=1e-10)


def test_seeded_golden_fixture():
    from theseus.synthetic import wkv7_inputs
    ref = np.load(GOLDEN / "wkv7_small_seeded.npz")
    inp = wkv7_inputs(1, 21, 2, 8, seed=int(ref["seed"]), dtype=torch.float32, s0_std=0.1, with_dsT=True)
    arr = {n: inp[n].numpy().astype(np.float64) for n in inp}
    y, sT = O.forward(*(arr[n] for n in "rwkvab"), arr["s0"])
    np.testing.assert_allclose(y, ref["y"], atol=1e-12)
    np.testing.assert_allclose(sT, ref["sT"], atol=1e-12)
    grads = O.backward(*(arr[n] for n in "rwkvab"), arr["s0"], arr["dy"], arr["dsT"])
    for name, g in zip(["dr", "dw", "dk", "dv", "da", "db", "ds0"], grads):
        np.testing.assert_allclose(g, ref[name], atol=1e-11, err_msg=name)


def test_oracle_flags_a_planted_mistake():
    """A restatement with a transposed state in sa (S^T a instead of S a) must
    fail the Kronecker/autograd style checks -- demonstrated on the CPU."""
    r, w, k, v, a, b, s0, _, _ = _inputs(1, 4, 1, 4, seed=9, s0_std=1.0)
    y, _ = O.forward(r, w, k, v, a, b, s0)
    S = s0[0, 0].copy()
    ys = []
    for t in range(4):
        sa = S.T @ a[0, t, 0]  # planted mistake
        S = S * O.decay(w[0, t, 0])[None, :] + np.outer(sa, b[0, t, 0]) + np.outer(v[0, t, 0], k[0, t, 0])
        ys.append(S @ r[0, t, 0])
    assert np.abs(np.array(ys) - y[0, :, 0]).max() > 1e-3
