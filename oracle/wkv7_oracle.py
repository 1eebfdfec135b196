"""CPU oracle for the WKV7 state recurrence -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The shipped path (``theseus.wkv7`` over the HIP C-ABI library) never
calls into this directory and fails loudly when the HIP library is missing.

Contents
--------
``forward`` / ``backward``
    float64 numpy restatement of the reference recurrence and of its
    hand-written adjoint, vectorised over (batch, head):

    * forward follows ``theseus/wkv7.py:16-28`` (formula, order of terms) and
      ``kernels/wkv7_state.cu:20-39`` (layouts: token vectors ``[B,T,H,N]``,
      state ``[B,H,value,key]``).
    * backward follows ``kernels/wkv7_state.cu:49-78`` line for line
      (``G += dy r^T``; column sums for dr/dw/dk/db/da; row sums for q and
      dv; ``G <- G*d + q a^T``; ``ds0 = G``).

``forward_c`` / ``backward_c``
    The same two functions restated in C (``oracle/wkv7_oracle.c``), float64,
    OpenMP over (batch, head), for sizes where numpy is slow.  Built by
    ``oracle/Makefile`` into ``oracle/_build/libwkv7_oracle.so``.

``reference_torch``
    The reference's PyTorch op sequence (``theseus/wkv7.py:16-28``) restated in
    torch, used (a) with float64 + autograd as an independent check of the
    hand-derived adjoint and (b) in float32 on the host cores as the CPU
    baseline that ``bench.py`` reports.

How each function is pinned (checks live in ``tests/test_oracle.py``)
-------------------------------------------------------------------
* forward: hand-computed N=2,T=2 closed form; dense Kronecker (vec(S))
  transition for tiny N; special cases (r=0 => y=0; a=b=k=v=0 => column
  scaling by the product of decays; w -> -inf with a=b=0 => plain linear
  attention cumulative sum); chunk-split invariance; numpy == C.
* backward: central finite differences of ``forward`` (float64);
  torch.autograd through ``reference_torch`` in float64 (an independent
  derivation); numpy == C.
No function here is left "parity unpinned".
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

# e^{-1/2}: the decay clamp constant of kernels/wkv7_state.cu:27 and
# theseus/wkv7.py:19.
DECAY_SCALE = 0.6065306597126334

_HERE = Path(__file__).resolve().parent


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def decay(w, mode="rwkv"):
    """Per-key decay of a step.

    mode "rwkv": d = exp(-e^{-1/2} * sigmoid(w)), w the pre-sigmoid logit (wkv7.py:19).
    mode "exp":  d = exp(w), no clamp or sigmoid -- the GDN teacher's decay as the
    converter's contract states it ("wkv_decay_operation": "exp(g), NO
    clamp/sigmoid/exp(-exp(w))", convert_qwen2rwkv_lightning.py:384).
    """
    w = np.asarray(w, dtype=np.float64)
    if mode == "exp":
        return np.exp(w)
    if mode != "rwkv":
        raise ValueError(mode)
    return np.exp(-DECAY_SCALE * _sigmoid(w))


def dlogd_dw(w, mode="rwkv"):
    """d(log d)/dw: -e^{-1/2} sigmoid(w)(1 - sigmoid(w)) for "rwkv" (cu:69), 1 for "exp"."""
    w = np.asarray(w, dtype=np.float64)
    if mode == "exp":
        return np.ones_like(w)
    sg = _sigmoid(w)
    return -DECAY_SCALE * sg * (1.0 - sg)


def _f64(*xs):
    return [np.ascontiguousarray(np.asarray(x, dtype=np.float64)) for x in xs]


def forward(r, w, k, v, a, b, s0, return_states=False, mode="rwkv"):
    """Forward recurrence (theseus/wkv7.py:16-28, kernels/wkv7_state.cu:24-38).

    r..b: [B,T,H,N]; s0: [B,H,N,N] (row = value i, column = key j).
    Returns y [B,T,H,N] float64 and sT [B,H,N,N] float64; with
    ``return_states`` also the stacked states [B,H,T+1,N,N] (S_0..S_T).
    ``mode`` picks the decay (``decay``).
    """
    r, w, k, v, a, b, s0 = _f64(r, w, k, v, a, b, s0)
    B, T, H, N = r.shape
    d = decay(w, mode)
    S = s0.copy()
    y = np.empty_like(r)
    states = [S.copy()] if return_states else None
    for t in range(T):
        # sa_i = sum_j S_ij a_j                       (wkv7.py:23, cu:31)
        sa = np.einsum("bhij,bhj->bhi", S, a[:, t])
        # S_ij = S_ij d_j + sa_i b_j + v_i k_j         (wkv7.py:24-26, cu:33)
        S = (S * d[:, t][:, :, None, :]
             + sa[..., None] * b[:, t][:, :, None, :]
             + v[:, t][..., None] * k[:, t][:, :, None, :])
        # y_i = sum_j S_ij r_j                         (wkv7.py:27, cu:34)
        y[:, t] = np.einsum("bhij,bhj->bhi", S, r[:, t])
        if return_states:
            states.append(S.copy())
    if return_states:
        return y, S, np.stack(states, axis=2)
    return y, S


def backward(r, w, k, v, a, b, s0, dy, dsT, mode="rwkv"):
    """Reverse-mode adjoint of ``forward`` (kernels/wkv7_state.cu:49-78).

    Returns (dr, dw, dk, dv, da, db, ds0), all float64; the first six are
    [B,T,H,N], ds0 is [B,H,N,N].  ``mode`` picks the decay; only dw's factor
    d(log d)/dw depends on it.
    """
    r, w, k, v, a, b, s0, dy, dsT = _f64(r, w, k, v, a, b, s0, dy, dsT)
    B, T, H, N = r.shape
    _, _, states = forward(r, w, k, v, a, b, s0, return_states=True, mode=mode)
    d = decay(w, mode)
    fw = dlogd_dw(w, mode)
    grads = [np.zeros_like(r) for _ in range(6)]
    dr, dw, dk, dv, da, db = grads
    G = dsT.copy()                                          # cu:50
    for t in range(T - 1, -1, -1):
        Sp = states[:, :, t]       # S_{t-1} in the 1-based notation (cu:61)
        Sn = states[:, :, t + 1]   # S_t (cu:68, hist[next])
        rt, dt, kt, at, bt = r[:, t], d[:, t], k[:, t], a[:, t], b[:, t]
        dyt, vt = dy[:, t], v[:, t]
        sa = np.einsum("bhij,bhj->bhi", Sp, at)             # cu:62 (dot)
        G = G + dyt[..., None] * rt[:, :, None, :]          # cu:63 (ds += dy r)
        q = np.einsum("bhij,bhj->bhi", G, bt)               # cu:64 (dotgrad)
        dr[:, t] = np.einsum("bhi,bhij->bhj", dyt, Sn)      # cu:68
        dw[:, t] = np.einsum("bhij,bhij->bhj", G, Sp) * dt * fw[:, t]  # cu:69
        dk[:, t] = np.einsum("bhij,bhi->bhj", G, vt)        # cu:70
        db[:, t] = np.einsum("bhij,bhi->bhj", G, sa)        # cu:71
        da[:, t] = np.einsum("bhi,bhij->bhj", q, Sp)        # cu:72
        dv[:, t] = np.einsum("bhij,bhj->bhi", G, kt)        # cu:73,76
        G = G * dt[:, :, None, :] + q[..., None] * at[:, :, None, :]  # cu:74
    return dr, dw, dk, dv, da, db, G                        # cu:78 (ds0 = G)


# ----------------------------------------------------------------------------
# C restatement (same arithmetic, float64, OpenMP over batch*head)
# ----------------------------------------------------------------------------
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "_build" / "libwkv7_oracle.so"
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is missing; build it with `make -C oracle`")
        lib = ctypes.CDLL(str(path))
        dp = ctypes.POINTER(ctypes.c_double)
        lib.wkv7_oracle_forward.argtypes = [ctypes.c_int] * 5 + [dp] * 9
        lib.wkv7_oracle_forward.restype = None
        lib.wkv7_oracle_backward.argtypes = [ctypes.c_int] * 5 + [dp] * 16
        lib.wkv7_oracle_backward.restype = None
        _LIB = lib
    return _LIB


def c_available():
    return (_HERE / "_build" / "libwkv7_oracle.so").exists()


def _ptr(x):
    return x.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


_MODES = {"rwkv": 0, "exp": 1}


def forward_c(r, w, k, v, a, b, s0, mode="rwkv"):
    r, w, k, v, a, b, s0 = _f64(r, w, k, v, a, b, s0)
    B, T, H, N = r.shape
    y = np.empty_like(r)
    sT = np.empty_like(s0)
    _lib().wkv7_oracle_forward(B, T, H, N, _MODES[mode], *map(_ptr, (r, w, k, v, a, b, s0, y, sT)))
    return y, sT


def backward_c(r, w, k, v, a, b, s0, dy, dsT, mode="rwkv"):
    r, w, k, v, a, b, s0, dy, dsT = _f64(r, w, k, v, a, b, s0, dy, dsT)
    B, T, H, N = r.shape
    outs = [np.empty_like(r) for _ in range(6)] + [np.empty_like(s0)]
    _lib().wkv7_oracle_backward(
        B, T, H, N, _MODES[mode], *map(_ptr, (r, w, k, v, a, b, s0, dy, dsT, *outs)))
    return tuple(outs)


# ----------------------------------------------------------------------------
# GDN (gated delta rule) as the recurrence in "exp" decay mode
# ----------------------------------------------------------------------------
def gdn_operands(q, k, v, g, beta):
    """The WKV operands of a GDN step, as the converter's contract maps them
    (convert_qwen2rwkv_lightning.py:385, "wkv_inputs": "r=q/sqrt(Dk), w=g, k=k,
    v=beta*v, a=k, b=-exp(g)*beta*k"): q, k, v [B,T,H,N] (q and k already
    L2-normalised if the layer does so), g, beta [B,T,H].  w is g broadcast
    over the keys, to be used with mode "exp"."""
    q, k, v, g, beta = _f64(q, k, v, g, beta)
    N = q.shape[-1]
    gb = np.broadcast_to(g[..., None], q.shape)
    return (q / np.sqrt(N), np.ascontiguousarray(gb), k, beta[..., None] * v, k.copy(),
            -np.exp(g)[..., None] * beta[..., None] * k)


def gdn_forward(q, k, v, g, beta, s0_kv):
    """GDN output and final state through ``forward`` in "exp" mode.  The GDN state
    is [B,H,key,value] ("gdn_state_layout": "B,Hv,K,V", :382), the transpose of
    the recurrence's [B,H,value,key]."""
    ops = gdn_operands(q, k, v, g, beta)
    y, sT = forward(*ops, np.swapaxes(np.asarray(s0_kv, dtype=np.float64), -1, -2), mode="exp")
    return y, np.ascontiguousarray(np.swapaxes(sT, -1, -2))


# ----------------------------------------------------------------------------
# Torch restatement of the reference op sequence (theseus/wkv7.py:16-28)
# ----------------------------------------------------------------------------
def reference_torch(r, w, k, v, a, b, state):
    """Same torch op sequence as ``theseus/wkv7.py:16-28``.

    Upcasts to float32 like the reference; when the inputs are float64 they
    stay float64 (used for the autograd cross-check).  Returns ``(y, sT)``
    with y cast back to the input dtype.
    """
    import torch

    dtype = r.dtype
    comp = torch.float64 if dtype == torch.float64 else torch.float32
    r, w, k, v, a, b = [x.to(comp) for x in (r, w, k, v, a, b)]
    dec = torch.exp(-DECAY_SCALE * torch.sigmoid(w))
    out = []
    state = state.to(comp)
    for t in range(r.shape[1]):
        sa = (state * a[:, t].unsqueeze(-2)).sum(-1)
        state = (state * dec[:, t].unsqueeze(-2)
                 + sa.unsqueeze(-1) * b[:, t].unsqueeze(-2)
                 + v[:, t].unsqueeze(-1) * k[:, t].unsqueeze(-2))
        out.append((state * r[:, t].unsqueeze(-2)).sum(-1))
    return torch.stack(out, 1).to(dtype), state


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_count():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
