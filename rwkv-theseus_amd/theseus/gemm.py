"""Few-row projections for TimeMix serving (C ABI: include/theseus_gemm.h).

A serving step runs every projection of the layer (theseus/timemix.py:63-69: receptance,
key, value, output and the w/a/g LoRAs) on one token per lane, so each product has as many
rows as lanes (64 at config 4) and streams its weight matrix.  ``linear(x, weight)`` is
``x @ weight.T`` and ``lora(x, down, up, act)`` is ``act(x @ down) @ up`` on the
``theseus_gemm_rows`` kernel (bf16, float32 accumulation, split-K with a deterministic
sum), for x with at most ``MAX_ROWS`` rows and no autograd; ``group`` runs several
independent products with the same rows in one launch (theseus_gemm_rows_group).

Weights are read in place when they are bf16 and already in the kernel's [out][in]
layout (nn.Linear weights); the LoRA matrices ([in][out]) and float32 weights need a
derived bf16 [out][in] copy, which is made per call -- or once, inside
``theseus.fused.param_cache(store)`` (theseus.serving.CapturedStep holds one).
"""
from __future__ import annotations

import ctypes

import torch

from . import fused
from .wkv7 import extension

MAX_ROWS = 128  # THESEUS_GEMM_MAX_ROWS
MAX_GROUP = 8  # THESEUS_GEMM_MAX_GROUP
NONE, TANH, SIGMOID = 0, 1, 2  # theseus_gemm_act

_bound = None


class Problem(ctypes.Structure):
    """theseus_gemm_problem: y [M][N] = act(x [M][K] w [N][K]^T)."""
    _fields_ = [("N", ctypes.c_int), ("K", ctypes.c_int), ("act", ctypes.c_int),
                ("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("y", ctypes.c_void_p)]


def _lib():
    global _bound
    lib = extension().lib
    if _bound is None:
        vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        lib.theseus_gemm_rows_workspace_size.argtypes = [i32] * 3
        lib.theseus_gemm_rows_workspace_size.restype = sz
        lib.theseus_gemm_rows.argtypes = [i32] * 4 + [vp] * 4 + [sz, vp]
        lib.theseus_gemm_rows.restype = i32
        lib.theseus_gemm_rows_group_workspace_size.argtypes = [i32, i32, ctypes.POINTER(Problem)]
        lib.theseus_gemm_rows_group_workspace_size.restype = sz
        lib.theseus_gemm_rows_group.argtypes = [i32, i32, ctypes.POINTER(Problem), vp, sz, vp]
        lib.theseus_gemm_rows_group.restype = i32
        _bound = True
    return lib


def supported(rows, n, k):
    """True when theseus_gemm_rows takes a [rows, k] x [n, k]^T product."""
    return 1 <= rows <= MAX_ROWS and n >= 16 and n % 16 == 0 and k >= 32 and k % 32 == 0


# Workspaces (the split-K partial tiles): one per (device, stream) for calls outside a
# parameter store, one in the store otherwise (so a captured graph owns the one it uses).
_workspaces = {}


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    store = fused._store
    if store is not None:
        key = ("gemm_workspace", device.index)
        hit = store.get(key)
        if hit is None or hit[2].numel() < nbytes:
            size = 1 << max(20, (nbytes - 1).bit_length())
            ws = torch.empty(size, dtype=torch.uint8, device=device)
            store[key] = ((), lambda: torch.empty(size, dtype=torch.uint8, device=device), ws)
            return ws
        return hit[2]
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(1 << max(20, (nbytes - 1).bit_length()), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _rows_bf16(x):
    return x.reshape(-1, x.shape[-1]).to(torch.bfloat16).contiguous()


def _out_in(w, transposed):
    """bf16 [out][in] view or copy of a weight ([out][in] unless ``transposed``)."""
    if not transposed and w.dtype == torch.bfloat16 and w.is_contiguous():
        return w.detach()
    make = (lambda: w.detach().t().to(torch.bfloat16).contiguous()) if transposed else \
        (lambda: w.detach().to(torch.bfloat16).contiguous())
    return fused._cached("gemm_t" if transposed else "gemm_bf16", (w,), make)


def _gemm(x2, w_oi, act):
    rows, k = x2.shape
    n = w_oi.shape[0]
    lib = _lib()
    y = torch.empty((rows, n), dtype=torch.bfloat16, device=x2.device)
    with torch.cuda.device(x2.device):
        nbytes = int(lib.theseus_gemm_rows_workspace_size(rows, n, k))
        ws = _workspace(nbytes, x2.device)
        st = lib.theseus_gemm_rows(rows, n, k, act, ctypes.c_void_p(x2.data_ptr()),
                                   ctypes.c_void_p(w_oi.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                   ctypes.c_void_p(ws.data_ptr() if ws is not None else 0),
                                   ctypes.c_size_t(ws.numel() if ws is not None else 0),
                                   ctypes.c_void_p(torch.cuda.current_stream(x2.device).cuda_stream))
    if st:
        raise RuntimeError("theseus_gemm: " + extension().lib.theseus_wkv7_error_string(st).decode())
    return y


def linear(x, weight, act=NONE):
    """act(x @ weight.T) in bf16 for x [..., in] (at most MAX_ROWS rows), weight [out, in]."""
    y = _gemm(_rows_bf16(x), _out_in(weight, False), act)
    return y.reshape(*x.shape[:-1], weight.shape[0])


def lora(x, down, up, act=NONE):
    """act(x @ down) @ up in bf16 for x [..., C], down [C, r], up [r, C] (timemix.py:64-67)."""
    mid = _gemm(_rows_bf16(x), _out_in(down, True), act)
    y = _gemm(mid, _out_in(up, True), NONE)
    return y.reshape(*x.shape[:-1], up.shape[1])


def group(items):
    """[(x, weight, act, transposed), ...] -> [act(x @ W^T), ...] in one launch
    (theseus_gemm_rows_group): every x [..., in] with the same number of rows (at most
    MAX_ROWS), weight [out, in], or [in, out] when ``transposed`` (a LoRA matrix)."""
    if not 1 <= len(items) <= MAX_GROUP:
        raise ValueError(f"theseus_gemm: 1 to {MAX_GROUP} products per group")
    xs = [_rows_bf16(x) for x, _, _, _ in items]
    rows = xs[0].shape[0]
    if any(x2.shape[0] != rows for x2 in xs):
        raise ValueError("theseus_gemm: the products of a group must have the same rows")
    ws_ = [_out_in(w, tr) for _, w, _, tr in items]
    dev = xs[0].device
    ys = [torch.empty((rows, w.shape[0]), dtype=torch.bfloat16, device=dev) for w in ws_]
    probs = (Problem * len(items))(*[Problem(w.shape[0], x2.shape[1], act, x2.data_ptr(), w.data_ptr(), y.data_ptr())
                                     for (_, _, act, _), x2, w, y in zip(items, xs, ws_, ys)])
    lib = _lib()
    with torch.cuda.device(dev):
        nbytes = int(lib.theseus_gemm_rows_group_workspace_size(rows, len(items), probs))
        ws = _workspace(nbytes, dev)
        st = lib.theseus_gemm_rows_group(rows, len(items), probs,
                                         ctypes.c_void_p(ws.data_ptr() if ws is not None else 0),
                                         ctypes.c_size_t(ws.numel() if ws is not None else 0),
                                         ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    if st:
        raise RuntimeError("theseus_gemm: " + extension().lib.theseus_wkv7_error_string(st).decode())
    return [y.reshape(*x.shape[:-1], y.shape[1]) for (x, _, _, _), y in zip(items, ys)]


def usable(x, *weights):
    """The serving path can take these products: CUDA, no autograd, few rows, and every
    weight's shape within the kernel's limits."""
    if not x.is_cuda or torch.is_grad_enabled() and (x.requires_grad or any(w.requires_grad for w in weights)):
        return False
    rows = x.numel() // x.shape[-1]
    if rows > MAX_ROWS:
        return False
    try:
        _lib()
    except AttributeError:
        return False
    return all(w.dim() == 2 and w.is_cuda for w in weights)
