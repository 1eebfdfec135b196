"""RWKV7 (WKV7) state recurrence for MI355X.  State layout: [batch, head, value, key].

Drop-in for the reference operator module ``theseus/wkv7.py``: the same public
names and meanings -- ``reference``, ``extension``, ``_WKV`` and
``wkv7(r, w, k, v, a, b, state, backend="cuda")`` (theseus/wkv7.py:16-70).

``backend="cuda"`` (the name is kept; on ROCm torch GPU tensors report
``is_cuda``) runs hand-written gfx950 HIP kernels from ``libtheseus_wkv7.so``
through its C ABI (``include/theseus_wkv7.h``), loaded with ctypes.  There is
no CPU fallback: if the library is missing, ``extension()`` raises.
``backend="reference"`` is the explicit pure-PyTorch loop for CPU use, as in
the reference.

Differences in what is saved for backward: the reference saves the full
float32 state history ``[B,H,T+1,N,N]`` (kernels/wkv7_state.cpp:21-22); this
implementation saves the state every 16 steps plus the final state
``[B,H,ceil(T/16)+1,N,N]`` and replays inside the backward kernels.  Gradients
come back in the input dtype (the reference computes float32 and casts,
theseus/wkv7.py:56) and ``ds0`` in float32, as in the reference.  The chunk
boundary is never detached by this operator; callers detach (wkv7.py:5).
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import warnings
from functools import lru_cache
from pathlib import Path

import torch

DECAY_SCALE = 0.6065306597126334  # e^{-1/2} (theseus/wkv7.py:19)
LIB_PATH = Path(__file__).resolve().parent / "libtheseus_wkv7.so"

_BF16, _FP32 = 0, 1

# theseus_wkv7_flags (include/theseus_wkv7.h)
DECAY_EXP = 1           # d = exp(w), unclamped (the GDN teacher's decay)
STATE_KEY_VALUE = 2     # states [B,H,key,value] (GDN's layout) instead of [B,H,value,key]

# theseus_wkv7_family codes (include/theseus_wkv7.h) -> why the step-serial kernels run
_FAMILY_FORCED = 1
_FAMILY_RECORDS = 6  # bf16, N=128: the chunk-record kernels
_FALLBACK_REASON = {
    2: "float32 token tensors",
    3: "a head size other than 64 or 128",
    4: "a token tensor of 2 GiB or more, or one head's saved states of 4 GiB or more",
}


def reference(r, w, k, v, a, b, state):
    """Pure-PyTorch recurrence, float32 (theseus/wkv7.py:16-28).

    Per step: sa = S a; S <- S*diag(d) + sa b^T + v k^T; y = S r, with
    d = exp(-e^{-1/2} sigmoid(w)).  Returns y in the input dtype and the
    float32 final state; differentiable through autograd.
    """
    dtype = r.dtype
    r, w, k, v, a, b = [x.float() for x in (r, w, k, v, a, b)]
    decay = torch.exp(-DECAY_SCALE * torch.sigmoid(w))
    state = state.float()
    ys = []
    for t in range(r.shape[1]):
        sa = (state * a[:, t, :, None, :]).sum(-1)
        state = (state * decay[:, t, :, None, :]
                 + sa[..., None] * b[:, t, :, None, :]
                 + v[:, t, :, :, None] * k[:, t, :, None, :])
        ys.append((state * r[:, t, :, None, :]).sum(-1))
    return torch.stack(ys, 1).to(dtype), state


def _ptr(x):
    return ctypes.c_void_p(x.data_ptr()) if x is not None else ctypes.c_void_p(0)


def _on(device):
    """The device guard of kernels/wkv7_state.cpp:17,27 (a no-op when it is already current)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _workspace(nbytes, device):
    return (torch.empty((nbytes,), dtype=torch.uint8, device=device), nbytes) if nbytes else (None, 0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class Extension:
    """ctypes binding of libtheseus_wkv7.so with the reference module's methods.

    ``forward``/``backward`` take and return the same things as the pybind11
    functions of kernels/wkv7_state.cpp:16-37, with the saved-state tensor in
    place of the history; ``decode_step`` is the in-place T=1 step.
    """

    def __init__(self, lib):
        self.lib = lib
        vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        lib.theseus_wkv7_abi_version.restype = i32
        lib.theseus_wkv7_error_string.argtypes = [i32]
        lib.theseus_wkv7_error_string.restype = ctypes.c_char_p
        lib.theseus_wkv7_checkpoint_interval.restype = i32
        lib.theseus_wkv7_checkpoint_count.argtypes = [i32]
        lib.theseus_wkv7_checkpoint_count.restype = ctypes.c_longlong
        for fn in (lib.theseus_wkv7_forward_workspace_size, lib.theseus_wkv7_backward_workspace_size):
            fn.argtypes = [i32] * 5
            fn.restype = sz
        lib.theseus_wkv7_forward.argtypes = [i32] * 5 + [vp] * 10 + [vp, sz, vp]
        lib.theseus_wkv7_forward.restype = i32
        lib.theseus_wkv7_backward.argtypes = [i32] * 5 + [vp] * 16 + [vp, sz, vp]
        lib.theseus_wkv7_backward.restype = i32
        lib.theseus_wkv7_decode_step.argtypes = [i32] * 4 + [vp] * 8 + [vp]
        lib.theseus_wkv7_decode_step.restype = i32
        # forward without a workspace argument (static device scratch; allocates nothing)
        lib.theseus_wkv7_forward_noalloc.argtypes = [i32] * 5 + [vp] * 10 + [vp]
        lib.theseus_wkv7_forward_noalloc.restype = i32
        lib.theseus_wkv7_forward_ex.argtypes = [i32] * 6 + [vp] * 10 + [vp, sz, vp]
        lib.theseus_wkv7_forward_ex.restype = i32
        lib.theseus_wkv7_backward_ex.argtypes = [i32] * 6 + [vp] * 16 + [vp, sz, vp]
        lib.theseus_wkv7_backward_ex.restype = i32
        lib.theseus_wkv7_workspace_size_ex.argtypes = [i32] * 7
        lib.theseus_wkv7_workspace_size_ex.restype = sz
        lib.theseus_wkv7_kernel_family.argtypes = [i32] * 5
        lib.theseus_wkv7_kernel_family.restype = i32
        lib.theseus_wkv7_wait_timeouts.argtypes = [ctypes.POINTER(ctypes.c_uint), i32]
        lib.theseus_wkv7_wait_timeouts.restype = i32
        lib.theseus_wkv7_set_waits.argtypes = [i32]
        lib.theseus_wkv7_set_waits.restype = i32
        # chunked gated-delta-rule forward (include/theseus_gdn.h)
        lib.theseus_gdn_forward.argtypes = [i32] * 6 + [vp] * 8 + [vp, sz, vp]
        lib.theseus_gdn_forward.restype = i32
        lib.theseus_gdn_forward_workspace_size.argtypes = [i32] * 4
        lib.theseus_gdn_forward_workspace_size.restype = sz
        lib.theseus_gdn_forward_train.argtypes = [i32] * 5 + [vp] * 9 + [vp, sz, vp]
        lib.theseus_gdn_forward_train.restype = i32
        lib.theseus_gdn_backward.argtypes = [i32] * 5 + [vp] * 14 + [vp, sz, vp]
        lib.theseus_gdn_backward.restype = i32
        lib.theseus_gdn_backward_workspace_size.argtypes = [i32] * 4
        lib.theseus_gdn_backward_workspace_size.restype = sz
        self.abi_version = lib.theseus_wkv7_abi_version()
        self.checkpoint_interval = lib.theseus_wkv7_checkpoint_interval()

    # -- helpers ---------------------------------------------------------
    def checkpoint_count(self, T):
        return int(self.lib.theseus_wkv7_checkpoint_count(T))

    def kernel_family(self, B, T, H, N, dtype):
        """theseus_wkv7_family code of a call (0: chunked MFMA kernels)."""
        return int(self.lib.theseus_wkv7_kernel_family(B, T, H, N, dtype))

    def _warn_fallback(self, B, T, H, N, dt):
        """Say so when a call runs on the step-serial kernels (exact, but one step at a
        time: ~75x slower than the chunked kernels at config 2).  THESEUS_WKV7_STRICT=1
        turns the warning into an error; THESEUS_WKV7_FAMILY=seq (an explicit request)
        is silent."""
        reason = _FALLBACK_REASON.get(self.kernel_family(B, T, H, N, dt))
        if reason is None:
            return
        msg = (f"theseus_wkv7: {reason} -> the step-serial kernels run this call "
               f"(B={B} T={T} H={H} N={N}); bf16 with N=64 or N=128 runs on the chunked MFMA kernels")
        if os.environ.get("THESEUS_WKV7_STRICT", "") == "1":
            raise RuntimeError(msg)
        warnings.warn(msg, RuntimeWarning, stacklevel=4)

    def _layout(self, B, T, H, N, dt, flags):
        """Order of the saved states a forward writes: "tiled" on the chunked kernels
        (every state but the last in their register tiling), "rows" ([value][key]) on the
        step-serial kernels.  The backward must read them with the family that wrote them."""
        return "rows" if flags or self.kernel_family(B, T, H, N, dt) else "tiled"

    def _raise(self, status):
        if status:
            msg = self.lib.theseus_wkv7_error_string(status).decode()
            raise RuntimeError(f"theseus_wkv7: {msg}")

    def wait_timeouts(self, reset=True):
        """Time-outs of the chunked kernels' bounded waits on the current device since the
        last reset (theseus_wkv7_wait_timeouts; synchronises the device).  A time-out
        leaves NaN where the result depended on the wait."""
        n = ctypes.c_uint(0)
        self._raise(self.lib.theseus_wkv7_wait_timeouts(ctypes.byref(n), 1 if reset else 0))
        return int(n.value)

    def set_waits(self, on):
        """Test hook (theseus_wkv7_set_waits): with on=False every bounded wait of the
        chunked kernels gives up at once, forcing the time-out path."""
        self._raise(self.lib.theseus_wkv7_set_waits(1 if on else 0))

    def _check_waits(self, device):
        """THESEUS_WKV7_CHECK_WAITS=1: after each call, synchronise and raise if a bounded
        wait timed out (a debug mode: it stalls the host on every call)."""
        if os.environ.get("THESEUS_WKV7_CHECK_WAITS", "") == "1":
            with _on(device):
                n = self.wait_timeouts(reset=True)
            if n:
                raise RuntimeError(f"theseus_wkv7: {n} bounded wait(s) timed out in the chunked kernels; "
                                   "the outputs hold NaN where they depended on them")

    @staticmethod
    def _check(r, xs):
        """Mirror of check() in kernels/wkv7_state.cpp:10-15 (same messages)."""
        if not (r.is_cuda and r.is_contiguous() and r.dim() == 4):
            raise RuntimeError("expected contiguous CUDA [B,T,H,N]")
        if not (r.size(1) > 0 and 2 <= r.size(3) <= 128):
            raise RuntimeError("invalid T or head size (2..128)")
        if r.dtype not in (torch.bfloat16, torch.float32):
            raise RuntimeError("expected BF16 or FP32")
        for x in xs:
            if not (x.device == r.device and x.shape == r.shape and x.dtype == r.dtype
                    and x.is_contiguous()):
                raise RuntimeError("input mismatch")

    # -- reference-compatible entry points --------------------------------
    def forward(self, r, w, k, v, a, b, s0, save_history, flags=0):
        """-> [y, end, saved]; saved is empty when save_history is False (cpp:16-25).
        ``flags`` (DECAY_EXP, STATE_KEY_VALUE) selects theseus_wkv7_forward_ex."""
        self._check(r, (w, k, v, a, b))
        B, T, H, N = r.shape
        if not (s0.device == r.device and s0.dtype == torch.float32 and s0.is_contiguous()):
            raise RuntimeError("s0 must be contiguous CUDA FP32")
        if tuple(s0.shape) != (B, H, N, N):
            raise RuntimeError("invalid s0 shape")
        with _on(r.device):
            y = torch.empty_like(r)
            end = torch.empty_like(s0)
            if save_history:
                saved = torch.empty((B, H, self.checkpoint_count(T), N, N),
                                    dtype=torch.float32, device=r.device)
            else:
                saved = torch.empty((0,), dtype=torch.float32, device=r.device)
            dt = _BF16 if r.dtype == torch.bfloat16 else _FP32
            ck = _ptr(saved) if save_history else ctypes.c_void_p(0)
            if flags:
                ws, ws_bytes = _workspace(int(self.lib.theseus_wkv7_workspace_size_ex(B, T, H, N, dt, flags, 0)),
                                          r.device)
                status = self.lib.theseus_wkv7_forward_ex(
                    B, T, H, N, dt, flags, *map(_ptr, (r, w, k, v, a, b, s0, y, end)), ck, _ptr(ws),
                    ctypes.c_size_t(ws_bytes), _stream(r.device))
            else:
                if T > 1 or save_history:  # (a T=1 step without saved states runs the single-step kernel)
                    self._warn_fallback(B, T, H, N, dt)
                ws, ws_bytes = _workspace(int(self.lib.theseus_wkv7_forward_workspace_size(B, T, H, N, dt)),
                                          r.device)
                status = self.lib.theseus_wkv7_forward(
                    B, T, H, N, dt, *map(_ptr, (r, w, k, v, a, b, s0, y, end)), ck, _ptr(ws),
                    ctypes.c_size_t(ws_bytes), _stream(r.device))
        self._raise(status)
        self._check_waits(r.device)
        if save_history:
            saved.theseus_layout = self._layout(B, T, H, N, dt, flags)
        return [y, end, saved]

    def gdn_forward(self, q, k, v, g, beta, s0, qk_l2norm=False):
        """Gated delta rule forward on the chunked kernels (theseus_gdn_forward): q, k, v
        [B,T,H,N] CUDA tensors of one dtype (bfloat16 or float32), g, beta [B,T,H] and s0
        [B,H,key,value] float32; N = 64 or 128.  qk_l2norm: L2-normalise q and k in the
        kernel (use_qk_l2norm_in_kernel).  q is scaled by 1/sqrt(N) inside.  Returns
        (o [B,T,H,N] in q's dtype, sT float32)."""
        B, T, H, N = q.shape
        if q.dtype not in (torch.bfloat16, torch.float32):
            raise RuntimeError("theseus_gdn: expected bfloat16 or float32 q, k, v")
        for x in (q, k, v):
            if not (x.is_cuda and x.dtype == q.dtype and x.is_contiguous() and x.shape == q.shape):
                raise RuntimeError("theseus_gdn: expected contiguous CUDA q, k, v [B,T,H,N] of one dtype")
        for x in (g, beta):
            if not (x.device == q.device and x.dtype == torch.float32 and x.is_contiguous()
                    and tuple(x.shape) == (B, T, H)):
                raise RuntimeError("theseus_gdn: expected contiguous float32 g, beta [B,T,H]")
        if not (s0.device == q.device and s0.dtype == torch.float32 and s0.is_contiguous()
                and tuple(s0.shape) == (B, H, N, N)):
            raise RuntimeError("theseus_gdn: expected contiguous float32 initial state [B,H,N,N]")
        with _on(q.device):
            o = torch.empty_like(q)
            sT = torch.empty_like(s0)
            ws, nbytes = _workspace(self.lib.theseus_gdn_forward_workspace_size(B, T, H, N), q.device)
            p = lambda t: t.data_ptr()  # noqa: E731
            self._raise(self.lib.theseus_gdn_forward(
                B, T, H, N, _BF16 if q.dtype == torch.bfloat16 else _FP32, 1 if qk_l2norm else 0, p(q), p(k), p(v), p(g), p(beta), p(s0),
                p(o), p(sT), None if ws is None else p(ws), nbytes, _stream(q.device)))
        return o, sT

    @staticmethod
    def _gdn_check(q, k, v, g, beta, s0):
        B, T, H, N = q.shape
        if q.dtype not in (torch.bfloat16, torch.float32):
            raise RuntimeError("theseus_gdn: expected bfloat16 or float32 q, k, v")
        for x in (q, k, v):
            if not (x.is_cuda and x.dtype == q.dtype and x.is_contiguous() and x.shape == q.shape):
                raise RuntimeError("theseus_gdn: expected contiguous CUDA q, k, v [B,T,H,N] of one dtype")
        for x in (g, beta):
            if not (x.device == q.device and x.dtype == torch.float32 and x.is_contiguous()
                    and tuple(x.shape) == (B, T, H)):
                raise RuntimeError("theseus_gdn: expected contiguous float32 g, beta [B,T,H]")
        if s0 is not None and not (s0.device == q.device and s0.dtype == torch.float32 and s0.is_contiguous()
                                   and tuple(s0.shape) == (B, H, N, N)):
            raise RuntimeError("theseus_gdn: expected contiguous float32 state [B,H,N,N]")

    def gdn_forward_train(self, q, k, v, g, beta, s0):
        """The gated delta rule forward of a call that needs gradients
        (theseus_gdn_forward_train): q and k used as given, and the saved states for
        ``gdn_backward``.  Returns (o in q's dtype, sT, saved [B,H,ceil(T/16)+1,N,N])."""
        self._gdn_check(q, k, v, g, beta, s0)
        B, T, H, N = q.shape
        with _on(q.device):
            o = torch.empty_like(q)
            sT = torch.empty_like(s0)
            saved = torch.empty((B, H, self.checkpoint_count(T), N, N), dtype=torch.float32, device=q.device)
            ws, nbytes = _workspace(self.lib.theseus_gdn_forward_workspace_size(B, T, H, N), q.device)
            p = lambda t: t.data_ptr()  # noqa: E731
            self._raise(self.lib.theseus_gdn_forward_train(
                B, T, H, N, _BF16 if q.dtype == torch.bfloat16 else _FP32, p(q), p(k), p(v), p(g), p(beta), p(s0),
                p(o), p(sT), p(saved), None if ws is None else p(ws), nbytes, _stream(q.device)))
        return o, sT, saved

    def gdn_backward(self, q, k, v, g, beta, saved, dout, dsT):
        """Backward of ``gdn_forward_train`` (theseus_gdn_backward, N = 128): dout in q's
        dtype, dsT [B,H,key,value] float32 or None.  Returns (dq, dk, dv in q's dtype, dg,
        dbeta [B,T,H] and ds0 [B,H,key,value] float32)."""
        self._gdn_check(q, k, v, g, beta, dsT)
        B, T, H, N = q.shape
        if not (dout.dtype == q.dtype and dout.is_contiguous() and dout.shape == q.shape
                and dout.device == q.device):
            raise RuntimeError("theseus_gdn: expected a contiguous output gradient like q")
        if not (saved.dtype == torch.float32 and saved.is_contiguous() and saved.device == q.device
                and tuple(saved.shape) == (B, H, self.checkpoint_count(T), N, N)):
            raise RuntimeError("theseus_gdn: invalid saved states")
        with _on(q.device):
            dq, dk, dv = (torch.empty_like(q) for _ in range(3))
            dg, dbeta = torch.empty_like(g), torch.empty_like(beta)
            ds0 = torch.empty((B, H, N, N), dtype=torch.float32, device=q.device)
            ws, nbytes = _workspace(self.lib.theseus_gdn_backward_workspace_size(B, T, H, N), q.device)
            p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
            self._raise(self.lib.theseus_gdn_backward(
                B, T, H, N, _BF16 if q.dtype == torch.bfloat16 else _FP32, p(q), p(k), p(v), p(g), p(beta),
                p(saved), p(dout), p(dsT), p(dq), p(dk), p(dv), p(dg), p(dbeta), p(ds0), p(ws), nbytes,
                _stream(q.device)))
        return dq, dk, dv, dg, dbeta, ds0

    def backward(self, r, w, k, v, a, b, saved, dy, dend, flags=0, layout=None):
        """-> [dr, dw, dk, dv, da, db, ds0] (cpp:26-37).  dend may be None (zero).
        ``flags`` must be those of the forward that made ``saved``; ``layout`` (default:
        the one that forward recorded on ``saved``) is the saved states' order, and a
        call that would read them with the other kernel family (THESEUS_WKV7_FAMILY
        changed in between) raises instead of returning wrong gradients."""
        self._check(r, (w, k, v, a, b, dy))
        B, T, H, N = r.shape
        layout = layout if layout is not None else getattr(saved, "theseus_layout", None)
        if layout is not None and layout != self._layout(B, T, H, N, _BF16 if r.dtype == torch.bfloat16 else _FP32,
                                                         flags):
            raise RuntimeError("saved states were written by the other kernel family (their order differs); "
                               "run the backward with the forward's THESEUS_WKV7_FAMILY")
        if not (saved.device == r.device and saved.dtype == torch.float32
                and saved.is_contiguous()
                and tuple(saved.shape) == (B, H, self.checkpoint_count(T), N, N)):
            raise RuntimeError("invalid history")
        if dend is not None and not (dend.device == r.device and dend.dtype == torch.float32
                                     and dend.is_contiguous()
                                     and tuple(dend.shape) == (B, H, N, N)):
            raise RuntimeError("invalid dend")
        with _on(r.device):
            grads = [torch.empty_like(r) for _ in range(6)]
            ds0 = torch.empty((B, H, N, N), dtype=torch.float32, device=r.device)
            dt = _BF16 if r.dtype == torch.bfloat16 else _FP32
            ptrs = map(_ptr, (r, w, k, v, a, b, saved, dy, dend, *grads, ds0))
            if flags:
                ws, ws_bytes = _workspace(int(self.lib.theseus_wkv7_workspace_size_ex(B, T, H, N, dt, flags, 1)),
                                          r.device)
                status = self.lib.theseus_wkv7_backward_ex(B, T, H, N, dt, flags, *ptrs, _ptr(ws),
                                                           ctypes.c_size_t(ws_bytes), _stream(r.device))
            else:
                self._warn_fallback(B, T, H, N, dt)
                ws, ws_bytes = _workspace(int(self.lib.theseus_wkv7_backward_workspace_size(B, T, H, N, dt)),
                                          r.device)
                status = self.lib.theseus_wkv7_backward(B, T, H, N, dt, *ptrs, _ptr(ws),
                                                        ctypes.c_size_t(ws_bytes), _stream(r.device))
        self._raise(status)
        self._check_waits(r.device)
        return grads + [ds0]

    def decode_step(self, r, w, k, v, a, b, state):
        """One step in place: r..b [B,1,H,N] (or [B,H,N]); state [B,H,N,N] fp32 is
        updated in place; returns y shaped like r."""
        xs = [x.reshape(x.shape[0], 1, x.shape[-2], x.shape[-1]) if x.dim() == 3 else x
              for x in (r, w, k, v, a, b)]
        self._check(xs[0], xs[1:])
        B, T, H, N = xs[0].shape
        if T != 1:
            raise RuntimeError("decode_step expects T == 1")
        if not (state.device == r.device and state.dtype == torch.float32
                and state.is_contiguous() and tuple(state.shape) == (B, H, N, N)):
            raise RuntimeError("invalid state")
        with _on(r.device):
            y = torch.empty_like(r)
            status = self.lib.theseus_wkv7_decode_step(
                B, H, N, _BF16 if r.dtype == torch.bfloat16 else _FP32,
                *map(_ptr, (*xs, state, y)), _stream(r.device))
        self._raise(status)
        return y


@lru_cache(maxsize=1)
def extension():
    """Load libtheseus_wkv7.so (built by ``make -C rwkv-theseus_amd/csrc``).

    Counterpart of the reference's lru-cached JIT build (theseus/wkv7.py:31-36);
    nothing is compiled at run time here.
    """
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C rwkv-theseus_amd/csrc` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
    return Extension(ctypes.CDLL(str(LIB_PATH)))


class _WKV(torch.autograd.Function):
    """Autograd Function over the HIP kernels (theseus/wkv7.py:39-56)."""

    @staticmethod
    def forward(ctx, r, w, k, v, a, b, state):
        xs = [x.contiguous() for x in (r, w, k, v, a, b)]
        state = state.float().contiguous()
        y, end, saved = extension().forward(*xs, state, True)
        ctx.save_for_backward(*xs, saved)
        ctx.layout = saved.theseus_layout
        return y, end

    @staticmethod
    def backward(ctx, dy, dend):
        *xs, saved = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(xs[0])
        dend = None if dend is None else dend.float().contiguous()
        grads = extension().backward(*xs, saved, dy.to(xs[0].dtype).contiguous(), dend, layout=ctx.layout)
        return tuple(g.to(x.dtype) for g, x in zip(grads[:6], xs)) + (grads[6],)


def wkv7(r, w, k, v, a, b, state, backend="cuda"):
    """(y, final_state) of the recurrence (theseus/wkv7.py:59-70)."""
    if backend == "reference":
        return reference(r, w, k, v, a, b, state)
    if backend != "cuda":
        raise ValueError(f"Unknown WKV backend: {backend}")
    if not r.is_cuda:
        raise ValueError("CUDA backend requested on CPU; use backend='reference' for tests")
    if not torch.is_grad_enabled() or not any(x.requires_grad for x in (r, w, k, v, a, b, state)):
        xs = [x.contiguous() for x in (r, w, k, v, a, b)]
        y, end, _ = extension().forward(*xs, state.float().contiguous(), False)
        return y, end
    return _WKV.apply(r, w, k, v, a, b, state)


class _WKVFlags(torch.autograd.Function):
    """_WKV with theseus_wkv7_flags (the *_ex entry points)."""

    @staticmethod
    def forward(ctx, flags, r, w, k, v, a, b, state):
        xs = [x.contiguous() for x in (r, w, k, v, a, b)]
        y, end, saved = extension().forward(*xs, state.float().contiguous(), True, flags=flags)
        ctx.save_for_backward(*xs, saved)
        ctx.flags = flags
        ctx.layout = saved.theseus_layout
        return y, end

    @staticmethod
    def backward(ctx, dy, dend):
        *xs, saved = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(xs[0])
        dend = None if dend is None else dend.float().contiguous()
        grads = extension().backward(*xs, saved, dy.to(xs[0].dtype).contiguous(), dend, flags=ctx.flags,
                                     layout=ctx.layout)
        return (None,) + tuple(g.to(x.dtype) for g, x in zip(grads[:6], xs)) + (grads[6],)


def wkv7_ex(r, w, k, v, a, b, state, flags=0):
    """``wkv7(..., backend="cuda")`` with theseus_wkv7_flags: DECAY_EXP (d = exp(w),
    unclamped) and/or STATE_KEY_VALUE (``state`` and the returned state are
    [B,H,key,value]).  flags=0 is ``wkv7`` itself."""
    if not r.is_cuda:
        raise ValueError("CUDA backend requested on CPU; use backend='reference' for tests")
    if not torch.is_grad_enabled() or not any(x.requires_grad for x in (r, w, k, v, a, b, state)):
        xs = [x.contiguous() for x in (r, w, k, v, a, b)]
        y, end, _ = extension().forward(*xs, state.float().contiguous(), False, flags=flags)
        return y, end
    return _WKVFlags.apply(flags, r, w, k, v, a, b, state)


def decode_step_(r, w, k, v, a, b, state):
    """In-place single step for serving: updates ``state`` and returns y.

    The reference decodes by calling the forward with T=1, which allocates a
    new end state per step (kernels/wkv7_state.cpp:21); this keeps the state
    resident and rewrites it in place.
    """
    return extension().decode_step(r, w, k, v, a, b, state)
