"""Autograd wrappers over the fused TimeMix kernels of libtheseus_wkv7.so
(C ABI: include/theseus_timemix.h).

Each Function replaces one torch op chain of TimeMix.forward
(theseus/timemix.py:70-71, 75, 78-80, 83-88) and returns the same values and
gradients (to bf16 rounding) with bf16 activations:

* ``shift_lerp(x, shift, coefs)`` -> 6 mixes (r, w, k, v, a, g order);
* ``add_param(z, p)`` -> (p + z).to(bf16), the decay input w = w0 + zw as the recurrence
  takes it (theseus/timemix.py:73, 80), without the float32 [B,T,C] sum;
* ``kk_kmod(k, za, a0, k_k, k_a, N, dtype)`` -> (kw, aw, bw, kmod) where, with the gate
  a = sigmoid(a0 + za) (za the LoRA output (x_a @ a1) @ a2), kw, aw, bw are the WKV
  operands k*(1+(a-1)k_a), -kk, kk*a as [B,T,H,N] tensors of ``dtype`` and kmod carries
  what the bonus term needs to recompute the modulation;
* ``gn_bonus_gate(y, r, kmod, v, g, r_k, ln_w, ln_b, eps, out_dtype)`` -> fp32
  GroupNorm over heads + (sum r*kmod*r_k) v, times g, as ``out_dtype``.

The gate is never materialised: both kernels that read it form it from za and a0, and
the GroupNorm backward hands its part of dL/da (times a (1 - a), float32) to the kk
backward through a float32 ``carrier`` output of kk_kmod, so that dL/dza is summed in
float32 and rounded to bf16 once, as autograd does for the reference's chain.

Parameters are handed to the kernels as float32 and their gradients come back
in the parameter's dtype.
"""
from __future__ import annotations

import contextlib
import ctypes

import torch

from .wkv7 import extension

_ready = None


def _lib():
    global _ready
    lib = extension().lib
    if _ready is None:
        vp, i32, sz, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
        try:
            lib.theseus_tm_shift_lerp_fwd.argtypes = [i32] * 3 + [vp] * 4 + [vp]
            lib.theseus_tm_shift_lerp_workspace.argtypes = [i32] * 3
            lib.theseus_tm_shift_lerp_workspace.restype = sz
            lib.theseus_tm_shift_lerp_bwd.argtypes = [i32] * 3 + [vp] * 8 + [sz, vp]
            lib.theseus_tm_add_param_fwd.argtypes = [i32] * 3 + [vp] * 3 + [vp]
            lib.theseus_tm_kk_fwd.argtypes = [i32] * 3 + [vp] * 8 + [vp]
            lib.theseus_tm_kk_workspace.argtypes = [i32] * 3
            lib.theseus_tm_kk_workspace.restype = sz
            lib.theseus_tm_kk_bwd.argtypes = [i32] * 3 + [vp] * 15 + [sz, vp]
            lib.theseus_tm_gn_fwd.argtypes = [i32] * 3 + [vp] * 11 + [f32, vp, vp]
            lib.theseus_tm_gn_workspace.argtypes = [i32] * 3
            lib.theseus_tm_gn_workspace.restype = sz
            lib.theseus_tm_gn_bwd.argtypes = [i32] * 3 + [vp] * 12 + [f32] + [vp] * 11 + [sz, vp]
            lib.theseus_tm_serving_step_workspace.argtypes = [ctypes.POINTER(TmLayer), i32]
            lib.theseus_tm_serving_step_workspace.restype = sz
            lib.theseus_tm_serving_step.argtypes = [ctypes.POINTER(TmLayer), i32] + [vp] * 7 + [sz, vp]
            for n in ("shift_lerp_fwd", "shift_lerp_bwd", "add_param_fwd", "kk_fwd", "kk_bwd", "gn_fwd", "gn_bwd",
                      "serving_step"):
                getattr(lib, "theseus_tm_" + n).restype = i32
            _ready = True
        except AttributeError:
            _ready = False
    return lib if _ready else None


class TmLayer(ctypes.Structure):
    """theseus_tm_layer (include/theseus_timemix.h): a TimeMix layer's parameters as the
    native serving step reads them."""
    _fields_ = ([(n, ctypes.c_int) for n in ("C", "H", "N", "rank_w", "rank_a", "rank_g")]
                + [(n, ctypes.c_void_p) for n in ("coef", "w_r", "w_k", "w_v", "w_o", "w1t", "a1t", "g1t", "w2t",
                                                   "a2t", "g2t", "w0", "a0", "k_k", "k_a", "r_k", "ln_w", "ln_b")]
                + [("ln_eps", ctypes.c_float)])


# The fused kernels' grids index token blocks of 64 in blockIdx.y (at most 65535).
MAX_TOKENS = 65535 * 64


def available(x, head_size):
    """True when the fused kernels cover this call: bf16 CUDA activations, N = 64, and
    B*T within the kernels' grid (longer inputs take the torch op sequence)."""
    return (x.dtype == torch.bfloat16 and head_size == 64 and x.shape[-1] % 64 == 0
            and x.shape[0] * x.shape[1] <= MAX_TOKENS and _lib() is not None)


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _s(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _check(status):
    if status:
        raise RuntimeError("theseus_timemix: " + extension().lib.theseus_wkv7_error_string(status).decode())


# Derived parameter tensors -- float32 copies of parameters kept in another dtype (bf16
# serving weights) and the stacked shift-lerp coefficients -- are made afresh on every
# call, so they always hold the parameters' current values, however those were updated
# (optimizer kernels that write through raw pointers change no version counter).  Only
# inside ``param_cache(store)`` are they made once and kept in the caller's ``store``:
# a serving loop or a captured graph (theseus.serving.CapturedStep) that owns the store
# then reuses them on every token, and calls ``refresh_param_cache(store)`` after a
# weight update.  Never filled while a stream is being captured into a graph: a copy
# made under capture holds its values only once the graph has run.
_store = None  # the store of the innermost param_cache, or None


@contextlib.contextmanager
def param_cache(store):
    """Keep the derived parameter tensors made inside this context in ``store`` (a dict
    the caller owns) and reuse them; they live as long as ``store``."""
    global _store
    prev, _store = _store, store
    try:
        yield store
    finally:
        _store = prev


def refresh_param_cache(store):
    """Rewrite every derived tensor held in ``store`` in place from its parameters'
    current values (same addresses, so graphs captured over them stay valid)."""
    global _store
    prev, _store = _store, None
    try:
        with torch.no_grad():
            for _srcs, make, out in store.values():
                if isinstance(out, torch.Tensor):  # (other entries point at these tensors)
                    out.copy_(make())
    finally:
        _store = prev


def _cached(slot, srcs, make):
    store = _store
    if store is None:
        return make()
    key = (slot,) + tuple(id(t) for t in srcs)
    hit = store.get(key)
    if hit is not None:
        return hit[2]
    out = make()
    on_gpu = out.is_cuda if isinstance(out, torch.Tensor) else True
    if not (on_gpu and torch.cuda.is_current_stream_capturing()):
        store[key] = (tuple(srcs), make, out)  # (the sources stay alive with the store)
    return out


class _NativeLayer:
    """A layer's TmLayer and the tensors its pointers refer to (kept alive with it)."""

    def __init__(self, struct, keep):
        self.struct, self.keep = struct, keep


def native_layer(m):
    """The TmLayer of TimeMix ``m`` for theseus_tm_serving_step, inside a param_cache
    store: the float32 parameter vectors and stacked coefficients, bf16 [out][in] weights
    and transposed LoRAs are the store's derived copies (or the parameters themselves),
    so refresh_param_cache(store) updates what it points at in place.  Keyed by the
    parameter objects, as every derived copy."""
    from . import gemm
    C = m.width
    params = (m.x_r, m.x_w, m.x_k, m.x_v, m.x_a, m.x_g, m.receptance.weight, m.key.weight, m.value.weight,
              m.output.weight, m.w1, m.a1, m.g1, m.w2, m.a2, m.g2, m.w0, m.a0, m.k_k, m.k_a, m.r_k,
              m.ln_x.weight, m.ln_x.bias)

    def make():
        coef = _coef_matrix(params[:6], C)
        mats = [gemm._out_in(w, False) for w in params[6:10]] + [gemm._out_in(w, True) for w in params[10:16]]
        vecs = [_vec(p, C) for p in params[16:]]
        keep = (coef, *mats, *vecs)
        st = TmLayer(C, m.heads, m.head_size, m.w1.shape[1], m.a1.shape[1], m.g1.shape[1],
                     *[t.data_ptr() for t in keep], float(m.ln_x.eps))
        return _NativeLayer(st, keep + params)

    return _cached("tm_layer", params, make)


def _vec(p, C):
    if p.dtype == torch.float32:
        return p.detach().reshape(C).contiguous()
    return _cached("vec", (p,), lambda: p.detach().reshape(C).float().contiguous())


def _coef_matrix(coefs, C):
    return _cached("coefs", tuple(coefs), lambda: torch.stack([_vec(c, C) for c in coefs]).contiguous())


class _ShiftLerp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, shift, *coefs):
        B, T, C = x.shape
        x = x.contiguous()
        shift = shift.to(x.dtype).contiguous()
        cf = _coef_matrix(coefs, C)
        outs = [torch.empty_like(x) for _ in range(6)]
        arr = (ctypes.c_void_p * 6)(*[o.data_ptr() for o in outs])
        with torch.cuda.device(x.device):
            _check(_lib().theseus_tm_shift_lerp_fwd(B, T, C, _p(x), _p(shift), _p(cf), arr, _s(x.device)))
        ctx.save_for_backward(x, shift, cf)
        ctx.coef_meta = [(c.shape, c.dtype) for c in coefs]
        ctx.shift_dtype = shift.dtype
        return tuple(outs)

    @staticmethod
    def backward(ctx, *douts):
        x, shift, cf = ctx.saved_tensors
        B, T, C = x.shape
        ds = [(d if d is not None else torch.zeros_like(x)).to(x.dtype).contiguous() for d in douts]
        dx = torch.empty_like(x)
        dshift = torch.empty_like(shift)
        dcoef = torch.empty(6, C, dtype=torch.float32, device=x.device)
        lib = _lib()
        ws_bytes = int(lib.theseus_tm_shift_lerp_workspace(B, T, C))
        ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=x.device)
        arr = (ctypes.c_void_p * 6)(*[d.data_ptr() for d in ds])
        with torch.cuda.device(x.device):
            _check(lib.theseus_tm_shift_lerp_bwd(B, T, C, arr, _p(x), _p(shift), _p(cf), _p(dx), _p(dshift),
                                                 _p(dcoef), _p(ws), ctypes.c_size_t(ws_bytes), _s(x.device)))
        dcs = [dcoef[n].reshape(shape).to(dt) for n, (shape, dt) in enumerate(ctx.coef_meta)]
        return (dx, dshift, *dcs)


def shift_lerp(x, shift, coefs):
    return _ShiftLerp.apply(x, shift, *coefs)


def _add_param_fwd(z, p):
    B, T, C = z.shape
    zs = z.to(torch.bfloat16).contiguous()
    out = torch.empty_like(zs)
    with torch.cuda.device(z.device):
        _check(_lib().theseus_tm_add_param_fwd(B, T, C, _p(zs), _p(_vec(p, C)), _p(out), _s(z.device)))
    return out


class _AddParam(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z, p):
        ctx.meta = (z.dtype, p.shape, p.dtype)
        return _add_param_fwd(z, p)

    @staticmethod
    def backward(ctx, dout):
        # as the reference's float32 add and cast: dL/dz is dL/dw, dL/dp its float32 sum
        z_dt, p_shape, p_dt = ctx.meta
        dp = torch.sum(dout, dim=(0, 1), dtype=torch.float32)
        return dout.to(z_dt), dp.reshape(p_shape).to(p_dt)


def add_param(z, p):
    """(p + z).to(bf16) for a bf16 [B,T,C] tensor z and a parameter p with C elements."""
    if torch.is_grad_enabled() and (z.requires_grad or p.requires_grad):
        return _AddParam.apply(z, p)
    return _add_param_fwd(z, p)  # (serving: no autograd node per token)


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in ts)


def _kk_fwd(k, za, a0, k_k, k_a, N, dtype):
    B, T, C = k.shape
    k = k.to(torch.bfloat16).contiguous()
    zs = za.to(torch.bfloat16).contiguous()
    a0v, kk_, ka = _vec(a0, C), _vec(k_k, C), _vec(k_a, C)
    kw, aw, bw = (torch.empty((B, T, C // N, N), dtype=torch.bfloat16, device=k.device) for _ in range(3))
    with torch.cuda.device(k.device):
        _check(_lib().theseus_tm_kk_fwd(B, T, C, _p(k), _p(zs), _p(a0v), _p(kk_), _p(ka), _p(kw), _p(aw),
                                        _p(bw), _s(k.device)))
    if dtype != torch.bfloat16:
        kw, aw, bw = kw.to(dtype), aw.to(dtype), bw.to(dtype)
    return (k, zs, a0v, kk_, ka), (kw, aw, bw)


class _KkKmod(torch.autograd.Function):
    @staticmethod
    def forward(ctx, k, za, a0, k_k, k_a, N, dtype):
        B, T, C = k.shape
        saved, (kw, aw, bw) = _kk_fwd(k, za, a0, k_k, k_a, N, dtype)
        ctx.save_for_backward(*saved)
        ctx.meta = (za.dtype, a0.shape, a0.dtype, k_k.shape, k_k.dtype, k_a.shape, k_a.dtype)
        # the channel through which gn_bonus_gate's backward returns its part of dL/da
        # (times a (1 - a)): a [B,T,C] float32 placeholder whose one element is never read
        # (so nothing is launched to fill it)
        carrier = torch.empty((), dtype=torch.float32, device=k.device).expand(B, T, C)
        return kw, aw, bw, carrier

    @staticmethod
    def backward(ctx, dkw, daw, dbw, dzg):
        k, zs, a0v, kk_, ka = ctx.saved_tensors
        B, T, C = k.shape
        z = torch.zeros(B, T, C, dtype=torch.bfloat16, device=k.device)
        g = [(d.to(torch.bfloat16).reshape(B, T, C).contiguous() if d is not None else z) for d in (dkw, daw, dbw)]
        gz = dzg.float().contiguous() if dzg is not None else None
        dk = torch.empty_like(k)
        dza = torch.empty_like(zs)
        da0, dkk, dka = (torch.empty(C, dtype=torch.float32, device=k.device) for _ in range(3))
        lib = _lib()
        ws_bytes = int(lib.theseus_tm_kk_workspace(B, T, C))
        ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=k.device)
        with torch.cuda.device(k.device):
            _check(lib.theseus_tm_kk_bwd(B, T, C, *map(_p, g), _p(k), _p(zs), _p(a0v),
                                         _p(gz) if gz is not None else ctypes.c_void_p(0), _p(kk_), _p(ka),
                                         _p(dk), _p(dza), _p(da0), _p(dkk), _p(dka), _p(ws),
                                         ctypes.c_size_t(ws_bytes), _s(k.device)))
        z_dt, a0_shape, a0_dt, kk_shape, kk_dt, ka_shape, ka_dt = ctx.meta
        return (dk, dza.to(z_dt), da0.reshape(a0_shape).to(a0_dt), dkk.reshape(kk_shape).to(kk_dt),
                dka.reshape(ka_shape).to(ka_dt), None, None)


def kk_kmod(k, za, a0, k_k, k_a, N, dtype):
    """WKV operands (kw, aw, bw) as [B,T,H,N], with a = sigmoid(a0 + za), plus what the
    bonus term needs (gn_bonus_gate)."""
    if not _needs_grad(k, za, a0, k_k, k_a):  # (serving: no autograd node, no carrier)
        return (*_kk_fwd(k, za, a0, k_k, k_a, N, dtype)[1], _KMod(k, za, a0, k_a, None))
    kw, aw, bw, carrier = _KkKmod.apply(k, za, a0, k_k, k_a, N, dtype)
    return kw, aw, bw, _KMod(k, za, a0, k_a, carrier)


class _KMod:
    """Carries (k, za, a0, k_a) to gn_bonus_gate, which recomputes a and k*(1+(a-1)k_a)
    itself, and the carrier through which its part of dL/da reaches kk_kmod's backward."""

    def __init__(self, k, za, a0, k_a, carrier):
        self.k, self.za, self.a0, self.k_a, self.carrier = k, za, a0, k_a, carrier


def _gn_fwd(y, r, k, za, a0, k_a, v, g, r_k, ln_w, ln_b, eps):
    B, T, C = r.shape
    bf = torch.bfloat16
    ys = y.reshape(B, T, C).to(bf).contiguous()
    rs, ks, zs, vs, gs = (t.to(bf).contiguous() for t in (r, k, za, v, g))
    a0v, ka, rk, lw, lb = _vec(a0, C), _vec(k_a, C), _vec(r_k, C), _vec(ln_w, C), _vec(ln_b, C)
    out = torch.empty(B, T, C, dtype=bf, device=r.device)
    with torch.cuda.device(r.device):
        _check(_lib().theseus_tm_gn_fwd(B, T, C, _p(ys), _p(rs), _p(ks), _p(zs), _p(a0v), _p(ka), _p(vs),
                                        _p(gs), _p(rk), _p(lw), _p(lb), ctypes.c_float(eps), _p(out),
                                        _s(r.device)))
    return (ys, rs, ks, zs, a0v, ka, vs, gs, rk, lw, lb), out


class _GnBonusGate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, r, k, carrier, za, a0, k_a, v, g, r_k, ln_w, ln_b, eps, out_dtype):
        bf = torch.bfloat16
        saved, out = _gn_fwd(y, r, k, za, a0, k_a, v, g, r_k, ln_w, ln_b, eps)
        ctx.save_for_backward(*saved)
        ctx.eps = eps
        ctx.meta = [(t.shape, t.dtype) for t in (y, r, k, k_a, v, g, r_k, ln_w, ln_b)]
        return out if out_dtype == bf else out.to(out_dtype)

    @staticmethod
    def backward(ctx, dout):
        ys, rs, ks, zs, a0v, ka, vs, gs, rk, lw, lb = ctx.saved_tensors
        B, T, C = rs.shape
        do = dout.to(torch.bfloat16).contiguous()
        dy, dr, dk, dv, dg = (torch.empty_like(rs) for _ in range(5))
        dzg = torch.empty(B, T, C, dtype=torch.float32, device=rs.device)
        drk, dlw, dlb, dka = (torch.empty(C, dtype=torch.float32, device=rs.device) for _ in range(4))
        lib = _lib()
        ws_bytes = int(lib.theseus_tm_gn_workspace(B, T, C))
        ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=rs.device)
        with torch.cuda.device(rs.device):
            _check(lib.theseus_tm_gn_bwd(B, T, C, _p(do), _p(ys), _p(rs), _p(ks), _p(zs), _p(a0v), _p(ka), _p(vs),
                                         _p(gs), _p(rk), _p(lw), _p(lb), ctypes.c_float(ctx.eps), _p(dy), _p(dr),
                                         _p(dk), _p(dv), _p(dg), _p(dzg), _p(drk), _p(dlw), _p(dlb), _p(dka),
                                         _p(ws), ctypes.c_size_t(ws_bytes), _s(rs.device)))
        y_, r_, k_, ka_, v_, g_, rk_, lw_, lb_ = [gr.reshape(shape).to(dt) for gr, (shape, dt) in
                                                  zip([dy, dr, dk, dka, dv, dg, drk, dlw, dlb], ctx.meta)]
        # za's and a0's share of the gradient goes to kk_kmod's backward through the carrier
        return (y_, r_, k_, dzg if ctx.needs_input_grad[3] else None, None, None, ka_, v_, g_, rk_, lw_, lb_,
                None, None)


def gn_bonus_gate(y, r, kmod, v, g, r_k, ln_w, ln_b, eps, out_dtype):
    if not _needs_grad(y, r, kmod.k, kmod.za, kmod.a0, kmod.k_a, v, g, r_k, ln_w, ln_b):
        out = _gn_fwd(y, r, kmod.k, kmod.za, kmod.a0, kmod.k_a, v, g, r_k, ln_w, ln_b, eps)[1]
        return out if out_dtype == torch.bfloat16 else out.to(out_dtype)
    return _GnBonusGate.apply(y, r, kmod.k, kmod.carrier, kmod.za, kmod.a0, kmod.k_a, v, g, r_k, ln_w, ln_b,
                              eps, out_dtype)
