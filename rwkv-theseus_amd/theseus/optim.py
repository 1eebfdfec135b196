"""Fused optimizer step after backward for TimeMix's float32 parameters on MI355X.

The reference updates each student layer after its backward with three torch steps
(train.py:202-208, optimizer from theseus/stage.py:39-42):

    for p in params: p.grad.mul_(world / count)
    norm = clip_grad_norm_(params, clip_norm, error_if_nonfinite=True)
    optimizer.step()        # torch.optim.AdamW(fused=True), groups decay / no decay

``FusedAdamW.step_after_backward(grad_scale, max_norm)`` does the same in one call of
``theseus_adamw_step`` (include/theseus_optim.h): per-chunk float64 sums of squared
gradients, a fixed-order final sum that forms the norm, the clip factor and a
non-finite flag in device memory, and the AdamW update reading that factor -- no
host synchronisation before the update, no scaled or clipped gradient written back,
deterministic results.  ``step()`` is plain AdamW (no scale, no clip), so the class is
also a drop-in ``torch.optim.AdamW`` for float32 CUDA parameters; its state uses
AdamW's keys ("step", "exp_avg", "exp_avg_sq"), so optimizer checkpoints keep their
format (theseus/checkpoint.py saves ``optimizer.state_dict()``), and LR schedulers
work on ``param_groups`` as usual.
"""
from __future__ import annotations

import ctypes
import math

import torch

from .wkv7 import extension


class _Tensor(ctypes.Structure):  # theseus_adamw_tensor
    _fields_ = [("param", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("exp_avg", ctypes.c_void_p),
                ("exp_avg_sq", ctypes.c_void_p), ("numel", ctypes.c_longlong), ("lr", ctypes.c_float),
                ("weight_decay", ctypes.c_float), ("step_size", ctypes.c_float),
                ("bias_correction2_sqrt", ctypes.c_float)]


_bound = None


def _lib():
    global _bound
    lib = extension().lib
    if _bound is None:
        lib.theseus_adamw_workspace_size.argtypes = [ctypes.POINTER(_Tensor), ctypes.c_int]
        lib.theseus_adamw_workspace_size.restype = ctypes.c_size_t
        lib.theseus_adamw_step.argtypes = ([ctypes.POINTER(_Tensor), ctypes.c_int] + [ctypes.c_float] * 5
                                           + [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                              ctypes.c_void_p])
        lib.theseus_adamw_step.restype = ctypes.c_int
        _bound = True
    return lib


NONFINITE_MSG = ("The total norm of order 2.0 for gradients from `parameters` is non-finite, so it cannot be "
                 "clipped. To disable this error and scale the gradients by the non-finite norm anyway, set "
                 "`error_if_nonfinite=False`")


class FusedAdamW(torch.optim.Optimizer):
    """AdamW over float32 CUDA parameters with the reference's post-backward step fused in."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta parameters: {betas}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))

    # -- the tensor list ------------------------------------------------------------------
    def _entries(self):
        hyper, entries, keep, device = None, [], [], None
        for group in self.param_groups:
            h = (float(group["betas"][0]), float(group["betas"][1]), float(group["eps"]))
            if hyper is None:
                hyper = h
            elif h != hyper:
                raise ValueError("FusedAdamW: all parameter groups must share betas and eps")
            for p in group["params"]:
                if p.grad is None:
                    continue
                g = p.grad
                if not (p.is_cuda and p.dtype == torch.float32 and p.is_contiguous()):
                    raise RuntimeError("FusedAdamW: parameters must be contiguous float32 CUDA tensors")
                if g.is_sparse or not (g.dtype == torch.float32 and g.is_contiguous() and g.shape == p.shape
                                       and g.device == p.device):
                    raise RuntimeError("FusedAdamW: gradients must be dense contiguous float32 like the parameter")
                if device is None:
                    device = p.device
                elif p.device != device:
                    raise RuntimeError("FusedAdamW: all parameters must be on one device")
                st = self.state[p]
                if not st:
                    st["step"] = torch.tensor(0.0)
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                elif st["step"].device.type != "cpu":  # e.g. loaded from torch's fused AdamW
                    st["step"] = st["step"].detach().float().cpu()
                step = float(st["step"]) + 1.0
                lr, wd = float(group["lr"]), float(group["weight_decay"])
                bc1 = 1.0 - hyper[0] ** step
                bc2 = 1.0 - hyper[1] ** step
                entries.append(_Tensor(p.data_ptr(), g.data_ptr(), st["exp_avg"].data_ptr(),
                                       st["exp_avg_sq"].data_ptr(), p.numel(), lr, wd, lr / bc1, math.sqrt(bc2)))
                keep.append(st)
        return hyper, entries, keep, device

    def _run(self, grad_scale, max_norm, error_if_nonfinite):
        hyper, entries, states, device = self._entries()
        if not entries:
            return None
        lib = _lib()
        arr = (_Tensor * len(entries))(*entries)
        norm_mode = max_norm is not None
        ws_bytes = int(lib.theseus_adamw_workspace_size(arr, len(entries))) if norm_mode else 0
        ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=device)
        result = torch.empty(3, dtype=torch.float32, device=device)
        with torch.cuda.device(device):
            status = lib.theseus_adamw_step(
                arr, len(entries), float(grad_scale), float(max_norm) if norm_mode else -1.0,
                hyper[0], hyper[1], hyper[2], 1 if error_if_nonfinite else 0,
                ctypes.c_void_p(result.data_ptr()), ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws_bytes),
                ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
        if status:
            raise RuntimeError("theseus_adamw: " + lib.theseus_wkv7_error_string(status).decode())
        if norm_mode and error_if_nonfinite and bool(result[2].item()):
            raise RuntimeError(NONFINITE_MSG)  # (the kernels left every parameter unchanged)
        for st in states:
            st["step"] += 1.0
        return result[0] if norm_mode else None

    # -- public ----------------------------------------------------------------------------
    @torch.no_grad()
    def step(self, closure=None):
        """torch.optim.AdamW's step for every parameter with a gradient."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._run(1.0, None, False)
        return loss

    @torch.no_grad()
    def step_after_backward(self, grad_scale=1.0, max_norm=None, error_if_nonfinite=True):
        """The reference's ``p.grad.mul_(grad_scale)`` loop, ``clip_grad_norm_(params,
        max_norm, error_if_nonfinite)`` and ``step()`` in one fused call
        (train.py:202-208).  Returns the total norm of the scaled gradients as a 0-d
        CUDA tensor, like clip_grad_norm_ (None when ``max_norm`` is None: no clipping
        and no norm).  The gradients themselves are left as they were.  With
        ``error_if_nonfinite`` a non-finite norm raises clip_grad_norm_'s RuntimeError
        and no parameter, moment or step count changes (this reads one flag back, a
        synchronisation the reference makes too); otherwise the update runs with the
        non-finite factor, as in torch."""
        return self._run(grad_scale, max_norm, error_if_nonfinite)
