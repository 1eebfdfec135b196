"""Gated delta rule (the GDN layers of the reference's Qwen3.5 teacher) on the WKV7
kernels in exp-decay mode.

The reference runs its teacher's GDN layers through transformers' torch functions
(``torch_chunk_gated_delta_rule`` / ``torch_recurrent_gated_delta_rule``, wrapped at
theseus/hf_model.py:28-52).  Its converter states the same recurrence as a WKV7 call
(convert_qwen2rwkv_lightning.py:381-385):

    decay d = exp(g), no clamp or sigmoid          ("wkv_decay_operation")
    r = q/sqrt(Dk), w = g, k = k, v = beta*v, a = k, b = -exp(g)*beta*k   ("wkv_inputs")
    state [B, Hv, K, V]                            ("gdn_state_layout")

``gated_delta_rule`` maps GDN's inputs that way and calls the HIP kernels through
``theseus_wkv7_forward_ex`` / ``_backward_ex`` with THESEUS_WKV7_DECAY_EXP and
THESEUS_WKV7_STATE_KEY_VALUE (no state transpose); the mapping is torch ops, so autograd
carries the kernels' gradients back to q, k, v, g and beta.  When no gradient is wanted
(the teacher's forward) and the head size is 64 or 128, it runs the chunked MFMA forward
of the gated delta rule instead (``theseus_gdn_forward``, include/theseus_gdn.h); with
gradients at head size 128, the chunked forward with saved states and the chunked backward
(``theseus_gdn_forward_train`` / ``theseus_gdn_backward``).  Like transformers'
functions it computes in float32 (the operands are passed to the kernels as float32)
and returns the output in the query's dtype.  The state must be square (K == V, the
kernels' N, 2..128).

``chunk_gated_delta_rule`` and ``recurrent_gated_delta_rule`` have transformers'
signatures; ``patch_transformers(module)`` installs them into a transformers model
module (e.g. ``transformers.models.qwen3_5.modeling_qwen3_5``) for CUDA tensors,
leaving CPU calls to transformers' own functions, as the reference's wrapper does.
"""
from __future__ import annotations

import functools

import torch

from .wkv7 import DECAY_EXP, STATE_KEY_VALUE, extension, wkv7_ex

# head sizes of the chunked forward (theseus_gdn_forward); others use the step-serial kernels
CHUNKED_HEAD_SIZES = (64, 128)
# head sizes of the chunked forward+backward (theseus_gdn_forward_train, theseus_gdn_backward)
CHUNKED_GRAD_HEAD_SIZES = (128,)


class _GDN(torch.autograd.Function):
    """The gated delta rule on the chunked kernels with gradients: q, k (as the layer
    normalised them), v, g, beta, s0 float32 or q/k/v bfloat16; saved states between
    the two calls."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, s0):
        ctx.set_materialize_grads(False)
        o, sT, saved = extension().gdn_forward_train(q, k, v, g, beta, s0)
        ctx.save_for_backward(q, k, v, g, beta, saved)
        return o, sT

    @staticmethod
    def backward(ctx, do, dsT):
        q, k, v, g, beta, saved = ctx.saved_tensors
        do = torch.zeros_like(q) if do is None else do.to(q.dtype).contiguous()
        dsT = None if dsT is None else dsT.float().contiguous()
        return extension().gdn_backward(q, k, v, g, beta, saved, do, dsT)


def l2norm(x, dim=-1, eps=1e-6):
    """x * rsqrt(sum(x*x) + eps): the q/k normalisation of GDN layers
    ("gdn_qk_normalization", convert_qwen2rwkv_lightning.py:381)."""
    return x * torch.rsqrt((x * x).sum(dim=dim, keepdim=True) + eps)


def gated_delta_rule(query, key, value, g, beta, initial_state=None, output_final_state=False,
                     use_qk_l2norm_in_kernel=False):
    """query, key [B,T,H,K]; value [B,T,H,V]; g, beta [B,T,H]; initial_state [B,H,K,V]
    (zeros if None).  Returns (output [B,T,H,V] in query's dtype, final state [B,H,K,V]
    float32 or None)."""
    B, T, H, K = query.shape
    V = value.shape[-1]
    if K != V or not 2 <= K <= 128:
        raise ValueError(f"gated_delta_rule on the WKV7 kernels needs K == V in 2..128 (got K={K}, V={V})")
    if key.shape != query.shape or value.shape[:3] != (B, T, H) or g.shape != (B, T, H) or beta.shape != (B, T, H):
        raise ValueError("gated_delta_rule: expected query/key [B,T,H,K], value [B,T,H,V], g/beta [B,T,H]")
    out_dtype = query.dtype
    s0 = (torch.zeros(B, H, K, V, device=query.device, dtype=torch.float32) if initial_state is None
          else initial_state.float().contiguous())
    leaves = (query, key, value, g, beta) + (() if initial_state is None else (initial_state,))
    if (K in CHUNKED_HEAD_SIZES and not (torch.is_grad_enabled() and any(x.requires_grad for x in leaves))
            and extension().lib.theseus_gdn_forward_workspace_size(B, T, H, K) > 0):
        # no gradients wanted (the teacher's case): the chunked MFMA forward, which takes
        # bf16 or fp32 q/k/v as they are and normalises q and k itself
        io = query.dtype if query.dtype in (torch.bfloat16, torch.float32) else torch.float32
        q, k, v = (x.to(io).contiguous() for x in (query, key, value))
        o, sT = extension().gdn_forward(q, k, v, g.float().contiguous(), beta.float().contiguous(), s0,
                                        qk_l2norm=use_qk_l2norm_in_kernel)
        return o.to(out_dtype), (sT if output_final_state else None)
    if use_qk_l2norm_in_kernel:
        query, key = l2norm(query), l2norm(key)
    if (K in CHUNKED_GRAD_HEAD_SIZES and query.is_cuda
            and extension().lib.theseus_gdn_backward_workspace_size(B, T, H, K) > 0):
        # gradients wanted: the chunked forward with saved states and the chunked backward,
        # in float32 as transformers' functions compute
        q, k, v, gf, bf = (x.float().contiguous() for x in (query, key, value, g, beta))
        o, sT = _GDN.apply(q, k, v, gf, bf, s0)
        return o.to(out_dtype), (sT if output_final_state else None)
    q, k, v, gf, bf = (x.float() for x in (query, key, value, g, beta))
    eg = torch.exp(gf)
    r = q * (K ** -0.5)
    w = gf.unsqueeze(-1).expand(B, T, H, K).contiguous()
    vb = v * bf.unsqueeze(-1)
    b = -(eg * bf).unsqueeze(-1) * k
    y, sT = wkv7_ex(r, w, k, vb, k, b, s0, flags=DECAY_EXP | STATE_KEY_VALUE)
    return y.to(out_dtype), (sT if output_final_state else None)


def _no_varlen(kwargs):
    if kwargs.get("cu_seqlens") is not None:
        raise NotImplementedError("packed variable-length sequences (cu_seqlens) are not supported")


def chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False, **kwargs):
    """transformers' ``torch_chunk_gated_delta_rule`` signature (chunk_size is not used)."""
    _no_varlen(kwargs)
    return gated_delta_rule(query, key, value, g, beta, initial_state, output_final_state,
                            use_qk_l2norm_in_kernel)


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state, output_final_state,
                               use_qk_l2norm_in_kernel=False, **kwargs):
    """transformers' ``torch_recurrent_gated_delta_rule`` signature."""
    _no_varlen(kwargs)
    return gated_delta_rule(query, key, value, g, beta, initial_state, output_final_state,
                            use_qk_l2norm_in_kernel)


def _wants_grad(args, kwargs):
    return torch.is_grad_enabled() and any(
        isinstance(x, torch.Tensor) and x.requires_grad for x in list(args) + list(kwargs.values()))


def patch_transformers(module):
    """Route ``module.torch_chunk_gated_delta_rule`` / ``torch_recurrent_gated_delta_rule``
    to the HIP kernels for CUDA tensors with a square state and no packed sequences
    (cu_seqlens): without gradients for K == V <= 128 (the teacher's forward, on the
    chunked kernels for 64 and 128), with gradients for K == V == 128 (the chunked forward
    and backward); any other call goes to the function that was there -- with gradients
    at other head sizes, transformers' own chunked torch function (37 ms forward+backward
    at B=1, T=2048, H=32, K=V=128 on MI355X) beats the step-serial backward.  Returns the
    previous pair."""
    old = (module.torch_chunk_gated_delta_rule, module.torch_recurrent_gated_delta_rule)

    def route(ours, theirs):
        @functools.wraps(theirs)
        def call(query, key, value, *args, **kwargs):
            K = query.shape[-1]
            if (query.is_cuda and 2 <= K == value.shape[-1] <= 128 and kwargs.get("cu_seqlens") is None
                    and (K in CHUNKED_GRAD_HEAD_SIZES or not _wants_grad((query, key, value) + args, kwargs))):
                return ours(query, key, value, *args, **kwargs)
            return theirs(query, key, value, *args, **kwargs)
        return call

    module.torch_chunk_gated_delta_rule = route(chunk_gated_delta_rule, old[0])
    module.torch_recurrent_gated_delta_rule = route(recurrent_gated_delta_rule, old[1])
    return old
