"""Seeded synthetic WKV7 inputs with the value distributions of the benchmark
configurations (r, w-logit, k, v ~ N(0,1); kk = per-head L2-normalised
N(0,1); alpha = sigmoid(N(0,1)); a = -kk; b = kk * alpha; optional
s0 ~ N(0,1)*s0_std; dy ~ N(0,1); dsT ~ N(0,1)).

Drawn in float32 on the CPU from ``torch.Generator().manual_seed(seed)`` in
that fixed order and only then cast, so the GPU path and the CPU oracle see
identical bits.  These are the operator inputs as TimeMix produces them
(theseus/timemix.py:78-80): ``w`` is the pre-sigmoid logit, the operator
derives the decay itself.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

SEED_BASE = 20260  # seed = SEED_BASE + config id


def wkv7_inputs(B, T, H, N, seed, dtype=torch.bfloat16, s0_std=0.0, with_dsT=False):
    g = torch.Generator().manual_seed(int(seed))
    shape = (B, T, H, N)

    def randn(*s):
        return torch.randn(*s, generator=g, dtype=torch.float32)

    r = randn(*shape)
    w = randn(*shape)
    k = randn(*shape)
    v = randn(*shape)
    kk = F.normalize(randn(*shape), dim=-1, eps=1e-12)
    alpha = torch.sigmoid(randn(*shape))
    a = -kk
    b = kk * alpha
    s0 = randn(B, H, N, N) * s0_std if s0_std else torch.zeros(B, H, N, N)
    dy = randn(*shape)
    dsT = randn(B, H, N, N) if with_dsT else torch.zeros(B, H, N, N)
    xs = [x.to(dtype).contiguous() for x in (r, w, k, v, a, b)]
    return dict(r=xs[0], w=xs[1], k=xs[2], v=xs[3], a=xs[4], b=xs[5], s0=s0.contiguous(),
                dy=dy.to(dtype).contiguous(), dsT=dsT.contiguous())
