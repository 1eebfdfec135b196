"""RWKV7 TimeMix layer on MI355X (drop-in for theseus/timemix.py).

Same constructor, parameter schema (23 tensors, names and shapes), initialisation
and forward contract as the reference module (theseus/timemix.py:18-93), so state
dicts, exports and seeds carry over unchanged: the schema is what
replace_timemix_lightning.py:66-72 and the checkpoints pin, and the
initialisation calls are issued in the reference's order so a seeded
construction consumes the RNG identically.

With ``backend="cuda"`` and CUDA tensors, the elementwise work around the
recurrence runs as three fused HIP kernel pairs (theseus.fused): the token-shift
lerp that produces the six mixes (timemix.py:70-71), the kk normalisation / k
modulation that produces the WKV operands (:78-80), and the fp32 GroupNorm +
r*k*r_k bonus + gate (:83-88).  Projections and LoRAs stay torch GEMMs
(hipBLASLt).  ``backend="reference"`` runs the reference's torch op sequence
for all of it.

Credit: the parameter schema and the initialisation formulas are those of
RWKV-LM-V7's RWKV_Tmix_x070 and generate_init_weight (RWKV-Vibe/RWKV-LM-V7,
src/model.py at commit 665472dab30952de9379a3a3a01eaa3453f1ad4e, Apache-2.0),
as adapted by the reference (theseus/timemix.py:1-10: independent blocks with
no cross-layer v_first, explicit shift/WKV state, fp32 normalisation).  They
are kept as the module's contract (state dicts, seeds and exports depend on
them), under that licence.
"""
from __future__ import annotations

import math
import os

import torch
from torch import nn
from torch.nn import functional as F

from .wkv7 import decode_step_, wkv7


def _group_norm(x, groups, weight, bias, eps):
    """F.group_norm(x, groups, weight, bias, eps) for x [M, C], written out (mean, biased
    variance, affine) so that its backward is plain elementwise autograd.

    Used for GPU tensors: torch 2.10+rocm7.0's group_norm backward returns wrong weight
    and bias gradients (relative error ~1) once x has about 1024 rows or more (measured
    against float64 on the CPU: M=1024..8192 rows at 4..80 groups), which would silently
    mistrain ln_x.  Same arithmetic as the reference's call (theseus/timemix.py:84)."""
    M, C = x.shape
    xg = x.reshape(M, groups, C // groups)
    mean = xg.mean(-1, keepdim=True)
    var = (xg - mean).square().mean(-1, keepdim=True)
    return ((xg - mean) * torch.rsqrt(var + eps)).reshape(M, C) * weight + bias


def _shift_lerp_ops(x, shift, coefs):
    """The reference's token-shift lerp as torch ops (theseus/timemix.py:70-71): the six
    mixes x + (x[t-1] - x) * coef, with x[-1] = the carried shift."""
    delta = torch.cat([shift.unsqueeze(1), x[:, :-1]], 1) - x
    return [(x + delta * c).to(x.dtype) for c in coefs]


class TimeMix(nn.Module):
    def __init__(self, width, layer_idx, depth, head_size=64, backend="cuda"):
        super().__init__()
        if width % head_size or head_size < 2:
            raise ValueError("width must be divisible by head_size >= 2")
        self.width, self.head_size = width, head_size
        self.heads, self.backend = width // head_size, backend
        C, N = width, head_size
        ratio = layer_idx / max(depth - 1, 1)       # 0 at the first layer, 1 at the last
        reverse = 1 - layer_idx / depth
        pos = torch.arange(C).reshape(1, 1, C) / C  # channel position in [0, 1)
        # token-shift mix coefficients x_r, x_w, x_k, x_v, x_a, x_g
        for name, power in (("r", .2), ("w", .9), ("k", .7), ("v", .7), ("a", .9), ("g", .2)):
            setattr(self, "x_" + name, nn.Parameter(1 - pos.pow(power * reverse)))
        ramp = torch.arange(C) / (C - 1) - .5
        zz = (torch.arange(C) % N - (N - 1) / 2) / ((N - 1) / 2)
        zz = zz * zz.abs()
        decay_base = -6 + 6 * (torch.arange(C) / (C - 1)).pow(1 + ratio ** .3)
        rank = max(32, round(2.5 * math.sqrt(C) / 32) * 32)
        gate_rank = max(32, round(5 * math.sqrt(C) / 32) * 32)
        for name in ("w", "a"):
            setattr(self, name + "1", nn.Parameter(torch.zeros(C, rank)))
            lora_out = nn.Parameter(torch.empty(rank, C))
            nn.init.orthogonal_(lora_out, gain=.1 * max(1, math.sqrt(rank / C)))
            setattr(self, name + "2", lora_out)
        self.w0 = nn.Parameter((decay_base + .5 + zz * 2.5).reshape(1, 1, C))
        self.a0 = nn.Parameter((-.19 + zz * .3 + ramp * .4).reshape(1, 1, C))
        self.g1 = nn.Parameter(torch.empty(C, gate_rank))
        self.g2 = nn.Parameter(torch.empty(gate_rank, C))
        nn.init.zeros_(self.g1)  # sigmoid(0) = 0.5, so the gate starts non-zero
        nn.init.orthogonal_(self.g2, gain=.1 * max(1, math.sqrt(gate_rank / C)))
        self.k_k = nn.Parameter((.71 - ramp * .1).reshape(1, 1, C))
        self.k_a = nn.Parameter(torch.full((1, 1, C), 1.02))
        self.r_k = nn.Parameter(torch.full((self.heads, N), -.04))
        for name, gain in (("receptance", 1.), ("key", .1), ("value", 1.), ("output", 0.)):
            lin = nn.Linear(C, C, bias=False)
            if gain:
                nn.init.orthogonal_(lin.weight, gain=gain)
            else:
                nn.init.zeros_(lin.weight)
            setattr(self, name, lin)
        self.ln_x = nn.GroupNorm(self.heads, C, eps=64e-5)
        nn.init.constant_(self.ln_x.weight, ((1 + layer_idx) / depth) ** .7)

    def initial_state(self, x):
        """Zero carried state: {"shift": [B,C] in x's dtype, "wkv": [B,H,N,N] fp32}."""
        return {"shift": torch.zeros(x.shape[0], self.width, device=x.device, dtype=x.dtype),
                "wkv": torch.zeros(x.shape[0], self.heads, self.head_size, self.head_size,
                                   device=x.device, dtype=torch.float32)}

    def _fused(self, x):
        if self.backend != "cuda" or not x.is_cuda:
            return False
        from . import fused
        return fused.available(x, self.head_size)

    def _few_rows(self, x):
        """Projections on the few-row GEMM kernel (theseus.gemm): a no-grad call with at
        most gemm.MAX_ROWS tokens in all (a serving step: one token per lane) and
        kernel-compatible widths and LoRA ranks."""
        from . import gemm
        C = self.width
        ranks = (self.w1.shape[1], self.a1.shape[1], self.g1.shape[1])
        if not (all(gemm.supported(1, C, C) and gemm.supported(1, r, C) and gemm.supported(1, C, r) for r in ranks)):
            return False
        return gemm.usable(x, self.receptance.weight, self.key.weight, self.value.weight, self.output.weight,
                           self.w1, self.w2, self.a1, self.a2, self.g1, self.g2)

    def forward(self, x, state=None):
        """x [B,T,C] -> (out [B,T,C] in x.dtype, {"shift": x[:, -1], "wkv": end state})."""
        if state is None:
            state = self.initial_state(x)
        return self._run(x, state, inplace=False)

    def step_(self, x, state):
        """Serving step that carries ``state`` in place: x [B,1,C] -> out [B,1,C].

        Same value as ``forward(x, state)[0]``, but the WKV state goes through the
        single-step kernel in place (theseus_wkv7_decode_step) and ``state["shift"]`` is
        overwritten with x[:, -1], so no new state is allocated per token and the state
        tensors keep their addresses (which lets a caller capture the step into a HIP
        graph, ``theseus.serving.CapturedStep``).  The reference's serving path calls
        ``forward`` with T=1 and gets a new state back each token (theseus/hf_model.py:104-106,
        kernels/wkv7_state.cpp:21); ``forward`` keeps doing that, since callers such as
        ``isolated_state`` (hf_model.py:240-252) hold on to earlier state objects.
        Needs backend="cuda", CUDA tensors, T == 1, no autograd, and ``state`` as
        ``initial_state``/``forward`` make it (shift [B,C] in x's dtype, wkv [B,H,N,N] fp32,
        both contiguous)."""
        if self.backend != "cuda" or not x.is_cuda:
            raise ValueError("step_ needs backend='cuda' and CUDA tensors")
        if x.dim() != 3 or x.shape[1] != 1:
            raise ValueError("step_ takes one token per call: x [B,1,C]")
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            raise RuntimeError("step_ updates the state in place and has no backward; call it under "
                               "torch.no_grad() (or use forward for training)")
        B, H, N = x.shape[0], self.heads, self.head_size
        sh, wkv = state["shift"], state["wkv"]
        if not (sh.shape == (B, self.width) and sh.dtype == x.dtype and sh.is_contiguous()
                and sh.device == x.device):
            raise ValueError("state['shift'] must be a contiguous [B,C] tensor of x's dtype and device")
        if not (wkv.shape == (B, H, N, N) and wkv.dtype == torch.float32 and wkv.is_contiguous()
                and wkv.device == x.device):
            raise ValueError("state['wkv'] must be a contiguous [B,H,N,N] float32 tensor on x's device")
        return self._run(x, state, inplace=True)[0]

    def _native_ok(self, x, state):
        """A one-token no-grad step inside a parameter store (theseus.fused.param_cache:
        the serving loop's or CapturedStep's) runs as one native call
        (theseus_tm_serving_step), the same kernels the few-row path below launches.
        THESEUS_TM_NATIVE=0 keeps the launches in Python (tests compare the two)."""
        from . import fused
        if x.shape[1] != 1 or fused._store is None or os.environ.get("THESEUS_TM_NATIVE", "1") == "0":
            return False
        wkv = state["wkv"]
        if not (wkv.dtype == torch.float32 and wkv.is_contiguous() and wkv.is_cuda
                and state["shift"].dim() == 2 and self._fused(x) and self._few_rows(x)):
            return False
        return all(p.is_cuda for p in (self.w1, self.a1, self.g1, self.w2, self.a2, self.g2))

    def _native_step(self, x, state, inplace):
        import ctypes
        from . import fused, gemm
        B, _, C = x.shape
        lib = fused._lib()
        lay = fused.native_layer(self)
        xs = x.contiguous()
        shift = state["shift"].to(x.dtype).contiguous()
        wkv = state["wkv"]
        out = torch.empty((B, 1, C), dtype=x.dtype, device=x.device)
        wkv_out = wkv if inplace else torch.empty_like(wkv)
        nbytes = int(lib.theseus_tm_serving_step_workspace(ctypes.byref(lay.struct), B))
        ws = gemm._workspace(nbytes, x.device)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        with torch.cuda.device(x.device):
            fused._check(lib.theseus_tm_serving_step(
                ctypes.byref(lay.struct), B, p(xs), p(shift), p(state["shift"]) if inplace else None, p(wkv),
                p(wkv_out), p(out), p(ws), ctypes.c_size_t(ws.numel()), fused._s(x.device)))
        if inplace:
            return out, state
        return out, {"shift": x[:, -1], "wkv": wkv_out}

    def _run(self, x, state, inplace):
        B, T, _ = x.shape
        if T == 1 and self._native_ok(x, state):
            return self._native_step(x, state, inplace)
        shape = (B, T, self.heads, self.head_size)
        fused_ok = self._fused(x)
        if fused_ok:
            from . import fused
            mixed = dict(zip("rwkvag", fused.shift_lerp(
                x, state["shift"], [getattr(self, "x_" + n) for n in "rwkvag"])))
        else:
            mixed = dict(zip("rwkvag", _shift_lerp_ops(
                x, state["shift"], [getattr(self, "x_" + n) for n in "rwkvag"])))
        rows = fused_ok and self._few_rows(x)
        if rows:
            # (as the torch products under bf16 autocast, with each activation applied to the
            # float32 accumulator before the bf16 rounding)
            from . import fused, gemm
            # one launch for every product of the step's mixes (r, k, v and, where their
            # [out][in] bf16 copies are kept -- a serving store -- or a float32 -> bf16 copy is
            # made anyway, the LoRAs' first halves), one for the LoRAs' second halves
            first = [(mixed["r"], self.receptance.weight, gemm.NONE, False),
                     (mixed["k"], self.key.weight, gemm.NONE, False),
                     (mixed["v"], self.value.weight, gemm.NONE, False)]
            loras = fused._store is not None or self.w1.dtype != torch.bfloat16
            if loras:
                first += [(mixed["w"], self.w1, gemm.TANH, True), (mixed["a"], self.a1, gemm.NONE, True),
                          (mixed["g"], self.g1, gemm.SIGMOID, True)]
            outs = gemm.group(first)
            r, k, v = outs[:3]
            if loras:
                zw, za, g = gemm.group([(outs[3], self.w2, gemm.NONE, True), (outs[4], self.a2, gemm.NONE, True),
                                        (outs[5], self.g2, gemm.NONE, True)])
            else:
                zw = torch.tanh(mixed["w"] @ self.w1) @ self.w2
                za = (mixed["a"] @ self.a1) @ self.a2
                g = torch.sigmoid(mixed["g"] @ self.g1) @ self.g2
        else:
            r = self.receptance(mixed["r"])
            zw = torch.tanh(mixed["w"] @ self.w1) @ self.w2
            k, v = self.key(mixed["k"]), self.value(mixed["v"])
            za = (mixed["a"] @ self.a1) @ self.a2
            g = torch.sigmoid(mixed["g"] @ self.g1) @ self.g2
        if fused_ok:
            from . import fused
            w = fused.add_param(zw, self.w0)  # (w0 + zw) in the recurrence's bf16, in one pass
        else:
            w = self.w0 + zw
        if fused_ok:
            from . import fused
            # a = sigmoid(a0 + za) (the reference's theseus/timemix.py:75) is formed inside the kernels
            kw, aw, bw, kmod = fused.kk_kmod(k, za, self.a0, self.k_k, self.k_a, self.head_size, r.dtype)
            args = [r.reshape(shape).to(r.dtype).contiguous(), w.reshape(shape).to(r.dtype).contiguous(),
                    kw, v.reshape(shape).to(r.dtype).contiguous(), aw, bw]
        else:
            a = torch.sigmoid(self.a0 + za)
            kk = F.normalize((k.float() * self.k_k).reshape(shape), dim=-1, eps=1e-12)
            k = k * (1 + (a - 1) * self.k_a)
            args = [z.reshape(shape).to(r.dtype).contiguous()
                    for z in (r, w, k, v, -kk, kk * a.reshape(shape))]
            kmod = k
        if inplace:
            y, end = decode_step_(*args, state["wkv"]), state["wkv"]
        else:
            y, end = wkv7(*args, state["wkv"], backend=self.backend)
        if fused_ok:
            from . import fused
            out = fused.gn_bonus_gate(y, r, kmod, v, g, self.r_k, self.ln_x.weight, self.ln_x.bias,
                                      self.ln_x.eps, x.dtype)
        else:
            # norms in fp32 with autocast off, cast back for the output projection
            with torch.autocast(x.device.type, enabled=False):
                gn = _group_norm if y.is_cuda else F.group_norm
                yn = gn(y.float().reshape(B * T, self.width), self.heads,
                        self.ln_x.weight.float(), self.ln_x.bias.float(),
                        self.ln_x.eps).reshape(B, T, self.width)
                bonus = ((r.float().reshape(shape) * kmod.float().reshape(shape) * self.r_k)
                         .sum(-1, keepdim=True) * v.float().reshape(shape)).reshape(B, T, self.width)
                out = ((yn + bonus) * g.float()).to(x.dtype)
        if rows:
            from . import gemm
            out = gemm.linear(out, self.output.weight).to(x.dtype)
        else:
            out = self.output(out).to(x.dtype)
        if inplace:
            state["shift"].copy_(x[:, -1])
            return out, state
        return out, {"shift": x[:, -1], "wkv": end}


def detach_state(state):
    """Cut the graph at a chunk boundary (theseus/timemix.py:92-93)."""
    return None if state is None else {k: v.detach() for k, v in state.items()}
