"""Config 3 at full size: one TimeMix layer forward+backward, B=2, T=4096, C=5120 (H=80,
N=64), bf16 autocast over fp32 parameters, 2-D weights ~ N(0, 0.02), x ~ N(0, 1), the
reference geometry (w/a LoRA rank 192, gate rank 352; theseus/timemix.py:18-59, :66-89).

The fused path (backend="cuda": HIP WKV7 + the fused shift-lerp, kk/k-modulation and
GroupNorm/bonus/gate kernels) is compared with the same module and weights with the fused
kernels switched off, i.e. the reference's torch op sequence around the same HIP
recurrence, whose parity with the fp64 oracle the WKV7 tests pin.  Every output the layer
produces is checked at the north-star bar rel-L2 <= 5e-3: y, the carried state (wkv and
shift), the gradients of x and of both initial states, and all 23 parameter gradients.

The fused shift-lerp reproduces the reference chain's forward rounding exactly (the
difference x[t-1] - x rounded to bf16, then x + delta * coef rounded once), so the two
passes see the same operands to ~1e-5.  Its backward sums the six lerp gradients of x in
float32 and rounds once, whereas autograd on the bf16 chain sums them in bf16, which alone
moves dx and the shift gradient by 5e-3 to 2e-2 from the float32 sum.  The reference pass
therefore runs the chain's lerp through a twin with bitwise the same forward values whose
gradients accumulate in float32 (straight-through bf16 rounding of the difference): the
rest of the op sequence is the reference's, unchanged.

A second test measures both against the truth instead: the same layer in float64 (up to
config 3's size), the fused layer and the reference's own unmodified bf16 chain
(backend="reference") each compared with it; the fused layer must be as close as the
reference chain is (its float32 gradient sums make dx and dshift closer).
"""
import pytest
import torch

from conftest import rel_l2
from theseus import fused
import theseus.timemix as TM
from theseus.timemix import TimeMix

BAR = 5e-3


def _layer(seed=20263, B=2, T=4096, H=80, N=64):
    C = H * N
    torch.manual_seed(seed)
    m = TimeMix(C, 3, 8, head_size=N, backend="cuda").cuda()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() == 2 and name != "r_k":
                p.normal_(0, .02)
    assert m.w1.shape[1] == 192 and m.g1.shape[1] == 352  # the reference geometry at C=5120
    bf = torch.bfloat16
    x = torch.randn(B, T, C, device="cuda", dtype=bf)
    st = {"shift": torch.randn(B, C, device="cuda", dtype=bf),
          "wkv": .1 * torch.randn(B, H, N, N, device="cuda")}
    gy = torch.randn(B, T, C, device="cuda", dtype=bf)
    gS = torch.randn(B, H, N, N, device="cuda")
    return m, x, st, gy, gS


def _shift_lerp_fp32_grad(x, shift, coefs):
    """The reference chain's six mixes, bit for bit (delta = prev - x rounded to bf16, then
    x + delta * coef in float32 rounded to bf16), with float32 gradient accumulation."""
    xf, sf = x.float(), shift.float()
    d = torch.cat([sf.unsqueeze(1), xf[:, :-1]], 1) - xf
    d = d + (d.to(x.dtype).float() - d).detach()  # value rounded to bf16, gradient 1
    return [(xf + d * c).to(x.dtype) for c in coefs]


def _run(m, x, st, gy, gS):
    m.zero_grad(set_to_none=True)
    xx = x.detach().clone().requires_grad_()  # fresh leaves on every pass
    sh = st["shift"].detach().clone().requires_grad_()
    s0 = st["wkv"].clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, s = m(xx, {"shift": sh, "wkv": s0})
    torch.autograd.backward((y, s["wkv"]), (gy, gS))
    torch.cuda.synchronize()
    out = {"y": y.detach().float(), "state.wkv": s["wkv"].detach(), "state.shift": s["shift"].detach().float(),
           "dx": xx.grad.float(), "dshift0": sh.grad.float(), "dwkv0": s0.grad.float()}
    for n, p in m.named_parameters():
        out["grad." + n] = p.grad.detach().float().clone()
    return out


@pytest.mark.gpu
def test_config3_layer_fused_matches_torch_op_chain(monkeypatch):
    m, x, st, gy, gS = _layer()
    assert fused.available(x, 64)
    got = _run(m, x, st, gy, gS)
    monkeypatch.setattr(fused, "available", lambda *a, **k: False)
    monkeypatch.setattr(TM, "_shift_lerp_ops", _shift_lerp_fp32_grad)
    ref = _run(m, x, st, gy, gS)
    assert len([k for k in got if k.startswith("grad.")]) == 23
    worst = []
    for k in ref:
        e = rel_l2(got[k].cpu(), ref[k].cpu())
        print(f"    {k}: rel_l2 {e:.2e}", flush=True)
        if not e <= BAR:
            worst.append((k, e))
    assert not worst, worst


def test_fp32_grad_twin_has_the_reference_chain_forward():
    """The twin's mixes are bitwise the reference chain's (CPU, bf16)."""
    torch.manual_seed(9)
    x = torch.randn(2, 33, 128, dtype=torch.bfloat16)
    sh = torch.randn(2, 128, dtype=torch.bfloat16)
    coefs = [torch.rand(1, 1, 128) for _ in range(6)]
    for a, b in zip(TM._shift_lerp_ops(x, sh, coefs), _shift_lerp_fp32_grad(x, sh, coefs)):
        assert a.dtype == b.dtype == torch.bfloat16 and torch.equal(a, b)



@pytest.mark.gpu
@pytest.mark.parametrize("B,T,H", [(2, 256, 16), (2, 4096, 80)], ids=["C1024", "config3"])
def test_fused_layer_is_as_close_to_float64_as_the_reference_chain(B, T, H):
    """Against the truth rather than against each other: the same layer and inputs in
    float64 (backend="reference", no autocast) give the exact values; the fused layer
    (backend="cuda", bf16 autocast) and the reference's own unmodified bf16 chain
    (backend="reference": its torch op sequence and its float32 recurrence loop, bf16
    autocast) are each measured against them.  Every output and all 23 parameter gradients
    of the fused layer must be within 1.25 times the reference chain's own error, or within
    2e-3 rel-L2 where that error is smaller."""
    print(f"  layer vs float64: B={B} T={T} H={H}", flush=True)
    torch.manual_seed(31)
    N = 64
    C = H * N
    m = TimeMix(C, 3, 8, head_size=N, backend="cuda").cuda()
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.dim() == 2 and name != "r_k":
                p.normal_(0, .02)
    bf = torch.bfloat16
    x = torch.randn(B, T, C, device="cuda", dtype=bf)
    st = {"shift": torch.randn(B, C, device="cuda", dtype=bf), "wkv": .1 * torch.randn(B, H, N, N, device="cuda")}
    gy = torch.randn(B, T, C, device="cuda", dtype=bf)
    gS = torch.randn(B, H, N, N, device="cuda")
    fused_out = _run(m, x, st, gy, gS)
    m.backend = "reference"
    ref_out = _run(m, x, st, gy, gS)
    m64 = TimeMix(C, 3, 8, head_size=N, backend="reference").cuda().double()
    m64.load_state_dict({k: v.double() for k, v in m.state_dict().items()})
    xx = x.double().requires_grad_()
    sh = st["shift"].double().requires_grad_()
    s0 = st["wkv"].double().requires_grad_()
    y, s = m64(xx, {"shift": sh, "wkv": s0})
    torch.autograd.backward((y, s["wkv"]), (gy.double(), gS.double()))
    truth = {"y": y.detach(), "state.wkv": s["wkv"].detach(), "state.shift": s["shift"].detach(),
             "dx": xx.grad, "dshift0": sh.grad, "dwkv0": s0.grad}
    for n, p in m64.named_parameters():
        truth["grad." + n] = p.grad.detach()
    bad = []
    for k, t in truth.items():
        ef = rel_l2(fused_out[k].double().cpu(), t.cpu())
        er = rel_l2(ref_out[k].double().cpu(), t.cpu())
        print(f"    {k}: fused {ef:.2e}  reference chain {er:.2e}", flush=True)
        if not ef <= max(1.25 * er, 2e-3):
            bad.append((k, ef, er))
    assert not bad, bad
