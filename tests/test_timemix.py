"""TimeMix drop-in: the reference's own TimeMix tests (tests/test_timemix.py of the
reference: CPU streaming/learning/TBPTT on backend="reference", the GPU stream and
fp32-optimizer tests) plus parity of the fused HIP elementwise kernels against the
reference's torch op sequence, op by op and for the whole layer."""
import math

import pytest
import torch
import torch.nn.functional as F

from conftest import rel_l2
from theseus.timemix import TimeMix, detach_state


# ---------------------------------------------------------------- CPU (reference backend)
def test_streaming_output_and_state():
    model = TimeMix(32, 3, 8, head_size=8, backend="reference")
    torch.nn.init.normal_(model.output.weight, std=.03)
    x = torch.randn(2, 9, 32)
    full, end = model(x)
    a, state = model(x[:, :4])
    b, state = model(x[:, 4:], state)
    torch.testing.assert_close(torch.cat([a, b], 1), full)
    for key in state:
        torch.testing.assert_close(state[key], end[key])


def test_initialization_can_learn():
    model = TimeMix(32, 3, 8, head_size=8, backend="reference")
    opt = torch.optim.AdamW(model.parameters(), lr=.01)
    x, target = torch.randn(1, 5, 32), torch.randn(1, 5, 32)
    for step in range(3):
        opt.zero_grad()
        y, _ = model(x)
        (y - target).square().mean().backward()
        assert model.output.weight.grad.abs().sum() > 0
        if step:
            assert model.receptance.weight.grad.abs().sum() > 0
            assert model.g1.grad.abs().sum() > 0
        opt.step()


def test_tbptt_detaches_only_at_chunk_boundary():
    model = TimeMix(16, 1, 4, head_size=4, backend="reference")
    torch.nn.init.normal_(model.output.weight, std=.05)
    x1 = torch.randn(1, 3, 16, requires_grad=True)
    x2 = torch.randn(1, 4, 16, requires_grad=True)
    _, state = model(x1)
    y, _ = model(x2, detach_state(state))
    y.sum().backward()
    assert x1.grad is None
    assert x2.grad is not None and x2.grad.abs().sum() > 0


def test_parameter_schema_and_init():
    """23 tensors with the reference's names and shapes (replace_timemix_lightning.py:66-72
    pins them), LoRA ranks max(32, round(k*sqrt(C)/32)*32), and the closed-form inits."""
    C, N, layer, depth = 5120, 64, 3, 8
    with torch.device("meta"):
        m = TimeMix(C, layer, depth, head_size=N, backend="reference")
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    rank, grank = 192, 352
    expect = {**{f"x_{n}": (1, 1, C) for n in "rwkvag"}, "w1": (C, rank), "w2": (rank, C), "a1": (C, rank),
              "a2": (rank, C), "w0": (1, 1, C), "a0": (1, 1, C), "g1": (C, grank), "g2": (grank, C),
              "k_k": (1, 1, C), "k_a": (1, 1, C), "r_k": (C // N, N), "receptance.weight": (C, C),
              "key.weight": (C, C), "value.weight": (C, C), "output.weight": (C, C), "ln_x.weight": (C,),
              "ln_x.bias": (C,)}
    assert shapes == expect
    small = TimeMix(128, 2, 4, head_size=64, backend="reference")
    c = torch.arange(128)
    reverse = 1 - 2 / 4
    torch.testing.assert_close(small.x_w.detach().reshape(-1), 1 - (c / 128).pow(.9 * reverse))
    assert torch.all(small.k_a == 1.02) and torch.all(small.r_k == -.04)
    assert torch.all(small.w1 == 0) and torch.all(small.g1 == 0) and torch.all(small.output.weight == 0)
    torch.testing.assert_close(small.ln_x.weight.detach(), torch.full((128,), (3 / 4) ** .7))
    w2 = small.w2.detach()
    gain = .1 * max(1, math.sqrt(32 / 128))
    torch.testing.assert_close(w2 @ w2.T, gain ** 2 * torch.eye(32), atol=1e-5, rtol=0)


# ---------------------------------------------------------------- GPU: fused ops vs torch
gpu = pytest.mark.gpu


def _torch_mix(x, shift, coefs):
    delta = torch.cat([shift.unsqueeze(1), x[:, :-1]], 1) - x
    return [(x + delta * c).to(x.dtype) for c in coefs]


# Op-level sizes: one partial token block at C=256 (4 heads); 19 heads (more than one
# 8-head group of the backward kernels and a partial last group) over 1203 tokens (18 token
# blocks of 64 plus a 51-token tail, so the fixed-order parameter-gradient reductions run
# over many blocks); and config 3's own size (B=2, T=4096, C=5120: 80 heads, 128 blocks).
OP_SIZES = [pytest.param(3, 37, 4, id="C256"), pytest.param(3, 401, 19, id="C1216-ragged"),
            pytest.param(2, 4096, 80, id="config3")]


@gpu
@pytest.mark.parametrize("B,T,H", OP_SIZES)
def test_fused_shift_lerp_matches_torch(B, T, H):
    from theseus import fused
    torch.manual_seed(1)
    C = 64 * H
    x = torch.randn(B, T, C, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    sh = torch.randn(B, C, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    coefs = [torch.rand(1, 1, C, device="cuda", requires_grad=True) for _ in range(6)]
    outs = fused.shift_lerp(x, sh, coefs)
    x2, sh2 = x.detach().clone().requires_grad_(), sh.detach().clone().requires_grad_()
    c2 = [c.detach().clone().requires_grad_() for c in coefs]
    refs = _torch_mix(x2, sh2, c2)
    for o, r in zip(outs, refs):
        torch.testing.assert_close(o.float(), r.float(), atol=1e-2, rtol=1e-2)
    gs = [torch.randn_like(o) for o in outs]
    torch.autograd.backward(outs, gs)
    torch.autograd.backward(refs, gs)
    # fp32 ground truth of the same math: the reference's bf16 chain rounds the
    # delta gradient several times, the fused kernel once, so compare both to it
    x3, sh3 = x.detach().float().requires_grad_(), sh.detach().float().requires_grad_()
    c3 = [c.detach().clone().requires_grad_() for c in coefs]
    d3 = torch.cat([sh3.unsqueeze(1), x3[:, :-1]], 1) - x3
    torch.autograd.backward([x3 + d3 * c for c in c3], [g.float() for g in gs])
    for got, ref_bf, truth in ((x.grad, x2.grad, x3.grad), (sh.grad, sh2.grad, sh3.grad),
                               *zip([c.grad for c in coefs], [c.grad for c in c2], [c.grad for c in c3])):
        e_fused = rel_l2(got.float().cpu(), truth.cpu())
        e_ref = rel_l2(ref_bf.float().cpu(), truth.cpu())
        print(f"    rel_l2 vs fp32: fused {e_fused:.2e}  reference-bf16 {e_ref:.2e}", flush=True)
        assert e_fused < 5e-3 and e_fused <= 1.5 * e_ref + 1e-4


def _kk_gn_chain(leaves, B, T, H, N, out_dtype):
    """The reference's op chains around the recurrence (theseus/timemix.py:75, 78-80, 83-88):
    the gate a = sigmoid(a0 + za), the WKV operands k*(1+(a-1)k_a), -kk, kk*a and the
    GroupNorm/bonus/gate output."""
    k, za, a0, k_k, k_a, r, v, g, y, r_k, ln_w, ln_b = leaves
    C = H * N
    f = torch.float64 if out_dtype == torch.float64 else torch.float32
    shape = (B, T, H, N)
    a = torch.sigmoid(a0 + za.to(f))
    kk = F.normalize((k.to(f) * k_k).reshape(shape), dim=-1, eps=1e-12)
    kmod = k * (1 + (a - 1) * k_a)
    ops = [z.reshape(shape).to(out_dtype) for z in (kmod, -kk, kk * a.reshape(shape))]
    yn = F.group_norm(y.to(f).reshape(B * T, C), H, ln_w, ln_b, 64e-5).reshape(B, T, C)
    bonus = ((r.to(f).reshape(shape) * kmod.to(f).reshape(shape) * r_k).sum(-1, keepdim=True)
             * v.to(f).reshape(shape)).reshape(B, T, C)
    return ops + [((yn + bonus) * g.to(f)).to(out_dtype)]


@gpu
@pytest.mark.parametrize("B,T,H", OP_SIZES)
def test_fused_decay_input_matches_torch(B, T, H):
    """w = (w0 + zw).to(bf16) (theseus/timemix.py:73, 80) in one kernel: the same bits as
    torch's float32 add and cast; dL/dzw is dL/dw, dL/dw0 its float32 sum over tokens."""
    from theseus import fused
    torch.manual_seed(4)
    C = 64 * H
    zw = torch.randn(B, T, C, device="cuda", dtype=torch.bfloat16).requires_grad_()
    w0 = torch.randn(1, 1, C, device="cuda").requires_grad_()
    z2, p2 = zw.detach().clone().requires_grad_(), w0.detach().clone().requires_grad_()
    got, ref = fused.add_param(zw, w0), (p2 + z2).to(torch.bfloat16)
    assert got.dtype == torch.bfloat16 and torch.equal(got, ref)
    dw = torch.randn_like(got)
    got.backward(dw)
    ref.backward(dw)
    assert torch.equal(zw.grad, z2.grad)
    torch.testing.assert_close(w0.grad, p2.grad, rtol=1e-5, atol=1e-4)


@gpu
@pytest.mark.parametrize("B,T,H", OP_SIZES)
def test_fused_kk_and_gn_match_torch(B, T, H):
    """The fused gate/kk/k-mod and GroupNorm/bonus/gate kernels against the same op chain in
    float64 on the CPU (outputs and all 12 input gradients at rel-L2 5e-3).  The torch
    chain on the GPU (bf16/fp32, as TimeMix runs it unfused) is measured against the same
    float64 truth and printed beside it."""
    from theseus import fused
    torch.manual_seed(2)
    N = 64
    C = H * N
    bf = torch.bfloat16
    mk = lambda *s, dt=bf: torch.randn(*s, device="cuda", dtype=dt)  # noqa: E731
    k = mk(B, T, C).requires_grad_()
    za = mk(B, T, C).requires_grad_()  # the LoRA output; the gate is sigmoid(a0 + za)
    a0 = (.3 * torch.randn(1, 1, C, device="cuda")).requires_grad_()
    k_k = (.71 + .1 * torch.rand(1, 1, C, device="cuda")).requires_grad_()
    k_a = torch.full((1, 1, C), 1.02, device="cuda").requires_grad_()
    r, v, g = (mk(B, T, C).requires_grad_() for _ in range(3))
    y = mk(B, T, H, N).requires_grad_()
    r_k = torch.full((H, N), -.04, device="cuda").requires_grad_()
    ln_w = (1 + .1 * torch.randn(C, device="cuda")).requires_grad_()
    ln_b = (.1 * torch.randn(C, device="cuda")).requires_grad_()
    leaves = [k, za, a0, k_k, k_a, r, v, g, y, r_k, ln_w, ln_b]
    refl = [t.detach().clone().requires_grad_() for t in leaves]
    truthl = [t.detach().cpu().double().requires_grad_() for t in leaves]

    kw, aw, bw, km = fused.kk_kmod(k, za, a0, k_k, k_a, N, bf)
    out = fused.gn_bonus_gate(y, r, km, v, g, r_k, ln_w, ln_b, 64e-5, bf)
    got = (kw, aw, bw, out)
    refs = _kk_gn_chain(refl, B, T, H, N, bf)
    truth = _kk_gn_chain(truthl, B, T, H, N, torch.float64)
    for n, o, rr, tt in zip(("kw", "aw", "bw", "out"), got, refs, truth):
        e, e_ref = rel_l2(o.float().cpu(), tt.detach()), rel_l2(rr.float().cpu(), tt.detach())
        print(f"    {n}: rel_l2 vs fp64 {e:.2e} (torch GPU chain {e_ref:.2e})", flush=True)
        assert e < 5e-3, (n, e)
    gs = [torch.randn_like(t) for t in got]
    torch.autograd.backward(got, gs)
    torch.autograd.backward(refs, gs)
    torch.autograd.backward(truth, [gg.cpu().double() for gg in gs])
    names = ["k", "za", "a0", "k_k", "k_a", "r", "v", "g", "y", "r_k", "ln_w", "ln_b"]
    bad = []
    for n, t, tr, tt in zip(names, leaves, refl, truthl):
        e = rel_l2(t.grad.float().cpu(), tt.grad)
        e_ref = rel_l2(tr.grad.float().cpu(), tt.grad)
        print(f"    grad {n}: rel_l2 vs fp64 {e:.2e} (torch GPU chain {e_ref:.2e})", flush=True)
        if not e < 5e-3:
            bad.append((n, e))
    assert not bad, bad


@gpu
def test_fused_timemix_layer_matches_reference_backend():
    """The whole layer: backend="cuda" (HIP WKV + fused elementwise) vs the reference torch
    sequence on the same weights, bf16 autocast over fp32 parameters.  The bars are the
    distance between two bf16 computations: the reference chain itself rounds its shift
    gradients 5e-3 to 2e-2 away from the float64 layer, so both sides are held to 5e-3
    against float64 in tests/test_timemix_c3.py (test_fused_layer_is_as_close_to_float64_
    as_the_reference_chain, up to config 3's size)."""
    torch.manual_seed(3)
    C, N = 256, 64
    m = TimeMix(C, 2, 6, head_size=N, backend="cuda").cuda()
    for p in (m.w1, m.a1, m.g1, m.output.weight):
        torch.nn.init.normal_(p, std=.05)
    ref = TimeMix(C, 2, 6, head_size=N, backend="reference").cuda()
    ref.load_state_dict(m.state_dict())
    x = torch.randn(2, 45, C, device="cuda", dtype=torch.bfloat16)
    st = {"shift": torch.randn(2, C, device="cuda", dtype=torch.bfloat16),
          "wkv": .1 * torch.randn(2, C // N, N, N, device="cuda")}
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, s = m(x, st)
        yr, sr = ref(x, st)
    assert rel_l2(y.float().cpu(), yr.float().cpu()) < 1e-2
    assert rel_l2(s["wkv"].cpu(), sr["wkv"].cpu()) < 5e-3
    gy = torch.randn_like(y)
    (y.float() * gy.float()).sum().backward()
    (yr.float() * gy.float()).sum().backward()
    for (n, p), (_, pr) in zip(m.named_parameters(), ref.named_parameters()):
        e = rel_l2(p.grad.float().cpu(), pr.grad.float().cpu())
        print(f"    {n}: rel_l2 {e:.2e}", flush=True)
        assert e < 2e-2, (n, e)


@gpu
@pytest.mark.parametrize("optim", ["FusedAdamW", "AdamW-fused"])
def test_fused_layer_computes_with_the_updated_parameters(optim):
    """Training: forward, backward and two optimizer steps on backend="cuda" -- through
    this build's FusedAdamW (it writes the parameters through raw pointers) or torch's
    AdamW(fused=True), as the reference's stage.py:42 -- then the next forward and backward
    against the reference backend on the same, updated parameters.  The steps move the
    shift-lerp coefficients far enough that the old values are detectably wrong."""
    from theseus.optim import FusedAdamW
    torch.manual_seed(8)
    C, N = 256, 64
    m = TimeMix(C, 2, 6, head_size=N, backend="cuda").cuda()
    for p in (m.w1, m.a1, m.g1, m.output.weight):
        torch.nn.init.normal_(p, std=.05)
    before = TimeMix(C, 2, 6, head_size=N, backend="reference").cuda()
    before.load_state_dict(m.state_dict())
    opt = (FusedAdamW(m.parameters(), lr=.05) if optim == "FusedAdamW"
           else torch.optim.AdamW(m.parameters(), lr=.05, fused=True))
    x = torch.randn(2, 33, C, device="cuda", dtype=torch.bfloat16)
    for _ in range(2):
        opt.zero_grad()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y, _ = m(x)
        y.float().square().mean().backward()
        opt.step()
    ref = TimeMix(C, 2, 6, head_size=N, backend="reference").cuda()
    ref.load_state_dict(m.state_dict())
    opt.zero_grad()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, _ = m(x)
        yr, _ = ref(x)
        with torch.no_grad():
            yb, _ = before(x)
    assert rel_l2(y.float().cpu(), yr.float().cpu()) < 1e-2
    assert rel_l2(yb.float().cpu(), yr.float().cpu()) > 5e-2  # (the steps changed the layer)
    gy = torch.randn_like(y)
    (y.float() * gy.float()).sum().backward()
    (yr.float() * gy.float()).sum().backward()
    for (n, p), (_, pr) in zip(m.named_parameters(), ref.named_parameters()):
        e = rel_l2(p.grad.float().cpu(), pr.grad.float().cpu())
        assert e < 2e-2, (n, e)


# ---------------------------------------------------------------- GPU: the reference's own tests
@gpu
def test_cuda_inference_chunking_and_current_stream():
    model = TimeMix(128, 3, 8, head_size=64, backend="cuda").cuda().to(torch.bfloat16)
    torch.nn.init.normal_(model.output.weight, std=.01)
    x = torch.randn(2, 17, 128, device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream), torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        full, final = model(x)
        a, state = model(x[:, :5])
        b, state = model(x[:, 5:], state)
    torch.cuda.current_stream().wait_stream(stream)
    torch.testing.assert_close(torch.cat([a, b], 1), full, atol=.006, rtol=.025)
    torch.testing.assert_close(state["wkv"], final["wkv"], atol=.0005, rtol=.02)


@gpu
def test_cuda_token_by_token_decode_matches_one_call():
    """Serving: the reference's Runner steps each TimeMix one token at a time with the
    carried {"shift", "wkv"} state (theseus/hf_model.py:96-108); on backend="cuda" every
    such step is a T=1 no-grad call, which runs the single-step kernel."""
    torch.manual_seed(5)
    model = TimeMix(256, 2, 6, head_size=64, backend="cuda").cuda().to(torch.bfloat16)
    torch.nn.init.normal_(model.output.weight, std=.02)
    x = torch.randn(2, 24, 256, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        full, final = model(x)
        state, outs = None, []
        for t in range(x.shape[1]):
            y, state = model(x[:, t:t + 1], state)
            outs.append(y)
    torch.testing.assert_close(torch.cat(outs, 1), full, atol=.006, rtol=.025)
    torch.testing.assert_close(state["wkv"], final["wkv"], atol=.0005, rtol=.02)
    assert torch.equal(state["shift"], final["shift"])


@gpu
def test_state_resumes_across_backends():
    """The carried state has the reference's format ({"shift": [B,C] in x's dtype,
    "wkv": [B,H,value,key] fp32}, theseus/checkpoint.py:100-102, the export's
    state_layout "B,H,value,key"): a prefix run on the reference backend (CPU, fp32)
    resumes on the HIP backend and matches the reference continuing itself."""
    torch.manual_seed(6)
    ref = TimeMix(128, 1, 4, head_size=64, backend="reference")
    torch.nn.init.normal_(ref.output.weight, std=.05)
    dev = TimeMix(128, 1, 4, head_size=64, backend="cuda").cuda()
    dev.load_state_dict(ref.state_dict())
    x = torch.randn(2, 20, 128)
    _, st = ref(x[:, :12])
    y_ref, st_ref = ref(x[:, 12:], st)
    assert set(st) == {"shift", "wkv"} and st["wkv"].shape == (2, 2, 64, 64) and st["wkv"].dtype == torch.float32
    with torch.no_grad():
        y_dev, st_dev = dev(x[:, 12:].cuda(), {k: v.cuda() for k, v in st.items()})
    assert rel_l2(y_dev.cpu(), y_ref.detach()) < 2e-3
    assert rel_l2(st_dev["wkv"].cpu(), st_ref["wkv"].detach()) < 2e-3


@gpu
def test_cuda_fp32_optimizer_states_and_learning():
    model = TimeMix(128, 3, 8, head_size=64, backend="cuda").cuda()
    optimizer = torch.optim.AdamW(model.parameters(), lr=.003)
    x = torch.randn(1, 7, 128, device="cuda", dtype=torch.bfloat16)
    target = torch.randn_like(x)
    losses = []
    for _ in range(4):
        optimizer.zero_grad()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y, _ = model(x)
        loss = (y.float() - target.float()).square().mean()
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1., error_if_nonfinite=True)
        optimizer.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0]
    for param, state in optimizer.state.items():
        assert param.dtype == param.grad.dtype == torch.float32
        assert state["exp_avg"].dtype == state["exp_avg_sq"].dtype == torch.float32


def test_explicit_group_norm_is_torch_group_norm():
    """The unfused GPU path's GroupNorm (written out, because torch's ROCm group_norm backward
    returns wrong weight/bias gradients at >= ~1024 rows) is the same function as
    F.group_norm: values and all three gradients, float64 on the CPU."""
    from theseus.timemix import _group_norm
    torch.manual_seed(4)
    M, G, C = 1500, 6, 6 * 16
    x = torch.randn(M, C, dtype=torch.float64, requires_grad=True)
    w = (1 + .1 * torch.randn(C, dtype=torch.float64)).requires_grad_()
    b = (.1 * torch.randn(C, dtype=torch.float64)).requires_grad_()
    go = torch.randn(M, C, dtype=torch.float64)
    ours = torch.autograd.grad(_group_norm(x, G, w, b, 64e-5), (x, w, b), go)
    ref = F.group_norm(x, G, w, b, 64e-5)
    torch.testing.assert_close(_group_norm(x, G, w, b, 64e-5), ref, rtol=1e-12, atol=1e-12)
    for g1, g2 in zip(ours, torch.autograd.grad(ref, (x, w, b), go)):
        torch.testing.assert_close(g1, g2, rtol=1e-10, atol=1e-10)
