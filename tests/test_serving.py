"""In-place serving step of TimeMix (``TimeMix.step_``) and its HIP-graph capture
(``theseus.serving.CapturedStep``), against the out-of-place serving step the
reference makes (``TimeMix.forward`` with T=1, theseus/hf_model.py:96-108), one
multi-token call, and the reference backend in float64 on the CPU."""
import pytest
import torch

from conftest import rel_l2
from theseus.serving import CapturedStep, serving_state
from theseus.timemix import TimeMix


def _model(C, seed, dtype=torch.bfloat16):
    torch.manual_seed(seed)
    m = TimeMix(C, 2, 6, head_size=64, backend="cuda")
    with torch.no_grad():
        for n, p in m.named_parameters():  # non-trivial LoRAs and output (zero at init)
            if n in ("w1", "a1", "g1", "output.weight"):
                p.normal_(0, .05)
    return m.cuda().to(dtype).eval()


def test_step_refuses_misuse_on_cpu():
    m = TimeMix(128, 0, 2, head_size=64, backend="reference")
    x = torch.randn(1, 1, 128)
    with pytest.raises(ValueError):
        m.step_(x, m.initial_state(x))


@pytest.mark.gpu
def test_step_in_place_matches_out_of_place_steps_and_references():
    """64 tokens at B=3, C=256 after an 8-token prefill: every in-place step equals the
    out-of-place T=1 forward bitwise (same kernels), the state keeps its storage, the
    outputs match one 64-token call (the chunked kernels), and the layer matches the
    reference backend in float64 on the CPU."""
    B, C, P, T = 3, 256, 8, 64
    m = _model(C, seed=11)
    x = torch.randn(B, P + T, C, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        _, pre = m(x[:, :P])
        st = serving_state(pre)
        ptr = (st["shift"].data_ptr(), st["wkv"].data_ptr())
        oop, outs = pre, []
        for t in range(P, P + T):
            y_ip = m.step_(x[:, t:t + 1], st)
            y_oop, oop = m(x[:, t:t + 1], oop)
            assert torch.equal(y_ip, y_oop), t
            outs.append(y_ip.clone())
        assert (st["shift"].data_ptr(), st["wkv"].data_ptr()) == ptr
        assert torch.equal(st["wkv"], oop["wkv"]) and torch.equal(st["shift"], oop["shift"])
        full, fin = m(x[:, P:], pre)
    got = torch.cat(outs, 1)
    torch.testing.assert_close(got, full, atol=.006, rtol=.025)
    torch.testing.assert_close(st["wkv"], fin["wkv"], atol=.0005, rtol=.02)

    ref = TimeMix(C, 2, 6, head_size=64, backend="reference").double()
    ref.load_state_dict({k: v.double().cpu() for k, v in m.state_dict().items()})
    with torch.no_grad():
        y_ref, s_ref = ref(x.double().cpu())
    e_y, e_s = rel_l2(got.cpu(), y_ref[:, P:]), rel_l2(st["wkv"].cpu(), s_ref["wkv"])
    print(f"    vs float64 reference backend: y rel-L2 {e_y:.2e}, wkv rel-L2 {e_s:.2e}", flush=True)
    assert e_y < 2e-2 and e_s < 1e-2


@pytest.mark.gpu
def test_step_rejects_states_it_cannot_update():
    m = _model(128, seed=2)
    x = torch.randn(2, 1, 128, device="cuda", dtype=torch.bfloat16)
    st = m.initial_state(x)
    with torch.no_grad():
        with pytest.raises(ValueError):
            m.step_(torch.randn(2, 2, 128, device="cuda", dtype=torch.bfloat16), st)
        with pytest.raises(ValueError):
            m.step_(x, {"shift": st["shift"], "wkv": st["wkv"].transpose(-1, -2)})
    m.float().requires_grad_(True)
    with pytest.raises(RuntimeError):
        m.step_(x.float(), {"shift": st["shift"].float(), "wkv": st["wkv"]})


@pytest.mark.gpu
@pytest.mark.parametrize("autocast", [None, torch.bfloat16], ids=["bf16-weights", "fp32-weights-autocast"])
def test_captured_step_replays_match_eager_steps(autocast):
    """A captured step replayed 64 times, with unrelated eager work and synchronisations
    between replays, gives every token's output and the final state of 64 eager steps."""
    B, C, T = 4, 320, 64
    m = _model(C, seed=12, dtype=torch.bfloat16 if autocast is None else torch.float32)
    x = torch.randn(B, T, C, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        st0 = {"shift": torch.randn(B, C, device="cuda", dtype=torch.bfloat16),
               "wkv": .1 * torch.randn(B, C // 64, 64, 64, device="cuda")}
        s_graph, s_eager = serving_state(st0), serving_state(st0)
        step = CapturedStep(m, s_graph, x[:, :1], autocast=autocast)
        assert torch.equal(s_graph["wkv"], st0["wkv"])  # capture leaves the state as it was
        junk = torch.randn(512, 512, device="cuda")
        for t in range(T):
            y_g = step(x[:, t:t + 1]).clone()
            junk = junk @ junk.T / 512  # eager work between replays
            torch.cuda.synchronize()
            if autocast is None:
                y_e = m.step_(x[:, t:t + 1], s_eager)
            else:
                with torch.autocast("cuda", dtype=autocast):
                    y_e = m.step_(x[:, t:t + 1], s_eager)
            assert rel_l2(y_g.float().cpu(), y_e.float().cpu()) < 1e-3, t
        assert rel_l2(s_graph["wkv"].cpu(), s_eager["wkv"].cpu()) < 1e-4
        assert torch.equal(s_graph["shift"], s_eager["shift"])


def test_parameter_copies_follow_every_update():
    """Outside a caller-owned store the fused wrappers make their float32 parameter copies
    (and the stacked lerp coefficients) afresh on every call, so even an update written
    through a raw pointer -- as optimizer kernels do, with no version-counter bump -- is
    seen by the next call.  Inside ``param_cache(store)`` the copies are reused, and
    ``refresh_param_cache`` rewrites them in place."""
    import ctypes
    from theseus import fused
    p = torch.nn.Parameter(torch.randn(1, 1, 8).to(torch.bfloat16))
    a = fused._vec(p, 8)
    assert torch.equal(a, p.detach().float().reshape(8))
    v0 = p._version
    new = torch.randn(1, 1, 8).to(torch.bfloat16)
    ctypes.memmove(p.data_ptr(), new.data_ptr(), 16)  # a raw-pointer write
    assert p._version == v0
    assert torch.equal(fused._vec(p, 8), new.float().reshape(8))
    cs = [torch.nn.Parameter(torch.randn(1, 1, 8)) for _ in range(6)]
    m1 = fused._coef_matrix(cs, 8)
    ctypes.memmove(cs[3].data_ptr(), torch.ones(8).data_ptr(), 32)
    m2 = fused._coef_matrix(cs, 8)
    assert torch.equal(m2, torch.stack([c.detach().reshape(8) for c in cs])) and not torch.equal(m1, m2)

    store = {}
    with fused.param_cache(store):
        c1 = fused._coef_matrix(cs, 8)
        assert fused._coef_matrix(cs, 8) is c1 and len(store) == 1
        b1 = fused._vec(p, 8)
        assert fused._vec(p, 8) is b1
    assert fused._coef_matrix(cs, 8) is not c1  # the store is used only inside the context
    with torch.no_grad():
        cs[0].add_(1)
        p.mul_(2)
    fused.refresh_param_cache(store)
    assert torch.equal(c1, torch.stack([c.detach().reshape(8) for c in cs]))
    assert torch.equal(b1, p.detach().float().reshape(8))
    with fused.param_cache(store):
        assert fused._coef_matrix(cs, 8) is c1


@pytest.mark.gpu
def test_captured_step_follows_refreshed_weights():
    """The graph reads parameter copies that the CapturedStep owns: an in-place weight
    update and eager calls with the new weights leave them alone (a replay still computes
    with the old small parameters), and after ``refresh_params()`` a replay equals an
    eager step with the new weights."""
    B, C = 2, 256
    m = _model(C, seed=13)
    x = torch.randn(B, 3, C, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        st0 = {"shift": torch.randn(B, C, device="cuda", dtype=torch.bfloat16),
               "wkv": .1 * torch.randn(B, C // 64, 64, 64, device="cuda")}
        s_graph = serving_state(st0)
        step = CapturedStep(m, s_graph, x[:, :1], autocast=None)
        step(x[:, :1])
        s1 = serving_state(s_graph)  # the state after token 0 (old weights)
        gen = torch.Generator(device="cuda").manual_seed(3)
        for p in m.parameters():
            if p.numel() == C:  # the small parameters (the graph reads float32 copies of them)
                p.add_((.2 * torch.randn(p.shape, generator=gen, device="cuda")).to(p.dtype))
        s_e = serving_state(s1)
        y_new = m.step_(x[:, 1:2], s_e).clone()  # eager, new weights
        y_stale = step(x[:, 1:2]).clone()        # replay before the refresh
        for k in s_graph:
            s_graph[k].copy_(s1[k])
        step.refresh_params()
        y_ref = step(x[:, 1:2]).clone()
    assert rel_l2(y_ref.float().cpu(), y_new.float().cpu()) < 1e-3
    assert rel_l2(s_graph["wkv"].cpu(), s_e["wkv"].cpu()) < 1e-4
    assert rel_l2(y_stale.float().cpu(), y_new.float().cpu()) > 2e-2  # (the update matters)


@pytest.mark.gpu
@pytest.mark.parametrize("B,C,dtype", [(4, 320, torch.bfloat16), (3, 640, torch.float32), (64, 5120, torch.bfloat16)],
                         ids=["C320", "C640-fp32-weights-autocast", "config4"])
def test_native_step_equals_the_python_launches(B, C, dtype, monkeypatch):
    """Inside a parameter store a one-token no-grad step runs as one native call
    (theseus_tm_serving_step) that launches the same kernels as the layer's Python path:
    8 tokens in place (step_) and out of place (forward, the reference's serving call) give
    bitwise the same outputs, WKV state and shift state on both paths."""
    import contextlib
    from theseus import fused
    m = _model(C, seed=31, dtype=dtype)
    x = torch.randn(B, 8, C, device="cuda", dtype=torch.bfloat16)
    st0 = {"shift": torch.randn(B, C, device="cuda", dtype=torch.bfloat16),
           "wkv": .1 * torch.randn(B, C // 64, 64, 64, device="cuda")}
    ac = (lambda: torch.autocast("cuda", dtype=torch.bfloat16)) if dtype == torch.float32 else contextlib.nullcontext
    for inplace in (True, False):
        res = {}
        for native in ("1", "0"):
            monkeypatch.setenv("THESEUS_TM_NATIVE", native)
            store, s, outs = {}, serving_state(st0), []
            with torch.no_grad(), fused.param_cache(store), ac():
                for t in range(8):
                    xt = x[:, t:t + 1].contiguous()
                    if inplace:
                        y = m.step_(xt, s)
                    else:
                        y, s = m(xt, s)
                    outs.append(y.clone())
            torch.cuda.synchronize()
            assert any(k[0] == "tm_layer" for k in store) == (native == "1")
            res[native] = (outs, s)
        (o1, s1), (o0, s0) = res["1"], res["0"]
        assert all(torch.equal(a, b) for a, b in zip(o1, o0)), inplace
        assert torch.equal(s1["wkv"], s0["wkv"]) and torch.equal(s1["shift"], s0["shift"]), inplace
