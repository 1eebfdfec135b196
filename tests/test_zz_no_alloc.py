"""theseus_wkv7_forward_noalloc (the forward whose handoff workspace is the
library's static device scratch array) against theseus_wkv7_forward (caller
workspace), both called through the C ABI with ctypes.

The two run the same kernels on the same inputs, so y, the final state and the
saved states must agree bitwise.  Two calls in a row, the second smaller, share
the scratch array: the second must not see the first's counters or states.  The
sizes cut heads between workgroups (B*H above the device's CUs), so the
handoffs really go through the scratch.
"""
import ctypes
import os

import pytest
import torch

from theseus import wkv7 as W
from theseus.synthetic import wkv7_inputs

pytestmark = pytest.mark.gpu

ERR_SCRATCH = 6
SCRATCH_BYTES = 8 << 20  # THESEUS_WKV7_NOALLOC_SCRATCH_BYTES


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _outputs(B, T, H, N, save, ext):
    y = torch.full((B, T, H, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    sT = torch.full((B, H, N, N), float("nan"), dtype=torch.float32, device="cuda")
    ck = (torch.full((B, H, ext.checkpoint_count(T), N, N), float("nan"), dtype=torch.float32,
                     device="cuda") if save else None)
    return y, sT, ck


def _run_both(B, T, H, seed, save):
    N = 64
    ext = W.extension()
    lib = ext.lib
    inp = wkv7_inputs(B, T, H, N, seed=seed, dtype=torch.bfloat16, s0_std=0.1)
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0 = inp["s0"].cuda()
    need = int(lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0))
    print(f"  noalloc case B={B} T={T} H={H} save={save} workspace={need} B", flush=True)
    assert 0 < need <= SCRATCH_BYTES  # heads are cut: the handoffs use the workspace

    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y1, s1, c1 = _outputs(B, T, H, N, save, ext)
    st = lib.theseus_wkv7_forward(B, T, H, N, 0, *map(_p, (*xs, s0, y1, s1, c1, ws)),
                                  ctypes.c_size_t(need), _stream())
    assert st == 0, st
    y2, s2, c2 = _outputs(B, T, H, N, save, ext)
    st = lib.theseus_wkv7_forward_noalloc(B, T, H, N, 0, *map(_p, (*xs, s0, y2, s2, c2)), _stream())
    assert st == 0, lib.theseus_wkv7_error_string(st)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(s1, s2)
    assert not torch.isnan(s2).any()
    if save:
        assert torch.equal(c1, c2)
        assert not torch.isnan(c2).any()


def test_noalloc_forward_matches_workspace_forward_twice():
    if torch.cuda.get_device_properties(0).multi_processor_count >= 320:
        pytest.skip("sizes below assume fewer than 320 CUs (cut heads)")
    _run_both(4, 2048, 80, seed=20262, save=True)   # config 2's forward, 320 heads
    _run_both(4, 300, 72, seed=5, save=False)       # smaller, 288 heads, partial last chunk
    _run_both(4, 300, 72, seed=6, save=True)


def test_noalloc_forward_refuses_sizes_beyond_its_scratch():
    """Planning for 4096 CUs cuts 4100 heads over ~3000 workgroups, whose handoffs would
    need ~48 MB: the call returns ERR_SCRATCH and enqueues nothing (outputs untouched)."""
    B, T, H, N = 50, 48, 82, 64
    lib = W.extension().lib
    inp = wkv7_inputs(1, T, H, N, seed=3, dtype=torch.bfloat16)
    xs = [inp[n].cuda().expand(B, T, H, N).contiguous() for n in "rwkvab"]
    s0 = torch.zeros(B, H, N, N, device="cuda")
    y = torch.full((B, T, H, N), 7.0, dtype=torch.bfloat16, device="cuda")
    sT = torch.full((B, H, N, N), 7.0, device="cuda")
    old = os.environ.get("THESEUS_WKV7_CUS")
    os.environ["THESEUS_WKV7_CUS"] = "4096"
    try:
        need = int(lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0))
        st = lib.theseus_wkv7_forward_noalloc(B, T, H, N, 0, *map(_p, (*xs, s0, y, sT, None)), _stream())
    finally:
        if old is None:
            del os.environ["THESEUS_WKV7_CUS"]
        else:
            os.environ["THESEUS_WKV7_CUS"] = old
    torch.cuda.synchronize()
    assert need > SCRATCH_BYTES
    assert st == ERR_SCRATCH
    assert b"THESEUS_WKV7_NOALLOC_SCRATCH_BYTES" in lib.theseus_wkv7_error_string(st)
    assert bool((y == 7.0).all()) and bool((sT == 7.0).all())


def test_noalloc_forward_on_two_ordered_streams():
    """The single-stream rule, as a caller on two streams keeps it: calls on stream A,
    then (after B waits for A) on stream B share the scratch array in order, and each
    result equals the caller-workspace forward bitwise."""
    if torch.cuda.get_device_properties(0).multi_processor_count >= 320:
        pytest.skip("sizes below assume fewer than 320 CUs (cut heads)")
    B, T, H, N = 4, 300, 72, 64
    ext = W.extension()
    lib = ext.lib
    need = int(lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    cases = []
    for seed in (11, 12):
        inp = wkv7_inputs(B, T, H, N, seed=seed, dtype=torch.bfloat16, s0_std=0.1)
        xs = [inp[n].cuda() for n in "rwkvab"]
        s0 = inp["s0"].cuda()
        y, s, c = _outputs(B, T, H, N, True, ext)
        assert lib.theseus_wkv7_forward(B, T, H, N, 0, *map(_p, (*xs, s0, y, s, c, ws)),
                                        ctypes.c_size_t(need), _stream()) == 0
        cases.append((xs, s0, (y, s, c)))
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    got = []
    for st, (xs, s0, _) in zip((sa, sb), cases):
        st.wait_stream(torch.cuda.current_stream())
        if st is sb:
            sb.wait_stream(sa)  # the ordering the shared scratch array requires
        with torch.cuda.stream(st):
            outs = _outputs(B, T, H, N, True, ext)
            assert lib.theseus_wkv7_forward_noalloc(B, T, H, N, 0, *map(_p, (*xs, s0, *outs)),
                                                    ctypes.c_void_p(st.cuda_stream)) == 0
        got.append(outs)
    torch.cuda.synchronize()
    for (_, _, want), outs in zip(cases, got):
        for a, b in zip(want, outs):
            assert torch.equal(a, b)
