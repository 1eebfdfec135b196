"""Head size 128 (bf16) on the chunk-record kernels, against the float64 oracle.

The reference's operator takes any head size from 2 to 128 (kernels/wkv7_state.cpp:12-13;
theseus/config.py:53-59 exposes head_size up to 128).  Here a bf16 forward with N = 128
runs on two kernels of gdn_chunk.hip -- every chunk's operands formed at once, then one
scan per head on the matrix cores -- when the caller's workspace holds the chunk records
(theseus_wkv7_forward_workspace_size counts them); the backward runs on the three of
wkv7_rec_bwd.hip (records, a reverse scan of dL/dS over the chunks, then every chunk's
gradients at once) from the [value][key] saved states either forward writes.  Bars as in
test_wkv7_gpu.py: rel-L2 <= 5e-3, fp32 outputs max-abs <= 2e-2, bf16 outputs
|err| <= 2e-2 + 2^-7 |ref| elementwise.
"""
import ctypes

import pytest
import torch

from oracle import wkv7_oracle as O
from test_wkv7_gpu import _check, _gpu_fwd_bwd, _oracle, _parity, _split_vs_one_pass
from theseus import wkv7 as W
from theseus.synthetic import wkv7_inputs

pytestmark = pytest.mark.gpu

N = 128
RECORD_BYTES = 43520  # one chunk's record: P, P2, the update operands, Q'^T, Q2^T, V, e^{gL}


def _fwd(lib, xs, s0, ws, ws_bytes, ckpt=None):
    B, T, H, _ = xs[0].shape
    y = torch.full((B, T, H, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    sT = torch.full((B, H, N, N), float("nan"), dtype=torch.float32, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    st = lib.theseus_wkv7_forward(B, T, H, N, 0, *map(p, (*xs, s0, y, sT)), p(ckpt), p(ws),
                                  ctypes.c_size_t(ws_bytes),
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, lib.theseus_wkv7_error_string(st)
    torch.cuda.synchronize()
    return y, sT


def _inputs(B, T, H, seed, w_mode=None):
    inp = wkv7_inputs(B, T, H, N, seed=seed, dtype=torch.bfloat16, s0_std=0.1, with_dsT=True)
    if w_mode is not None:
        w = inp["w"].float()
        w = {"wide": 8.0 * w, "max_decay": torch.full_like(w, 30.0), "no_decay": torch.full_like(w, -30.0)}[w_mode]
        inp["w"] = w.to(torch.bfloat16).contiguous()
    return inp


def _oracle_fwd(inp):
    return O.forward_c(*(inp[n].double().numpy() for n in "rwkvab"), inp["s0"].double().numpy())


@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 15, 2), (2, 16, 1), (1, 17, 3), (2, 100, 2), (1, 333, 4),
                                   (3, 64, 5)])
def test_record_forward_against_oracle(B, T, H, monkeypatch):
    """One-pass scan (the library's own CU count: no time split at these head counts or
    below 8 chunks), tails of every length; the workspace, filled with NaN first, holds
    finite records afterwards (the record path ran); no workspace runs the step-serial
    kernels, which agree to fp32 rounding."""
    monkeypatch.setenv("THESEUS_WKV7_CUS", "1")
    lib = W.extension().lib
    assert W.extension().kernel_family(B, T, H, N, 0) == 6
    need = int(lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0))
    nrec = B * H * (-(-T // 16))
    assert need == nrec * RECORD_BYTES
    print(f"  records B={B} T={T} H={H}", flush=True)
    inp = _inputs(B, T, H, seed=5000 + T + H)
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0 = inp["s0"].cuda()
    ws = torch.full((need // 4,), float("nan"), dtype=torch.float32, device="cuda")
    y, sT = _fwd(lib, xs, s0, ws, need)
    if T > 1:  # (one step without saved states runs the single-step kernel)
        assert bool(torch.isfinite(ws).all())
    y_ref, s_ref = _oracle_fwd(inp)
    _check("y", y, y_ref, torch.bfloat16)
    _check("sT", sT, s_ref, torch.bfloat16)
    y_q, s_q = _fwd(lib, xs, s0, None, 0)
    _check("y", y_q, y_ref, torch.bfloat16)
    torch.testing.assert_close(sT, s_q, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 15, 2), (2, 16, 1), (1, 18, 1), (2, 100, 2), (1, 257, 3),
                                   (3, 48, 4)])
def test_record_backward_against_oracle(B, T, H):
    """Training calls through autograd: all nine outputs (y, sT, the six input gradients
    and ds0) against the oracle, dsT ~ N(0,1), tails of every length."""
    _parity(B, T, H, N, torch.bfloat16, seed=5100 + T)


def test_record_backward_without_state_gradient():
    """dsT = 0 (the training case: the final state is not used), B=2, T=200, H=3."""
    _parity(2, 200, 3, N, torch.bfloat16, seed=5150, with_dsT=False)


@pytest.mark.parametrize("fwd_fam", ["auto", "seq"])
def test_record_backward_reads_either_forwards_saved_states(fwd_fam, monkeypatch):
    """Both forwards keep [value][key] saved states: the record backward given the
    step-serial forward's (and the step-serial backward given the record forward's) gives
    the gradients of the all-record call to fp32 rounding, nothing raises."""
    B, T, H = 1, 90, 2
    inp = _inputs(B, T, H, seed=5170)
    ext = W.extension()
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0, dy, dsT = inp["s0"].cuda(), inp["dy"].cuda(), inp["dsT"].cuda()
    _, _, saved = ext.forward(*xs, s0, True)
    ref = ext.backward(*xs, saved, dy, dsT)
    monkeypatch.setenv("THESEUS_WKV7_FAMILY", fwd_fam)
    _, _, saved2 = ext.forward(*xs, s0, True)
    monkeypatch.setenv("THESEUS_WKV7_FAMILY", "seq" if fwd_fam == "auto" else "auto")
    got = ext.backward(*xs, saved2, dy, dsT)
    torch.cuda.synchronize()
    for name, x, z in zip(["dr", "dw", "dk", "dv", "da", "db", "ds0"], got, ref):
        rel = ((x.float() - z.float()).norm() / z.float().norm()).item()
        print(f"    {name} rel {rel:.2e}", flush=True)
        assert rel < 5e-3, (name, rel)


def test_record_backward_at_the_ends_of_the_decay_range():
    """w ~ N(0, 8^2) (decays from none to the strongest within a chunk), fwd+bwd against
    the oracle."""
    B, T, H = 1, 120, 2
    inp = _inputs(B, T, H, seed=5180, w_mode="wide")
    got = _gpu_fwd_bwd(inp, torch.bfloat16, inp["dsT"])
    ref = _oracle(inp, inp["dsT"])
    for name, g, r in zip(["y", "sT", "dr", "dw", "dk", "dv", "da", "db", "ds0"], got, ref):
        _check(name, g, r, torch.bfloat16)


def test_saved_states_equal_the_step_serial_forwards(monkeypatch):
    """The record forward's saved states are [value][key] states after every 16 steps and
    the final one, as the step-serial forward saves them: state 0 is s0 bit for bit, the
    last is the returned final state, the rest agree to fp32 rounding."""
    B, T, H = 2, 70, 3
    inp = _inputs(B, T, H, seed=5200)
    ext = W.extension()
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0 = inp["s0"].cuda()
    _, end, saved = ext.forward(*xs, s0, True)
    assert saved.theseus_layout == "rows"
    monkeypatch.setenv("THESEUS_WKV7_FAMILY", "seq")
    _, end_q, saved_q = ext.forward(*xs, s0, True)
    torch.cuda.synchronize()
    assert saved.shape == saved_q.shape == (B, H, 6, N, N)
    assert torch.equal(saved[:, :, 0], s0)
    assert torch.equal(saved[:, :, -1], end)
    rel = ((saved - saved_q).norm() / saved_q.norm()).item()
    assert rel <= 1e-5, rel


@pytest.mark.parametrize("B,T,H", [(1, 2048, 4), (2, 300, 3), (1, 130, 1)])
def test_record_forward_time_split(B, T, H, monkeypatch):
    """Few heads and no saved states: with the split's buffers in the workspace the scan
    runs in k = min(4, CUs / (2 B H)) segments at once and the fix-up kernels chain them;
    y and the final state against the oracle and the one-pass scan."""
    monkeypatch.setenv("THESEUS_WKV7_CUS", "256")
    lib = W.extension().lib
    need = int(lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0))
    recs = B * H * (-(-T // 16)) * RECORD_BYTES
    assert need > recs
    print(f"  records time split B={B} T={T} H={H}", flush=True)
    inp = _inputs(B, T, H, seed=5300 + T)
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0 = inp["s0"].cuda()
    ws = torch.empty((need,), dtype=torch.uint8, device="cuda")
    y_s, s_s = _fwd(lib, xs, s0, ws, need)
    y_1, s_1 = _fwd(lib, xs, s0, ws, recs)
    y_ref, s_ref = _oracle_fwd(inp)
    for name, got, ref, one in [("y", y_s, y_ref, y_1), ("sT", s_s, s_ref, s_1)]:
        _check(name, got, ref, torch.bfloat16)
        _split_vs_one_pass(name, got, one)
    with torch.no_grad():
        y_op, s_op = W.wkv7(*xs, s0)
    torch.cuda.synchronize()
    assert torch.equal(y_op, y_s) and torch.equal(s_op, s_s)


@pytest.mark.parametrize("mode", ["wide", "max_decay", "no_decay"])
def test_record_forward_at_the_ends_of_the_decay_range(mode, monkeypatch):
    """w ~ N(0, 8^2), w = +30 (the strongest decay on every step: e^{-g} reaches its
    largest, about 1.6e4 at the end of a chunk) and w = -30 (no decay): one pass with
    saved states and the time split, against the oracle."""
    monkeypatch.setenv("THESEUS_WKV7_CUS", "256")
    B, T, H = 1, 400, 3
    print(f"  records decays={mode}", flush=True)
    inp = _inputs(B, T, H, seed=5400, w_mode=mode)
    ext = W.extension()
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0 = inp["s0"].cuda()
    y_ref, s_ref = _oracle_fwd(inp)
    y_h, s_h, _ = ext.forward(*xs, s0, True)
    with torch.no_grad():
        y_s, s_s = W.wkv7(*xs, s0)
    torch.cuda.synchronize()
    for name, got, ref in [("y", y_h, y_ref), ("sT", s_h, s_ref), ("y", y_s, y_ref), ("sT", s_s, s_ref)]:
        _check(name, got, ref, torch.bfloat16)


def test_teacher_geometry_against_oracle():
    """B=1, T=2048, H=32 (a 4096-wide layer of 128-key heads), forward with saved states
    and backward, all nine outputs against the oracle."""
    _parity(1, 2048, 32, N, torch.bfloat16, seed=5500)


def test_noalloc_forward_stays_step_serial():
    """theseus_wkv7_forward_noalloc brings no workspace, so N = 128 runs step-serial there
    (the records need one): same results as the step-serial forward, to fp32 rounding."""
    B, T, H = 1, 40, 2
    lib = W.extension().lib
    inp = _inputs(B, T, H, seed=5600)
    xs = [inp[n].cuda() for n in "rwkvab"]
    s0 = inp["s0"].cuda()
    y = torch.empty((B, T, H, N), dtype=torch.bfloat16, device="cuda")
    sT = torch.empty_like(s0)
    p = lambda t: ctypes.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    st = lib.theseus_wkv7_forward_noalloc(B, T, H, N, 0, *map(p, (*xs, s0, y, sT)), p(None),
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0
    y_q, s_q = _fwd(lib, xs, s0, None, 0)
    assert torch.equal(y, y_q) and torch.equal(sT, s_q)
    y_ref, s_ref = _oracle_fwd(inp)
    _check("y", y, y_ref, torch.bfloat16)
    _check("sT", sT, s_ref, torch.bfloat16)
