"""CPU checks of the C-ABI library and of the Python boundary's host logic.

No kernel is launched here: the library is loaded, every symbol declared in
include/theseus_wkv7.h is looked up, and argument validation is exercised
(it returns before any HIP call).
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import theseus.wkv7 as W

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "theseus_wkv7.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(theseus_wkv7_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_symbols()
    for required in ("theseus_wkv7_forward", "theseus_wkv7_backward", "theseus_wkv7_decode_step",
                     "theseus_wkv7_error_string", "theseus_wkv7_abi_version"):
        assert required in names


def test_library_loads_and_exports_every_declared_symbol():
    assert W.LIB_PATH.exists(), "build first: make -C rwkv-theseus_amd/csrc"
    lib = ctypes.CDLL(str(W.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def declared_arity(header=HEADER):
    """{function: number of parameters} parsed from a header."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(theseus_\w+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_bindings_match_header_arity():
    ext = W.extension()
    arity = declared_arity()
    assert arity["theseus_wkv7_forward"] == 18 and arity["theseus_wkv7_backward"] == 24
    for name, n in arity.items():
        fn = getattr(ext.lib, name)
        bound = len(fn.argtypes) if fn.argtypes is not None else 0
        assert bound == n, (name, bound, n)


def test_timemix_abi_exported_and_bound_with_header_arity():
    from theseus import fused
    lib = fused._lib()
    assert lib is not None
    arity = declared_arity(ROOT / "include" / "theseus_timemix.h")
    assert len(arity) == 12
    for name, n in arity.items():
        fn = getattr(lib, name)
        assert fn.argtypes is not None and len(fn.argtypes) == n, (name, n)


def test_timemix_abi_rejects_shapes_before_launching():
    """Every fused TimeMix entry point checks B, T, C first (status 1, nothing enqueued):
    C must be a positive multiple of 64, and B*T may not exceed 65535 blocks of 64 tokens
    along the grid's y dimension.  Null pointers are never reached."""
    from theseus import fused
    lib = fused._lib()
    names = ["theseus_tm_shift_lerp_fwd", "theseus_tm_shift_lerp_bwd", "theseus_tm_add_param_fwd",
             "theseus_tm_kk_fwd", "theseus_tm_kk_bwd", "theseus_tm_gn_fwd", "theseus_tm_gn_bwd"]
    for B, T, C in [(1 << 16, 1 << 13, 64), (65535, 65, 64), (1, 4, 96), (0, 4, 64), (1, 0, 64)]:
        for name in names:
            fn = getattr(lib, name)
            rest = [0.0 if t is ctypes.c_float else 0 if t is ctypes.c_size_t else None for t in fn.argtypes[3:]]
            assert fn(B, T, C, *rest) == 1, (name, B, T, C)
    # exactly 65535 blocks of 64 tokens passes the shape check and stops at the null pointers
    assert lib.theseus_tm_shift_lerp_fwd(65535, 64, 64, None, None, None, None, None) not in (0, 1)


def test_host_queries():
    ext = W.extension()
    assert ext.abi_version == 2
    assert ext.checkpoint_interval == 16
    lib = ext.lib
    assert ext.checkpoint_count(1) == 2
    assert ext.checkpoint_count(16) == 2
    assert ext.checkpoint_count(17) == 3
    assert ext.checkpoint_count(2048) == 129
    assert lib.theseus_wkv7_checkpoint_count(0) == 0
    assert lib.theseus_wkv7_error_string(0) == b"ok"
    assert lib.theseus_wkv7_error_string(1) == b"invalid T or head size (2..128)"
    assert lib.theseus_wkv7_error_string(2) == b"expected BF16 or FP32"
    assert lib.theseus_wkv7_error_string(99) == b"unknown status"
    assert lib.theseus_wkv7_backward_workspace_size(1, 0, 1, 64, 0) == 0  # invalid T
    assert lib.theseus_wkv7_forward_workspace_size(1, 0, 1, 64, 0) == 0
    assert lib.theseus_wkv7_backward_workspace_size(2, 32, 3, 64, 1) > 0   # step-serial replay
    assert lib.theseus_wkv7_forward_workspace_size(2, 32, 3, 64, 1) == 0


def test_schedule_workspace_follows_the_cu_count(monkeypatch):
    """Chunked kernels: a workspace only when heads are cut between workgroups.

    With c CUs, J = B*H heads of n chunks go L = max(n, ceil(J n / c)) to a
    workgroup; a head is cut when L is not a multiple of n, and then every one
    of the G = ceil(J n / L) workgroups has a 256-byte-aligned counter block
    plus a handoff of N*N floats (forward: the state) or N*N + N floats (backward:
    dL/dS and the decay-gradient carry).
    """
    lib = W.extension().lib
    N = 64

    def expect(B, T, H, cus, per):
        n = -(-T // 16)
        J = B * H
        L = max(n, -(-J * n // cus))
        if L % n == 0:
            return 0
        G = -(-J * n // L)
        return -(-4 * G // 256) * 256 + G * per * 4

    for B, T, H, cus in [(2, 32, 3, 6), (2, 32, 3, 5), (1, 100, 6, 4), (4, 2048, 80, 256),
                         (4, 2048, 64, 256), (4, 2048, 80, 255), (1, 16, 7, 3), (3, 33, 5, 1)]:
        monkeypatch.setenv("THESEUS_WKV7_CUS", str(cus))
        f = lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0)
        b = lib.theseus_wkv7_backward_workspace_size(B, T, H, N, 0)
        assert f == expect(B, T, H, cus, N * N), (B, T, H, cus)
        assert b == expect(B, T, H, cus, N * N + N), (B, T, H, cus)
    monkeypatch.setenv("THESEUS_WKV7_CUS", "256")
    # config 2: 320 heads of 128 chunks on 256 CUs -> L = 160, G = 256, cut
    assert lib.theseus_wkv7_forward_workspace_size(4, 2048, 80, 64, 0) == 1024 + 256 * 4096 * 4
    # 256 heads: one each, nothing cut
    assert lib.theseus_wkv7_backward_workspace_size(4, 2048, 64, 64, 0) == 0


@pytest.mark.parametrize("B,T,H,N,dtype,code", [
    (1, 0, 1, 64, 0, 1), (1, 4, 1, 1, 0, 1), (1, 4, 1, 129, 0, 1), (0, 4, 1, 64, 0, 1),
    (1, 4, 1, 64, 7, 2), (1, 4, 1, 64, 0, 3)])
def test_c_abi_rejects_bad_arguments_without_launching(B, T, H, N, dtype, code):
    lib = W.extension().lib
    null = ctypes.c_void_p(0)
    status = lib.theseus_wkv7_forward(B, T, H, N, dtype, *([null] * 11), 0, null)
    assert status == code
    status = lib.theseus_wkv7_backward(B, T, H, N, dtype, *([null] * 17), 0, null)
    assert status == code


def test_c_abi_rejects_a_small_workspace_without_launching(monkeypatch):
    """With heads cut between workgroups the chunked kernels need the workspace;
    a smaller one is refused before anything is enqueued (THESEUS_WKV7_ERR_WORKSPACE)."""
    lib = W.extension().lib
    monkeypatch.setenv("THESEUS_WKV7_CUS", "5")
    B, T, H, N = 2, 100, 3, 64
    need_f = lib.theseus_wkv7_forward_workspace_size(B, T, H, N, 0)
    need_b = lib.theseus_wkv7_backward_workspace_size(B, T, H, N, 0)
    assert need_f > 0 and need_b > 0
    p = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    null = ctypes.c_void_p(0)
    assert lib.theseus_wkv7_forward(B, T, H, N, 0, *([p] * 9), null, p, need_f - 1, null) == 4
    assert lib.theseus_wkv7_forward(B, T, H, N, 0, *([p] * 9), null, null, need_f, null) == 4
    assert lib.theseus_wkv7_backward(B, T, H, N, 0, *([p] * 8), null, *([p] * 7), p, need_b - 1, null) == 4


def test_backend_errors_match_reference():
    x = torch.zeros(1, 2, 1, 4)
    s = torch.zeros(1, 1, 4, 4)
    with pytest.raises(ValueError, match="Unknown WKV backend"):
        W.wkv7(x, x, x, x, x, x, s, backend="triton")
    with pytest.raises(ValueError, match="CUDA backend requested on CPU"):
        W.wkv7(x, x, x, x, x, x, s, backend="cuda")


def test_extension_checks_match_reference_messages():
    ext = W.extension()
    x = torch.zeros(1, 2, 1, 4)
    with pytest.raises(RuntimeError, match=r"expected contiguous CUDA \[B,T,H,N\]"):
        ext.forward(x, x, x, x, x, x, torch.zeros(1, 1, 4, 4), True)
    with pytest.raises(RuntimeError, match=r"expected contiguous CUDA \[B,T,H,N\]"):
        ext.backward(x, x, x, x, x, x, torch.zeros(1, 1, 2, 4, 4), x, None)


def test_reference_backend_on_cpu_matches_oracle():
    import numpy as np
    from oracle import wkv7_oracle as O
    from theseus.synthetic import wkv7_inputs
    inp = wkv7_inputs(1, 12, 2, 8, seed=11, dtype=torch.float32, s0_std=0.1)
    y, sT = W.wkv7(*(inp[n] for n in "rwkvab"), inp["s0"], backend="reference")
    yo, sTo = O.forward(*(inp[n].numpy() for n in "rwkvab"), inp["s0"].numpy())
    np.testing.assert_allclose(y.numpy(), yo, atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(sT.numpy(), sTo, atol=1e-4, rtol=1e-4)


def test_kernel_family_dispatch_predicate(monkeypatch):
    """theseus_wkv7_kernel_family: the chunked MFMA kernels (0) cover bf16 with N = 64 only
    while both 32-bit buffer ranges hold: every [B,T,H,64] token tensor under 2 GiB and one
    head's saved states (ceil(T/16)+1 states of 16 KiB) under 4 GiB.  Anything else runs on
    the step-serial kernels, with the reason as the code."""
    monkeypatch.delenv("THESEUS_WKV7_FAMILY", raising=False)
    lib = W.extension().lib
    fam = lib.theseus_wkv7_kernel_family
    assert fam(4, 2048, 80, 64, 0) == 0
    assert fam(4, 2048, 80, 64, 1) == 2   # fp32
    assert fam(4, 2048, 80, 32, 0) == 3   # head size
    assert fam(1, 2048, 32, 128, 0) == 6  # N = 128, bf16: the chunk-record kernels
    assert fam(1, 2048, 32, 128, 1) == 2
    assert fam(1, 16 * 98689, 1, 128, 0) == 6   # one head's records (43520 B per chunk) < 4 GiB
    assert fam(1, 16 * 98690, 1, 128, 0) == 3
    assert fam(65535, 32, 1, 128, 0) == 6 and fam(65536, 32, 1, 128, 0) == 3  # B*H on grid y
    # token tensors: B*T*H*64*2 bytes must stay below 2^31
    assert fam(1, (1 << 21) - 1, 8, 64, 0) == 0
    assert fam(1, 1 << 21, 8, 64, 0) == 4
    # saved states of one head: (ceil(T/16) + 1) * 64 * 64 * 4 bytes must stay below 2^32,
    # i.e. ceil(T/16) + 1 < 262144 -- reached long before 2 GiB of tokens when B*H is small
    t_max = 16 * (262144 - 2)
    assert fam(1, t_max, 1, 64, 0) == 0
    assert fam(1, t_max + 1, 1, 64, 0) == 4
    assert fam(1, 0, 1, 64, 0) == -1      # invalid sizes: minus the status code
    assert fam(1, 4, 1, 64, 9) == -2
    monkeypatch.setenv("THESEUS_WKV7_FAMILY", "seq")
    assert fam(4, 2048, 80, 64, 0) == 1


def test_step_serial_fallback_warns_and_strict_mode_refuses(monkeypatch):
    monkeypatch.delenv("THESEUS_WKV7_FAMILY", raising=False)
    ext = W.extension()
    with pytest.warns(RuntimeWarning, match="float32 token tensors"):
        ext._warn_fallback(1, 32, 2, 64, 1)
    with pytest.warns(RuntimeWarning, match="head size other than 64"):
        ext._warn_fallback(1, 32, 2, 8, 0)
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        ext._warn_fallback(1, 32, 2, 64, 0)  # chunked: silent
        ext._warn_fallback(1, 32, 2, 128, 0)  # the chunk-record kernels: silent
        monkeypatch.setenv("THESEUS_WKV7_FAMILY", "seq")
        ext._warn_fallback(1, 32, 2, 64, 0)  # an explicit request: silent
    monkeypatch.delenv("THESEUS_WKV7_FAMILY")
    monkeypatch.setenv("THESEUS_WKV7_STRICT", "1")
    with pytest.raises(RuntimeError, match="step-serial kernels"):
        ext._warn_fallback(1, 32, 2, 64, 1)


def test_fused_timemix_covers_only_what_its_grid_addresses():
    """Above 65535 token blocks of 64 the fused kernels refuse the shape; TimeMix must then
    take the reference's torch op sequence instead of raising."""
    from theseus import fused
    lim = 65535 * 64
    assert fused.MAX_TOKENS == lim
    ok = torch.empty((1, lim, 128), dtype=torch.bfloat16, device="meta")
    big = torch.empty((1, lim + 1, 128), dtype=torch.bfloat16, device="meta")
    two = torch.empty((2, lim // 2 + 1, 128), dtype=torch.bfloat16, device="meta")
    assert fused.available(ok, 64)
    assert not fused.available(big, 64) and not fused.available(two, 64)
    assert not fused.available(ok.float(), 64) and not fused.available(ok, 32)


def test_gdn_abi_exported_bound_and_validated():
    """include/theseus_gdn.h: every declared function exported and bound with the header's
    arity; sizes are checked before anything is enqueued (N must be 64 or 128)."""
    ext = W.extension()
    arity = declared_arity(ROOT / "include" / "theseus_gdn.h")
    assert arity == {"theseus_gdn_forward": 17, "theseus_gdn_forward_workspace_size": 4,
                     "theseus_gdn_forward_train": 17, "theseus_gdn_backward": 22,
                     "theseus_gdn_backward_workspace_size": 4}
    for name, n in arity.items():
        fn = getattr(ext.lib, name)
        assert fn.argtypes is not None and len(fn.argtypes) == n, (name, n)
    lib = ext.lib
    # one record per 16-step chunk: 43264 bytes at N = 128, 22784 at N = 64
    assert lib.theseus_gdn_forward_workspace_size(1, 2048, 32, 128) == 32 * 128 * 43264
    assert lib.theseus_gdn_forward_workspace_size(2, 17, 3, 64) == 2 * 3 * 2 * 22784
    # a head's records must stay under 4 GiB: 99273 chunks of 43264 bytes do, 99274 do not
    assert lib.theseus_gdn_forward_workspace_size(1, 16 * 99273, 1, 128) == 99273 * 43264
    assert lib.theseus_gdn_forward_workspace_size(1, 16 * 99274, 1, 128) == 0
    for B, T, H, N in [(1, 4, 1, 32), (1, 4, 1, 100), (0, 4, 1, 64), (1, 0, 1, 64), (1, 4, 70000, 64)]:
        assert lib.theseus_gdn_forward_workspace_size(B, T, H, N) == 0
        assert lib.theseus_gdn_forward(B, T, H, N, 1, 0, *[None] * 8, None, 0, None) == 1
    assert lib.theseus_gdn_forward(1, 4, 1, 64, 5, 0, *[None] * 8, None, 0, None) == 2  # dtype
    assert lib.theseus_gdn_forward(1, 4, 1, 64, 0, 1, *[None] * 8, None, 0, None) == 3  # null pointers
    # the training pair: saved states required; the backward takes N = 128 only, its
    # workspace 25088 bytes of scan record and a 64 KiB float32 dL/dS per chunk
    assert lib.theseus_gdn_forward_train(1, 4, 1, 64, 1, *[None] * 9, None, 0, None) == 3
    assert lib.theseus_gdn_forward_train(1, 4, 1, 100, 1, *[None] * 9, None, 0, None) == 1
    assert lib.theseus_gdn_backward_workspace_size(1, 2048, 32, 128) == 32 * 128 * (25088 + 65536)
    assert lib.theseus_gdn_backward_workspace_size(1, 2048, 32, 64) == 0
    assert lib.theseus_gdn_backward(1, 4, 1, 64, 1, *[None] * 14, None, 0, None) == 1
    assert lib.theseus_gdn_backward(1, 4, 1, 128, 5, *[None] * 14, None, 0, None) == 2
    assert lib.theseus_gdn_backward(1, 4, 1, 128, 1, *[None] * 14, None, 0, None) == 3
