"""Few-row GEMM of the TimeMix serving path (include/theseus_gemm.h, theseus.gemm):
Y = act(X W^T) for at most 128 rows, against float32 torch products of the same bf16
operands, on the shapes a C=5120 serving step runs (the r/k/v/output projections and the
w/a/g LoRAs) and ragged ones; split-K results deterministic; argument errors before
anything is enqueued."""
import ctypes

import pytest
import torch

from test_capi import ROOT, declared_arity
from theseus import gemm
from theseus import wkv7 as W

ERR_SHAPE, ERR_NULL, ERR_WORKSPACE, ERR_FLAGS = 1, 3, 4, 7


def test_gemm_abi_exported_bound_and_validated():
    """Every function of include/theseus_gemm.h is exported and bound with the header's
    arity; sizes, activation codes, pointers and workspace are checked on the host."""
    arity = declared_arity(ROOT / "include" / "theseus_gemm.h")
    assert arity == {"theseus_gemm_rows_workspace_size": 3, "theseus_gemm_rows": 10,
                     "theseus_gemm_rows_group_workspace_size": 3, "theseus_gemm_rows_group": 6}
    lib = gemm._lib()
    for name, n in arity.items():
        assert len(getattr(lib, name).argtypes) == n, name
    for M, N, K in [(0, 64, 64), (129, 64, 64), (4, 24, 64), (4, 64, 48), (4, 0, 64)]:
        assert lib.theseus_gemm_rows_workspace_size(M, N, K) == 0
        assert lib.theseus_gemm_rows(M, N, K, 0, None, None, None, None, 0, None) == ERR_SHAPE
    assert lib.theseus_gemm_rows(4, 64, 64, 3, None, None, None, None, 0, None) == ERR_FLAGS
    assert lib.theseus_gemm_rows(4, 64, 64, 0, None, None, None, None, 0, None) == ERR_NULL
    # groups: 1..8 products, every one of them valid, pointers checked
    pr = (gemm.Problem * 9)(*[gemm.Problem(64, 64, 0, None, None, None)] * 9)
    for count in (0, 9):
        assert lib.theseus_gemm_rows_group_workspace_size(4, count, pr) == 0
        assert lib.theseus_gemm_rows_group(4, count, pr, None, 0, None) == ERR_SHAPE
    assert lib.theseus_gemm_rows_group(129, 2, pr, None, 0, None) == ERR_SHAPE
    pr[1].N = 24
    assert lib.theseus_gemm_rows_group(4, 2, pr, None, 0, None) == ERR_SHAPE
    pr[1].N, pr[1].act = 64, 3
    assert lib.theseus_gemm_rows_group(4, 2, pr, None, 0, None) == ERR_FLAGS
    pr[1].act = 0
    assert lib.theseus_gemm_rows_group(4, 2, pr, None, 0, None) == ERR_NULL
    assert gemm.supported(64, 5120, 5120) and gemm.supported(1, 352, 5120) and gemm.supported(128, 5120, 192)
    assert not gemm.supported(129, 64, 64) and not gemm.supported(4, 24, 64) and not gemm.supported(4, 64, 48)


def _ref(x, w, act):
    """float32 product; an activation takes it rounded to bf16 (as torch under autocast).
    Returns (reference, bound on the error a bf16 result may carry): one bf16 rounding of
    the result, and with an activation one bf16 rounding of its input, whose last bit the
    summation order may flip, times the activation's slope."""
    y = x.float() @ w.float().t()
    if act == gemm.NONE:
        return y, 2.0 ** -8 * y.abs()
    yb = y.to(torch.bfloat16).float()
    r = torch.tanh(yb) if act == gemm.TANH else torch.sigmoid(yb)
    slope = 1 - r * r if act == gemm.TANH else r * (1 - r)
    return r, 2.0 ** -8 * r.abs() + 2.0 ** -7 * yb.abs() * slope


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,act", [
    (64, 5120, 5120, gemm.NONE),      # r, k, v, output projections at config 4
    (64, 192, 5120, gemm.TANH),       # LoRA down-projections (w: tanh, a: none, g: sigmoid)
    (64, 352, 5120, gemm.SIGMOID),
    (64, 5120, 192, gemm.NONE),       # LoRA up-projections
    (64, 5120, 352, gemm.NONE),
    (1, 5120, 5120, gemm.NONE), (7, 96, 640, gemm.TANH), (33, 16, 32, gemm.NONE),
    (100, 1040, 4096, gemm.SIGMOID), (128, 5120, 5120, gemm.NONE), (17, 272, 9984, gemm.NONE),
])
def test_gemm_rows_matches_float32_products(M, N, K, act):
    """Within one bf16 rounding of the float32 product (plus float32 summation-order
    noise), bitwise repeatable, whatever the workspace held before."""
    print(f"  gemm M={M} N={N} K={K} act={act}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, device="cuda", generator=g) / K ** .5).to(torch.bfloat16)
    lib = gemm._lib()
    nbytes = int(lib.theseus_gemm_rows_workspace_size(M, N, K))
    ws = torch.full((max(nbytes, 1),), 0xFF, dtype=torch.uint8, device="cuda")  # (NaN-filled partials)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    ys = []
    for _ in range(2):
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert lib.theseus_gemm_rows(M, N, K, act, P(x), P(w), P(y), P(ws), ctypes.c_size_t(nbytes), s) == 0
        ys.append(y)
    if nbytes:
        assert lib.theseus_gemm_rows(M, N, K, act, P(x), P(w), P(ys[0]), P(ws), ctypes.c_size_t(nbytes - 1), s) \
            == ERR_WORKSPACE
    torch.cuda.synchronize()
    ref, tol = _ref(x, w, act)
    err = (ys[0].float() - ref).abs()
    bar = tol + 1e-5 * ref.abs().max() + 1e-6
    print(f"    max err {err.max().item():.3e}, max |ref| {ref.abs().max().item():.3e}", flush=True)
    assert bool((err <= bar).all())
    assert torch.equal(ys[0], ys[1])


@pytest.mark.gpu
def test_gemm_python_wrappers_and_layouts():
    """gemm.linear takes nn.Linear's [out][in] weight as it is; gemm.lora the [in][out]
    LoRA matrices (transposed copies made per call, or once inside fused.param_cache),
    for [B,T,C] inputs and float32 weights (rounded to bf16 as autocast would)."""
    from theseus import fused
    g = torch.Generator(device="cuda").manual_seed(9)
    C, r = 512, 96
    x = torch.randn(4, 1, C, device="cuda", generator=g).to(torch.bfloat16)
    lin = (torch.randn(C, C, device="cuda", generator=g) / C ** .5).to(torch.bfloat16)
    down = torch.randn(C, r, device="cuda", generator=g) / C ** .5
    up = torch.randn(r, C, device="cuda", generator=g) / r ** .5
    with torch.no_grad():
        y = gemm.linear(x, lin)
        z = gemm.lora(x, down, up, gemm.TANH)
        store = {}
        with fused.param_cache(store):
            z2 = gemm.lora(x, down, up, gemm.TANH)
            assert len([k for k in store if k[0] == "gemm_t"]) == 2
    assert y.shape == (4, 1, C) and z.shape == (4, 1, C) and torch.equal(z, z2)
    yr = x.float() @ lin.float().t()
    mid = torch.tanh((x.float() @ down.to(torch.bfloat16).float()).to(torch.bfloat16).float()).to(torch.bfloat16)
    zr = mid.float() @ up.to(torch.bfloat16).float()
    assert ((y.float() - yr).abs() <= 2.0 ** -8 * yr.abs() + 1e-4).all()
    # (the middle product is rounded to bf16 on both sides; one bf16 ULP of it may flip)
    assert ((z.float() - zr).norm() / zr.norm()).item() < 4e-3


@pytest.mark.gpu
@pytest.mark.parametrize("M", [64, 5, 128])
def test_gemm_group_matches_single_products(M):
    """theseus_gemm_rows_group on a serving step's two groups at C=5120 (r, k, v and the
    LoRA first halves, 3 x 5120 + 192 + 192 + 352 columns; then the LoRA second halves)
    and on a ragged group whose small products split K: every product within the single
    call's bar of its float32 reference, and within twice that bar of theseus_gemm_rows (the
    two differ in the order of the float32 sums); repeatable bitwise."""
    g = torch.Generator(device="cuda").manual_seed(M + 5)
    rn = lambda *s: torch.randn(*s, device="cuda", generator=g)  # noqa: E731
    C = 5120
    shapes = [[(C, C, gemm.NONE)] * 3 + [(192, C, gemm.TANH), (192, C, gemm.NONE), (352, C, gemm.SIGMOID)],
              [(C, 192, gemm.NONE), (C, 192, gemm.NONE), (C, 352, gemm.NONE)],
              [(96, 640, gemm.TANH), (16, 4096, gemm.NONE), (1040, 1024, gemm.SIGMOID)]]
    for group in shapes:
        print(f"  group M={M}: {[(n, k) for n, k, _ in group]}", flush=True)
        xs = [rn(M, k).to(torch.bfloat16) for n, k, a in group]
        ws = [(rn(n, k) / k ** .5).to(torch.bfloat16) for n, k, a in group]
        with torch.no_grad():
            outs = gemm.group([(x, w, a, False) for x, w, (n, k, a) in zip(xs, ws, group)])
            again = gemm.group([(x, w, a, False) for x, w, (n, k, a) in zip(xs, ws, group)])
            single = [gemm.linear(x, w, a) for x, w, (n, k, a) in zip(xs, ws, group)]
        torch.cuda.synchronize()
        for y, y2, y1, x, w, (n, k, a) in zip(outs, again, single, xs, ws, group):
            assert torch.equal(y, y2)
            ref, tol = _ref(x, w, a)
            bar = tol + 1e-5 * ref.abs().max() + 1e-6  # (as test_gemm_rows_matches_float32_products)
            assert bool(((y.float() - ref).abs() <= bar).all()), (n, k)
            # (both within that bar of the float32 product, in different summation orders)
            assert bool(((y.float() - y1.float()).abs() <= 2 * bar).all()), (n, k)
