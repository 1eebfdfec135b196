"""The fused optimizer step after backward (theseus.optim.FusedAdamW, C ABI
include/theseus_optim.h) against the reference's own sequence
(train.py:202-208: scale the gradients, clip_grad_norm_, torch.optim.AdamW
fused, the two parameter groups of theseus/stage.py:36-42) on identical
gradients, and the C ABI's host-side checks on the CPU."""
import ctypes
import math
import re
import subprocess
from pathlib import Path

import pytest
import torch

from theseus.timemix import TimeMix

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "theseus_optim.h"


# ------------------------------------------------------------------------- CPU
def test_optim_header_symbols_are_exported():
    from theseus import optim
    lib = optim._lib()
    names = set(re.findall(r"\b(theseus_adamw_\w+)\s*\(", HEADER.read_text()))
    assert names == {"theseus_adamw_workspace_size", "theseus_adamw_step"}
    for n in names:
        assert hasattr(lib, n)


def test_ctypes_struct_matches_the_c_layout(tmp_path):
    """Field offsets and size of theseus_adamw_tensor as a C compiler lays it out."""
    from theseus.optim import _Tensor
    src = tmp_path / "layout.c"
    fields = [f[0] for f in _Tensor._fields_]
    src.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"theseus_optim.h\"\nint main(void){\n"
                   + "".join(f'printf("%zu\\n", offsetof(theseus_adamw_tensor, {f}));\n' for f in fields)
                   + 'printf("%zu\\n", sizeof(theseus_adamw_tensor));\nreturn 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(_Tensor, f).offset for f in fields] + [ctypes.sizeof(_Tensor)]
    assert got == want


def test_adamw_abi_rejects_bad_arguments_before_launching():
    from theseus.optim import _Tensor, _lib
    lib = _lib()
    one = (_Tensor * 1)(_Tensor(16, 16, 16, 16, 100000, 1e-3, 0.0, 1e-3, 1.0))
    res = ctypes.c_void_p(16)
    assert lib.theseus_adamw_workspace_size(one, 1) == math.ceil(100000 / 16384) * 8
    # (status codes of theseus_wkv7.h: 1 shape, 3 null pointer, 4 workspace)
    assert lib.theseus_adamw_step(one, -1, 1, 1, .9, .999, 1e-8, 1, res, None, 0, None) == 1
    assert lib.theseus_adamw_step(one, 1, 1, 1, .9, .999, 1e-8, 1, None, None, 0, None) == 3
    assert lib.theseus_adamw_step(one, 1, 1, 1, .9, .999, 1e-8, 1, res, None, 0, None) == 4
    assert lib.theseus_adamw_step(one, 1, 1, 1, .9, .999, 1e-8, 1, res, ctypes.c_void_p(16), 8, None) == 4
    neg = (_Tensor * 1)(_Tensor(16, 16, 16, 16, -5, 1e-3, 0.0, 1e-3, 1.0))
    assert lib.theseus_adamw_step(neg, 1, 1, 1, .9, .999, 1e-8, 1, res, None, 0, None) == 1
    nul = (_Tensor * 1)(_Tensor(16, None, 16, 16, 5, 1e-3, 0.0, 1e-3, 1.0))
    assert lib.theseus_adamw_step(nul, 1, 1, 1, .9, .999, 1e-8, 1, res, ctypes.c_void_p(16), 64, None) == 3


def test_fused_adamw_validates_like_adamw():
    from theseus.optim import FusedAdamW
    p = [torch.nn.Parameter(torch.zeros(3))]
    for bad in (dict(lr=-1.0), dict(eps=-1.0), dict(betas=(1.0, .9)), dict(weight_decay=-.1)):
        with pytest.raises(ValueError):
            FusedAdamW(p, **bad)


# ------------------------------------------------------------------------- GPU
def _groups(model):
    """theseus/stage.py:36-38: 2-D ``.weight`` tensors decay, everything else does not."""
    decay, no_decay = [], []
    for name, p in model.named_parameters():
        (decay if name.endswith(".weight") and p.ndim == 2 else no_decay).append(p)
    return decay, no_decay


def _pair(C, seed, wd=.1, lr=3e-3, betas=(.9, .95), eps=1e-8):
    from theseus.optim import FusedAdamW
    # the layer's parameter schema at width C, filled with seeded N(0, 0.02) values
    with torch.device("meta"):
        a = TimeMix(C, 1, 4, head_size=64, backend="cuda")
        b = TimeMix(C, 1, 4, head_size=64, backend="cuda")
    a, b = a.to_empty(device="cuda"), b.to_empty(device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(seed)
    with torch.no_grad():
        for pa, pb in zip(a.parameters(), b.parameters()):
            pa.copy_(torch.randn(pa.shape, generator=gen, device="cuda") * .02)
            pb.copy_(pa)
    da, na = _groups(a)
    db, nb = _groups(b)
    ours = FusedAdamW([{"params": da, "weight_decay": wd}, {"params": na, "weight_decay": 0.}],
                      lr=lr, betas=betas, eps=eps)
    ref = torch.optim.AdamW([{"params": db, "weight_decay": wd}, {"params": nb, "weight_decay": 0.}],
                            lr=lr, betas=betas, eps=eps, fused=True)
    return a, b, ours, ref


def _grads(a, b, gen, mag):
    for pa, pb in zip(a.parameters(), b.parameters()):
        g = torch.randn(pa.shape, generator=gen, device="cuda") * mag
        pa.grad, pb.grad = g.clone(), g.clone()


def _close(x, y, what, atol=1e-7):
    """fp32 rounding-order differences only: a few ulps of the values, which is ~1e-4 of
    one step's update (lr) at atol."""
    torch.testing.assert_close(x, y, rtol=2e-5, atol=atol, msg=lambda m: f"{what}: {m}")


@pytest.mark.gpu
@pytest.mark.parametrize("C", [256, 5120], ids=["C256", "config3-layer-112M"])
def test_step_after_backward_matches_the_reference_sequence(C):
    """Five steps with gradient scale 3/7 and clip norm 1.0 (gradient sizes chosen so
    that some steps clip and others do not); parameters, both moments and the norm
    against p.grad.mul_ + clip_grad_norm_ + AdamW(fused=True)."""
    a, b, ours, ref = _pair(C, seed=7)
    gen = torch.Generator(device="cuda").manual_seed(5)
    n_params = sum(p.numel() for p in a.parameters())
    steps = 5 if C == 256 else 2
    for s in range(steps):
        mag = (.3 if s % 2 else 3.0) / math.sqrt(n_params)  # norms ~0.13 / ~1.3 after scaling
        _grads(a, b, gen, mag)
        norm = ours.step_after_backward(grad_scale=3 / 7, max_norm=1.0)
        for p in b.parameters():
            p.grad.mul_(3 / 7)
        rnorm = torch.nn.utils.clip_grad_norm_(b.parameters(), 1.0, error_if_nonfinite=True)
        ref.step()
        print(f"    step {s}: norm {float(norm):.6f} (reference {float(rnorm):.6f})", flush=True)
        torch.testing.assert_close(norm, rnorm, rtol=1e-5, atol=0)
        for (n, pa), pb in zip(a.named_parameters(), b.parameters()):
            _close(pa, pb, n)
            sa, sb = ours.state[pa], ref.state[pb]
            _close(sa["exp_avg"], sb["exp_avg"], n + ".exp_avg")
            _close(sa["exp_avg_sq"], sb["exp_avg_sq"], n + ".exp_avg_sq")
            assert float(sa["step"]) == float(sb["step"]) == s + 1
        ours.zero_grad(set_to_none=True)
        ref.zero_grad(set_to_none=True)


@pytest.mark.gpu
def test_plain_step_is_adamw_and_many_odd_tensors():
    """step() against torch's AdamW over 45 tensors (two kernel launches of at most 32)
    of odd sizes, one a view at a 4-byte offset (no 16-byte vector path), tails that
    are not multiples of 4, and one bigger than a chunk."""
    from theseus.optim import FusedAdamW
    torch.manual_seed(3)
    sizes = [1, 3, 5, 7, 17, 33, 100, 1023, 16384, 16385, 40001] + [64 * i + 3 for i in range(34)]
    base = torch.randn(sum(sizes) + 1, device="cuda")
    pa = [torch.nn.Parameter(torch.randn(n, device="cuda")) for n in sizes]
    pa[5] = torch.nn.Parameter(base[1:1 + sizes[5]])  # data at a 4-byte offset
    assert pa[5].data_ptr() % 16 != 0
    pb = [torch.nn.Parameter(p.detach().clone()) for p in pa]
    ours = FusedAdamW(pa, lr=1e-2, weight_decay=.05)
    ref = torch.optim.AdamW(pb, lr=1e-2, weight_decay=.05, foreach=False)
    for _ in range(3):
        for x, y in zip(pa, pb):
            g = torch.randn_like(x)
            x.grad, y.grad = g.clone(), g.clone()
        ours.step()
        ref.step()
    for i, (x, y) in enumerate(zip(pa, pb)):
        _close(x, y, f"tensor {i} (n={sizes[i]})", atol=1e-6)  # |p| ~ 1, lr 1e-2


@pytest.mark.gpu
def test_nonfinite_norm_raises_and_changes_nothing():
    from theseus.optim import NONFINITE_MSG
    a, b, ours, _ = _pair(256, seed=9)
    gen = torch.Generator(device="cuda").manual_seed(1)
    _grads(a, b, gen, 1e-3)
    ours.step_after_backward(grad_scale=1.0, max_norm=1.0)
    before = {n: p.detach().clone() for n, p in a.named_parameters()}
    moments = {n: ours.state[p]["exp_avg"].clone() for n, p in a.named_parameters()}
    _grads(a, b, gen, 1e-3)
    a.w1.grad[3, 4] = float("inf")
    with pytest.raises(RuntimeError, match="non-finite"):
        ours.step_after_backward(grad_scale=1.0, max_norm=1.0)
    for n, p in a.named_parameters():
        assert torch.equal(p, before[n]) and torch.equal(ours.state[p]["exp_avg"], moments[n]), n
        assert float(ours.state[p]["step"]) == 1.0
    assert "error_if_nonfinite=False" in NONFINITE_MSG
    norm = ours.step_after_backward(grad_scale=1.0, max_norm=1.0, error_if_nonfinite=False)
    assert not torch.isfinite(norm)
    assert torch.isnan(a.w1).any()  # the update ran with the non-finite factor, as torch's would


@pytest.mark.gpu
def test_fused_step_is_deterministic():
    runs = []
    for _ in range(2):
        a, b, ours, _ = _pair(320, seed=4)
        gen = torch.Generator(device="cuda").manual_seed(2)
        for _ in range(3):
            _grads(a, b, gen, 1e-2)
            norm = ours.step_after_backward(grad_scale=.5, max_norm=.7)
        runs.append([p.detach().clone() for p in a.parameters()] + [norm.clone()])
    for x, y in zip(*runs):
        assert torch.equal(x, y)
