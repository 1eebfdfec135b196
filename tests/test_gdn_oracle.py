"""Pins the oracle's "exp" decay mode and its GDN operand mapping (the gated delta
rule of the reference's teacher layers as the converter's contract writes it,
convert_qwen2rwkv_lightning.py:382-385) before it checks the GDN kernels.

Independent checks: the published library routine the reference's teacher runs
(transformers' ``torch_recurrent_gated_delta_rule`` and ``torch_chunk_gated_delta_rule``,
theseus/hf_model.py:28-52 dispatches to them; they compute in float32); special cases with
textbook answers (no decay and no write leaves the state; the delta rule's exact
write S^T k = v for a unit key and beta = 1; a decay of exp(-60) forgets the past);
central finite differences and float64 torch autograd for the backward; numpy == C.
"""
import numpy as np
import pytest
import torch

from oracle import wkv7_oracle as O


def _gdn_inputs(B, T, H, N, seed, g_scale=1.0, normalise=True):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((B, T, H, N)) for _ in range(3))
    if normalise:  # the layer's q/k L2 norm ("gdn_qk_normalization", :381)
        q /= np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        k /= np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    g = -np.exp(rng.standard_normal((B, T, H))) * g_scale  # -exp(A_log) softplus(.) < 0
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    s0 = rng.standard_normal((B, H, N, N)) * .1           # [B,H,key,value]
    return q, k, v, g, beta, s0


def _near(got, ref, rl=1e-5):
    """transformers' GDN functions compute in float32 whatever the input dtype (they cast
    with .to(torch.float32)), so the pin is at float32 accuracy: a dropped term, a wrong
    sign or a transposed state moves the result by O(1), far beyond this."""
    ref = np.asarray(ref, dtype=np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < rl
    assert np.max(np.abs(got - ref)) < 1e-4


def _hf():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as M
    import inspect
    # the undecorated torch functions (the hub-kernel wrapper only dispatches on CUDA)
    return inspect.unwrap(M.torch_recurrent_gated_delta_rule), inspect.unwrap(M.torch_chunk_gated_delta_rule)


@pytest.mark.parametrize("l2", [False, True])
def test_gdn_matches_transformers_recurrent_rule(l2):
    rec, _ = _hf()
    q, k, v, g, beta, s0 = _gdn_inputs(2, 19, 3, 8, seed=1, normalise=False)
    t = [torch.from_numpy(x) for x in (q, k, v, g, beta, s0)]
    o_hf, s_hf = rec(*t[:5], initial_state=t[5], output_final_state=True, use_qk_l2norm_in_kernel=l2)
    if l2:  # the function normalises q and k itself (l2norm, eps 1e-6)
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    y, sT = O.gdn_forward(q, k, v, g, beta, s0)
    _near(y, o_hf.numpy())
    _near(sT, s_hf.numpy())


def test_gdn_matches_transformers_chunk_rule():
    """The chunked form HF uses for long or differentiable work (same recurrence)."""
    _, chunk = _hf()
    q, k, v, g, beta, s0 = _gdn_inputs(1, 70, 2, 16, seed=2)
    t = [torch.from_numpy(x) for x in (q, k, v, g, beta, s0)]
    o_hf, s_hf = chunk(*t[:5], chunk_size=64, initial_state=t[5], output_final_state=True)
    y, sT = O.gdn_forward(q, k, v, g, beta, s0)
    _near(y, o_hf.numpy())
    _near(sT, s_hf.numpy())


def test_exp_mode_special_cases():
    B, T, H, N = 1, 5, 2, 6
    q, k, v, g, beta, s0 = _gdn_inputs(B, T, H, N, seed=3)
    # g = 0 and beta = 0: no decay, no write -> the state stays, y_t = S0^T q / sqrt(N)
    y, sT = O.gdn_forward(q, k, v, np.zeros_like(g), np.zeros_like(beta), s0)
    np.testing.assert_allclose(sT, s0, atol=1e-15)
    np.testing.assert_allclose(y, np.einsum("bhkv,bthk->bthv", s0, q) / np.sqrt(N), atol=1e-14)
    # beta = 1, g = 0, unit key: the delta rule writes v exactly, S_1^T k = v
    k1 = k / np.linalg.norm(k, axis=-1, keepdims=True)
    _, s1 = O.gdn_forward(q[:, :1], k1[:, :1], v[:, :1], np.zeros((B, 1, H)), np.ones((B, 1, H)), s0)
    np.testing.assert_allclose(np.einsum("bhkv,bhk->bhv", s1, k1[:, 0]), v[:, 0], atol=1e-13)
    # g = -60 on every step: exp(g) ~ 1e-26 wipes the past, so the state is the last write
    yl, sl = O.gdn_forward(q, k, v, np.full_like(g, -60.0), beta, s0)
    last = beta[:, -1, :, None, None] * np.einsum("bhk,bhv->bhkv", k[:, -1], v[:, -1])
    np.testing.assert_allclose(sl, last, atol=1e-20)
    # the "exp" decay itself, and rwkv mode untouched
    np.testing.assert_allclose(O.decay(np.array([-2.0, 0.0, .5]), "exp"), np.exp([-2.0, 0.0, .5]))
    with pytest.raises(ValueError):
        O.decay(np.zeros(2), "sigmoid")


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_exp_mode_backward_by_finite_differences(impl):
    rng = np.random.default_rng(4)
    B, T, H, N = 1, 4, 1, 3
    r, k, v, dy = (rng.standard_normal((B, T, H, N)) for _ in range(4))
    w = -np.abs(rng.standard_normal((B, T, H, N)))
    a, b = rng.standard_normal((B, T, H, N)) * .5, rng.standard_normal((B, T, H, N)) * .5
    s0, dsT = rng.standard_normal((B, H, N, N)), rng.standard_normal((B, H, N, N))
    args = [r, w, k, v, a, b, s0]
    bwd = O.backward if impl == "numpy" else O.backward_c
    grads = bwd(*args, dy, dsT, mode="exp")

    def loss(xs):
        y, sT = O.forward(*xs, mode="exp")
        return float((y * dy).sum() + (sT * dsT).sum())

    eps = 1e-6
    for idx, g in zip(range(7), grads):
        num = np.zeros_like(args[idx])
        it = np.nditer(args[idx], flags=["multi_index"])
        for _ in it:
            m = it.multi_index
            hi = [x.copy() for x in args]
            lo = [x.copy() for x in args]
            hi[idx][m] += eps
            lo[idx][m] -= eps
            num[m] = (loss(hi) - loss(lo)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-7, err_msg=f"grad {idx}")


def test_exp_mode_backward_against_torch_autograd_and_c():
    rng = np.random.default_rng(5)
    B, T, H, N = 2, 21, 2, 5
    r, k, v, dy = (rng.standard_normal((B, T, H, N)) for _ in range(4))
    w = -3 * np.abs(rng.standard_normal((B, T, H, N)))
    a, b = rng.standard_normal((B, T, H, N)) * .4, rng.standard_normal((B, T, H, N)) * .4
    s0, dsT = rng.standard_normal((B, H, N, N)), rng.standard_normal((B, H, N, N))
    xs = [torch.tensor(x, requires_grad=True) for x in (r, w, k, v, a, b, s0)]
    S = xs[6]
    ys = []
    for t in range(T):  # the recurrence written directly in torch (exp decay)
        sa = (S * xs[4][:, t, :, None, :]).sum(-1)
        S = S * torch.exp(xs[1][:, t, :, None, :]) + sa[..., None] * xs[5][:, t, :, None, :] \
            + xs[3][:, t, :, :, None] * xs[2][:, t, :, None, :]
        ys.append((S * xs[0][:, t, :, None, :]).sum(-1))
    y = torch.stack(ys, 1)
    ((y * torch.from_numpy(dy)).sum() + (S * torch.from_numpy(dsT)).sum()).backward()
    ours = O.backward(r, w, k, v, a, b, s0, dy, dsT, mode="exp")
    ours_c = O.backward_c(r, w, k, v, a, b, s0, dy, dsT, mode="exp")
    for x, g, gc in zip(xs, ours, ours_c):
        np.testing.assert_allclose(g, x.grad.numpy(), rtol=1e-10, atol=1e-11)
        np.testing.assert_allclose(gc, g, rtol=1e-11, atol=1e-12)
    yf, sf = O.forward(r, w, k, v, a, b, s0, mode="exp")
    yc, sc = O.forward_c(r, w, k, v, a, b, s0, mode="exp")
    np.testing.assert_allclose(yf, y.detach().numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(yc, yf, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(sc, sf, rtol=1e-12, atol=1e-13)
