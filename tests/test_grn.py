"""GRN on the CPU: the oracle pinned against independent checks, the module
API (mirrors the reference's tests/ops/test_grn.py) and the fused entry's
argument contract under fake tensors (mirrors tests/ops/test_grn_triton.py).

The oracle's backward is hand-derived; it is pinned against torch float64
autograd of the forward formula, central finite differences, the reference
tests' closed-form channel-coupling case and the all-zero input, and a planted
mistake (the cross-channel term dropped) must fail the autograd check.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode

from mednext_accel_amd import GlobalResponseNorm3d, global_response_norm3d_reference
from oracle import grn as ogrn


def torch_formula(x, gamma, beta, eps=1e-6):
    """GRN written independently with torch.norm (not the package's code)."""
    n = torch.stack([x[:, c].flatten(1).norm(dim=1) for c in range(x.shape[1])], dim=1)
    r = n / (n.sum(dim=1, keepdim=True) + eps)
    g = gamma.reshape(1, -1, 1, 1, 1)
    return x + g * x * r[..., None, None, None] + beta.reshape(1, -1, 1, 1, 1)


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("shape", [(2, 3, 2, 3, 4), (1, 5, 3, 1, 7), (3, 1, 2, 2, 2)])
def test_oracle_forward_and_backward_match_torch_autograd(shape):
    x, dy = rand(shape, 1), rand(shape, 2)
    gamma, beta = rand(shape[1], 3), rand(shape[1], 4)
    xt = torch.from_numpy(x).requires_grad_()
    gt = torch.from_numpy(gamma).requires_grad_()
    bt = torch.from_numpy(beta).requires_grad_()
    y = torch_formula(xt, gt, bt)
    dx, dg, db = torch.autograd.grad(y, (xt, gt, bt), torch.from_numpy(dy))
    np.testing.assert_allclose(ogrn.forward(x, gamma, beta), y.detach().numpy(), rtol=1e-13, atol=1e-13)
    odx, odg, odb = ogrn.backward(dy, x, gamma)
    np.testing.assert_allclose(odx, dx.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(odg, dg.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(odb, db.numpy(), rtol=1e-11, atol=1e-12)


def test_oracle_backward_matches_finite_differences():
    shape = (2, 3, 2, 2, 3)
    x, dy = rand(shape, 5), rand(shape, 6)
    gamma, beta = rand(3, 7), rand(3, 8)
    dx, dg, db = ogrn.backward(dy, x, gamma)
    h = 1e-6

    def loss(xv, gv, bv):
        return float((ogrn.forward(xv, gv, bv) * dy).sum())

    for idx in [(0, 0, 0, 0, 0), (1, 2, 1, 1, 2), (0, 1, 1, 0, 1)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        assert abs((loss(xp, gamma, beta) - loss(xm, gamma, beta)) / (2 * h) - dx[idx]) < 1e-6
    for c in range(3):
        gp, gm = gamma.copy(), gamma.copy()
        gp[c] += h
        gm[c] -= h
        assert abs((loss(x, gp, beta) - loss(x, gm, beta)) / (2 * h) - dg[c]) < 1e-6
        bp, bm = beta.copy(), beta.copy()
        bp[c] += h
        bm[c] -= h
        assert abs((loss(x, gamma, bp) - loss(x, gamma, bm)) / (2 * h) - db[c]) < 1e-6


def test_oracle_channel_coupling_closed_form():
    """x = (1, 2, 4), gamma = (2, 3, -4), dy only in channel 0: S = 7, g_0 = 1,
    T = gamma_0 g_0 n_0 = 2, so channels 1 and 2 get x (-T / (S + eps)^2) / n = -2 / (7 + eps)^2."""
    x = np.array([1.0, 2.0, 4.0]).reshape(1, 3, 1, 1, 1)
    gamma = np.array([2.0, 3.0, -4.0])
    dy = np.zeros_like(x)
    dy[:, 0] = 1.0
    dx, _, _ = ogrn.backward(dy, x, gamma)
    np.testing.assert_allclose(dx[0, 1:].ravel(), -2.0 / (7.0 + 1e-6) ** 2, rtol=1e-14)
    # channel 0: 1 + gamma_0 r_0 + x_0 (gamma_0 g_0 / (S + eps) - T / (S + eps)^2) / n_0
    s = 7.0 + 1e-6
    np.testing.assert_allclose(dx[0, 0].item(), 1 + 2 * (1 / s) + (2 / s - 2 / s**2), rtol=1e-14)


def test_oracle_zero_input_is_identity_gradient():
    shape = (2, 3, 2, 3, 5)
    x = np.zeros(shape)
    dy = rand(shape, 9)
    gamma, beta = rand(3, 10), rand(3, 11)
    y = ogrn.forward(x, gamma, beta)
    np.testing.assert_array_equal(y, np.broadcast_to(beta.reshape(1, 3, 1, 1, 1), shape))
    dx, dg, db = ogrn.backward(dy, x, gamma)
    np.testing.assert_array_equal(dx, dy)
    np.testing.assert_array_equal(dg, np.zeros(3))
    np.testing.assert_allclose(db, dy.sum(axis=(0, 2, 3, 4)))


def test_oracle_closed_forms():
    x = rand((2, 4, 3, 3, 3), 12)
    # zero affine parameters: identity
    np.testing.assert_array_equal(ogrn.forward(x, None, None), x)
    # one channel: r = n / (n + eps)
    n = np.sqrt((x[:, :1] ** 2).sum(axis=(2, 3, 4)))
    y = ogrn.forward(x[:, :1], np.array([2.0]), np.array([0.5]))
    np.testing.assert_allclose(y, x[:, :1] * (1 + 2 * (n / (n + 1e-6)))[..., None, None, None] + 0.5, rtol=1e-14)
    # ratios sum to S / (S + eps) per sample
    norms, r = ogrn.norms(x)
    np.testing.assert_allclose(r.sum(axis=1), norms.sum(axis=1) / (norms.sum(axis=1) + 1e-6), rtol=1e-14)


def test_planted_mistake_is_caught():
    """Dropping the cross-channel term T must fail the autograd pin."""
    shape = (1, 3, 2, 2, 2)
    x, dy, gamma = rand(shape, 13), rand(shape, 14), rand(3, 15)
    xt = torch.from_numpy(x).requires_grad_()
    y = torch_formula(xt, torch.from_numpy(gamma), torch.zeros(3, dtype=torch.float64))
    (dx_true,) = torch.autograd.grad(y, (xt,), torch.from_numpy(dy))
    n, r = ogrn.norms(x)
    flat_x, flat_dy = x.reshape(1, 3, -1), dy.reshape(1, 3, -1)
    gc = (flat_dy * flat_x).sum(axis=2)
    s = n.sum(axis=1, keepdims=True) + 1e-6
    wrong = flat_dy * (1 + gamma * r)[..., None] + flat_x * (gamma * gc / s / n)[..., None]
    assert np.abs(wrong.reshape(shape) - dx_true.numpy()).max() > 1e-3


# ------------------------------------------------------------------ module API


def test_reference_formula_matches_oracle_and_keeps_half_dtype():
    torch.manual_seed(0)
    module = GlobalResponseNorm3d(3).double()
    module.gamma.data.normal_()
    module.beta.data.normal_()
    x = torch.randn(2, 3, 2, 3, 4, dtype=torch.double)
    want = ogrn.forward(x.numpy(), module.gamma.detach().numpy(), module.beta.detach().numpy())
    np.testing.assert_allclose(module(x).detach().numpy(), want, rtol=1e-13, atol=1e-13)
    for dtype in (torch.float16, torch.bfloat16):
        half = GlobalResponseNorm3d(3)
        half.gamma.data.normal_()
        out = half(torch.randn(2, 3, 2, 3, 4, dtype=dtype))
        assert out.dtype is dtype


def test_zero_input_gradient_is_finite():
    module = GlobalResponseNorm3d(4).double()
    x = torch.zeros(2, 4, 3, 5, 7, dtype=torch.double, requires_grad=True)
    module(x).sum().backward()
    assert torch.isfinite(x.grad).all()


@pytest.mark.parametrize("shape", [(3, 2, 3, 4), (2, 3, 2, 3)])
def test_reference_rejects_non_ncdhw(shape):
    with pytest.raises(ValueError, match="NCDHW"):
        global_response_norm3d_reference(torch.randn(shape), torch.zeros(1, 3, 1, 1, 1), torch.zeros(1, 3, 1, 1, 1))


@pytest.mark.parametrize("channels", [0, -1])
def test_rejects_nonpositive_channels(channels):
    with pytest.raises(ValueError, match="channels"):
        GlobalResponseNorm3d(channels)


@pytest.mark.parametrize("eps", [0.0, -1e-6, float("nan")])
def test_rejects_bad_epsilon(eps):
    with pytest.raises(ValueError, match="eps"):
        GlobalResponseNorm3d(3, eps=eps)


def test_parameters_zero_initialised_with_broadcast_shape():
    module = GlobalResponseNorm3d(5)
    assert tuple(module.gamma.shape) == tuple(module.beta.shape) == (1, 5, 1, 1, 1)
    assert torch.count_nonzero(module.gamma) == 0 and torch.count_nonzero(module.beta) == 0
    assert list(module.state_dict()) == ["gamma", "beta"]


def _fake(mode, shape, dtype, *, device="cuda", stride=None):
    elem = (
        torch.empty(shape, device="meta", dtype=dtype)
        if stride is None
        else torch.empty_strided(shape, stride, device="meta", dtype=dtype)
    )
    return FakeTensor(mode, elem, torch.device(device))


@pytest.mark.parametrize(
    "case,message",
    [
        ("rank", "fused GRN expects a rank-5 NCDHW input"),
        ("cpu", "fused GRN requires CUDA tensors"),
        ("fp32", "fused GRN requires a float16 or bfloat16 input"),
        ("strided", "fused GRN requires a contiguous NCDHW input"),
        ("affine_dtype", "fused GRN requires float32 gamma and beta"),
        ("affine_shape", "fused GRN requires gamma and beta with shape"),
        ("affine_stride", "fused GRN requires contiguous gamma and beta"),
        ("device", "fused GRN requires all tensors on the same CUDA device"),
        ("empty", "fused GRN requires nonempty input dimensions"),
        ("epsilon", "fused GRN requires eps to be finite and positive"),
    ],
)
def test_fused_entry_rejects_unsupported_arguments(case, message):
    from mednext_accel_amd import hip_ops

    mode = FakeTensorMode()
    with mode:
        x = _fake(mode, (2, 3, 2, 3, 5), torch.float16)
        gamma = _fake(mode, (1, 3, 1, 1, 1), torch.float32)
        beta = _fake(mode, (1, 3, 1, 1, 1), torch.float32)
        eps = 1e-6
        if case == "rank":
            x = _fake(mode, (3, 2, 3, 5), torch.float16)
        elif case == "cpu":
            x = _fake(mode, (2, 3, 2, 3, 5), torch.float16, device="cpu")
        elif case == "fp32":
            x = _fake(mode, (2, 3, 2, 3, 5), torch.float32)
        elif case == "strided":
            x = _fake(mode, (2, 3, 2, 5, 3), torch.float16, stride=(90, 30, 15, 1, 5))
        elif case == "affine_dtype":
            gamma = _fake(mode, (1, 3, 1, 1, 1), torch.float16)
        elif case == "affine_shape":
            beta = _fake(mode, (3,), torch.float32)
        elif case == "affine_stride":
            gamma = _fake(mode, (1, 3, 1, 1, 1), torch.float32, stride=(6, 2, 1, 1, 1))
        elif case == "device":
            beta = _fake(mode, (1, 3, 1, 1, 1), torch.float32, device="cuda:1")
        elif case == "empty":
            x = _fake(mode, (0, 3, 2, 3, 5), torch.float16)
        elif case == "epsilon":
            eps = 0.0
        with pytest.raises(ValueError, match=message):
            hip_ops.fused_global_response_norm3d(x, gamma, beta, eps)
