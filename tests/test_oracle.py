"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against (i) the library routine the reference
calls, in float64 (torch F.conv3d / F.group_norm / F.gelu + autograd), (ii) the
committed golden fixtures, and (iii) closed forms / brute force chosen so that
a plausible slip (flipped taps, wrong shift sign, dropped term, transposed
operand) fails at least one of them.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import depthwise as odw
from oracle import groupnorm as ogn
from oracle import pointwise as opw

GOLDEN = np.load(Path(__file__).with_name("golden") / "golden_ops.npz")


def _t(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


# ----------------------------------------------------------------- depthwise


@pytest.mark.parametrize("k", [1, 3, 5])
def test_depthwise_oracle_matches_golden(k):
    g = {n: GOLDEN[f"dw_k{k}_{n}"] for n in ("x", "w", "b", "y", "dy", "dx", "dw", "db")}
    np.testing.assert_allclose(odw.forward(g["x"], g["w"], g["b"]), g["y"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.input_grad(g["dy"], g["w"]), g["dx"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.weight_grad(g["x"], g["dy"], k), g["dw"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.bias_grad(g["dy"]), g["db"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("shape", [(1, 2, 4, 9, 3), (2, 1, 7, 2, 8), (1, 3, 1, 1, 6)])
def test_depthwise_oracle_matches_torch_float64(k, shape):
    rng = np.random.default_rng(k + sum(shape))
    x = rng.standard_normal(shape)
    w = rng.standard_normal((shape[1], 1, k, k, k))
    b = rng.standard_normal(shape[1])
    xt, wt, bt = (_t(a).requires_grad_() for a in (x, w, b))
    y = F.conv3d(xt, wt, bt, padding=k // 2, groups=shape[1])
    dy = rng.standard_normal(y.shape)
    dx, dw, db = torch.autograd.grad(y, (xt, wt, bt), _t(dy))
    np.testing.assert_allclose(odw.forward(x, w, b), y.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.input_grad(dy, w), dx.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.weight_grad(x, dy, k), dw.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.bias_grad(dy), db.numpy(), rtol=1e-12, atol=1e-12)


def test_depthwise_oracle_brute_force_loops():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 2, 3, 4, 5))
    for k in (1, 3, 5):
        w = rng.standard_normal((2, 1, k, k, k))
        b = rng.standard_normal(2)
        np.testing.assert_allclose(odw.forward(x, w, b), odw.forward_loops(x, w, b), rtol=1e-12, atol=1e-12)


def test_depthwise_closed_forms():
    rng = np.random.default_rng(1)
    k, p = 3, 1
    w = rng.standard_normal((1, 1, k, k, k))
    # Impulse input: the forward (a correlation) returns the kernel reversed
    # around the impulse; the input gradient returns it unreversed.
    x = np.zeros((1, 1, 7, 7, 7))
    x[0, 0, 3, 3, 3] = 1.0
    y = odw.forward(x, w)
    np.testing.assert_allclose(y[0, 0, 2:5, 2:5, 2:5], w[0, 0, ::-1, ::-1, ::-1])
    dx = odw.input_grad(x, w)
    np.testing.assert_allclose(dx[0, 0, 2:5, 2:5, 2:5], w[0, 0])
    # All-ones input: interior output is sum(w) + b.
    ones = np.ones((1, 1, 6, 6, 6))
    y = odw.forward(ones, w, np.array([0.25]))
    np.testing.assert_allclose(y[0, 0, p:-p, p:-p, p:-p], w.sum() + 0.25)
    # k = 1 reduces to a per-channel scale.
    x = rng.standard_normal((2, 3, 2, 3, 4))
    w1 = rng.standard_normal((3, 1, 1, 1, 1))
    np.testing.assert_allclose(odw.forward(x, w1), x * w1.reshape(1, 3, 1, 1, 1))
    # dW of an impulse grad_output is the input window around it.
    dy = np.zeros((1, 1, 7, 7, 7))
    dy[0, 0, 3, 3, 3] = 1.0
    xi = rng.standard_normal((1, 1, 7, 7, 7))
    np.testing.assert_allclose(odw.weight_grad(xi, dy, 3)[0, 0], xi[0, 0, 2:5, 2:5, 2:5])


def test_planted_oracle_mistake_is_caught():
    """A plausible slip (taps applied without the -p shift) must fail a check."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 2, 4, 5, 6))
    w = rng.standard_normal((2, 1, 3, 3, 3))

    def wrong_forward(x, w):
        y = np.zeros_like(x)
        for kd in range(3):
            for kh in range(3):
                for kw in range(3):
                    y += w[None, :, 0, kd, kh, kw, None, None, None] * odw._shifted(x, kd, kh, kw)
        return y

    ref = F.conv3d(_t(x), _t(w), padding=1, groups=2).numpy()
    assert not np.allclose(wrong_forward(x, w), ref, atol=1e-6)
    np.testing.assert_allclose(odw.forward(x, w), ref, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------- groupnorm


def test_group_norm_oracle_matches_golden_and_torch():
    g = {n: GOLDEN[f"gn_{n}"] for n in ("x", "g", "b", "y", "dy", "dx", "dg", "db")}
    y, mean, rstd = ogn.forward(g["x"], g["g"], g["b"])
    np.testing.assert_allclose(y, g["y"], rtol=1e-10, atol=1e-10)
    dx, dg, db = ogn.backward(g["dy"], g["x"], g["g"])
    np.testing.assert_allclose(dx, g["dx"], rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(dg, g["dg"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(db, g["db"], rtol=1e-10, atol=1e-10)
    # Independent torch check at another shape.
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 5, 2, 3, 4)) * 2 - 1
    gam, bet = rng.standard_normal(5), rng.standard_normal(5)
    xt, gt, bt = (_t(a).requires_grad_() for a in (x, gam, bet))
    yt = F.group_norm(xt, 5, gt, bt, eps=1e-5)
    dy = rng.standard_normal(x.shape)
    ref = torch.autograd.grad(yt, (xt, gt, bt), _t(dy))
    np.testing.assert_allclose(ogn.forward(x, gam, bet)[0], yt.detach().numpy(), rtol=1e-10, atol=1e-10)
    for got, want in zip(ogn.backward(dy, x, gam), ref):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-9, atol=1e-9)


def test_group_norm_invariants():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 4, 4, 4)) * 5 + 11
    y, _, _ = ogn.forward(x)
    flat = y.reshape(2, 3, -1)
    np.testing.assert_allclose(flat.mean(axis=2), 0, atol=1e-12)
    np.testing.assert_allclose(flat.var(axis=2), 1 / (1 + 1e-5 / x.reshape(2, 3, -1).var(axis=2)), rtol=1e-9)
    # With gamma = 1, dx sums to zero per (n, c) and its projection on x̂ is
    # rstd * sum(dy x̂) * (1 - mean(x̂^2)) (zero only when eps = 0).
    dy = rng.standard_normal(x.shape)
    dx, _, _ = ogn.backward(dy, x)
    _, _, rstd = ogn.forward(x)
    xh = y.reshape(2, 3, -1)
    g = dy.reshape(2, 3, -1)
    np.testing.assert_allclose(dx.reshape(2, 3, -1).sum(axis=2), 0, atol=1e-9)
    expected = rstd * (g * xh).sum(axis=2) * (1 - (xh**2).mean(axis=2))
    np.testing.assert_allclose((dx.reshape(2, 3, -1) * xh).sum(axis=2), expected, rtol=1e-6, atol=1e-12)


# ----------------------------------------------------------------- pointwise


def test_pointwise_oracle_matches_golden():
    g = {n: GOLDEN[f"pw_{n}"] for n in ("x", "w1", "b1", "w2", "b2", "a", "h", "y", "dy", "dx", "dw1", "db1", "dw2", "db2")}
    a = opw.conv1x1(g["x"], g["w1"], g["b1"])
    np.testing.assert_allclose(a, g["a"], rtol=1e-12, atol=1e-12)
    h = opw.gelu(a)
    np.testing.assert_allclose(h, g["h"], rtol=1e-12, atol=1e-12)
    y = opw.conv1x1(h, g["w2"], g["b2"]) + g["x"]
    np.testing.assert_allclose(y, g["y"], rtol=1e-12, atol=1e-12)
    dh, dw2, db2 = opw.conv1x1_backward(g["dy"], h, g["w2"])
    da = dh * opw.gelu_grad(a)
    dxa, dw1, db1 = opw.conv1x1_backward(da, g["x"], g["w1"])
    np.testing.assert_allclose(dw2, g["dw2"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(db2, g["db2"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(dw1, g["dw1"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(db1, g["db1"], rtol=1e-11, atol=1e-11)
    np.testing.assert_allclose(dxa + g["dy"], g["dx"], rtol=1e-11, atol=1e-11)


def test_gelu_special_values_and_torch():
    a = np.linspace(-9, 9, 1001)
    np.testing.assert_allclose(opw.gelu(a), F.gelu(_t(a), approximate="none").numpy(), rtol=1e-14, atol=1e-15)
    assert opw.gelu(np.array([0.0]))[0] == 0.0
    # gelu(a) - gelu(-a) = a (the odd part is identity/2 * 2)
    np.testing.assert_allclose(opw.gelu(a) - opw.gelu(-a), a, atol=1e-14)
    at = _t(a).requires_grad_()
    (g,) = torch.autograd.grad(F.gelu(at, approximate="none").sum(), at)
    np.testing.assert_allclose(opw.gelu_grad(a), g.numpy(), rtol=1e-12, atol=1e-14)


def test_pointwise_oracle_is_not_transposed():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 3, 2, 2, 2))
    w = rng.standard_normal((5, 3, 1, 1, 1))
    y = opw.conv1x1(x, w)
    ref = F.conv3d(_t(x), _t(w)).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)
    dy = rng.standard_normal(y.shape)
    dx, dw, db = opw.conv1x1_backward(dy, x, w)
    xt, wt = _t(x).requires_grad_(), _t(w).requires_grad_()
    rdx, rdw = torch.autograd.grad(F.conv3d(xt, wt), (xt, wt), _t(dy))
    np.testing.assert_allclose(dx, rdx.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dw, rdw.numpy(), rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ stride 2


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("shape", [(2, 3, 5, 6, 7), (1, 2, 8, 8, 8), (1, 1, 3, 9, 4)])
def test_strided_oracle_matches_torch_float64(k, shape):
    rng = np.random.default_rng(k * 13 + shape[-1])
    c = shape[1]
    x, w, b = rng.standard_normal(shape), rng.standard_normal((c, 1, k, k, k)), rng.standard_normal(c)
    xt, wt, bt = (torch.tensor(a, requires_grad=True) for a in (x, w, b))
    yt = F.conv3d(xt, wt, bt, stride=2, padding=k // 2, groups=c)
    assert yt.shape[2:] == odw.strided_output_shape(shape[2:])
    dy = rng.standard_normal(yt.shape)
    gx, gw, gb = torch.autograd.grad(yt, (xt, wt, bt), torch.tensor(dy))
    np.testing.assert_allclose(odw.strided_forward(x, w, b), yt.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.strided_input_grad(dy, w, shape[2:]), gx.numpy(), rtol=1e-12, atol=1e-12)
    dw, db = odw.strided_weight_grad(x, dy, k)
    np.testing.assert_allclose(dw, gw.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(db, gb.numpy(), rtol=1e-12, atol=1e-12)
    # The transposed conv (MedNeXt up block): forward, dX and dW.
    s = rng.standard_normal((shape[0], c) + tuple(max(1, v // 2) for v in shape[2:]))
    st_, wt2 = torch.tensor(s, requires_grad=True), torch.tensor(w, requires_grad=True)
    yt2 = F.conv_transpose3d(st_, wt2, torch.tensor(b), stride=2, padding=k // 2, groups=c)
    np.testing.assert_allclose(odw.transposed_forward(s, w, b), yt2.detach().numpy(), rtol=1e-12, atol=1e-12)
    g2 = rng.standard_normal(yt2.shape)
    gs, gw2 = torch.autograd.grad(yt2, (st_, wt2), torch.tensor(g2))
    np.testing.assert_allclose(odw.strided_forward(g2, w), gs.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(odw.strided_weight_grad(g2, s, k)[0], gw2.numpy(), rtol=1e-12, atol=1e-12)


def test_strided_oracle_brute_force_and_adjoint():
    """Brute-force loops, and <forward(a), b> == <a, input_grad(b)> (the scatter
    is the adjoint of the gather), which fixes the transposed relation without
    any library."""
    rng = np.random.default_rng(77)
    for k in (3, 5):
        x = rng.standard_normal((1, 2, 5, 4, 7))
        w = rng.standard_normal((2, 1, k, k, k))
        b = rng.standard_normal(2)
        np.testing.assert_allclose(odw.strided_forward(x, w, b), odw.strided_forward_loops(x, w, b), rtol=1e-12)
        y = odw.strided_forward(x, w)
        g = rng.standard_normal(y.shape)
        lhs = float((y * g).sum())
        rhs = float((x * odw.strided_input_grad(g, w, x.shape[2:])).sum())
        assert abs(lhs - rhs) <= 1e-10 * max(1.0, abs(lhs))
        # dW is the derivative of <forward(x; w), g> with respect to w.
        dw, _ = odw.strided_weight_grad(x, g, k)
        eps = 1e-6
        e = np.zeros_like(w)
        e[1, 0, 1, 0, 2] = eps
        num = ((odw.strided_forward(x, w + e) - odw.strided_forward(x, w - e)) * g).sum() / (2 * eps)
        assert abs(num - dw[1, 0, 1, 0, 2]) <= 1e-6 * max(1.0, abs(num))
