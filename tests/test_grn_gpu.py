"""HIP GRN forward/backward parity on the GPU.

The reference's path is its fused Triton GRN (reference ops/_triton/grn.py)
behind the formula of ops/grn.py:16-30. Checked against the CPU oracle in
float64 (1e-12 / 1e-11) and float32 (1e-5 outputs / input grads, 1e-4
parameter grads), and against the PyTorch formula for f16 / bf16 inputs with
the reference's own fused-GRN tolerances (tests/ops/test_grn_triton.py:40-53:
activations and dX rtol 2e-3 / atol 2e-3 for f16, rtol 1e-2 / atol 1.6e-2 for
bf16; float32 parameter grads rtol 2e-4 / atol 3e-5).
"""

from __future__ import annotations

import copy

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

from helpers import FP32_OUT, FP32_WGRAD, max_rel
from mednext_accel_amd import AdaptiveGlobalResponseNorm3d, GlobalResponseNorm3d, global_response_norm3d_reference
from mednext_accel_amd import hip_ops
from mednext_accel_amd.adaptive import ModelOptimizationContext
from mednext_accel_amd.optimization import PolicyRegistry
from oracle import grn as ogrn

pytestmark = pytest.mark.gpu
DEV = "cuda"
GRN_OP = "mednext_accel_amd::grn_forward"
GRN_BWD_OP = "mednext_accel_amd::grn_backward"


class Observe(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops: list[str] = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.ops.append(func._schema.name)
        return func(*args, **(kwargs or {}))


def oracle_all(x, gamma, beta, dy):
    xn, gn, bn, dyn = (t.detach().cpu().double().numpy() for t in (x, gamma, beta, dy))
    return ogrn.forward(xn, gn, bn), *ogrn.backward(dyn, xn, gn)


SHAPES = [((2, 3, 5, 6, 7), None), ((1, 4, 9, 9, 9), 3), ((3, 2, 1, 1, 5), 2), ((1, 8, 16, 16, 16), 7),
          ((1, 3, 13, 15, 17), 5), ((2, 5, 7, 9, 11), 9), ((1, 1, 3, 3, 3), 1)]


@pytest.mark.parametrize("shape,splits", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_against_oracle(shape, splits, dtype):
    print(f"[grn {dtype}] shape={shape} splits={splits}", flush=True)
    gen = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(shape, generator=gen, dtype=torch.float64) * 2 + 0.5
    gamma = torch.randn(shape[1], generator=gen, dtype=torch.float64)
    beta = torch.randn(shape[1], generator=gen, dtype=torch.float64)
    dy = torch.randn(shape, generator=gen, dtype=torch.float64)
    xg, gg, bg, dyg = (t.to(DEV, dtype) for t in (x, gamma, beta, dy))
    y, coef = hip_ops.grn_forward(xg, gg, bg, splits=splits)
    dx, dgam, dbet = hip_ops.grn_backward(dyg, xg, coef, gg, splits=splits)
    y_ref, dx_ref, dg_ref, db_ref = oracle_all(xg, gg, bg, dyg)
    out_tol, w_tol = (1e-12, 1e-11) if dtype == torch.float64 else (FP32_OUT, FP32_WGRAD)
    assert y.dtype == dx.dtype == dtype
    assert max_rel(y, y_ref) <= out_tol
    assert max_rel(dx, dx_ref) <= out_tol
    assert max_rel(dgam, dg_ref) <= w_tol
    assert max_rel(dbet, db_ref) <= w_tol
    n_ref, r_ref = ogrn.norms(xg.cpu().double().numpy())
    assert max_rel(coef[..., 3], n_ref) <= out_tol
    assert max_rel(coef[..., 2], r_ref) <= out_tol


def reference_grads(x, gamma, beta, upstream, eps=1e-6):
    inputs = tuple(t.detach().clone().requires_grad_() for t in (x, gamma, beta))
    out = global_response_norm3d_reference(*inputs, eps)
    return out, torch.autograd.grad(out, inputs, upstream)


def fused_grads(x, gamma, beta, upstream, eps=1e-6):
    inputs = tuple(t.detach().clone().requires_grad_() for t in (x, gamma, beta))
    out = hip_ops.fused_global_response_norm3d(*inputs, eps)
    return out, torch.autograd.grad(out, inputs, upstream)


def compare(x, gamma, beta, upstream):
    want, wants = reference_grads(x, gamma, beta, upstream)
    got, gots = fused_grads(x, gamma, beta, upstream)
    act = dict(rtol=1e-2, atol=1.6e-2) if x.dtype == torch.bfloat16 else dict(rtol=2e-3, atol=2e-3)
    assert got.dtype == x.dtype
    torch.testing.assert_close(got, want, **act)
    for i, (a, b) in enumerate(zip(gots, wants, strict=True)):
        assert torch.isfinite(a).all()
        assert a.dtype == (x.dtype if i == 0 else torch.float32)
        torch.testing.assert_close(a, b, **(act if i == 0 else dict(rtol=2e-4, atol=3e-5)))
    return got, gots


@pytest.mark.parametrize("batch", (1, 2, 3))
@pytest.mark.parametrize("channels", (3, 32, 96))
@pytest.mark.parametrize("spatial", ((2, 3, 5), (8, 8, 8), (17, 9, 5)))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_half_inputs_match_reference_formula(batch, channels, spatial, dtype):
    torch.manual_seed(902)
    x = torch.randn(batch, channels, *spatial, device=DEV, dtype=dtype)
    gamma = torch.randn(1, channels, 1, 1, 1, device=DEV)
    beta = torch.randn_like(gamma)
    compare(x, gamma, beta, torch.randn_like(x))


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("case", ("zero", "tiny", "one_zero_channel", "multiple_tiles", "split_loop"))
def test_zero_norms_tiny_values_and_tails(dtype, case):
    print(f"[grn edge] {case} {dtype}", flush=True)
    torch.manual_seed(903)
    spatial = {"multiple_tiles": (17, 13, 11), "split_loop": (41, 41, 41)}.get(case, (2, 3, 5))
    x = torch.randn(2, 3, *spatial, device=DEV, dtype=dtype)
    gamma = torch.randn(1, 3, 1, 1, 1, device=DEV)
    beta = torch.randn_like(gamma)
    if case == "zero":
        x.zero_()
    elif case == "tiny":
        x = torch.sign(x) * torch.finfo(dtype).tiny
    elif case == "one_zero_channel":
        x[:, 1].zero_()
    upstream = torch.randn_like(x)
    _, grads = compare(x, gamma, beta, upstream)
    if case == "zero":
        torch.testing.assert_close(grads[0], upstream, rtol=0, atol=0)
        torch.testing.assert_close(grads[1], torch.zeros_like(gamma), rtol=0, atol=0)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
def test_backward_couples_channels_through_the_denominator(dtype):
    x = torch.tensor([1.0, 2.0, 4.0], device=DEV, dtype=dtype).view(1, 3, 1, 1, 1)
    gamma = torch.tensor([2.0, 3.0, -4.0], device=DEV)
    upstream = torch.zeros_like(x)
    upstream[:, 0] = 1
    _, coef = hip_ops.grn_forward(x, gamma.to(dtype), None)
    dx, _, _ = hip_ops.grn_backward(upstream, x, coef, gamma.to(dtype))
    torch.testing.assert_close(dx[:, 1:].float(), torch.full((1, 2, 1, 1, 1), -2 / (7 + 1e-6) ** 2, device=DEV),
                               rtol=5e-3, atol=1e-4)


def test_fp32_upstream_with_bf16_activation():
    torch.manual_seed(5)
    x = torch.randn(2, 16, 9, 10, 11, device=DEV, dtype=torch.bfloat16)
    gamma, beta = torch.randn(16, device=DEV), torch.randn(16, device=DEV)
    dy = torch.randn(x.shape, device=DEV)
    _, coef = hip_ops.grn_forward(x, gamma, beta)
    dx, dgam, dbet = hip_ops.grn_backward(dy, x, coef, gamma)
    assert dx.dtype == torch.bfloat16
    _, dx_ref, dg_ref, db_ref = oracle_all(x, gamma, beta, dy)
    assert max_rel(dx, dx_ref) <= 1e-2  # one bf16 rounding of dx
    assert max_rel(dgam, dg_ref) <= FP32_WGRAD
    assert max_rel(dbet, db_ref) <= FP32_WGRAD


def test_results_are_bit_reproducible():
    torch.manual_seed(6)
    x = torch.randn(2, 64, 24, 24, 24, device=DEV, dtype=torch.bfloat16)
    gamma = torch.randn(1, 64, 1, 1, 1, device=DEV)
    beta = torch.randn_like(gamma)
    dy = torch.randn_like(x)
    first = fused_grads(x, gamma, beta, dy)
    second = fused_grads(x, gamma, beta, dy)
    assert torch.equal(first[0], second[0])
    for a, b in zip(first[1], second[1], strict=True):
        assert torch.equal(a, b)


def test_large_stage_shape_against_oracle_properties():
    """A MedNeXt v2 stage-0 expansion shape (C=96, 64^3, bf16): the forward
    norms and dbeta are checked against float64 reductions on the GPU. The
    kernels accumulate half inputs per thread in float32 (as the reference's
    fused GRN does) and combine in float64, so the bound is float32's."""
    torch.manual_seed(8)
    x = torch.randn(1, 96, 64, 64, 64, device=DEV, dtype=torch.bfloat16)
    gamma = torch.randn(1, 96, 1, 1, 1, device=DEV)
    beta = torch.randn_like(gamma)
    dy = torch.randn_like(x)
    _, coef = hip_ops.grn_forward_op(x, gamma, beta, 1e-6)
    norms = x.double().flatten(2).norm(dim=2)
    assert max_rel(coef[..., 3], norms) <= 1e-6
    _, dgam, dbet = hip_ops.grn_backward_op(dy, x, gamma, coef, 1e-6)
    assert max_rel(dbet.flatten(), dy.double().sum(dim=(0, 2, 3, 4))) <= 1e-6
    gc = (dy.double() * x.double()).sum(dim=(2, 3, 4))
    assert max_rel(dgam.flatten(), (gc * coef[..., 2]).sum(0)) <= 1e-5


def test_adaptive_wrapper_routes_training_to_hip():
    torch.manual_seed(9)
    ref = GlobalResponseNorm3d(24).to(DEV)
    with torch.no_grad():
        ref.gamma.normal_()
        ref.beta.normal_()
    cand = AdaptiveGlobalResponseNorm3d(copy.deepcopy(ref), PolicyRegistry().resolver(),
                                        ModelOptimizationContext("mednext_v2", "base", "none"))
    assert cand.gamma is not ref.gamma
    x = torch.randn(2, 24, 10, 11, 12, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    with Observe() as seen:
        got = cand(y)
    assert GRN_OP in seen.ops
    want = ref(x)
    torch.testing.assert_close(got, want, rtol=1e-2, atol=1.6e-2)
    g = torch.randn_like(want)
    wants = torch.autograd.grad(want, (x, ref.gamma, ref.beta), g)
    with Observe() as seen_bwd:
        gots = torch.autograd.grad(got, (y, cand.gamma, cand.beta), g)
    assert GRN_BWD_OP in seen_bwd.ops
    torch.testing.assert_close(gots[0], wants[0], rtol=1e-2, atol=1.6e-2)
    for a, b in zip(gots[1:], wants[1:], strict=True):
        torch.testing.assert_close(a, b, rtol=2e-4, atol=3e-5)
    # evaluation, no-grad and float32 stay on the PyTorch formula
    for mode in ("eval", "no_grad", "fp32"):
        c = copy.deepcopy(cand).train(mode != "eval")
        inp = y.detach().float() if mode == "fp32" else y.detach()
        with torch.set_grad_enabled(mode != "no_grad"), Observe() as seen_other:
            c(inp)
        assert GRN_OP not in seen_other.ops, mode


def test_opcheck_grn_ops():
    torch.manual_seed(904)
    x = torch.randn(2, 3, 2, 3, 5, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    gamma = torch.randn(1, 3, 1, 1, 1, device=DEV, requires_grad=True)
    beta = torch.randn_like(gamma, requires_grad=True)
    result = torch.library.opcheck(hip_ops.grn_forward_op, (x, gamma, beta, 1e-6), raise_exception=False)
    assert all(v == "SUCCESS" for v in result.values()), result
    _, coef = hip_ops.grn_forward_op(x.detach(), gamma.detach(), beta.detach(), 1e-6)
    result = torch.library.opcheck(
        hip_ops.grn_backward_op, (torch.randn_like(x), x.detach(), gamma.detach(), coef, 1e-6), raise_exception=False
    )
    assert all(v == "SUCCESS" for v in result.values()), result


def test_fullgraph_compile_forward_and_backward():
    torch.manual_seed(905)
    fused = hip_ops.fused_global_response_norm3d

    def loss_and_output(x, gamma, beta, upstream):
        out = fused(x, gamma, beta)
        return (out.float() * upstream).sum(), out

    compiled = torch.compile(loss_and_output, fullgraph=True, backend="aot_eager")
    x = torch.randn(2, 3, 17, 13, 11, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    gamma = torch.randn(1, 3, 1, 1, 1, device=DEV, requires_grad=True)
    beta = torch.randn_like(gamma, requires_grad=True)
    upstream = torch.randn(x.shape, device=DEV)
    expected_in = tuple(t.detach().clone().requires_grad_() for t in (x, gamma, beta))
    e_loss, e_out = loss_and_output(*expected_in, upstream)
    e_grads = torch.autograd.grad(e_loss, expected_in)
    a_loss, a_out = compiled(x, gamma, beta, upstream)
    a_grads = torch.autograd.grad(a_loss, (x, gamma, beta))
    torch.testing.assert_close(a_out, e_out)
    for a, b in zip(a_grads, e_grads, strict=True):
        torch.testing.assert_close(a, b)


def test_autograd_saves_input_gamma_and_compact_coefficients():
    x = torch.randn(2, 3, 17, 13, 11, device=DEV, dtype=torch.float16, requires_grad=True)
    gamma = torch.randn(1, 3, 1, 1, 1, device=DEV, requires_grad=True)
    beta = torch.randn_like(gamma, requires_grad=True)
    saved = []

    def pack(t):
        saved.append(t)
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out = hip_ops.fused_global_response_norm3d(x, gamma, beta)
    assert len(saved) == 3 and saved[0] is x and saved[1] is gamma
    assert tuple(saved[2].shape) == (2, 3, 4) and saved[2].dtype == torch.float64
    grads = torch.autograd.grad(out.sum(), (x, gamma, beta))  # expanded (non-contiguous) upstream
    assert all(torch.isfinite(g).all() for g in grads)
