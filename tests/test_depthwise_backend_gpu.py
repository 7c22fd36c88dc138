"""The reference-schema ``mednext_accel::`` depthwise ops on the GPU.

``reference_regular_flow`` restates the argument flow of the reference's
``_setup_regular_context`` / ``_regular_backward`` (reference
``ops/_triton/depthwise.py:583-648``) with both custom phases on: the forward
op, then ``depthwise_input_grad_odd_regular(grad_output, weight, kernel_size,
channels, spatial_size, dx_block)``, ``depthwise_weight_grad_odd_regular(x,
grad_output, kernel_size, channels, spatial_size, dw_splits, dw_block)`` and the
bias gradient from ATen's ``convolution_backward`` with mask
``[False, False, True]``. Its results are checked against the CPU oracle on the
dtype-rounded inputs. Launch parameters are the reference's NVIDIA defaults
(``dw_splits = min(512, max(1, round(B*V / 32768)))``, ``dw_block`` 512,
``dx_block`` 128; reference ``optimization/parameters.py:52-87``).

Tolerances (normwise max relative error, tests/helpers.py): fp64 1e-12;
fp32 1e-5 outputs / dX, 1e-4 dW and dB; bf16 2e-2.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import mednext_accel_amd.depthwise_backend as backend
from helpers import BF16, FP32_OUT, FP32_WGRAD, max_rel
from oracle import depthwise as odw

pytestmark = pytest.mark.gpu

DEV = "cuda"
OPS = torch.ops.mednext_accel
TOL = {torch.float64: (1e-12, 1e-12), torch.float32: (FP32_OUT, FP32_WGRAD), torch.bfloat16: (BF16, BF16)}


def reference_launch(batch: int, size: int) -> tuple[int, int, int]:
    splits = min(512, max(1, round(batch * size**3 / 32768)))
    return splits, 512, 128


def reference_regular_flow(x, w, b, dy, k):
    """Forward + the reference's backward argument flow, custom dX and dW."""
    channels, size = int(x.shape[1]), int(x.shape[2])
    splits, dw_block, dx_block = reference_launch(int(x.shape[0]), size)
    y = OPS.depthwise_conv3d_odd_regular(x, w, b, k, channels, size, splits, dw_block, dx_block)
    pad = k // 2
    _, _, db = torch.ops.aten.convolution_backward(
        dy, x, w, [channels], [1, 1, 1], [pad] * 3, [1, 1, 1], False, [0, 0, 0], channels, [False, False, True]
    )
    dx = OPS.depthwise_input_grad_odd_regular(dy, w, k, channels, size, dx_block)
    dw = OPS.depthwise_weight_grad_odd_regular(x, dy, k, channels, size, splits, dw_block)
    torch.cuda.synchronize()
    return y, dx, dw, db


def inputs(shape, k, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    c = shape[1]
    x = torch.randn(shape, generator=gen).to(dtype)
    bound = 1.0 / k**1.5
    w = ((torch.rand(c, 1, k, k, k, generator=gen) * 2 - 1) * bound).to(dtype)
    b = (torch.randn(c, generator=gen) * 0.1).to(dtype)
    dy = torch.randn(shape, generator=gen).to(dtype)
    return x, w, b, dy


@pytest.mark.parametrize(
    "shape,k,dtype",
    [
        ((2, 3, 7, 7, 7), 3, torch.float64),
        ((2, 3, 7, 7, 7), 5, torch.float64),
        ((1, 32, 64, 64, 64), 3, torch.float32),  # configs[0]
        ((2, 4, 9, 9, 9), 5, torch.float32),
        ((1, 32, 128, 128, 128), 3, torch.bfloat16),  # configs[1] headline
        ((1, 64, 64, 64, 64), 5, torch.bfloat16),
        ((1, 256, 16, 16, 16), 3, torch.bfloat16),
        ((1, 512, 8, 8, 8), 5, torch.bfloat16),
    ],
)
def test_reference_regular_flow_against_oracle(shape, k, dtype):
    print(f"[mednext_accel regular flow] shape={shape} k={k} dtype={dtype}", flush=True)
    x, w, b, dy = inputs(shape, k, dtype, seed=17 + k)
    y, dx, dw, db = reference_regular_flow(*(t.to(DEV) for t in (x, w, b, dy)), k)
    out_tol, w_tol = TOL[dtype]
    assert y.dtype == dx.dtype == dw.dtype == dtype and dw.shape == w.shape
    if dtype == torch.bfloat16:
        # Large bf16 shapes: the reference's own torch path in fp32 on the same
        # bf16-rounded inputs (the oracle's float64 loops would take minutes).
        xf, wf, bf = (t.to(DEV).float().requires_grad_() for t in (x, w, b))
        yf = F.conv3d(xf, wf, bf, padding=k // 2, groups=shape[1])
        expect = (yf, *torch.autograd.grad(yf, (xf, wf, bf), dy.to(DEV).float()))
    else:
        xn, wn, bn, dyn = (t.double().numpy() for t in (x, w, b, dy))
        expect = (odw.forward(xn, wn, bn), odw.input_grad(dyn, wn), odw.weight_grad(xn, dyn, k), odw.bias_grad(dyn))
    for name, got, want, tol in zip(("y", "dx", "dw", "db"), (y, dx, dw, db), expect, (out_tol, out_tol, w_tol, w_tol)):
        assert max_rel(got, want) <= tol, name


@pytest.mark.parametrize("custom_dx,custom_dw", [(True, True), (True, False), (False, True), (False, False)])
def test_autograd_phase_mask_matches_float64(custom_dx, custom_dw):
    """Autograd through the registered formula: each combination of the
    reference's per-phase flags gives the float64 gradients (dB fused into the
    HIP dW pass when ``custom_dw``, ATen's otherwise)."""
    x, w, b, dy = inputs((2, 5, 8, 8, 8), 3, torch.float32, seed=41)
    xs = [t.to(DEV).requires_grad_() for t in (x, w, b)]
    y = OPS.depthwise_conv3d_odd_regular(*xs, 3, 5, 8, 1, 512, 128, custom_dx, custom_dw)
    got = torch.autograd.grad(y, xs, dy.to(DEV))
    ref = [t.double().requires_grad_() for t in (x, w, b)]
    want = torch.autograd.grad(F.conv3d(ref[0], ref[1], ref[2], padding=1, groups=5), ref, dy.double())
    assert max_rel(y, F.conv3d(ref[0], ref[1], ref[2], padding=1, groups=5)) <= FP32_OUT
    for name, a, e, tol in zip(("dx", "dw", "db"), got, want, (FP32_OUT, FP32_WGRAD, FP32_WGRAD), strict=True):
        assert max_rel(a, e) <= tol, name


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("size", [9, 16])
def test_stride2_and_transpose_ops_against_oracle(k, size):
    """Down block (stride-2 conv) and up block (transposed conv) ops, every
    gradient, fp32, against the oracle's strided restatements."""
    print(f"[mednext_accel stride2] k={k} size={size}", flush=True)
    c = 6
    gen = torch.Generator().manual_seed(3 * k + size)
    x = torch.randn(2, c, size, size, size, generator=gen)
    w = torch.randn(c, 1, k, k, k, generator=gen) / k**1.5
    b = torch.randn(c, generator=gen)
    xn, wn, bn = (t.double().numpy() for t in (x, w, b))

    xs = [t.to(DEV).requires_grad_() for t in (x, w, b)]
    small = OPS.depthwise_conv3d_stride2_regular(*xs, k, c, size, 128)
    assert max_rel(small, odw.strided_forward(xn, wn, bn)) <= FP32_OUT
    g = torch.randn(small.shape, generator=gen)
    dx, dw, db = torch.autograd.grad(small, xs, g.to(DEV))
    gn = g.double().numpy()
    dw_ref, db_ref = odw.strided_weight_grad(xn, gn, k)
    assert max_rel(dx, odw.strided_input_grad(gn, wn, (size,) * 3)) <= FP32_OUT
    assert max_rel(dw, dw_ref) <= FP32_WGRAD
    assert max_rel(db, db_ref) <= FP32_WGRAD
    direct = OPS.depthwise_input_grad_stride2_regular(g.to(DEV), w.to(DEV), c, size, 256)
    assert max_rel(direct, odw.strided_input_grad(gn, wn, (size,) * 3)) <= FP32_OUT

    ts = [t.to(DEV).requires_grad_() for t in (x, w, b)]
    big = OPS.depthwise_conv_transpose3d_odd_regular(*ts, k, c, size, 8, 256)
    assert tuple(big.shape[2:]) == (2 * size - 1,) * 3
    assert max_rel(big, odw.transposed_forward(xn, wn, bn)) <= FP32_OUT
    gb = torch.randn(big.shape, generator=gen)
    tdx, tdw, tdb = torch.autograd.grad(big, ts, gb.to(DEV))
    gbn = gb.double().numpy()
    # Transposed conv: dX is the stride-2 conv of dy, dW[t] = sum_o x[o] dy[2o + t - p].
    tdw_ref, _ = odw.strided_weight_grad(gbn, xn, k)
    assert max_rel(tdx, odw.strided_forward(gbn, wn)) <= FP32_OUT
    assert max_rel(tdw, tdw_ref) <= FP32_WGRAD
    assert max_rel(tdb, gbn.sum(axis=(0, 2, 3, 4))) <= FP32_WGRAD
    direct = OPS.depthwise_transpose_weight_grad_odd_regular(x.to(DEV), gb.to(DEV), k, c, size, 8, 256)
    assert max_rel(direct, tdw_ref) <= FP32_WGRAD


def test_low_level_launchers_match_the_oracle():
    """The reference module's plain launchers (``depthwise.py:271-442``)."""
    x, w, _b, dy = inputs((1, 4, 10, 12, 16), 3, torch.float32, seed=7)
    xg, wg, dyg = (t.to(DEV) for t in (x, w, dy))
    xn, wn, dyn = (t.double().numpy() for t in (x, w, dy))
    assert max_rel(backend.depthwise_input_grad(dyg, wg), odw.input_grad(dyn, wn)) <= FP32_OUT
    assert max_rel(backend.depthwise_weight_grad(xg, dyg, kernel_size=3), odw.weight_grad(xn, dyn, 3)) <= FP32_WGRAD
    small = torch.randn(1, 4, 5, 6, 8).to(DEV)
    got = backend.depthwise_stride2_input_grad(small, wg, (10, 12, 16))
    assert max_rel(got, odw.strided_input_grad(small.double().cpu().numpy(), wn, (10, 12, 16))) <= FP32_OUT
    big = torch.randn(1, 4, 19, 23, 31).to(DEV)
    got = backend.depthwise_transpose_weight_grad(xg, big, kernel_size=3)
    want, _ = odw.strided_weight_grad(big.double().cpu().numpy(), xn, 3)
    assert max_rel(got, want) <= FP32_WGRAD


def test_opcheck_reference_schema_ops():
    torch.manual_seed(5)
    x = torch.randn(1, 3, 6, 6, 6, device=DEV, requires_grad=True)
    w = torch.randn(3, 1, 3, 3, 3, device=DEV, requires_grad=True)
    b = torch.randn(3, device=DEV, requires_grad=True)
    dy = torch.randn(1, 3, 6, 6, 6, device=DEV)
    torch.library.opcheck(OPS.depthwise_conv3d_odd_regular, (x, w, b, 3, 3, 6, 1, 512, 128, True, True))
    torch.library.opcheck(OPS.depthwise_conv3d_odd_regular, (x, w, b, 3, 3, 6, 1, 512, 128, False, True))
    torch.library.opcheck(OPS.depthwise_input_grad_odd_regular, (dy, w.detach(), 3, 3, 6, 128))
    torch.library.opcheck(OPS.depthwise_weight_grad_odd_regular, (x.detach(), dy, 3, 3, 6, 1, 512))
    torch.library.opcheck(OPS.depthwise_conv3d_stride2_regular, (x, w, b, 3, 3, 6, 128))
    small = torch.randn(1, 3, 3, 3, 3, device=DEV)
    torch.library.opcheck(OPS.depthwise_input_grad_stride2_regular, (small, w.detach(), 3, 6, 128))
    torch.library.opcheck(OPS.depthwise_conv_transpose3d_odd_regular, (x, w, b, 3, 3, 6, 8, 256))
    big = torch.randn(1, 3, 11, 11, 11, device=DEV)
    torch.library.opcheck(OPS.depthwise_transpose_weight_grad_odd_regular, (x.detach(), big, 3, 3, 6, 8, 256))


def test_regular_op_compiles_fullgraph():
    def step(x, w, b):
        return OPS.depthwise_conv3d_odd_regular(x, w, b, 3, 4, 8, 1, 512, 128).square().sum()

    x, w, b, _ = inputs((1, 4, 8, 8, 8), 3, torch.float32, seed=13)
    compiled = torch.compile(step, fullgraph=True, backend="aot_eager")
    xs = [t.to(DEV).requires_grad_() for t in (x, w, b)]
    ys = [t.to(DEV).requires_grad_() for t in (x, w, b)]
    got = torch.autograd.grad(compiled(*xs), xs)
    want = torch.autograd.grad(step(*ys), ys)
    for a, e in zip(got, want, strict=True):
        assert max_rel(a, e) <= FP32_WGRAD
