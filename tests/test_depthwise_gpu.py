"""HIP depthwise Conv3d (fwd, dgrad, wgrad + fused dB) parity on the GPU.

Small shapes are checked against the CPU oracle and the golden fixtures; the
BASELINE sizes (cfg0 fp32 1x32x64^3, cfg1 bf16 stage shapes) against the oracle
(cfg0) or the reference's own torch path in fp32 on the same device (cfg1).
Tolerances (normwise max relative error, tests/helpers.py): fp64 1e-12;
fp32 1e-5 outputs / dX, 1e-4 dW and dB; bf16 / fp16 2e-2.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import BF16, FP32_OUT, FP32_WGRAD, max_rel
from mednext_accel_amd import hip_ops
from mednext_accel_amd.tiles import depthwise_recipe
from oracle import depthwise as odw

pytestmark = pytest.mark.gpu

GOLDEN = np.load(Path(__file__).with_name("golden") / "golden_ops.npz")
DEV = "cuda"
TOL = {
    torch.float64: (1e-12, 1e-12),
    torch.float32: (FP32_OUT, FP32_WGRAD),
    torch.bfloat16: (BF16, BF16),
    torch.float16: (BF16, BF16),
}


def run_all(x, w, b, dy, recipe=None):
    k = w.shape[-1]
    y = hip_ops.depthwise_forward(x, w, b, recipe)
    dx = hip_ops.depthwise_input_grad(dy, w, recipe)
    dw, db = hip_ops.depthwise_weight_grad(x, dy, k, recipe)
    torch.cuda.synchronize()
    return y, dx, dw, db


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
def test_golden_shape_all_dtypes(k, dtype):
    print(f"[depthwise golden] k={k} dtype={dtype}", flush=True)
    g = {n: GOLDEN[f"dw_k{k}_{n}"] for n in ("x", "w", "b", "dy", "y", "dx", "dw", "db")}
    cast = lambda a: torch.from_numpy(a).to(dtype)  # noqa: E731
    x, w, b, dy = (cast(g[n]) for n in ("x", "w", "b", "dy"))
    y, dx, dw, db = run_all(*(t.to(DEV) for t in (x, w, b, dy)))
    out_tol, w_tol = TOL[dtype]
    if dtype == torch.float64:
        expect = g
    else:  # oracle on the dtype-rounded inputs
        xn, wn, bn, dyn = (t.double().numpy() for t in (x, w, b, dy))
        expect = {
            "y": odw.forward(xn, wn, bn),
            "dx": odw.input_grad(dyn, wn),
            "dw": odw.weight_grad(xn, dyn, k),
            "db": odw.bias_grad(dyn),
        }
    assert max_rel(y, expect["y"]) <= out_tol
    assert max_rel(dx, expect["dx"]) <= out_tol
    assert max_rel(dw, expect["dw"]) <= w_tol
    assert max_rel(db, expect["db"]) <= w_tol
    assert y.dtype == dx.dtype == dw.dtype == db.dtype == dtype


@pytest.mark.parametrize(
    "shape,recipe",
    [
        ((1, 2, 9, 11, 13), [0, 4, 2]),  # W not a multiple of 4 -> scalar path
        ((2, 3, 3, 5, 8), [0, 8, 1]),  # depth_chunk 1, tiny D
        ((1, 1, 17, 33, 70), [0, 64, 5]),  # ragged tiles in every direction
        ((3, 2, 6, 2, 4), [0, 4, 100]),  # depth_chunk > D
        ((1, 4, 8, 8, 64), [0, 16, 3]),
    ],
)
@pytest.mark.parametrize("k", [3, 5])
def test_ragged_shapes_and_recipes_fp32(shape, recipe, k):
    print(f"[depthwise ragged] shape={shape} recipe={recipe} k={k}", flush=True)
    gen = torch.Generator().manual_seed(k + shape[-1])
    x = torch.randn(shape, generator=gen)
    w = torch.randn(shape[1], 1, k, k, k, generator=gen)
    b = torch.randn(shape[1], generator=gen)
    dy = torch.randn(shape, generator=gen)
    y, dx, dw, db = run_all(*(t.to(DEV) for t in (x, w, b, dy)), recipe=recipe)
    xn, wn, bn, dyn = (t.double().numpy() for t in (x, w, b, dy))
    assert max_rel(y, odw.forward(xn, wn, bn)) <= FP32_OUT
    assert max_rel(dx, odw.input_grad(dyn, wn)) <= FP32_OUT
    assert max_rel(dw, odw.weight_grad(xn, dyn, k)) <= FP32_WGRAD
    assert max_rel(db, odw.bias_grad(dyn)) <= FP32_WGRAD


def test_cfg0_fp32_1x32x64_against_oracle():
    """fp32 1x32x64^3, k3, w ~ U(+-1/sqrt(27)), b = 0."""
    print("[depthwise cfg0] fp32 1x32x64^3", flush=True)
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(1, 32, 64, 64, 64, generator=gen)
    bound = 1.0 / 27**0.5
    w = (torch.rand(32, 1, 3, 3, 3, generator=gen) * 2 - 1) * bound
    b = torch.zeros(32)
    dy = torch.randn(1, 32, 64, 64, 64, generator=torch.Generator().manual_seed(2))
    y, dx, dw, db = run_all(*(t.to(DEV) for t in (x, w, b, dy)))
    xn, wn, bn, dyn = (t.double().numpy() for t in (x, w, b, dy))
    assert max_rel(y, odw.forward(xn, wn, bn)) <= FP32_OUT
    assert max_rel(dx, odw.input_grad(dyn, wn)) <= FP32_OUT
    assert max_rel(dw, odw.weight_grad(xn, dyn, 3)) <= FP32_WGRAD
    assert max_rel(db, odw.bias_grad(dyn)) <= FP32_WGRAD


STAGES = [(32, 128), (64, 64), (128, 32), (256, 16), (512, 8)]


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("channels,size", STAGES)
def test_cfg1_bf16_stage_shapes_against_torch(channels, size, k):
    """bf16 in / fp32 accumulate at the MedNeXt stage shapes;
    reference = the reference's torch path (F.conv3d + autograd) in fp32 on the
    same bf16-rounded inputs."""
    print(f"[depthwise cfg1] C={channels} S={size} k={k}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(channels * 7 + k)
    shape = (1, channels, size, size, size)
    x = torch.randn(shape, generator=gen, device=DEV).bfloat16()
    dy = torch.randn(shape, generator=gen, device=DEV).bfloat16()
    bound = 1.0 / (k**3) ** 0.5
    w = ((torch.rand(channels, 1, k, k, k, generator=gen, device=DEV) * 2 - 1) * bound).bfloat16()
    b = (torch.rand(channels, generator=gen, device=DEV) - 0.5).bfloat16()
    y, dx, dw, db = run_all(x, w, b, dy)
    xf, wf, bf = (t.float().requires_grad_() for t in (x, w, b))
    yf = F.conv3d(xf, wf, bf, padding=k // 2, groups=channels)
    rdx, rdw, rdb = torch.autograd.grad(yf, (xf, wf, bf), dy.float())
    assert max_rel(y, yf) <= BF16
    assert max_rel(dx, rdx) <= BF16
    assert max_rel(dw, rdw) <= BF16
    assert max_rel(db, rdb) <= BF16


@pytest.mark.parametrize(
    "shape,fwd_recipe,dw_recipe",
    [
        ((1, 2, 9, 33, 40), [1, 64, 4], None),  # ragged H and W, forward/dgrad only
        ((2, 3, 5, 32, 32), [1, 32, 2], [1, 32, 2]),
        ((1, 2, 7, 35, 64), [1, 128, 3], [1, 64, 3]),  # tile wider than W, ragged H
        ((1, 1, 19, 48, 96), [1, 32, 19], [1, 32, 100]),  # depth_chunk >= D
        ((1, 2, 3, 64, 128), [1, 128, 1], [1, 64, 1]),  # depth_chunk 1
    ],
)
@pytest.mark.parametrize("k", [3, 5])
def test_mfma_engine_bf16_against_oracle(shape, fwd_recipe, dw_recipe, k):
    print(f"[depthwise mfma] shape={shape} fwd={fwd_recipe} dw={dw_recipe} k={k}", flush=True)
    gen = torch.Generator().manual_seed(k * 31 + shape[2])
    x = torch.randn(shape, generator=gen).bfloat16()
    w = (torch.randn(shape[1], 1, k, k, k, generator=gen) / k).bfloat16()
    b = torch.randn(shape[1], generator=gen).bfloat16()
    dy = torch.randn(shape, generator=gen).bfloat16()
    xg, wg, bg, dyg = (t.to(DEV) for t in (x, w, b, dy))
    y = hip_ops.depthwise_forward(xg, wg, bg, fwd_recipe)
    dx = hip_ops.depthwise_input_grad(dyg, wg, fwd_recipe)
    xn, wn, bn, dyn = (t.double().numpy() for t in (x, w, b, dy))
    assert max_rel(y, odw.forward(xn, wn, bn)) <= BF16
    assert max_rel(dx, odw.input_grad(dyn, wn)) <= BF16
    # The MFMA path must agree with the fp32-accumulating VALU path to bf16 rounding.
    y_valu = hip_ops.depthwise_forward(xg, wg, bg, [0, 32, 4])
    assert max_rel(y, y_valu) <= 1e-2
    if dw_recipe is not None:
        dw, db = hip_ops.depthwise_weight_grad(xg, dyg, k, dw_recipe)
        assert max_rel(dw, odw.weight_grad(xn, dyn, k)) <= BF16
        assert max_rel(db, odw.bias_grad(dyn)) <= BF16


def test_recipe_default_is_valid_for_stage_shapes():
    for channels, size in STAGES:
        for k in (3, 5):
            for dtype in ("bfloat16", "float32"):
                for phase in ("forward", "input_grad", "weight_grad"):
                    engine, tile_w, depth_chunk = depthwise_recipe(1, channels, (size,) * 3, k, dtype, phase)
                    assert engine in (0, 1, 2)
                    assert engine != 1 or dtype == "bfloat16"
                    assert 1 <= depth_chunk <= size


def test_deterministic_weight_grad():
    gen = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(1, 16, 32, 32, 32, generator=gen, device=DEV)
    dy = torch.randn(1, 16, 32, 32, 32, generator=gen, device=DEV)
    a = hip_ops.depthwise_weight_grad(x, dy, 3)
    b = hip_ops.depthwise_weight_grad(x, dy, 3)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_mfma_weight_grad_repeats_and_replays():
    """The MFMA weight gradient (partials kernel + fixed-order finish kernel):
    back-to-back launches, a launch of another shape in between and HIP-graph
    replays (with eager work between them) all give the first launch's bits,
    and those match the oracle."""
    print("[depthwise mfma wgrad repeats / replays]", flush=True)
    gen = torch.Generator().manual_seed(19)
    xc = torch.randn(2, 24, 16, 64, 64, generator=gen).bfloat16()
    dyc = torch.randn(2, 24, 16, 64, 64, generator=gen).bfloat16()
    x, dy = xc.to(DEV), dyc.to(DEV)
    recipe = [1, 64, 4]
    first = hip_ops.depthwise_weight_grad(x, dy, 3, recipe)
    xn, dyn = xc.double().numpy(), dyc.double().numpy()
    assert max_rel(first[0], odw.weight_grad(xn, dyn, 3)) <= BF16
    assert max_rel(first[1], odw.bias_grad(dyn)) <= BF16
    hip_ops.depthwise_weight_grad(x[:1, :5].contiguous(), dy[:1, :5].contiguous(), 3, [1, 32, 16])
    again = hip_ops.depthwise_weight_grad(x, dy, 3, recipe)
    assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hip_ops.depthwise_weight_grad(x, dy, 3, recipe)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = hip_ops.depthwise_weight_grad(x, dy, 3, recipe)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured[0], first[0]) and torch.equal(captured[1], first[1])
        hip_ops.depthwise_weight_grad(x[:1, :5].contiguous(), dy[:1, :5].contiguous(), 3, [1, 32, 16])


def test_launcher_argument_errors():
    x = torch.randn(1, 2, 4, 4, 4, device=DEV)
    with pytest.raises(ValueError):
        hip_ops.depthwise_input_grad(x, torch.randn(2, 1, 2, 2, 2, device=DEV))  # even k
    with pytest.raises(ValueError):
        hip_ops.depthwise_input_grad(x.transpose(2, 3), torch.randn(2, 1, 3, 3, 3, device=DEV))
    with pytest.raises(ValueError):
        hip_ops.depthwise_weight_grad(x, torch.randn(1, 2, 4, 4, 5, device=DEV), 3)
    with pytest.raises(ValueError):
        hip_ops.depthwise_forward(x.cpu(), torch.randn(2, 1, 3, 3, 3))
    with pytest.raises(ValueError):
        hip_ops.depthwise_forward(x, torch.randn(2, 1, 7, 7, 7, device=DEV))  # k=7 unsupported


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("shape,recipe", [((1, 16, 12, 64, 64), [1, 64, 4]), ((2, 8, 9, 33, 96), [1, 32, 3])])
def test_residual_tap_sums_both_gradients_in_the_kernel(shape, recipe, k):
    """DepthwiseResidualTap: (depthwise(x), x) whose backward adds the residual
    branch's gradient inside the matrix-core input-gradient kernel; the result
    is the separate kernel + bf16 add, bit for bit."""
    print(f"[depthwise residual tap] shape={shape} recipe={recipe} k={k}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(shape, generator=gen, device=DEV).bfloat16().requires_grad_()
    w = (torch.randn(shape[1], 1, k, k, k, generator=gen, device=DEV) / k).bfloat16().requires_grad_()
    b = torch.randn(shape[1], generator=gen, device=DEV).bfloat16().requires_grad_()
    d, xr = hip_ops.DepthwiseResidualTap.apply(x, w, b, k, recipe, recipe, recipe)
    assert torch.equal(d, hip_ops.depthwise_forward(x.detach(), w.detach(), b.detach(), recipe))
    assert torch.equal(xr, x)
    gd = torch.randn(shape, generator=gen, device=DEV).bfloat16()
    gr = torch.randn(shape, generator=gen, device=DEV).bfloat16()
    dx, dw, db = torch.autograd.grad((d, xr), (x, w, b), (gd, gr))
    want_dx = hip_ops.depthwise_input_grad(gd, w.detach(), recipe) + gr
    want_dw, want_db = hip_ops.depthwise_weight_grad(x.detach(), gd, k, recipe)
    assert torch.equal(dx, want_dx)
    assert torch.equal(dw, want_dw) and torch.equal(db, want_db)
