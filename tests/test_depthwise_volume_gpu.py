"""The small-plane volume engine (engine 2: whole zero-padded planes in LDS)
against the CPU oracle: forward, input gradient, weight gradient and fused
bias gradient, every dtype, k in {1, 3, 5}.

Cases cover both reduction paths of the weight gradient (H * W a multiple of
64: per-wave sums; otherwise per-lane sums), several slabs per workgroup
(small planes), D-runs that are not a multiple of the 4 planes a lane owns,
D-runs longer than D, and the MedNeXt stage shapes 16^3 / 8^3 in bf16.
Tolerances (normwise max relative error, tests/helpers.py): fp64 1e-12;
fp32 1e-5 outputs / dX, 1e-4 dW and dB; bf16 / fp16 2e-2.
"""

from __future__ import annotations

import pytest
import torch

from helpers import BF16, FP32_OUT, FP32_WGRAD, max_rel
from mednext_accel_amd import hip_ops
from mednext_accel_amd.tiles import ENGINE_VOLUME, VOLUME_BAND, depthwise_recipe
from oracle import depthwise as odw

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {
    torch.float64: (1e-12, 1e-12),
    torch.float32: (FP32_OUT, FP32_WGRAD),
    torch.bfloat16: (BF16, BF16),
    torch.float16: (BF16, BF16),
}


def check(shape, k, dtype, depth_chunk, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=gen).to(dtype)
    w = (torch.randn(shape[1], 1, k, k, k, generator=gen) / k**1.5).to(dtype)
    b = torch.randn(shape[1], generator=gen).to(dtype)
    dy = torch.randn(shape, generator=gen).to(dtype)
    recipe = [ENGINE_VOLUME, VOLUME_BAND, depth_chunk]
    xg, wg, bg, dyg = (t.to(DEV) for t in (x, w, b, dy))
    y = hip_ops.depthwise_forward(xg, wg, bg, recipe)
    y_nobias = hip_ops.depthwise_forward(xg, wg, None, recipe)
    dx = hip_ops.depthwise_input_grad(dyg, wg, recipe)
    dw, db = hip_ops.depthwise_weight_grad(xg, dyg, k, recipe)
    torch.cuda.synchronize()
    xn, wn, bn, dyn = (t.double().numpy() for t in (x, w, b, dy))
    out_tol, w_tol = TOL[dtype]
    assert max_rel(y, odw.forward(xn, wn, bn)) <= out_tol
    assert max_rel(y_nobias, odw.forward(xn, wn)) <= out_tol
    assert max_rel(dx, odw.input_grad(dyn, wn)) <= out_tol
    assert max_rel(dw, odw.weight_grad(xn, dyn, k)) <= w_tol
    assert max_rel(db, odw.bias_grad(dyn)) <= w_tol
    assert y.dtype == dx.dtype == dw.dtype == db.dtype == dtype


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "shape,depth_chunk",
    [
        ((2, 3, 8, 8, 8), 4),  # H*W = 64: wave sums, four slabs per workgroup
        ((1, 5, 7, 16, 16), 3),  # H*W = 256, D-run not a multiple of 4, ragged last run
        ((2, 3, 9, 5, 9), 8),  # H*W = 45: per-lane sums, slabs straddle waves
        ((1, 2, 3, 4, 6), 16),  # D-run longer than D, tiny plane
        ((3, 4, 5, 12, 12), 1),  # one plane per workgroup
    ],
)
def test_volume_engine_against_oracle(shape, depth_chunk, dtype, k):
    print(f"[depthwise volume] shape={shape} dchunk={depth_chunk} dtype={dtype} k={k}", flush=True)
    check(shape, k, dtype, depth_chunk, seed=sum(shape) + k + depth_chunk)


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("channels,size", [(256, 16), (512, 8)])
def test_volume_engine_stage_shapes_bf16(channels, size, k):
    """MedNeXt stage shapes with the tile policy's own recipe (which picks the
    volume engine for them)."""
    recipe = depthwise_recipe(1, channels, (size,) * 3, k, "bfloat16", "forward")
    assert recipe[0] == ENGINE_VOLUME
    print(f"[depthwise volume stage] C={channels} S={size} k={k} recipe={recipe}", flush=True)
    check((1, channels, size, size, size), k, torch.bfloat16, recipe[2], seed=channels + k)


def test_volume_weight_grad_is_deterministic():
    gen = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(2, 64, 16, 16, 16, generator=gen, device=DEV)
    dy = torch.randn(2, 64, 16, 16, 16, generator=gen, device=DEV)
    recipe = [ENGINE_VOLUME, VOLUME_BAND, 4]
    a = hip_ops.depthwise_weight_grad(x, dy, 5, recipe)
    b = hip_ops.depthwise_weight_grad(x, dy, 5, recipe)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
