"""HIP GroupNorm(C, C) forward/backward parity on the GPU.

The reference's path is ``nn.GroupNorm(C, C)`` (reference models/blocks.py:74),
which under bf16 autocast reads a bf16 tensor, computes in fp32 and returns
fp32. Checked against the CPU oracle (small and cfg2 stage-0 shapes) with the
fp32 bound 1e-5 on outputs / input grads and 1e-4 on parameter grads.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import BF16, FP32_OUT, FP32_WGRAD, max_rel
from mednext_accel_amd import hip_ops
from oracle import groupnorm as ogn

pytestmark = pytest.mark.gpu

GOLDEN = np.load(Path(__file__).with_name("golden") / "golden_ops.npz")
DEV = "cuda"


def test_golden_fp64():
    g = {n: torch.from_numpy(GOLDEN[f"gn_{n}"]) for n in ("x", "g", "b", "y", "dy", "dx", "dg", "db")}
    x, gam, bet, dy = (g[n].to(DEV) for n in ("x", "g", "b", "dy"))
    y, mean, rstd = hip_ops.group_norm_forward(x, gam, bet)
    dx, dg, db = hip_ops.group_norm_backward(dy, x, mean, rstd, gam)
    assert max_rel(y, g["y"]) <= 1e-12
    assert max_rel(dx, g["dx"]) <= 1e-11
    assert max_rel(dg, g["dg"]) <= 1e-11
    assert max_rel(db, g["db"]) <= 1e-11


@pytest.mark.parametrize(
    "shape,splits",
    [((2, 3, 5, 6, 7), None), ((1, 4, 9, 9, 9), 3), ((3, 2, 1, 1, 5), 2), ((1, 8, 16, 16, 16), 7),
     ((1, 3, 13, 15, 17), 5), ((2, 5, 7, 9, 11), 9)],
)
def test_fp32_against_oracle(shape, splits):
    print(f"[groupnorm fp32] shape={shape} splits={splits}", flush=True)
    gen = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(shape, generator=gen) * 2 + 3
    gam = torch.randn(shape[1], generator=gen)
    bet = torch.randn(shape[1], generator=gen)
    dy = torch.randn(shape, generator=gen)
    y, mean, rstd = hip_ops.group_norm_forward(x.to(DEV), gam.to(DEV), bet.to(DEV), splits=splits)
    dx, dg, db = hip_ops.group_norm_backward(dy.to(DEV), x.to(DEV), mean, rstd, gam.to(DEV), splits=splits)
    xn, gn, bn, dyn = (t.double().numpy() for t in (x, gam, bet, dy))
    y_ref, mean_ref, rstd_ref = ogn.forward(xn, gn, bn)
    dx_ref, dg_ref, db_ref = ogn.backward(dyn, xn, gn)
    assert max_rel(y, y_ref) <= FP32_OUT
    assert max_rel(mean, mean_ref.reshape(-1)) <= FP32_OUT
    assert max_rel(rstd, rstd_ref.reshape(-1)) <= FP32_OUT
    assert max_rel(dx, dx_ref) <= FP32_OUT
    assert max_rel(dg, dg_ref) <= FP32_WGRAD
    assert max_rel(db, db_ref) <= FP32_WGRAD


def test_autocast_bf16_in_fp32_out_stage0():
    """cfg2 stage 0: bf16 depthwise output 1x32x128^3 -> fp32 GroupNorm output,
    as autocast does in the reference; dx comes back in bf16 (the cast's
    backward)."""
    print("[groupnorm autocast] 1x32x128^3", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(1, 32, 128, 128, 128, generator=gen, device=DEV).bfloat16()
    gam = torch.randn(32, generator=gen, device=DEV)
    bet = torch.randn(32, generator=gen, device=DEV)
    dy = torch.randn(1, 32, 128, 128, 128, generator=gen, device=DEV)
    y, mean, rstd = hip_ops.group_norm_forward(x, gam, bet, out_dtype=torch.float32)
    dx, dg, db = hip_ops.group_norm_backward(dy, x, mean, rstd, gam)
    assert y.dtype == torch.float32 and dx.dtype == torch.bfloat16
    xf = x.float().requires_grad_()
    gf, bf = gam.clone().requires_grad_(), bet.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yr = F.group_norm(xf, 32, gf, bf)
    assert yr.dtype == torch.float32
    rdx, rdg, rdb = torch.autograd.grad(yr, (xf, gf, bf), dy)
    assert max_rel(y, yr) <= FP32_OUT
    assert max_rel(dx, rdx) <= BF16
    assert max_rel(dg, rdg) <= FP32_WGRAD
    assert max_rel(db, rdb) <= FP32_WGRAD


@pytest.mark.parametrize("size,splits", [(63, None), (31, 7), (15, 2)])
def test_autocast_bf16_odd_volumes(size, splits):
    """Up-block volumes (2s - 1)^3: every row starts at a different alignment,
    so the scalar head / 16-byte body / scalar tail split is exercised."""
    print(f"[groupnorm odd] 1x6x{size}^3 splits={splits}", flush=True)
    gen = torch.Generator().manual_seed(size)
    x = torch.randn(1, 6, size, size, size, generator=gen).bfloat16()
    gam, bet = torch.randn(6, generator=gen), torch.randn(6, generator=gen)
    dy = torch.randn(1, 6, size, size, size, generator=gen)
    y, mean, rstd = hip_ops.group_norm_forward(x.to(DEV), gam.to(DEV), bet.to(DEV), out_dtype=torch.float32,
                                               splits=splits)
    dx, dg, db = hip_ops.group_norm_backward(dy.to(DEV), x.to(DEV), mean, rstd, gam.to(DEV), splits=splits)
    xn, gn, bn, dyn = (t.double().numpy() for t in (x, gam, bet, dy))
    y_ref, _, _ = ogn.forward(xn, gn, bn)
    dx_ref, dg_ref, db_ref = ogn.backward(dyn, xn, gn)
    assert max_rel(y, y_ref) <= FP32_OUT
    assert max_rel(dx, dx_ref) <= BF16
    assert max_rel(dg, dg_ref) <= FP32_WGRAD
    assert max_rel(db, db_ref) <= FP32_WGRAD


def test_large_mean_is_stable():
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(1, 2, 32, 32, 32, generator=gen) + 1000.0
    y, _, _ = hip_ops.group_norm_forward(x.to(DEV), None, None)
    y_ref, _, _ = ogn.forward(x.double().numpy())
    assert max_rel(y, y_ref) <= 1e-4


def test_deterministic():
    gen = torch.Generator(device=DEV).manual_seed(12)
    x = torch.randn(2, 16, 24, 24, 24, generator=gen, device=DEV)
    dy = torch.randn_like(x)
    a = hip_ops.group_norm_forward(x, None, None)
    b = hip_ops.group_norm_forward(x, None, None)
    assert all(torch.equal(p, q) for p, q in zip(a, b))
    ga = hip_ops.group_norm_backward(dy, x, a[1], a[2], None)
    gb = hip_ops.group_norm_backward(dy, x, a[1], a[2], None)
    assert all(torch.equal(p, q) for p, q in zip(ga, gb))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_one_sample_parameter_gradients_match_the_batched_sum(dtype):
    """With one sample the apply kernel stores dgamma / dbeta itself (no
    parameter-gradient launch); they are the bits the batched path gives when
    a second sample contributes a zero gradient."""
    print(f"[gn one-sample param grads] dtype={dtype}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(2, 24, 9, 10, 11, generator=gen, device=DEV).to(dtype)
    dy = torch.randn(2, 24, 9, 10, 11, generator=gen, device=DEV).to(dtype)
    dy[1] = 0
    gam = torch.randn(24, generator=gen, device=DEV)
    bet = torch.randn(24, generator=gen, device=DEV)
    for splits in (1, 3):
        _, mean1, rstd1 = hip_ops.group_norm_forward(x[:1].contiguous(), gam, bet, 1e-5, None, splits=splits)
        _, dg1, db1 = hip_ops.group_norm_backward(dy[:1].contiguous(), x[:1].contiguous(), mean1, rstd1, gam,
                                                  splits=splits)
        _, mean2, rstd2 = hip_ops.group_norm_forward(x, gam, bet, 1e-5, None, splits=splits)
        _, dg2, db2 = hip_ops.group_norm_backward(dy, x, mean2, rstd2, gam, splits=splits)
        assert torch.equal(dg1, dg2) and torch.equal(db1, db2), splits
