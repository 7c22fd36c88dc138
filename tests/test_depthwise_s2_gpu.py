"""Stride-2 depthwise (MedNeXt down block) and its transpose (up block) on the GPU.

Raw maps (gather / scatter / weight-grad) against the float64 oracle on the
same dtype-rounded inputs, for every dtype, k in {1, 3, 5}, odd and even sizes
and batch 2, through both the band kernels and (rows too wide for them) the
row-task kernels; the two autograd ops against PyTorch's F.conv3d /
F.conv_transpose3d at MedNeXt down / up shapes. Tolerances: fp64 1e-12; fp32
1e-5 outputs / input grads, 1e-4 weight grads; bf16 / fp16 2e-2.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from helpers import BF16, FP32_OUT, FP32_WGRAD, max_rel
from mednext_accel_amd import hip_ops
from mednext_accel_amd.adaptive import AdaptiveDepthwise3d, ModelOptimizationContext
from mednext_accel_amd.optimization import PolicyRegistry
from oracle import depthwise as odw

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {
    torch.float64: (1e-12, 1e-12),
    torch.float32: (FP32_OUT, FP32_WGRAD),
    torch.bfloat16: (BF16, BF16),
    torch.float16: (BF16, BF16),
}


def rounded(shape, gen, dtype, scale=1.0):
    return (torch.randn(shape, generator=gen, dtype=torch.float64) * scale).to(dtype)


def f64(t):
    return t.double().cpu().numpy()


@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("big", [(8, 8, 8), (7, 9, 6), (5, 12, 13)])
def test_maps_against_oracle(k, dtype, big):
    print(f"[s2 maps] k={k} dtype={dtype} big={big}", flush=True)
    gen = torch.Generator().manual_seed(k * 100 + sum(big))
    n, c = 2, 3
    small = tuple((s - 1) // 2 + 1 for s in big)
    x = rounded((n, c, *big), gen, dtype)
    w = rounded((c, 1, k, k, k), gen, dtype, 1.0 / k)
    b = rounded((c,), gen, dtype)
    g = rounded((n, c, *small), gen, dtype)
    out_tol, w_tol = TOL[dtype]
    y = hip_ops.depthwise_s2_gather(x.to(DEV), w.to(DEV), b.to(DEV), small)
    assert max_rel(y, odw.strided_forward(f64(x), f64(w), f64(b))) <= out_tol
    dx = hip_ops.depthwise_s2_scatter(g.to(DEV), w.to(DEV), None, big)
    assert max_rel(dx, odw.strided_input_grad(f64(g), f64(w), big)) <= out_tol
    dw, ds = hip_ops.depthwise_s2_wgrad(x.to(DEV), g.to(DEV), k)
    want_dw, want_db = odw.strided_weight_grad(f64(x), f64(g), k)
    assert max_rel(dw, want_dw) <= w_tol
    assert max_rel(ds, want_db) <= w_tol
    assert y.dtype == dx.dtype == dw.dtype == ds.dtype == dtype


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize(
    "n,c,big",
    [
        (1, 1000, (8, 40, 32)),  # band kernels: 5 bands per small plane, 2 per reduce workgroup (last group ragged)
        (2, 2, (3, 3, 2000)),  # rows too wide for the staged LDS block: the row-task kernels
    ],
)
def test_maps_band_and_row_paths(n, c, big, k):
    print(f"[s2 maps paths] n={n} c={c} big={big} k={k}", flush=True)
    gen = torch.Generator().manual_seed(c + k + sum(big))
    dtype = torch.float32
    small = tuple((s - 1) // 2 + 1 for s in big)
    x = rounded((n, c, *big), gen, dtype)
    w = rounded((c, 1, k, k, k), gen, dtype, 1.0 / k)
    b = rounded((c,), gen, dtype)
    g = rounded((n, c, *small), gen, dtype)
    y = hip_ops.depthwise_s2_gather(x.to(DEV), w.to(DEV), b.to(DEV), small)
    assert max_rel(y, odw.strided_forward(f64(x), f64(w), f64(b))) <= FP32_OUT
    dw, ds = hip_ops.depthwise_s2_wgrad(x.to(DEV), g.to(DEV), k)
    want_dw, want_db = odw.strided_weight_grad(f64(x), f64(g), k)
    assert max_rel(dw, want_dw) <= FP32_WGRAD and max_rel(ds, want_db) <= FP32_WGRAD


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize(
    "n,c,big",
    [
        (2, 3, (6, 48, 64)),  # even big dims (down block)
        (1, 2, (10, 34, 96)),
        (1, 1, (4, 32, 32 * 9)),
        (2, 3, (7, 47, 63)),  # big = 2 small - 1 (up block): odd rows, element-exact big access
        (1, 2, (9, 33, 79)),
    ],
)
def test_mfma_route_maps_against_oracle(n, c, big, k):
    """bf16 maps whose small plane exceeds the band kernels (big = 2 small or
    2 small - 1): the matrix-core stencil with the output subsampled (gather),
    over the zero-upsampled small tensor (scatter), and the weight gradient
    with dy upsampled. Batch 2, row tiles past H (33 .. 48 rows), column tiles
    past W (63 .. 96 columns), odd widths, short D-runs."""
    print(f"[s2 mfma maps] n={n} c={c} big={big} k={k}", flush=True)
    gen = torch.Generator().manual_seed(7 * k + sum(big))
    dtype = torch.bfloat16
    small = tuple((s + 1) // 2 for s in big)
    x = rounded((n, c, *big), gen, dtype)
    w = rounded((c, 1, k, k, k), gen, dtype, 1.0 / k)
    b = rounded((c,), gen, dtype)
    g = rounded((n, c, *small), gen, dtype)
    y = hip_ops.depthwise_s2_gather(x.to(DEV), w.to(DEV), b.to(DEV), small)
    assert max_rel(y, odw.strided_forward(f64(x), f64(w), f64(b))) <= BF16
    dx = hip_ops.depthwise_s2_scatter(g.to(DEV), w.to(DEV), b.to(DEV), big)
    want_dx = odw.strided_input_grad(f64(g), f64(w), big) + f64(b).reshape(1, c, 1, 1, 1)
    assert max_rel(dx, want_dx) <= BF16
    dw, ds = hip_ops.depthwise_s2_wgrad(x.to(DEV), g.to(DEV), k)
    want_dw, want_db = odw.strided_weight_grad(f64(x), f64(g), k)
    assert max_rel(dw, want_dw) <= BF16 and max_rel(ds, want_db) <= BF16
    dw2, _ = hip_ops.depthwise_s2_wgrad(x.to(DEV), g.to(DEV), k)
    assert torch.equal(dw, dw2)


DOWN_UP = [(32, 128, 3), (64, 64, 3), (128, 32, 3), (64, 64, 5), (32, 128, 5)]


@pytest.mark.parametrize("channels,size,k", DOWN_UP)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_down_and_up_ops_against_torch(channels, size, k, dtype):
    """The down-block op on C x S^3 and the up-block op on C x (S/2)^3 -> (S-1)^3,
    forward and all gradients, against PyTorch (fp32 reference on the same
    dtype-rounded operands)."""
    print(f"[s2 ops] C={channels} S={size} k={k} {dtype}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(channels + size + k)
    out_tol, w_tol = TOL[dtype]
    # Down block: Conv3d(stride 2).
    x = torch.randn(1, channels, size, size, size, generator=gen, device=DEV).to(dtype)
    w = (torch.randn(channels, 1, k, k, k, generator=gen, device=DEV) / k**1.5).to(dtype)
    b = torch.randn(channels, generator=gen, device=DEV).to(dtype)
    leaves = [t.clone().requires_grad_() for t in (x, w, b)]
    y = hip_ops.depthwise_conv3d_stride2(*leaves, k)
    ref_leaves = [t.float().requires_grad_() for t in (x, w, b)]
    yr = F.conv3d(*ref_leaves, stride=2, padding=k // 2, groups=channels)
    assert y.shape == yr.shape and max_rel(y, yr) <= out_tol
    g = torch.randn_like(yr).to(dtype)
    got = torch.autograd.grad(y, leaves, g)
    want = torch.autograd.grad(yr, ref_leaves, g.float())
    assert max_rel(got[0], want[0]) <= out_tol
    assert max_rel(got[1], want[1]) <= w_tol and max_rel(got[2], want[2]) <= w_tol
    # Up block: ConvTranspose3d(stride 2) from (S/2)^3 to (S-1)^3.
    s = size // 2
    x2 = torch.randn(1, channels, s, s, s, generator=gen, device=DEV).to(dtype)
    leaves2 = [t.clone().requires_grad_() for t in (x2, w, b)]
    y2 = hip_ops.depthwise_conv_transpose3d_stride2(*leaves2, k)
    ref2 = [t.float().requires_grad_() for t in (x2, w, b)]
    yr2 = F.conv_transpose3d(*ref2, stride=2, padding=k // 2, groups=channels)
    assert y2.shape == yr2.shape == (1, channels, 2 * s - 1, 2 * s - 1, 2 * s - 1)
    assert max_rel(y2, yr2) <= out_tol
    g2 = torch.randn_like(yr2).to(dtype)
    got2 = torch.autograd.grad(y2, leaves2, g2)
    want2 = torch.autograd.grad(yr2, ref2, g2.float())
    assert max_rel(got2[0], want2[0]) <= out_tol
    assert max_rel(got2[1], want2[1]) <= w_tol and max_rel(got2[2], want2[2]) <= w_tol


def test_wrappers_route_strided_and_transposed_through_hip():
    from torch.utils._python_dispatch import TorchDispatchMode

    class Observe(TorchDispatchMode):
        def __init__(self):
            super().__init__()
            self.ops = []

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            self.ops.append(func._schema.name)
            return func(*args, **(kwargs or {}))

    mc = ModelOptimizationContext("mednext_v1", "base", "none")
    torch.manual_seed(3)
    down = nn.Conv3d(16, 16, 3, stride=2, padding=1, groups=16, device=DEV)
    up = nn.ConvTranspose3d(16, 16, 3, stride=2, padding=1, groups=16, device=DEV)
    for ref, name in ((down, "depthwise_conv3d_stride2"), (up, "depthwise_conv_transpose3d_stride2")):
        cand = AdaptiveDepthwise3d(copy.deepcopy(ref), PolicyRegistry().resolver(), mc)
        x = torch.randn(2, 16, 12, 10, 8, device=DEV, requires_grad=True)
        y = x.detach().clone().requires_grad_()
        with torch.autocast(DEV, dtype=torch.bfloat16), Observe() as seen:
            got = cand(y)
        assert f"mednext_accel_amd::{name}" in seen.ops
        with torch.autocast(DEV, dtype=torch.bfloat16):
            want = ref(x)
        assert got.shape == want.shape and max_rel(got, want) <= BF16
        gr = torch.randn_like(want)
        a = torch.autograd.grad(got, (y, *cand.parameters()), gr)
        bb = torch.autograd.grad(want, (x, *ref.parameters()), gr)
        for u, v in zip(a, bb, strict=True):
            assert max_rel(u, v) <= BF16


def test_opcheck_stride2_ops():
    gen = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(1, 3, 5, 6, 7, generator=gen, device=DEV, requires_grad=True)
    w = torch.randn(3, 1, 3, 3, 3, generator=gen, device=DEV, requires_grad=True)
    b = torch.randn(3, generator=gen, device=DEV, requires_grad=True)
    torch.library.opcheck(hip_ops.depthwise_conv3d_stride2, (x, w, b, 3))
    torch.library.opcheck(hip_ops.depthwise_conv_transpose3d_stride2, (x, w, b, 3))


def test_stride2_argument_errors():
    x = torch.randn(1, 2, 4, 4, 4, device=DEV)
    with pytest.raises(ValueError):
        hip_ops.depthwise_s2_gather(x, torch.randn(2, 1, 2, 2, 2, device=DEV), None, (2, 2, 2))  # even k
    with pytest.raises(ValueError):
        hip_ops.depthwise_s2_gather(x, torch.randn(3, 1, 3, 3, 3, device=DEV), None, (2, 2, 2))  # channels
    with pytest.raises(ValueError):
        hip_ops.depthwise_s2_scatter(x.transpose(2, 3), torch.randn(2, 1, 3, 3, 3, device=DEV), None, (8, 8, 8))
    with pytest.raises(ValueError):
        hip_ops.depthwise_s2_wgrad(x, x.double(), 3)
    assert np.isfinite(hip_ops.depthwise_s2_gather(x, torch.randn(2, 1, 3, 3, 3, device=DEV), None, (2, 2, 2)).cpu().numpy()).all()


@pytest.mark.parametrize("recipe", [[1, 32, 16], [1, 64, 16]])
def test_stencil_fill_sink_leaves_staged_rows_alone(recipe):
    """Regression: fill threads without a chunk once wrote their zeros at an
    offset from the plane buffer being filled, which for the second buffer
    fell inside the k = 3 output staging tile (32- and 64-column tiles) and
    raced with the staged-row stores. Three repeats must agree bit for bit and
    match the reference: the up-block forward at 63^3 (where the race showed)
    and the stride-1 forward at the affected tile widths."""
    gen = torch.Generator().manual_seed(5)
    c, k = 64, 3
    small = torch.randn(1, c, 32, 32, 32, generator=gen, dtype=torch.float64).bfloat16()
    w = (torch.randn(c, 1, k, k, k, generator=gen, dtype=torch.float64) / k).bfloat16()
    b = torch.randn(c, generator=gen, dtype=torch.float64).bfloat16()
    big = (63, 63, 63)
    outs = [hip_ops.depthwise_s2_scatter(small.to(DEV), w.to(DEV), b.to(DEV), big) for _ in range(3)]
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    want = odw.strided_input_grad(f64(small), f64(w), big) + f64(b).reshape(1, c, 1, 1, 1)
    assert max_rel(outs[0], want) <= BF16
    x = torch.randn(1, c, 64, 64, 64, generator=gen).bfloat16().to(DEV)
    ys = [hip_ops.depthwise_forward(x, w.to(DEV), b.to(DEV), recipe) for _ in range(3)]
    assert all(torch.equal(ys[0], y) for y in ys[1:])
    ref = F.conv3d(x.float(), w.to(DEV).float(), b.to(DEV).float(), padding=1, groups=c)
    assert max_rel(ys[0], ref) <= BF16
