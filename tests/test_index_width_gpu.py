"""Tensors past 2^31 elements: the kernels address them correctly.

The reference pins 64-bit addressing at the signed 32-bit element boundary:
batch 32 and 33 at C32 128^3 (N*C*V = 2^31 and above), the transposed
weight gradient at N=40, C=64, 64^3 -> 127^3, and a weight-gradient
reduction whose own length crosses 2^31 (N=2^22, C=1, 8^3) (reference
``tests/ops/test_depthwise_indexing.py:22-106``). The reference checks its
compiled IR; here the kernels run at those sizes.

Here each kernel forms a 64-bit base per (n, c) slab or per sample, and 32-bit
offsets inside it (the host rejects slabs >= 2 GiB). Every sample of a launch
holds the same data, so every sample's output must equal a one-sample launch's
bit for bit (an addressing error past 2^31 would show up as a wrong sample),
and a reduction over the batch (weight and bias gradients) must equal N times
the one-sample reduction within bf16 rounding.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from helpers import max_rel
from mednext_accel_amd import hip_ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
LIMIT = 2**31


def batch_of(one: torch.Tensor, n: int) -> torch.Tensor:
    return one.expand(n, *one.shape[1:]).contiguous()


def same_as_one(big: torch.Tensor, one: torch.Tensor) -> bool:
    return bool(torch.equal(big, one.expand_as(big)))


def fp32_weight_grad(x1, dy1, k, stride=1, transpose=False):
    """dW (and dB) of one sample in fp32 by PyTorch on the GPU."""
    c = x1.shape[1]
    w = torch.zeros(c, 1, k, k, k, device=DEV, requires_grad=True)
    b = torch.zeros(c, device=DEV, requires_grad=True)
    xf = x1.float()
    if transpose:
        y = F.conv_transpose3d(xf, w, b, stride=stride, padding=k // 2, groups=c)
    else:
        y = F.conv3d(xf, w, b, stride=stride, padding=k // 2, groups=c)
    return torch.autograd.grad(y, (w, b), dy1.float())


def cleanup():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("n", [32, 33])
def test_depthwise_regular_bf16_past_2_31(n):
    """Matrix-core forward, input gradient and weight gradient, C32 128^3."""
    print(f"[index width] regular k3 bf16 N={n} C=32 128^3", flush=True)
    c, s, k = 32, 128, 3
    assert n * c * s**3 >= LIMIT
    gen = torch.Generator(device=DEV).manual_seed(n)
    x1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    dy1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    w = (torch.randn(c, 1, k, k, k, generator=gen, device=DEV) / k**1.5).bfloat16()
    b = torch.randn(c, generator=gen, device=DEV).bfloat16()
    x, dy = batch_of(x1, n), batch_of(dy1, n)
    assert same_as_one(hip_ops.depthwise_forward(x, w, b), hip_ops.depthwise_forward(x1, w, b))
    assert same_as_one(hip_ops.depthwise_input_grad(dy, w), hip_ops.depthwise_input_grad(dy1, w))
    assert same_as_one(hip_ops.depthwise_input_grad_acc(dy, w, x, None), hip_ops.depthwise_input_grad_acc(dy1, w, x1, None))
    dw, db = hip_ops.depthwise_weight_grad(x, dy, k)
    rw, rb = fp32_weight_grad(x1, dy1, k)
    assert max_rel(dw, n * rw) <= 1e-2 and max_rel(db, n * rb) <= 1e-2
    del x, dy
    cleanup()


def test_depthwise_regular_fp32_past_2_31():
    """VALU engine (fp32), N=33 at C32 128^3: 8.9 GB per tensor."""
    print("[index width] regular k3 fp32 N=33 C=32 128^3", flush=True)
    n, c, s, k = 33, 32, 128, 3
    gen = torch.Generator(device=DEV).manual_seed(5)
    x1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV)
    dy1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV)
    w = torch.randn(c, 1, k, k, k, generator=gen, device=DEV) / k**1.5
    x, dy = batch_of(x1, n), batch_of(dy1, n)
    assert same_as_one(hip_ops.depthwise_forward(x, w), hip_ops.depthwise_forward(x1, w))
    assert same_as_one(hip_ops.depthwise_input_grad(dy, w), hip_ops.depthwise_input_grad(dy1, w))
    dw, db = hip_ops.depthwise_weight_grad(x, dy, k)
    rw, rb = fp32_weight_grad(x1, dy1, k)
    assert max_rel(dw, n * rw) <= 1e-4 and max_rel(db, n * rb) <= 1e-4
    del x, dy
    cleanup()


def test_stride2_down_block_past_2_31():
    """Stride-2 conv (gather), its input gradient (scatter) and weight
    gradient, bf16, N=33 C=32 128^3 -> 64^3."""
    print("[index width] stride-2 k3 bf16 N=33 C=32 128^3", flush=True)
    n, c, s, k = 33, 32, 128, 3
    gen = torch.Generator(device=DEV).manual_seed(7)
    x1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    g1 = torch.randn(1, c, s // 2, s // 2, s // 2, generator=gen, device=DEV).bfloat16()
    w = (torch.randn(c, 1, k, k, k, generator=gen, device=DEV) / k**1.5).bfloat16()
    x, g = batch_of(x1, n), batch_of(g1, n)
    small = [s // 2] * 3
    assert same_as_one(hip_ops.depthwise_s2_gather(x, w, None, small), hip_ops.depthwise_s2_gather(x1, w, None, small))
    assert same_as_one(hip_ops.depthwise_s2_scatter(g, w, None, [s] * 3), hip_ops.depthwise_s2_scatter(g1, w, None, [s] * 3))
    dw, db = hip_ops.depthwise_s2_wgrad(x, g, k)
    rw, rb = fp32_weight_grad(x1, g1, k, stride=2)
    assert max_rel(dw, n * rw) <= 1e-2 and max_rel(db, n * rb) <= 1e-2
    del x, g
    cleanup()


def test_transposed_up_block_past_2_31():
    """Transposed stride-2 conv at the reference's case N=40, C=64, 64^3 ->
    127^3 (5.2e9 output elements): forward (scatter), input gradient
    (gather) and weight gradient."""
    print("[index width] transposed k3 bf16 N=40 C=64 64^3 -> 127^3", flush=True)
    n, c, s, k = 40, 64, 64, 3
    big = [2 * s - 1] * 3
    gen = torch.Generator(device=DEV).manual_seed(9)
    x1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    g1 = torch.randn(1, c, *big, generator=gen, device=DEV).bfloat16()
    w = (torch.randn(c, 1, k, k, k, generator=gen, device=DEV) / k**1.5).bfloat16()
    x, g = batch_of(x1, n), batch_of(g1, n)
    assert n * c * big[0] ** 3 >= LIMIT
    assert same_as_one(hip_ops.depthwise_s2_scatter(x, w, None, big), hip_ops.depthwise_s2_scatter(x1, w, None, big))
    assert same_as_one(hip_ops.depthwise_s2_gather(g, w, None, [s] * 3), hip_ops.depthwise_s2_gather(g1, w, None, [s] * 3))
    dw, _ = hip_ops.depthwise_s2_wgrad(g, x, k)
    rw, _ = fp32_weight_grad(x1, g1, k, stride=2, transpose=True)
    assert max_rel(dw, n * rw) <= 1e-2
    del x, g
    cleanup()


def test_weight_grad_reduction_longer_than_2_31():
    """N=2^22, C=1, 8^3: the weight-gradient reduction itself runs over
    2^31 elements per tap."""
    print("[index width] wgrad reduction N=2^22 C=1 8^3 bf16", flush=True)
    n, c, s, k = 2**22, 1, 8, 3
    gen = torch.Generator(device=DEV).manual_seed(11)
    x1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    dy1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    x, dy = batch_of(x1, n), batch_of(dy1, n)
    assert x.numel() >= LIMIT
    dw, db = hip_ops.depthwise_weight_grad(x, dy, k)
    rw, rb = fp32_weight_grad(x1, dy1, k)
    assert max_rel(dw, n * rw) <= 1e-2 and max_rel(db, n * rb) <= 1e-2
    del x, dy
    cleanup()


def test_group_norm_and_pointwise_past_2_31():
    """GroupNorm (bf16 in, fp32 out as under autocast) and the 32 -> 64
    pointwise GEMM with its weight gradient, N=33 at C32 128^3."""
    print("[index width] group norm + pointwise bf16 N=33 C=32 128^3", flush=True)
    n, c, s = 33, 32, 128
    gen = torch.Generator(device=DEV).manual_seed(13)
    x1 = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    x = batch_of(x1, n)
    gamma = torch.rand(c, generator=gen, device=DEV) + 0.5
    beta = torch.randn(c, generator=gen, device=DEV)
    # The default row split depends on the batch (fewer chunks per row when
    # there are many rows); the same split gives every row the same arithmetic.
    y, mean, rstd = hip_ops.group_norm_forward(x, gamma, beta, out_dtype=torch.float32, splits=16)
    y1, mean1, rstd1 = hip_ops.group_norm_forward(x1, gamma, beta, out_dtype=torch.float32, splits=16)
    assert same_as_one(y, y1)
    assert torch.equal(mean.view(n, c), mean1.view(1, c).expand(n, c))
    assert torch.equal(rstd.view(n, c), rstd1.view(1, c).expand(n, c))
    del y
    cleanup()
    w = (torch.randn(64, c, 1, 1, 1, generator=gen, device=DEV) / c**0.5).bfloat16()
    bias = torch.randn(64, generator=gen, device=DEV).bfloat16()
    out = hip_ops.pointwise_conv(x, w, bias)
    out1 = hip_ops.pointwise_conv(x1, w, bias)
    assert same_as_one(out, out1)
    dy = batch_of(torch.randn(1, 64, s, s, s, generator=gen, device=DEV).bfloat16(), n)
    dw, db = hip_ops.pointwise_weight_grad(dy, x, with_bias=True)
    dw1, db1 = hip_ops.pointwise_weight_grad(dy[:1].contiguous(), x1, with_bias=True)
    assert max_rel(dw, n * dw1.float()) <= 1e-2 and max_rel(db, n * db1.float()) <= 1e-2
    del x, out, dy
    cleanup()
