"""HIP pointwise (1x1x1) GEMMs with fused GELU / residual epilogues on the GPU.

Small and ragged shapes are checked against the float64 oracle on the same
bf16-rounded inputs; the MedNeXt stage shapes against PyTorch in fp32. The
kernels take bf16 operands and accumulate in fp32, so the bar is the bf16
autocast tolerance (normwise max relative error <= 2e-2).
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import BF16, max_rel
from mednext_accel_amd import hip_ops
from mednext_accel_amd.hip_ops import (
    PW_EPILOGUE_BIAS,
    PW_EPILOGUE_BIAS_GELU,
    PW_EPILOGUE_BIAS_RESIDUAL,
    PW_EPILOGUE_GELU_GRAD,
    PW_PROLOGUE_GELU,
    PW_PROLOGUE_NONE,
)
from oracle import pointwise as opw

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).bfloat16()


def f64(t):
    return t.double().cpu().numpy()


SHAPES = [
    # (n, cin, cout, spatial)
    (1, 32, 64, (4, 8, 8)),  # V = 256: two full chunks
    (2, 64, 32, (3, 5, 8)),  # V = 120: ragged last chunk, batch 2
    (1, 96, 48, (2, 4, 16)),  # K = 3 x 32, M = 48 (partial 64-row block)
    (1, 32, 192, (1, 8, 17 * 8)),  # M = 192: three row blocks
    (1, 512, 128, (2, 2, 8)),  # K = 512 (largest LDS weight block)
]


@pytest.mark.parametrize("n,cin,cout,spatial", SHAPES)
@pytest.mark.parametrize("epilogue", ["bias", "bias_gelu", "bias_residual", "none"])
def test_forward_epilogues_against_oracle(n, cin, cout, spatial, epilogue):
    print(f"[pw fwd] n={n} cin={cin} cout={cout} spatial={spatial} epi={epilogue}", flush=True)
    gen = torch.Generator().manual_seed(cin * 7 + cout)
    x = bf((n, cin, *spatial), gen)
    w = bf((cout, cin, 1, 1, 1), gen, cin**-0.5)
    b = bf((cout,), gen)
    res = bf((n, cout, *spatial), gen)
    code = {"bias": PW_EPILOGUE_BIAS, "none": PW_EPILOGUE_BIAS, "bias_gelu": PW_EPILOGUE_BIAS_GELU,
            "bias_residual": PW_EPILOGUE_BIAS_RESIDUAL}[epilogue]
    bias = None if epilogue == "none" else b
    y = hip_ops.pointwise_conv(
        x.to(DEV), w.to(DEV), None if bias is None else bias.to(DEV),
        aux=res.to(DEV) if epilogue == "bias_residual" else None, epilogue=code,
    )
    expect = opw.conv1x1(f64(x), f64(w), None if bias is None else f64(bias))
    if epilogue == "bias_gelu":
        expect = opw.gelu(expect)
    if epilogue == "bias_residual":
        expect = expect + f64(res)
    assert y.dtype == torch.bfloat16 and y.shape == (n, cout, *spatial)
    assert max_rel(y, expect) <= BF16


# Shapes valid in both directions (the transposed product has K = cout).
BOTH_WAYS = [(1, 32, 64, (4, 8, 8)), (2, 64, 32, (3, 5, 8)), (1, 32, 192, (1, 8, 17 * 8)), (1, 96, 64, (2, 4, 16))]


@pytest.mark.parametrize("n,cin,cout,spatial", BOTH_WAYS)
def test_gelu_prologue_and_transposed_product(n, cin, cout, spatial):
    gen = torch.Generator().manual_seed(3 * cin + cout)
    x = bf((n, cin, *spatial), gen, 2.0)
    w = bf((cout, cin, 1, 1, 1), gen, cin**-0.5)
    b = bf((cout,), gen)
    y = hip_ops.pointwise_conv(x.to(DEV), w.to(DEV), b.to(DEV), prologue=PW_PROLOGUE_GELU)
    assert max_rel(y, opw.conv1x1(opw.gelu(f64(x)), f64(w), f64(b))) <= BF16
    # Input gradient: dX = W^T dY, weight given in the conv's own [Cout, Cin] layout.
    dy = bf((n, cout, *spatial), gen)
    dx = hip_ops.pointwise_conv(dy.to(DEV), w.to(DEV), transpose=True)
    want_dx, _, _ = opw.conv1x1_backward(f64(dy), f64(x), f64(w))
    assert dx.shape == x.shape and max_rel(dx, want_dx) <= BF16
    # GELU backward fused into the input gradient: dH = (W^T dY) * GELU'(h).
    h = bf((n, cin, *spatial), gen, 2.0)
    dh = hip_ops.pointwise_conv(dy.to(DEV), w.to(DEV), aux=h.to(DEV), epilogue=PW_EPILOGUE_GELU_GRAD, transpose=True)
    assert max_rel(dh, want_dx * opw.gelu_grad(f64(h))) <= BF16


@pytest.mark.parametrize("n,cin,cout,spatial", SHAPES)
@pytest.mark.parametrize("gelu_input", [False, True])
def test_weight_and_bias_grad_against_oracle(n, cin, cout, spatial, gelu_input):
    print(f"[pw wgrad] n={n} cin={cin} cout={cout} spatial={spatial} gelu={gelu_input}", flush=True)
    gen = torch.Generator().manual_seed(11 * cin + cout)
    x = bf((n, cin, *spatial), gen)
    dy = bf((n, cout, *spatial), gen)
    w0 = np.zeros((cout, cin, 1, 1, 1))
    prologue = PW_PROLOGUE_GELU if gelu_input else PW_PROLOGUE_NONE
    dw, db = hip_ops.pointwise_weight_grad(dy.to(DEV), x.to(DEV), prologue=prologue)
    xin = opw.gelu(f64(x)) if gelu_input else f64(x)
    _, want_dw, want_db = opw.conv1x1_backward(f64(dy), xin, w0)
    assert dw.shape == (cout, cin, 1, 1, 1) and db.shape == (cout,)
    assert max_rel(dw, want_dw) <= BF16
    assert max_rel(db, want_db) <= BF16


@pytest.mark.parametrize("splits", [1, 3, 64])
def test_weight_grad_splits_and_determinism(splits):
    gen = torch.Generator().manual_seed(5)
    x = bf((2, 64, 8, 8, 24), gen).to(DEV)
    dy = bf((2, 96, 8, 8, 24), gen).to(DEV)
    a = hip_ops.pointwise_weight_grad(dy, x, splits=splits)
    b = hip_ops.pointwise_weight_grad(dy, x, splits=splits)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    _, want_dw, want_db = opw.conv1x1_backward(f64(dy), f64(x), np.zeros((96, 64, 1, 1, 1)))
    assert max_rel(a[0], want_dw) <= BF16 and max_rel(a[1], want_db) <= BF16


@pytest.mark.parametrize(
    "n,cin,cout,spatial,splits,with_bias",
    [
        (2, 32, 96, (16, 32, 128), 512, True),  # 1024 slots, 16 outputs per block, 16 waves
        (2, 32, 96, (16, 32, 128), 512, False),
        (1, 128, 160, (8, 8, 40), 7, True),  # 32 outputs per block, one wave
        (3, 256, 192, (4, 4, 50), 20, False),  # 64 outputs per block, two waves
    ],
)
def test_weight_grad_reduction_shapes(n, cin, cout, spatial, splits, with_bias):
    """The one-launch partial reduction at each of its block shapes (outputs
    per block, waves), with and without the bias gradient; run twice."""
    print(f"[pw wgrad reduce] n={n} cin={cin} cout={cout} spatial={spatial} splits={splits}", flush=True)
    gen = torch.Generator().manual_seed(cin + cout + splits)
    x = bf((n, cin, *spatial), gen).to(DEV)
    dy = bf((n, cout, *spatial), gen).to(DEV)
    a = hip_ops.pointwise_weight_grad(dy, x, splits=splits, with_bias=with_bias)
    b = hip_ops.pointwise_weight_grad(dy, x, splits=splits, with_bias=with_bias)
    assert torch.equal(a[0], b[0])
    assert (a[1] is None) == (not with_bias)
    _, want_dw, want_db = opw.conv1x1_backward(f64(dy), f64(x), np.zeros((cout, cin, 1, 1, 1)))
    assert max_rel(a[0], want_dw) <= BF16
    if with_bias:
        assert torch.equal(a[1], b[1]) and max_rel(a[1], want_db) <= BF16


STAGES = [(32, 64, 128), (64, 32, 128), (64, 192, 64), (192, 64, 64), (128, 512, 32), (512, 128, 32)]


@pytest.mark.parametrize("cin,cout,size", STAGES)
def test_stage_shapes_against_torch_fp32(cin, cout, size):
    """MedNeXt-B expand / project shapes (configs[2]/[3]) vs PyTorch fp32 on the
    same bf16 inputs: forward, input gradient, weight and bias gradients."""
    print(f"[pw stage] {cin}->{cout} @ {size}^3", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(cin + cout)
    x = torch.randn(1, cin, size, size, size, generator=gen, device=DEV).bfloat16()
    w = (torch.randn(cout, cin, 1, 1, 1, generator=gen, device=DEV) * cin**-0.5).bfloat16()
    b = torch.randn(cout, generator=gen, device=DEV).bfloat16()
    dy = torch.randn(1, cout, size, size, size, generator=gen, device=DEV).bfloat16()
    xf, wf, bf_ = (t.float().requires_grad_() for t in (x, w, b))
    yf = F.conv3d(xf, wf, bf_)
    rdx, rdw, rdb = torch.autograd.grad(yf, (xf, wf, bf_), dy.float())
    y = hip_ops.pointwise_conv(x, w, b)
    dx = hip_ops.pointwise_conv(dy, w, transpose=True)
    dw, db = hip_ops.pointwise_weight_grad(dy, x)
    assert max_rel(y, yf) <= BF16
    assert max_rel(dx, rdx) <= BF16
    assert max_rel(dw, rdw) <= BF16
    assert max_rel(db, rdb) <= BF16


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("residual,c,r,s", [(True, 32, 2, 32), (False, 32, 2, 32), (True, 64, 3, 20), (True, 96, 4, 9)])
def test_fused_mlp_expansion_matches_unfused_fp32(residual, c, r, s, stored):
    """mlp_expansion (GELU recomputed from h) and mlp_expansion_stored (GELU
    and GELU' stored by the expand GEMM) = project(GELU(expand(x))) + residual,
    fwd + bwd, vs the same composition in fp32 PyTorch on the bf16-rounded
    operands."""
    gen = torch.Generator(device=DEV).manual_seed(2)
    x = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    res = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    w1 = (torch.randn(r * c, c, 1, 1, 1, generator=gen, device=DEV) * c**-0.5).bfloat16()
    b1 = (torch.randn(r * c, generator=gen, device=DEV) * 0.1).bfloat16()
    w2 = (torch.randn(c, r * c, 1, 1, 1, generator=gen, device=DEV) * (r * c) ** -0.5).bfloat16()
    b2 = (torch.randn(c, generator=gen, device=DEV) * 0.1).bfloat16()
    leaves = [t.clone().requires_grad_() for t in (x, w1, b1, w2, b2, res)]
    op = hip_ops.mlp_expansion_stored if stored else hip_ops.mlp_expansion
    out = op(*leaves[:5], leaves[5] if residual else None)[0]
    ref_leaves = [t.float().requires_grad_() for t in (x, w1, b1, w2, b2, res)]
    xf, w1f, b1f, w2f, b2f, rf = ref_leaves
    ref = F.conv3d(F.gelu(F.conv3d(xf, w1f, b1f)), w2f, b2f) + (rf if residual else 0)
    assert max_rel(out, ref) <= BF16
    g = torch.randn_like(ref).bfloat16()
    inputs = leaves if residual else leaves[:5]
    got = torch.autograd.grad(out, inputs, g)
    want = torch.autograd.grad(ref, ref_leaves if residual else ref_leaves[:5], g.float())
    for name, a, b in zip(["x", "w1", "b1", "w2", "b2", "res"], got, want):
        assert max_rel(a, b) <= BF16, name


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("n,c,r,s,residual", [(1, 32, 2, 32, True), (2, 64, 3, 12, True), (1, 96, 4, 9, False)])
def test_groupnorm_folded_expansion_matches_fp32(n, c, r, s, residual, stored):
    """gn_mlp_expansion = project(GELU(expand(GroupNorm(d)))) + residual with the
    GroupNorm folded into the expand GEMM's NORM prologue, fwd + bwd (d, gamma,
    beta, both weights and biases, residual) vs the same composition in fp32
    PyTorch on the bf16 operands."""
    print(f"[gn folded expansion] n={n} c={c} r={r} s={s} residual={residual} stored={stored}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(3 + c)
    d = (torch.randn(n, c, s, s, s, generator=gen, device=DEV) * 2 + 0.5).bfloat16()
    res = torch.randn(n, c, s, s, s, generator=gen, device=DEV).bfloat16()
    gamma = 1 + 0.2 * torch.randn(c, generator=gen, device=DEV)
    beta = 0.1 * torch.randn(c, generator=gen, device=DEV)
    w1 = (torch.randn(r * c, c, 1, 1, 1, generator=gen, device=DEV) * c**-0.5).bfloat16()
    b1 = (torch.randn(r * c, generator=gen, device=DEV) * 0.1).bfloat16()
    w2 = (torch.randn(c, r * c, 1, 1, 1, generator=gen, device=DEV) * (r * c) ** -0.5).bfloat16()
    b2 = (torch.randn(c, generator=gen, device=DEV) * 0.1).bfloat16()
    leaves = [t.clone().requires_grad_() for t in (d, gamma, beta, w1, b1, w2, b2, res)]
    out = hip_ops.gn_mlp_expansion(*leaves[:7], leaves[7] if residual else None, 1e-5, stored)[0]
    ref_leaves = [t.float().requires_grad_() for t in (d, gamma, beta, w1, b1, w2, b2, res)]
    df, gf, bf_, w1f, b1f, w2f, b2f, rf = ref_leaves
    ref = F.conv3d(F.gelu(F.conv3d(F.group_norm(df, c, gf, bf_, 1e-5), w1f, b1f)), w2f, b2f) + (rf if residual else 0)
    assert max_rel(out, ref) <= BF16
    g = torch.randn_like(ref).bfloat16()
    inputs = leaves if residual else leaves[:7]
    got = torch.autograd.grad(out, inputs, g)
    want = torch.autograd.grad(ref, ref_leaves if residual else ref_leaves[:7], g.float())
    for name, a, b in zip(["d", "gamma", "beta", "w1", "b1", "w2", "b2", "res"], got, want):
        assert max_rel(a, b) <= BF16, name


def test_groupnorm_stats_match_the_forward():
    """group_norm_stats: mean / rstd bit-identical to group_norm_forward's, and
    the NORM records (rstd * gamma, beta, mean, rstd) reproduce its output."""
    gen = torch.Generator(device=DEV).manual_seed(9)
    x = (torch.randn(2, 24, 9, 10, 11, generator=gen, device=DEV) * 3 + 1).bfloat16()
    w = torch.randn(24, generator=gen, device=DEV)
    b = torch.randn(24, generator=gen, device=DEV)
    y, mean, rstd = hip_ops.group_norm_forward(x, w, b, 1e-5, torch.float32)
    coef, m2, r2 = hip_ops.group_norm_stats(x, w, b, 1e-5)
    assert torch.equal(mean, m2) and torch.equal(rstd, r2)
    assert torch.equal(coef[..., 2].flatten().float(), mean) and torch.equal(coef[..., 3].flatten().float(), rstd)
    assert torch.equal(coef[..., 0], coef[..., 3] * w.double())  # rstd * gamma in fp64
    assert torch.equal(coef[..., 1], b.double().expand(2, 24))
    s_, t_, c_ = (coef[..., i].float().view(2, 24, 1, 1, 1) for i in range(3))
    assert torch.allclose((x.float() - c_) * s_ + t_, y, rtol=1e-5, atol=1e-5)


# (n, k, m, s): streaming kernels (K 32 / 96), split-K (K 256), and shapes the
# tiled product takes under AUTO (K 256 with a wide M).
NORM_SHAPES = [(1, 32, 64, 16), (2, 96, 192, 9), (1, 256, 64, 8), (1, 256, 1024, 16)]


@pytest.mark.parametrize("n,k,m,s", NORM_SHAPES)
def test_norm_prologue_reproduces_the_group_norm_output_bitwise(n, k, m, s):
    """The NORM prologue hands the MFMAs exactly the bf16 values
    group_norm_forward writes: every kernel family (streaming / split-K,
    tiled at 128 and 64 rows) and epilogue gives bit-identical outputs with
    the normalisation folded or run first."""
    print(f"[norm prologue bitwise] n={n} k={k} m={m} s={s}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(k + m)
    d = (torch.randn(n, k, s, s, s, generator=gen, device=DEV) * 2 - 0.7).bfloat16()
    gamma = 1 + 0.3 * torch.randn(k, generator=gen, device=DEV)
    beta = 0.2 * torch.randn(k, generator=gen, device=DEV)
    w = (torch.randn(m, k, 1, 1, 1, generator=gen, device=DEV) * k**-0.5).bfloat16()
    b = (torch.randn(m, generator=gen, device=DEV) * 0.1).bfloat16()
    res = torch.randn(n, m, s, s, s, generator=gen, device=DEV).bfloat16()
    h, _, _ = hip_ops.group_norm_forward(d, gamma, beta, 1e-5, torch.bfloat16)
    coef, _, _ = hip_ops.group_norm_stats(d, gamma, beta, 1e-5)
    cases = [
        (hip_ops.PW_EPILOGUE_BIAS, None),
        (hip_ops.PW_EPILOGUE_BIAS_RESIDUAL, res),
        (hip_ops.PW_EPILOGUE_BIAS_GELU_PAIR, None),
    ]
    try:
        for choice in (hip_ops.PW_KERNELS_AUTO, hip_ops.PW_KERNELS_STREAMING, hip_ops.PW_KERNELS_TILED,
                       hip_ops.PW_KERNELS_TILED_64):
            hip_ops.set_pointwise_kernels(choice)
            for epi, aux in cases:
                folded = hip_ops.pointwise_conv(d, w, b, aux=aux, epilogue=epi, prologue=hip_ops.PW_PROLOGUE_NORM,
                                                prologue_coef=coef)
                plain = hip_ops.pointwise_conv(h, w, b, aux=aux, epilogue=epi)
                for a, c in zip(folded if isinstance(folded, tuple) else (folded,),
                                plain if isinstance(plain, tuple) else (plain,)):
                    assert torch.equal(a, c), (choice, epi)
    finally:
        hip_ops.set_pointwise_kernels(hip_ops.PW_KERNELS_AUTO)


@pytest.mark.parametrize("n,k,m,s", [(2, 32, 64, 12), (1, 128, 256, 16), (2, 96, 160, 10)])
def test_norm_weight_grad_is_the_exact_map_of_the_raw_product(n, k, m, s):
    """NORM / AFFINE weight gradients: the library sums dy x over voxels and
    maps each sample's sums with its records, so dW matches
    sum dy ((x - c) s + t) in float64 (records taken as floats) to the bf16
    rounding of the output, on every weight-gradient tile (64 x 64 and
    128 x 128)."""
    print(f"[norm wgrad] n={n} k={k} m={m} s={s}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(7 * k + m)
    x = (torch.randn(n, k, s, s, s, generator=gen, device=DEV) * 1.5 + 2.0).bfloat16()
    dy = torch.randn(n, m, s, s, s, generator=gen, device=DEV).bfloat16()
    gamma = 1 + 0.3 * torch.randn(k, generator=gen, device=DEV)
    beta = 0.2 * torch.randn(k, generator=gen, device=DEV)
    coef, _, _ = hip_ops.group_norm_stats(x, gamma, beta, 1e-5)
    cf = coef.float().double()
    v = s**3
    xs = (x.double().view(n, k, v) - cf[..., 2:3]) * cf[..., :1] + cf[..., 1:2]
    dyd = dy.double().view(n, m, v)
    want_dw = torch.einsum("nmv,nkv->mk", dyd, xs)
    want_db = dyd.sum(dim=(0, 2))
    try:
        for choice in (hip_ops.PW_KERNELS_STREAMING, hip_ops.PW_KERNELS_TILED):
            hip_ops.set_pointwise_kernels(choice)
            dw, db = hip_ops.pointwise_weight_grad(dy, x, prologue=hip_ops.PW_PROLOGUE_NORM, prologue_coef=coef)
            err = (dw.view(m, k).double() - want_dw).abs() / want_dw.abs().clamp_min(1e-3 * want_dw.abs().max())
            assert float(err.max()) <= 2**-8, choice  # one bf16 rounding of the output
            assert max_rel(db, want_db) <= 2**-8
    finally:
        hip_ops.set_pointwise_kernels(hip_ops.PW_KERNELS_AUTO)


def test_opcheck_pointwise_ops():
    gen = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(1, 32, 2, 4, 8, generator=gen, device=DEV).bfloat16().requires_grad_()
    w = (torch.randn(64, 32, 1, 1, 1, generator=gen, device=DEV) / 6).bfloat16().requires_grad_()
    b = torch.randn(64, generator=gen, device=DEV).bfloat16().requires_grad_()
    torch.library.opcheck(hip_ops.pointwise_conv3d, (x, w, b))
    w2 = (torch.randn(32, 64, 1, 1, 1, generator=gen, device=DEV) / 8).bfloat16().requires_grad_()
    res = torch.randn(1, 32, 2, 4, 8, generator=gen, device=DEV).bfloat16().requires_grad_()
    torch.library.opcheck(hip_ops.mlp_expansion, (x, w, b, w2, None, res))
    torch.library.opcheck(hip_ops.mlp_expansion_stored, (x, w, b, w2, None, res))
    gamma = torch.randn(x.shape[1], device=DEV).requires_grad_()
    beta = torch.randn(x.shape[1], device=DEV).requires_grad_()
    for stored in (False, True):
        torch.library.opcheck(hip_ops.gn_mlp_expansion, (x, gamma, beta, w, b, w2, None, res, 1e-5, stored))


def test_channels_above_2048_take_the_tiled_product():
    """K above the streaming kernels' 2048-channel weight block runs the tiled
    product (K <= 8192, K % 32 == 0, M % 16 == 0): the tile policy selects the
    kernels exactly there, and the C ABI refuses the rest with a message."""
    from mednext_accel_amd.tiles import pointwise_supported

    assert pointwise_supported(4096, 512, 8**3) and pointwise_supported(512, 4096, 8**3)
    assert pointwise_supported(8192, 16, 8) and not pointwise_supported(8224, 32, 8)
    assert not pointwise_supported(4112, 512, 8**3) and not pointwise_supported(4096, 520, 8**3)
    assert pointwise_supported(2048, 520, 8**3) and pointwise_supported(1, 32, 127**3)
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(2, 4096, 2, 4, 9, generator=gen).bfloat16()
    w = (torch.randn(256, 4096, 1, 1, 1, generator=gen) / 64).bfloat16()
    b = torch.randn(256, generator=gen).bfloat16()
    res = torch.randn(2, 256, 2, 4, 9, generator=gen).bfloat16()
    want = torch.einsum("mk,nkv->nmv", w.double().view(256, 4096), x.double().flatten(2)).view(2, 256, 2, 4, 9)
    y = hip_ops.pointwise_conv(x.to(DEV), w.to(DEV), b.to(DEV), aux=res.to(DEV), epilogue=PW_EPILOGUE_BIAS_RESIDUAL)
    assert max_rel(y, want + b.double().view(1, -1, 1, 1, 1) + res.double()) <= BF16
    # transposed product (input gradient of a 4096 -> 256 conv's twin): K = 4096 rows of a [K][M] weight
    wt = (torch.randn(4096, 256, 1, 1, 1, generator=gen) / 64).bfloat16()
    dx = hip_ops.pointwise_conv(x.to(DEV), wt.to(DEV), transpose=True)
    want_t = torch.einsum("km,nkv->nmv", wt.double().view(4096, 256), x.double().flatten(2)).view(2, 256, 2, 4, 9)
    assert max_rel(dx, want_t) <= BF16
    with pytest.raises(hip_ops._hip.HipLibraryError, match="tiled product only"):
        hip_ops.pointwise_conv(x.to(DEV), w.to(DEV), prologue=PW_PROLOGUE_GELU)
    xr = torch.randn(1, 4112, 1, 1, 8, device=DEV).bfloat16()
    with pytest.raises(hip_ops._hip.HipLibraryError, match="tiled product only"):
        hip_ops.pointwise_conv(xr, torch.randn(256, 4112, 1, 1, 1, device=DEV).bfloat16())
    hip_ops.set_pointwise_kernels(hip_ops.PW_KERNELS_STREAMING)
    try:
        with pytest.raises(hip_ops._hip.HipLibraryError, match="tiled product only"):
            hip_ops.pointwise_conv(x.to(DEV), w.to(DEV))
    finally:
        hip_ops.set_pointwise_kernels(hip_ops.PW_KERNELS_AUTO)


@pytest.mark.parametrize("s", [8, 5])
def test_fused_mlp_expansion_at_4096_hidden_channels(s):
    """The MedNeXt-L bottleneck block's expansion (512 -> 4096 -> 512, expansion
    ratio 8) fwd + bwd through the fused op vs the same composition in fp32
    PyTorch: the project product and the expand input gradient reduce over
    4096 channels (tiled product with K split over workgroups)."""
    gen = torch.Generator(device=DEV).manual_seed(8)
    c, h = 512, 4096
    x = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    res = torch.randn(1, c, s, s, s, generator=gen, device=DEV).bfloat16()
    w1 = (torch.randn(h, c, 1, 1, 1, generator=gen, device=DEV) * c**-0.5).bfloat16()
    b1 = (torch.randn(h, generator=gen, device=DEV) * 0.1).bfloat16()
    w2 = (torch.randn(c, h, 1, 1, 1, generator=gen, device=DEV) * h**-0.5).bfloat16()
    b2 = (torch.randn(c, generator=gen, device=DEV) * 0.1).bfloat16()
    leaves = [t.clone().requires_grad_() for t in (x, w1, b1, w2, b2, res)]
    out = hip_ops.mlp_expansion_stored(*leaves)[0]
    ref_leaves = [t.float().requires_grad_() for t in (x, w1, b1, w2, b2, res)]
    xf, w1f, b1f, w2f, b2f, rf = ref_leaves
    ref = F.conv3d(F.gelu(F.conv3d(xf, w1f, b1f)), w2f, b2f) + rf
    assert max_rel(out, ref) <= BF16
    g = torch.randn_like(ref).bfloat16()
    got = torch.autograd.grad(out, leaves, g)
    want = torch.autograd.grad(ref, ref_leaves, g.float())
    for name, a, b in zip(["x", "w1", "b1", "w2", "b2", "res"], got, want):
        assert max_rel(a, b) <= BF16, name


# Ragged and odd shapes: K not a multiple of 32 (stem K = 1, head dgrad K = 3),
# M not a multiple of 16 (head M = 3), V not a multiple of 8 (the up blocks'
# (2s-1)^3 volumes), large K (stage 3-4 and the bottleneck), and single-
# workgroup launches whose waves loop over many chunks (odd chunk counts, so
# the next-chunk prefetch and the odd-KS buffer alternation both run).
ODD = [
    # (n, cin, cout, spatial, blocks)
    (1, 1, 32, (5, 7, 9), None),
    (1, 32, 3, (5, 7, 9), None),
    (2, 3, 32, (3, 3, 3), None),
    (1, 40, 24, (2, 3, 41), None),
    (1, 32, 64, (3, 5, 347), 1),  # KS = 1, MT = 4, 41 chunks over 4 waves
    (1, 64, 32, (3, 5, 347), 1),  # KS = 2
    (1, 96, 64, (7, 9, 83), 1),  # KS = 3
    (2, 128, 48, (2, 9, 131), 1),  # KS = 4, partial row group
    (1, 160, 32, (1, 11, 107), 1),  # KS = 5: runtime slice loop, odd count
    (1, 1024, 256, (4, 4, 4), None),  # split-K: the four waves share each chunk
    (1, 2048, 64, (3, 3, 3), None),  # K = 2048: 16-row groups
    (1, 288, 32, (3, 5, 43), 1),  # split-K, 9 slices over 4 waves, 6 chunks in one workgroup
    (2, 256, 48, (2, 3, 130), 1),  # split-K, partial row group, ragged V
]


@pytest.mark.parametrize("n,cin,cout,spatial,blocks", ODD)
@pytest.mark.parametrize("epilogue", ["bias", "bias_residual", "gelu_grad"])
def test_odd_shapes_forward_against_oracle(n, cin, cout, spatial, blocks, epilogue):
    print(f"[pw odd] n={n} cin={cin} cout={cout} spatial={spatial} blocks={blocks} epi={epilogue}", flush=True)
    gen = torch.Generator().manual_seed(cin * 13 + cout + 7 * spatial[-1])
    x = bf((n, cin, *spatial), gen)
    w = bf((cout, cin, 1, 1, 1), gen, cin**-0.5)
    b = bf((cout,), gen)
    aux = bf((n, cout, *spatial), gen, 1.5)
    code = {"bias": PW_EPILOGUE_BIAS, "bias_residual": PW_EPILOGUE_BIAS_RESIDUAL, "gelu_grad": PW_EPILOGUE_GELU_GRAD}
    pro = PW_PROLOGUE_GELU if epilogue == "bias_residual" else PW_PROLOGUE_NONE
    y = hip_ops.pointwise_conv(
        x.to(DEV), w.to(DEV), None if epilogue == "gelu_grad" else b.to(DEV),
        aux=None if epilogue == "bias" else aux.to(DEV), prologue=pro, epilogue=code[epilogue], blocks=blocks,
    )
    xin = opw.gelu(f64(x)) if pro == PW_PROLOGUE_GELU else f64(x)
    if epilogue == "gelu_grad":
        expect = opw.conv1x1(xin, f64(w)) * opw.gelu_grad(f64(aux))
    else:
        expect = opw.conv1x1(xin, f64(w), f64(b))
        if epilogue == "bias_residual":
            expect = expect + f64(aux)
    assert y.shape == (n, cout, *spatial)
    assert max_rel(y, expect) <= BF16


@pytest.mark.parametrize("n,cin,cout,spatial,blocks", ODD)
def test_odd_shapes_transposed_and_weight_grad(n, cin, cout, spatial, blocks):
    gen = torch.Generator().manual_seed(cin + 17 * cout)
    x = bf((n, cin, *spatial), gen)
    dy = bf((n, cout, *spatial), gen)
    w = bf((cout, cin, 1, 1, 1), gen, cin**-0.5)
    want_dx, want_dw, want_db = opw.conv1x1_backward(f64(dy), f64(x), f64(w))
    if cout <= 2048:
        dx = hip_ops.pointwise_conv(dy.to(DEV), w.to(DEV), transpose=True, blocks=blocks)
        assert max_rel(dx, want_dx) <= BF16
    splits = 1 if blocks == 1 else None
    dw, db = hip_ops.pointwise_weight_grad(dy.to(DEV), x.to(DEV), splits=splits)
    assert max_rel(dw, want_dw) <= BF16 and max_rel(db, want_db) <= BF16


def test_transposed_conv_op_matches_native_fp32():
    """The output-head route: 1x1x1 ConvTranspose3d (weight [Cin, Cout]) against
    PyTorch in fp32, forward and all three gradients, V = 9^3 (odd)."""
    gen = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(1, 32, 9, 9, 9, device=DEV, generator=gen).bfloat16().requires_grad_()
    w = (torch.randn(32, 3, 1, 1, 1, device=DEV, generator=gen) / 6).bfloat16().requires_grad_()
    b = torch.randn(3, device=DEV, generator=gen).bfloat16().requires_grad_()
    y = hip_ops.pointwise_conv_transpose3d(x, w, b)
    dy = torch.randn_like(y)
    y.backward(dy)
    xr, wr, br = (t.detach().float().requires_grad_() for t in (x, w, b))
    yr = F.conv_transpose3d(xr, wr, br)
    yr.backward(dy.float())
    assert max_rel(y, yr.detach().double().cpu().numpy()) <= BF16
    for got, want in ((x.grad, xr.grad), (w.grad, wr.grad), (b.grad, br.grad)):
        assert got.shape == want.shape
        assert max_rel(got, want.double().cpu().numpy()) <= BF16
    torch.library.opcheck(hip_ops.pointwise_conv_transpose3d, (x.detach().requires_grad_(), w, b))


def test_pointwise_argument_errors():
    x = torch.randn(1, 32, 2, 2, 8, device=DEV).bfloat16()
    w = torch.randn(64, 32, 1, 1, 1, device=DEV).bfloat16()
    with pytest.raises(ValueError):
        hip_ops.pointwise_conv(x.float(), w)  # dtype
    with pytest.raises(ValueError):
        hip_ops.pointwise_conv(x, torch.randn(64, 16, 1, 1, 1, device=DEV).bfloat16())  # channel mismatch
    with pytest.raises(ValueError):
        hip_ops.pointwise_conv(x.transpose(3, 4), w)  # non-contiguous
    with pytest.raises(hip_ops._hip.HipLibraryError):
        hip_ops.pointwise_conv(x, w, aux=None, epilogue=PW_EPILOGUE_BIAS_RESIDUAL)  # missing aux


@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("cin,cout,spatial", [(32, 64, (16, 16, 16)), (64, 32, (9, 10, 11)), (16, 8, (7, 8, 9))])
def test_stride2_residual_convs_match_native(transposed, cin, cout, spatial):
    """The down block's Conv3d(k=1, stride=2) and the up block's
    ConvTranspose3d(k=1, stride=2) residual convolutions through the wrapper
    (gather / scatter around the matrix-core GEMM) vs PyTorch's own convs under
    bf16 autocast: output and all gradients within the bf16 bound."""
    from mednext_accel_amd.adaptive import AdaptivePointwise3d, ModelOptimizationContext
    from mednext_accel_amd.optimization import PolicyRegistry

    torch.manual_seed(cin + cout)
    if transposed:
        ref = torch.nn.ConvTranspose3d(cin, cout, kernel_size=1, stride=2).to(DEV)
    else:
        ref = torch.nn.Conv3d(cin, cout, kernel_size=1, stride=2).to(DEV)
    cand = AdaptivePointwise3d(
        copy.deepcopy(ref), PolicyRegistry().resolver(), ModelOptimizationContext("mednext_v1", "base", "none")
    ).train()
    x = torch.randn(2, cin, *spatial, device=DEV, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    with torch.autocast(DEV, dtype=torch.bfloat16):
        want = ref(x)
        got = cand(y)
    assert got.shape == want.shape and got.dtype == want.dtype == torch.bfloat16
    assert max_rel(got, want) <= BF16
    g = torch.randn_like(want)
    wants = torch.autograd.grad(want, (x, ref.weight, ref.bias), g)
    gots = torch.autograd.grad(got, (y, cand.weight, cand.bias), g)
    for name, a, b in zip(("x", "weight", "bias"), gots, wants):
        assert max_rel(a, b) <= BF16, name
