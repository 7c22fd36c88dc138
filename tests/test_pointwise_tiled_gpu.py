"""The LDS-tiled pointwise product against float64 ground truth, mode by mode,
next to the streaming kernels on the same inputs.

Every case runs twice: with the streaming kernels only and with the tiled
kernel forced wherever it applies (``set_pointwise_kernels``). Shapes cover
64- and 128-row workgroups, workgroups whose last waves have no live rows
(M = 48, 80), several row groups (M = 272), odd
slice counts (K = 32, 96), both weight layouts, and ragged volumes (V % 128
and V % 8 non-zero). The bar is the one of the other GEMM-mode tests:
rel-L2 <= 8e-3 against the same chain in float64 on the bf16 inputs.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from helpers import rel_l2
from mednext_accel_amd import hip_ops as P

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 8e-3


@pytest.fixture(autouse=True)
def _restore_choice():
    yield
    P.set_pointwise_kernels(P.PW_KERNELS_AUTO)


def run_both(fn):
    """fn() with the streaming kernels, the tiled kernel (64- or 128-row
    workgroups by the library's choice) and the tiled kernel at 64 rows."""
    outs = []
    for choice in (P.PW_KERNELS_STREAMING, P.PW_KERNELS_TILED, P.PW_KERNELS_TILED_64):
        P.set_pointwise_kernels(choice)
        outs.append(fn())
    P.set_pointwise_kernels(P.PW_KERNELS_AUTO)
    return outs


def product(w2, x, transpose):
    """float64 W . x (W^T . x) per sample over flattened voxels."""
    a = w2.t() if transpose else w2
    return torch.matmul(a, x.flatten(2))


# (n, k, m, spatial): K input rows of the product, M output rows. Grids of
# fewer than 256 128-row workgroups run 64-row ones (the first four shapes);
# the last two are large enough for 128-row workgroups.
SHAPES = [
    (2, 256, 128, (8, 8, 9)),     # two slices per step, V = 576 (partial chunk)
    (1, 96, 80, (3, 5, 7)),       # odd slice count, M = 80, V % 8 != 0
    (2, 32, 48, (4, 6, 11)),      # one slice, M = 48 (one wave idle)
    (1, 512, 272, (2, 4, 16)),    # five 64-row groups, the last one 16 rows
    (1, 96, 80, (15, 33, 67)),    # 128-row workgroups: M = 80 (waves 2-3 partly idle), V % 8 != 0
    (1, 512, 272, (16, 32, 64)),  # 128-row workgroups, three row groups, the last one 16 rows
]


@pytest.mark.parametrize("n,k,m,spatial", SHAPES)
@pytest.mark.parametrize("mode", ["bias", "none", "bias_gelu", "bias_residual", "pair"])
def test_forward_modes(n, k, m, spatial, mode):
    print(f"[pw tiled fwd] n={n} k={k} m={m} spatial={spatial} mode={mode}", flush=True)
    g = torch.Generator().manual_seed(k + m + len(mode))
    x = torch.randn(n, k, *spatial, generator=g).bfloat16()
    w = (torch.randn(m, k, 1, 1, 1, generator=g) / k**0.5).bfloat16()
    b = (torch.randn(m, generator=g) * 0.3).bfloat16()
    r = torch.randn(n, m, *spatial, generator=g).bfloat16()
    epi = {"bias": P.PW_EPILOGUE_BIAS, "none": P.PW_EPILOGUE_BIAS, "bias_gelu": P.PW_EPILOGUE_BIAS_GELU,
           "bias_residual": P.PW_EPILOGUE_BIAS_RESIDUAL, "pair": P.PW_EPILOGUE_BIAS_GELU_PAIR}[mode]
    v = x[0, 0].numel()
    P.set_pointwise_kernels(P.PW_KERNELS_TILED)
    assert P.pointwise_uses_tiled(n, k, m, v, P.PW_PROLOGUE_NONE, epi)
    xd, wd, bd, rd = (t.to(DEV) for t in (x, w, b, r))
    outs = run_both(lambda: P.pointwise_conv(
        xd, wd, None if mode == "none" else bd, aux=rd if mode == "bias_residual" else None, epilogue=epi))
    u = product(w.double().view(m, k), x.double(), False)
    if mode != "none":
        u = u + b.double()[None, :, None]
    if mode == "bias_residual":
        u = u + r.double().flatten(2)
    for out in outs:
        if mode == "pair":
            ud = u.clone().requires_grad_()
            gelu = F.gelu(ud)
            (dgelu,) = torch.autograd.grad(gelu.sum(), ud)
            assert rel_l2(out[0].cpu().flatten(2), gelu.detach()) <= TOL
            assert rel_l2(out[1].cpu().flatten(2), dgelu) <= TOL
        else:
            want = F.gelu(u) if mode == "bias_gelu" else u
            assert out.shape == (n, m, *spatial)
            assert rel_l2(out.cpu().flatten(2), want) <= TOL


@pytest.mark.parametrize("n,k,m,spatial", SHAPES)
@pytest.mark.parametrize("mode", ["plain", "gelu_grad", "aux_scale", "affine_scale"])
def test_transposed_modes(n, k, m, spatial, mode):
    """Input-gradient products: the weight arrives as the conv's [K][M]
    (weight_layout 1, transposed through registers on its way to LDS)."""
    print(f"[pw tiled bwd] n={n} k={k} m={m} spatial={spatial} mode={mode}", flush=True)
    g = torch.Generator().manual_seed(3 * k + m + len(mode))
    dy = torch.randn(n, k, *spatial, generator=g).bfloat16()
    w = (torch.randn(k, m, 1, 1, 1, generator=g) / m**0.5).bfloat16()  # conv weight [Cout = k][Cin = m]
    a = torch.randn(n, m, *spatial, generator=g).bfloat16()
    d = torch.rand(n, m, *spatial, generator=g).bfloat16()
    c = torch.randn(n, m, 2, generator=g, dtype=torch.float64)
    epi = {"plain": P.PW_EPILOGUE_BIAS, "gelu_grad": P.PW_EPILOGUE_GELU_GRAD, "aux_scale": P.PW_EPILOGUE_AUX_SCALE,
           "affine_scale": P.PW_EPILOGUE_AFFINE_SCALE}[mode]
    dyd, wd, ad, dd, cd = (t.to(DEV) for t in (dy, w, a, d, c))
    kw = {}
    if mode != "plain":
        kw["aux"] = ad
    if mode == "affine_scale":
        kw.update(aux2=dd, epilogue_coef=cd)
    outs = run_both(lambda: P.pointwise_conv(dyd, wd, epilogue=epi, transpose=True, **kw))
    dz = product(w.double().view(k, m), dy.double(), True)
    af = a.double().flatten(2)
    if mode == "gelu_grad":
        ar = af.clone().requires_grad_()
        (gd,) = torch.autograd.grad(F.gelu(ar).sum(), ar)
        want = dz * gd
    elif mode == "aux_scale":
        want = dz * af
    elif mode == "affine_scale":
        want = (dz * c[..., :1] + af * c[..., 1:]) * d.double().flatten(2)
    else:
        want = dz
    for out in outs:
        assert out.shape == (n, m, *spatial)
        assert rel_l2(out.cpu().flatten(2), want) <= TOL


@pytest.mark.parametrize("n,k,m,spatial", [(2, 96, 32, (5, 6, 7)), (1, 1024, 128, (4, 8, 8)), (2, 256, 80, (8, 8, 9)),
                                            (1, 1024, 128, (16, 32, 64))])
@pytest.mark.parametrize("residual", [False, True])
def test_affine_prologue(n, k, m, spatial, residual):
    """The GRN-consuming project GEMM: W . (x s + t) + b (+ residual). The
    tiled kernel rounds x s + t to bf16 per element, the streaming kernels
    fold s into the weight; both against the exact float64 chain."""
    print(f"[pw tiled affine] n={n} k={k} m={m} spatial={spatial} residual={residual}", flush=True)
    g = torch.Generator().manual_seed(k + m + residual)
    x = torch.randn(n, k, *spatial, generator=g).bfloat16()
    w = (torch.randn(m, k, 1, 1, 1, generator=g) / k**0.5).bfloat16()
    b = (torch.randn(m, generator=g) * 0.1).bfloat16()
    r = torch.randn(n, m, *spatial, generator=g).bfloat16()
    coef = torch.randn(n, k, 4, generator=g, dtype=torch.float64)
    coef[..., 0] = 1 + 0.3 * coef[..., 0]
    epi = P.PW_EPILOGUE_BIAS_RESIDUAL if residual else P.PW_EPILOGUE_BIAS
    xd, wd, bd, rd, cd = (t.to(DEV) for t in (x, w, b, r, coef))
    outs = run_both(lambda: P.pointwise_conv(xd, wd, bd, aux=rd if residual else None, prologue=P.PW_PROLOGUE_AFFINE,
                                             epilogue=epi, prologue_coef=cd))
    z = x.double().flatten(2) * coef[..., :1] + coef[..., 1:2]
    want = torch.matmul(w.double().view(m, k), z) + b.double()[None, :, None]
    if residual:
        want = want + r.double().flatten(2)
    for out in outs:
        assert rel_l2(out.cpu().flatten(2), want) <= TOL


def test_tiled_is_deterministic_and_matches_streaming_closely():
    """Same inputs, same bits on a second launch; streaming and tiled agree to
    bf16 rounding (both accumulate in fp32, in different K orders)."""
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(2, 1024, 16, 16, 16, generator=g, device=DEV).bfloat16()
    w = (torch.randn(128, 1024, 1, 1, 1, generator=g, device=DEV) / 32).bfloat16()
    b = torch.randn(128, generator=g, device=DEV).bfloat16()
    P.set_pointwise_kernels(P.PW_KERNELS_TILED)
    y1 = P.pointwise_conv(x, w, b)
    y2 = P.pointwise_conv(x, w, b)
    assert torch.equal(y1, y2)
    P.set_pointwise_kernels(P.PW_KERNELS_STREAMING)
    ys = P.pointwise_conv(x, w, b)
    assert rel_l2(y1.float(), ys.float()) <= 4e-3


@pytest.mark.parametrize("n,k,m,spatial", [(1, 128, 128, (8, 8, 16)), (2, 160, 272, (5, 7, 9)), (1, 64, 96, (4, 4, 33)),
                                            (2, 256, 1024, (4, 8, 8))])
@pytest.mark.parametrize("prologue", ["none", "gelu", "affine"])
def test_weight_grad_tiles(n, k, m, spatial, prologue):
    """dW = dY . prologue(X)^T and dB = sum dY with 64 x 64 workgroup tiles
    (streaming) and 128 x 128 ones (tiled): ragged sides (M = 96, 272; K = 64,
    160), V % 8 != 0, several splits and samples."""
    print(f"[pw wgrad tiles] n={n} k={k} m={m} spatial={spatial} prologue={prologue}", flush=True)
    g = torch.Generator().manual_seed(5 * k + m + len(prologue))
    x = torch.randn(n, k, *spatial, generator=g).bfloat16()
    dy = torch.randn(n, m, *spatial, generator=g).bfloat16()
    coef = torch.randn(n, k, 4, generator=g, dtype=torch.float64)
    coef[..., 0] = 1 + 0.3 * coef[..., 0]
    pro = {"none": P.PW_PROLOGUE_NONE, "gelu": P.PW_PROLOGUE_GELU, "affine": P.PW_PROLOGUE_AFFINE}[prologue]
    xd, dyd, cd = x.to(DEV), dy.to(DEV), coef.to(DEV)
    outs = run_both(lambda: P.pointwise_weight_grad(dyd, xd, prologue=pro,
                                                    prologue_coef=cd if prologue == "affine" else None))
    xf = x.double().flatten(2)
    if prologue == "gelu":
        xf = F.gelu(xf)
    elif prologue == "affine":
        cf = coef.float().double()  # records as floats; the map of the raw product's sums is exact
        xf = xf * cf[..., :1] + cf[..., 1:2]
    dyf = dy.double().flatten(2)
    want_dw = torch.einsum("nmv,nkv->mk", dyf, xf)
    want_db = dyf.sum(dim=(0, 2))
    for dw, db in outs:
        assert dw.shape == (m, k, 1, 1, 1)
        assert rel_l2(dw.cpu().view(m, k), want_dw) <= TOL
        assert rel_l2(db.cpu(), want_db) <= TOL
