"""Fused MedNeXt v2 block expansion on the GPU: ``out = W2 . GRN(GELU(W1 . x +
b1)) + b2 (+ residual)`` with GELU and GRN folded into the matrix-core GEMMs
(hip_ops.grn_expansion), and each GEMM mode it uses on its own.

Ground truth is the same chain in float64 on the same bf16 inputs (reference
models/blocks_v2.py:44-45 with ops/grn.py:16-30). The bar is the bf16
autocast one: every output and gradient within 2e-2 (rel-L2) of the truth, or
no worse than twice the error of the reference's own unfused bf16 path
(PyTorch convs, GELU and the GRN formula under autocast).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from helpers import BF16, check_against_truth, max_rel, rel_l2
from mednext_accel_amd import global_response_norm3d_reference
from mednext_accel_amd import hip_ops as P

pytestmark = pytest.mark.gpu
DEV = "cuda"


def chain(x, w1, b1, w2, b2, gamma, beta, residual, eps=1e-6):
    u = F.conv3d(x, w1, b1)
    z = global_response_norm3d_reference(F.gelu(u), gamma, beta, eps)
    out = F.conv3d(z, w2, b2)
    return out if residual is None else out + residual


def make(n, c, hidden, cout, spatial, seed, residual=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, c, *spatial, generator=g)
    w1 = torch.randn(hidden, c, 1, 1, 1, generator=g) / c**0.5
    b1 = torch.randn(hidden, generator=g) * 0.1
    w2 = torch.randn(cout, hidden, 1, 1, 1, generator=g) / hidden**0.5
    b2 = torch.randn(cout, generator=g) * 0.1
    gamma = torch.randn(1, hidden, 1, 1, 1, generator=g)
    beta = torch.randn(1, hidden, 1, 1, 1, generator=g) * 0.5
    res = torch.randn(n, cout, *spatial, generator=g) if residual else None
    bf = [t.to(DEV, torch.bfloat16) for t in (x, w1, b1, w2, b2)]
    gb = [t.to(DEV) for t in (gamma, beta)]
    return bf, gb, (res.to(DEV, torch.bfloat16) if residual else None)


CASES = [
    (2, 32, 96, 32, (24, 24, 24), True),    # v2 stage 0: K = 96 project
    (1, 64, 256, 64, (16, 16, 16), True),   # v2 stage 1: split-K project
    (2, 8, 40, 12, (7, 9, 11), False),      # odd widths and volume, no residual
    (1, 32, 128, 64, (12, 12, 12), False),  # down-block shape: Cout = 2 C
    (1, 128, 1024, 128, (16, 16, 16), True),  # v2 stage 2: split-K project, K = 128 backward GEMMs
]


@pytest.mark.parametrize("n,c,hidden,cout,spatial,residual", CASES)
def test_fused_expansion_matches_float64_chain(n, c, hidden, cout, spatial, residual):
    print(f"[grn expansion] n={n} c={c} hidden={hidden} cout={cout} spatial={spatial} residual={residual}", flush=True)
    (x, w1, b1, w2, b2), (gamma, beta), res = make(n, c, hidden, cout, spatial, hidden + cout, residual)
    leaves = [t.clone().requires_grad_() for t in (x, w1, b1, w2, b2, gamma, beta)] + (
        [res.clone().requires_grad_()] if residual else [])
    hip_in = leaves
    out, a, dgelu, coef = P.grn_expansion(*hip_in[:7], hip_in[7] if residual else None, 1e-6)
    assert out.dtype == a.dtype == dgelu.dtype == torch.bfloat16 and coef.dtype == torch.float64
    # reference path: the unfused chain under bf16 autocast (fp32 GRN parameters)
    ref_in = [t.detach().float().clone().requires_grad_() if i in (5, 6) else t.detach().clone().requires_grad_()
              for i, t in enumerate(leaves)]
    with torch.autocast(DEV, dtype=torch.bfloat16):
        ref_out = chain(*ref_in[:7], ref_in[7] if residual else None)
    truth_in = [t.detach().double().clone().requires_grad_() for t in leaves]
    truth = chain(*truth_in[:7], truth_in[7] if residual else None)
    check_against_truth("output", out, ref_out, truth, BF16)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(DEV)
    got = torch.autograd.grad(out, hip_in, g.bfloat16())
    want = torch.autograd.grad(ref_out, ref_in, g.bfloat16())
    exact = torch.autograd.grad(truth, truth_in, g.double())
    names = ["x", "w1", "b1", "w2", "b2", "gamma", "beta", "residual"]
    for name, a, b, t in zip(names, got, want, exact):
        assert a.dtype == hip_in[names.index(name)].dtype, name
        check_against_truth(name, a, b, t, BF16)


def test_fused_expansion_is_bit_reproducible():
    (x, w1, b1, w2, b2), (gamma, beta), res = make(1, 32, 96, 32, (20, 20, 20), 3)
    runs = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_() for t in (x, w1, b1, w2, b2, gamma, beta)]
        out, _, _, _ = P.grn_expansion(*leaves, res, 1e-6)
        grads = torch.autograd.grad(out, leaves, torch.ones_like(out))
        runs.append((out, *grads))
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_row_reduce_epilogue_matches_torch():
    torch.manual_seed(11)
    n, k, m, s = 2, 32, 96, 20
    dy = torch.randn(n, k, s, s, s, device=DEV).bfloat16()
    a = torch.randn(n, m, s, s, s, device=DEV).bfloat16()
    w = (torch.randn(k, m, 1, 1, 1, device=DEV) / m**0.5).bfloat16()  # conv weight [Cout=k][Cin=m]
    v = s**3
    slots = P.pointwise_row_slots(n, k, m, v, 0)
    rows = torch.empty(n, m, slots, 2, device=DEV, dtype=torch.float64)
    assert P.pointwise_conv(dy, w, aux=a, epilogue=P.PW_EPILOGUE_ROW_REDUCE, transpose=True, row_partial=rows) is None
    dz = torch.einsum("km,nkv->nmv", w.double().view(k, m), dy.double().view(n, k, v))
    sums = rows.sum(dim=2)
    assert max_rel(sums[..., 0], (dz * a.double().view(n, m, v)).sum(-1)) <= 1e-5
    assert max_rel(sums[..., 1], dz.sum(-1)) <= 1e-5


@pytest.mark.parametrize("k,m,s", [(64, 256, 12), (32, 96, 9), (96, 192, 8), (128, 64, 8), (320, 40, 6)])
def test_affine_scale_epilogue_matches_torch(k, m, s):
    torch.manual_seed(12)
    n = 2
    dy = torch.randn(n, k, s, s, s, device=DEV).bfloat16()
    a = torch.randn(n, m, s, s, s, device=DEV).bfloat16()
    d = torch.rand(n, m, s, s, s, device=DEV).bfloat16()
    w = (torch.randn(k, m, 1, 1, 1, device=DEV) / m**0.5).bfloat16()
    c = torch.randn(n, m, 2, device=DEV, dtype=torch.float64)
    du = P.pointwise_conv(dy, w, aux=a, aux2=d, epilogue=P.PW_EPILOGUE_AFFINE_SCALE, transpose=True,
                          epilogue_coef=c)
    v = s**3
    dz = torch.einsum("km,nkv->nmv", w.double().view(k, m), dy.double().view(n, k, v))
    want = (dz * c[..., :1] + a.double().view(n, m, v) * c[..., 1:]) * d.double().view(n, m, v)
    assert rel_l2(du.view(n, m, v), want) <= 8e-3


@pytest.mark.parametrize("k,m,s", [(32, 96, 20), (64, 256, 10), (8, 40, 7)])
def test_bias_gelu_pair_epilogue_matches_torch(k, m, s):
    torch.manual_seed(15)
    n = 2
    x = torch.randn(n, k, s, s, s, device=DEV).bfloat16()
    w = (torch.randn(m, k, 1, 1, 1, device=DEV) / k**0.5).bfloat16()
    b = (torch.randn(m, device=DEV) * 0.3).bfloat16()
    g, dg = P.pointwise_conv(x, w, b, epilogue=P.PW_EPILOGUE_BIAS_GELU_PAIR)
    u = (F.conv3d(x.double(), w.double(), b.double())).requires_grad_()
    want = F.gelu(u)
    (want_d,) = torch.autograd.grad(want.sum(), u)
    assert rel_l2(g, want) <= 8e-3
    assert rel_l2(dg, want_d) <= 8e-3


def test_affine_prologue_forward_and_weight_grad():
    torch.manual_seed(13)
    n, k, m, s = 2, 96, 32, 16
    a = torch.randn(n, k, s, s, s, device=DEV).bfloat16()
    w = (torch.randn(m, k, 1, 1, 1, device=DEV) / k**0.5).bfloat16()
    b = (torch.randn(m, device=DEV) * 0.1).bfloat16()
    coef = torch.randn(n, k, 4, device=DEV, dtype=torch.float64)
    coef[..., 0] = 1 + 0.3 * coef[..., 0]
    y = P.pointwise_conv(a, w, b, prologue=P.PW_PROLOGUE_AFFINE, prologue_coef=coef)
    v = s**3
    z = a.double().view(n, k, v) * coef[..., :1] + coef[..., 1:2]
    want = torch.einsum("mk,nkv->nmv", w.double().view(m, k), z) + b.double()[None, :, None]
    assert rel_l2(y.view(n, m, v), want) <= 8e-3
    dy = torch.randn(n, m, s, s, s, device=DEV).bfloat16()
    dw, db = P.pointwise_weight_grad(dy, a, prologue=P.PW_PROLOGUE_AFFINE, prologue_coef=coef)
    cf = coef.float().double()  # the records as the kernels take them
    zx = a.double().view(n, k, v) * cf[..., :1] + cf[..., 1:2]  # exact: the library maps the raw product's sums
    want_dw = torch.einsum("nmv,nkv->mk", dy.double().view(n, m, v), zx)
    assert rel_l2(dw.view(m, k), want_dw) <= 8e-3
    assert rel_l2(db, dy.double().sum(dim=(0, 2, 3, 4))) <= 8e-3


def test_grn_stats_match_torch():
    torch.manual_seed(14)
    x = torch.randn(2, 48, 10, 11, 12, device=DEV).bfloat16()
    gamma = torch.randn(48, device=DEV)
    beta = torch.randn(48, device=DEV)
    coef = P.grn_stats(x, gamma, beta, 1e-6)
    norms = x.double().flatten(2).norm(dim=2)
    r = norms / (norms.sum(dim=1, keepdim=True) + 1e-6)
    assert max_rel(coef[..., 3], norms) <= 1e-6
    assert max_rel(coef[..., 2], r) <= 1e-6
    assert max_rel(coef[..., 0], 1 + gamma.double() * r) <= 1e-6
    assert max_rel(coef[..., 1], beta.double().expand(2, 48)) == 0


def test_opcheck_grn_expansion():
    (x, w1, b1, w2, b2), (gamma, beta), res = make(1, 8, 40, 8, (5, 6, 7), 21)
    args = [t.clone().requires_grad_() for t in (x, w1, b1, w2, b2, gamma, beta)]
    result = torch.library.opcheck(P.grn_expansion, (*args, res, 1e-6), raise_exception=False)
    assert all(v == "SUCCESS" for v in result.values()), result
