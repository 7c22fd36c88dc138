"""The up-block join (hip_ops.up_block_join): pad(main) + pad(residual) of a
MedNeXt up block in one pass, against the same pad-and-add in PyTorch on the
same bf16 operands (reference models/blocks.py:179-181 with the pad at the
start, models/blocks_v2.py:131-133 at the end), forward and backward, and its
use inside the models."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch.utils._python_dispatch import TorchDispatchMode

from helpers import rel_l2
from mednext_accel_amd import hip_ops as P
from mednext_accel_amd import mednext_base, mednext_v2_base

pytestmark = pytest.mark.gpu
DEV = "cuda"


def residual_grid(small, bias, full):
    """The transposed stride-2 1x1x1 conv's output from its GEMM values: small
    at the even points of the (2s - 1)^3 grid, the bias elsewhere."""
    n, c = small.shape[:2]
    res = (bias if bias is not None else small.new_zeros(c)).view(1, c, 1, 1, 1).expand(n, c, *full).clone()
    res[:, :, ::2, ::2, ::2] = small
    return res


@pytest.mark.parametrize("lead", [0, 1])
@pytest.mark.parametrize("n,c,s,with_bias", [(1, 32, (8, 8, 8), True), (2, 3, (4, 6, 8), False),
                                             (1, 5, (3, 2, 4), True)])
@pytest.mark.parametrize("bias_in_small", [False, True])
def test_join_is_pad_and_add(lead, n, c, s, with_bias, bias_in_small):
    if bias_in_small and not with_bias:
        pytest.skip("the flag only changes the bias gradient")
    print(f"[up join] lead={lead} n={n} c={c} s={s} bias={with_bias} bias_in_small={bias_in_small}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(sum(s) + c + lead)
    full = tuple(2 * v - 1 for v in s)
    main = torch.randn(n, c, *full, generator=g, device=DEV).bfloat16().requires_grad_()
    small = torch.randn(n, c, *s, generator=g, device=DEV).bfloat16().requires_grad_()
    bias = torch.randn(c, generator=g, device=DEV).bfloat16().requires_grad_() if with_bias else None
    out = P.up_block_join(main, small, bias, lead, bias_in_small)
    pad = (1, 0) * 3 if lead else (0, 1) * 3
    ref = F.pad(main, pad) + F.pad(residual_grid(small, bias, full), pad)
    assert out.shape == ref.shape and torch.equal(out, ref)
    dout = torch.randn(out.shape, generator=g, device=DEV).bfloat16()
    inputs = (main, small) + ((bias,) if with_bias else ())
    got = torch.autograd.grad(out, inputs, dout)
    want = torch.autograd.grad(ref, inputs, dout)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    if with_bias:
        grid = dout[:, :, lead:lead + full[0], lead:lead + full[1], lead:lead + full[2]].double()
        whole = grid.sum(dim=(0, 2, 3, 4))
        odd = whole - grid[:, :, ::2, ::2, ::2].sum(dim=(0, 2, 3, 4))
        assert rel_l2(got[2].double(), whole if bias_in_small else odd) <= 1e-2


def bf16_ulps(a, b):
    """Distance in bf16 steps between two bf16 tensors of the same sign pattern."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


@pytest.mark.parametrize("lead", [0, 1])
def test_residual_bias_gradient_is_one_rounding(lead):
    """The up block's residual bias through the join (GEMM with the bias's
    value, join with bias_in_small): its gradient is the whole-grid sum of
    grad_out rounded once to bf16, within one bf16 step of the fp64 sum and
    within bf16 tolerance of the fp32 conv_transpose3d + pad + add reference
    (reference models/blocks.py:176-181)."""
    print(f"[up join bias] lead={lead}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7 + lead)
    n, cin, cout, s = 1, 16, 8, (8, 8, 8)
    full = tuple(2 * v - 1 for v in s)
    x = torch.randn(n, cin, *s, generator=g, device=DEV)
    w = torch.randn(cin, cout, 1, 1, 1, generator=g, device=DEV) * cin**-0.5
    b = torch.randn(cout, generator=g, device=DEV).requires_grad_()
    main = torch.randn(n, cout, *full, generator=g, device=DEV)
    bb = b.bfloat16()
    small = P.pointwise_conv_transpose3d(x.bfloat16(), w.bfloat16(), bb.detach())
    out = P.up_block_join(main.bfloat16(), small, bb, lead, True)
    dout = torch.randn(out.shape, generator=g, device=DEV).bfloat16()
    (gb,) = torch.autograd.grad(out, (b,), dout)
    grid = dout[:, :, lead:lead + full[0], lead:lead + full[1], lead:lead + full[2]].double()
    exact = grid.sum(dim=(0, 2, 3, 4))
    assert int(bf16_ulps(gb.bfloat16(), exact.float().bfloat16()).max()) <= 1
    b32 = b.detach().clone().requires_grad_()
    pad = (1, 0) * 3 if lead else (0, 1) * 3
    res = F.conv_transpose3d(x, w, b32, stride=2)
    ref = F.pad(main, pad) + F.pad(res, pad)
    (gb32,) = torch.autograd.grad(ref, (b32,), dout.float())
    assert rel_l2(gb.double(), gb32.double()) <= 8e-3


class Observe(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops: list[str] = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.ops.append(func._schema.name)
        return func(*args, **(kwargs or {}))


@pytest.mark.parametrize("family", ["v1", "v2"])
def test_models_join_their_up_blocks(family):
    torch.manual_seed(2)
    build = mednext_base if family == "v1" else mednext_v2_base
    model = build(in_channels=1, out_channels=3, deep_supervision=True).to(DEV).train()
    x = torch.randn(1, 1, 64, 64, 64, device=DEV)
    with torch.autocast(DEV, dtype=torch.bfloat16), Observe() as seen:
        outs = model(x)
    assert seen.ops.count("mednext_accel_amd::up_block_join") >= 2
    sum(o.float().square().mean() for o in outs).backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in model.parameters())
