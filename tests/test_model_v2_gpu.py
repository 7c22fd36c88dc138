"""MedNeXt v2 through the HIP path on the GPU: block and model parity against
the reference's plain PyTorch modules (and against float64 ground truth), and
one MedNeXt v2 Base training step.

Tolerances as for v1: rel-L2 1e-4 for whole fp32 models, bf16 autocast 2e-2
(each result within 2e-2 of the float64 truth, or no worse than twice the
reference path's own error).
"""

from __future__ import annotations

import copy
from dataclasses import replace

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

from helpers import BF16, check_against_truth
from mednext_accel_amd import MedNeXtV2, MedNeXtV2Block, get_mednext_v2_config, mednext_v2_base
from mednext_accel_amd.adaptive import ModelOptimizationContext, install_adaptive_operators
from mednext_accel_amd.grn import install_adaptive_grn, install_fused_grn_expansions
from mednext_accel_amd.mednext_v2 import configure_optimization
from mednext_accel_amd.optimization import PolicyRegistry
from mednext_accel_amd.step import make_training_step

pytestmark = pytest.mark.gpu
DEV = "cuda"
GRN_OP = "mednext_accel_amd::grn_forward"
GRN_BWD_OP = "mednext_accel_amd::grn_backward"
DW_OP = "mednext_accel_amd::depthwise_conv3d_odd_regular"
GN_OP = "mednext_accel_amd::group_norm_channels"
PW_OP = "mednext_accel_amd::pointwise_conv3d"
EXP_OP = "mednext_accel_amd::grn_expansion"
EXP_BWD_OP = "mednext_accel_amd::grn_expansion_backward"
MC = ModelOptimizationContext("mednext_v2", "base", "none")


class Observe(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops: list[str] = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.ops.append(func._schema.name)
        return func(*args, **(kwargs or {}))


def randomize_grn(model):
    """GRN parameters start at zero (GRN is then the identity); give them values."""
    gen = torch.Generator().manual_seed(77)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("grn.gamma") or name.endswith("grn.beta"):
                p.copy_(torch.randn(p.shape, generator=gen) * 0.5)


@pytest.mark.parametrize("channels,size,ratio,fused", [(32, 64, 3, False), (64, 32, 8, False), (32, 64, 3, True),
                                                       (64, 32, 4, True)])
def test_block_bf16_autocast_matches_reference_block(channels, size, ratio, fused):
    print(f"[v2 block] C={channels} S={size} R={ratio} fused={fused}", flush=True)
    torch.manual_seed(12)
    ref = MedNeXtV2Block(in_channels=channels, out_channels=channels, expansion_ratio=ratio).to(DEV).train()
    randomize_grn(ref)
    cand = copy.deepcopy(ref)
    truth = copy.deepcopy(ref).double()
    resolver = PolicyRegistry().resolver()
    assert install_adaptive_operators(cand, resolver=resolver, model_context=MC) == 4
    assert install_adaptive_grn(cand, resolver=resolver, model_context=MC) == 1
    if fused:
        assert install_fused_grn_expansions(cand, resolver=resolver, model_context=MC) == 1
    x = torch.randn(2, channels, size, size, size, device=DEV, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    z = x.detach().double().requires_grad_()
    with torch.autocast(DEV, dtype=torch.bfloat16):
        want = ref(x)
        with Observe() as seen:
            got = cand(y)
    assert DW_OP in seen.ops and GN_OP in seen.ops
    if fused:
        assert EXP_OP in seen.ops and GRN_OP not in seen.ops
    else:
        assert GRN_OP in seen.ops and PW_OP in seen.ops
    exact = truth(z)
    g = torch.randn_like(want)
    wants = torch.autograd.grad(want, (x, *ref.parameters()), g)
    with Observe() as seen_bwd:
        gots = torch.autograd.grad(got, (y, *cand.parameters()), g)
    assert (EXP_BWD_OP if fused else GRN_BWD_OP) in seen_bwd.ops
    exacts = torch.autograd.grad(exact, (z, *truth.parameters()), g.double())
    names = ["output", "x", *(n for n, _ in ref.named_parameters())]
    for name, a, b, t in zip(names, (got, *gots), (want, *wants), (exact, *exacts), strict=True):
        check_against_truth(name, a, b, t, BF16)


def small_config(deep_supervision=True):
    return replace(
        get_mednext_v2_config("base", in_channels=1, out_channels=3, deep_supervision=deep_supervision),
        base_channels=8,
        block_counts=(1,) * 9,
        expansion_ratios=(2,) * 9,
        downsample_expansion_ratios=(2,) * 4,
        upsample_expansion_ratios=(2,) * 4,
    )


def test_small_model_fp32_matches_reference_model():
    """fp32 (depthwise, GroupNorm on HIP; GRN stays on the formula in fp32, as
    the reference's fused GRN takes half inputs only) at an odd extent that
    exercises the right-edge reconcile path."""
    print("[v2 model fp32] C8 (33, 40, 47)", flush=True)
    torch.manual_seed(23)
    ref = MedNeXtV2(small_config())
    randomize_grn(ref)
    cand = configure_optimization(copy.deepcopy(ref), "auto")
    truth = copy.deepcopy(ref).double()
    ref, cand, truth = ref.to(DEV).train(), cand.to(DEV).train(), truth.to(DEV).train()
    x = torch.randn(1, 1, 33, 40, 47, device=DEV)
    with Observe() as seen:
        outs = cand(x)
    want, exact = ref(x), truth(x.double())
    assert DW_OP in seen.ops and GN_OP in seen.ops
    for i, (a, b, t) in enumerate(zip(outs, want, exact, strict=True)):
        check_against_truth(f"head {i}", a, b, t, 1e-4)
    for heads in (outs, want, exact):
        sum(o.square().mean() for o in heads).backward()
    for (name, p), q, t in zip(cand.named_parameters(), ref.parameters(), truth.parameters(), strict=True):
        check_against_truth(name, p.grad, q.grad, t.grad, 1e-4)


def test_small_model_bf16_autocast_matches_reference_model():
    print("[v2 model bf16] C8 48^3 batch 2", flush=True)
    torch.manual_seed(29)
    ref = MedNeXtV2(small_config())
    randomize_grn(ref)
    cand = configure_optimization(copy.deepcopy(ref), "auto")
    truth = copy.deepcopy(ref).double()
    ref, cand, truth = ref.to(DEV).train(), cand.to(DEV).train(), truth.to(DEV).train()
    x = torch.randn(2, 1, 48, 48, 48, device=DEV)
    with torch.autocast(DEV, dtype=torch.bfloat16):
        with Observe() as seen:
            outs = cand(x)
        want = ref(x)
    exact = truth(x.double())
    assert seen.ops.count(GRN_OP) + seen.ops.count(EXP_OP) == 17
    assert seen.ops.count(EXP_OP) > 0
    for i, (a, b, t) in enumerate(zip(outs, want, exact, strict=True)):
        check_against_truth(f"head {i}", a, b, t, BF16)
    for heads in (outs, want, exact):
        sum(o.float().square().mean() for o in heads).backward()
    for (name, p), q, t in zip(cand.named_parameters(), ref.parameters(), truth.parameters(), strict=True):
        check_against_truth(name, p.grad, q.grad, t.grad, BF16)


def test_v2_base_training_step_matches_reference():
    """One MedNeXt v2 Base bf16 AdamW step with deep supervision at 64^3
    through the HIP ops: same loss as the reference model within the bf16
    tolerance and matching per-parameter gradient norms."""
    print("[v2 model step] base 64^3 bf16", flush=True)
    torch.manual_seed(4321)
    ref = mednext_v2_base(in_channels=1, out_channels=3, deep_supervision=True, optimization="reference")
    randomize_grn(ref)
    cand = mednext_v2_base(in_channels=1, out_channels=3, deep_supervision=True)
    cand.load_state_dict(ref.state_dict())
    ref, cand = ref.to(DEV).train(), cand.to(DEV).train()
    losses, norms = [], []
    for model in (cand, ref):
        step = make_training_step(model, size=64, device=DEV)
        with Observe() as seen:
            loss = step()
        losses.append(float(loss.detach()))
        norms.append(torch.stack([p.grad.float().norm() for p in model.parameters()]))
        if model is cand:
            assert EXP_OP in seen.ops and EXP_BWD_OP in seen.ops and DW_OP in seen.ops and PW_OP in seen.ops
        del step
    print(f"  loss hip {losses[0]:.6f} reference {losses[1]:.6f}", flush=True)
    assert abs(losses[0] - losses[1]) / abs(losses[1]) < BF16
    assert torch.isfinite(norms[0]).all()
    assert float((norms[0] - norms[1]).norm() / norms[1].norm()) < 5e-2
    torch.cuda.empty_cache()
