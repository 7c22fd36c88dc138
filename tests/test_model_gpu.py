"""Wrapper / model path on the GPU: per-phase routing through the HIP ops,
GroupNorm autocast semantics, block and model parity against the reference's
plain PyTorch modules, one MedNeXt-Base 128^3 training step, torch.compile and
opcheck (mirrors the reference's tests/ops/test_phase_routing.py and
tests/ops/test_depthwise.py).

Tolerances: fp32 normwise 1e-5 on outputs / input grads and 1e-4 on weight
grads for single ops, rel-L2 1e-4 for whole fp32 models (accumulated over
~60 layers, as the reference's phase-routing test uses), bf16 autocast 2e-2.
"""

from __future__ import annotations

import copy

import pytest
import torch
from torch import nn
from torch.utils._python_dispatch import TorchDispatchMode

from helpers import BF16, FP32_OUT, FP32_WGRAD, check_against_truth, max_rel, rel_l2
from mednext_accel_amd import CheckpointConfig, MedNeXtBlock, mednext_base, mednext_small
from mednext_accel_amd.adaptive import (
    AdaptiveDepthwise3d,
    AdaptiveExpansion,
    AdaptiveGroupNorm3d,
    ModelOptimizationContext,
    install_adaptive_operators,
)
from mednext_accel_amd.optimization import PolicyRegistry, PolicyResolver, parse_policy
from mednext_accel_amd.step import make_training_step

pytestmark = pytest.mark.gpu
DEV = "cuda"
MC = ModelOptimizationContext("mednext_v1", "base", "none")
DW_OP = "mednext_accel_amd::depthwise_conv3d_odd_regular"
DX_OP = "mednext_accel_amd::depthwise_input_grad_odd_regular"
DWG_OP = "mednext_accel_amd::depthwise_weight_grad_odd_regular"
GN_OP = "mednext_accel_amd::group_norm_channels"
GN_MLP_OP = "mednext_accel_amd::gn_mlp_expansion"  # GroupNorm folded into the expand GEMM
MLP_OP = "mednext_accel_amd::mlp_expansion"
MLP_STORED_OP = "mednext_accel_amd::mlp_expansion_stored"


class Observe(TorchDispatchMode):
    def __init__(self):
        super().__init__()
        self.ops: list[str] = []
        self.masks: list[tuple[bool, ...]] = []

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        name = func._schema.name
        self.ops.append(name)
        if name == "aten::convolution_backward":
            self.masks.append(tuple(args[-1]))
        return func(*args, **(kwargs or {}))


def phase_policy(fwd: bool, dx: bool, dw: bool):
    def sel(on, impl):
        return {"implementation": impl, "parameters": "auto"} if on else {"implementation": "reference"}

    return parse_policy(
        {
            "version": 2, "kind": "mednext-accel-policy", "name": "phases", "target": {"vendor": "amd"},
            "rules": [{"id": "dw", "when": {"family": "depthwise_conv3d", "direction": "regular"},
                       "use": {"forward": sel(fwd, "hip_depthwise_fwd"), "backward_input": sel(dx, "hip_depthwise_dx"),
                               "backward_weight": sel(dw, "hip_split_dw")},
                       "confidence": "measured-exact-context"}],
        }
    )


@pytest.mark.parametrize("fwd,dx,dw", [(1, 1, 1), (0, 1, 0), (0, 0, 1), (1, 0, 0), (0, 0, 0)])
@pytest.mark.parametrize("autocast", [False, True])
def test_depthwise_phases_route_independently(fwd, dx, dw, autocast):
    print(f"[routing] fwd={fwd} dx={dx} dw={dw} autocast={autocast}", flush=True)
    torch.manual_seed(19)
    ref = nn.Conv3d(4, 4, 3, padding=1, groups=4, device=DEV)
    cand = AdaptiveDepthwise3d(copy.deepcopy(ref), PolicyResolver(external=phase_policy(fwd, dx, dw)), MC)
    x = torch.randn(2, 4, 8, 40, 40, device=DEV, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    with torch.autocast(DEV, dtype=torch.bfloat16, enabled=autocast):
        want = ref(x)
        with Observe() as seen_fwd:
            got = cand(y)
    custom = bool(fwd or dx or dw)
    assert (DW_OP in seen_fwd.ops) == custom
    g = torch.randn_like(want)
    wants = torch.autograd.grad(want, (x, *ref.parameters()), g)
    with Observe() as seen_bwd:
        gots = torch.autograd.grad(got, (y, *cand.parameters()), g)
    if custom:
        assert (DX_OP in seen_bwd.ops) == bool(dx)
        assert (DWG_OP in seen_bwd.ops) == bool(dw)
        native = (not dx, not dw, not dw)  # dB rides with the HIP dW pass
        assert seen_bwd.masks == ([native] if any(native) else [])
    assert got.dtype == want.dtype
    out_tol, w_tol = (BF16, BF16) if autocast else (FP32_OUT, FP32_WGRAD)
    assert max_rel(got, want) <= out_tol
    assert max_rel(gots[0], wants[0]) <= out_tol
    for a, b in zip(gots[1:], wants[1:], strict=True):
        assert a.dtype == torch.float32
        assert max_rel(a, b) <= w_tol


@pytest.mark.parametrize("guard", ["noncontiguous", "unbatched", "no-grad", "eval"])
def test_tensor_guards_keep_the_native_route(guard):
    cand = AdaptiveDepthwise3d(nn.Conv3d(2, 2, 3, padding=1, groups=2, device=DEV), PolicyRegistry().resolver(), MC)
    x = torch.randn(1, 2, 5, 6, 7, device=DEV, requires_grad=True)
    if guard == "noncontiguous":
        x = x.transpose(2, 3)
    if guard == "unbatched":
        x = x.squeeze(0)
    if guard == "eval":
        cand.eval()
    with torch.set_grad_enabled(guard != "no-grad"), Observe() as seen:
        cand(x)
    assert DW_OP not in seen.ops


@pytest.mark.parametrize("autocast", [False, True])
@pytest.mark.parametrize("affine", [True, False])
def test_group_norm_wrapper_matches_native(autocast, affine):
    print(f"[gn wrapper] autocast={autocast} affine={affine}", flush=True)
    torch.manual_seed(7)
    ref = nn.GroupNorm(16, 16, affine=affine).to(DEV)
    if affine:
        with torch.no_grad():
            ref.weight.uniform_(0.5, 1.5)
            ref.bias.uniform_(-0.5, 0.5)
    cand = AdaptiveGroupNorm3d(copy.deepcopy(ref), PolicyRegistry().resolver(), MC)
    dtype = torch.bfloat16 if autocast else torch.float32
    x = (torch.randn(2, 16, 12, 20, 24, device=DEV) * 3 + 1).to(dtype).requires_grad_()
    y = x.detach().clone().requires_grad_()
    with torch.autocast(DEV, dtype=torch.bfloat16, enabled=autocast):
        want = ref(x)
        with Observe() as seen:
            got = cand(y)
    assert GN_OP in seen.ops
    assert got.dtype == want.dtype == torch.float32
    g = torch.randn_like(want)
    wants = torch.autograd.grad(want, (x, *ref.parameters()), g)
    gots = torch.autograd.grad(got, (y, *cand.parameters()), g)
    assert max_rel(got, want) <= FP32_OUT  # GroupNorm runs in fp32 either way
    assert gots[0].dtype == x.dtype
    assert max_rel(gots[0], wants[0]) <= (FP32_OUT if not autocast else BF16)
    for a, b in zip(gots[1:], wants[1:], strict=True):
        assert max_rel(a, b) <= FP32_WGRAD


@pytest.mark.parametrize("channels,size,ratio", [(32, 128, 2), (128, 32, 4)])
def test_block_cfg2_bf16_autocast_matches_reference_block(channels, size, ratio):
    """one MedNeXt block (dw -> GN -> expand -> GELU ->
    project -> +res) under bf16 autocast, fwd + bwd.

    Both the HIP-backed block and the reference block (plain PyTorch under the
    same autocast) are compared with the block evaluated in float64 on the same
    input. Each output / gradient must be within the bf16 tolerance of that
    ground truth, or no worse than 2x the reference's own error: sums such as
    the depthwise bias gradient (2M terms per channel with heavy cancellation)
    amplify bf16 rounding of the upstream gradient in both paths alike; the
    depthwise bias gradient is exactly zero (GroupNorm follows it)."""
    print(f"[block cfg2] C={channels} S={size} R={ratio}", flush=True)
    torch.manual_seed(11)
    ref = MedNeXtBlock(spatial_dims=3, in_channels=channels, out_channels=channels, expansion_ratio=ratio, kernel_size=3)
    ref = ref.to(DEV).train()
    cand = copy.deepcopy(ref)
    truth = copy.deepcopy(ref).double()
    assert install_adaptive_operators(cand, resolver=PolicyRegistry().resolver(), model_context=MC) == 4
    x = torch.randn(1, channels, size, size, size, device=DEV, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    z = x.detach().double().requires_grad_()
    with torch.autocast(DEV, dtype=torch.bfloat16):
        want = ref(x)
        with Observe() as seen:
            got = cand(y)
    # The block's GroupNorm folds into the expand GEMM (gn_mlp_expansion).
    assert DW_OP in seen.ops and GN_MLP_OP in seen.ops and GN_OP not in seen.ops
    exact = truth(z)
    g = torch.randn_like(want)
    wants = torch.autograd.grad(want, (x, *ref.parameters()), g)
    gots = torch.autograd.grad(got, (y, *cand.parameters()), g)
    exacts = torch.autograd.grad(exact, (z, *truth.parameters()), g.double())
    names = ["output", "x", *(n for n, _ in ref.named_parameters())]
    for name, a, b, t in zip(names, (got, *gots), (want, *wants), (exact, *exacts), strict=True):
        check_against_truth(name, a, b, t, BF16)


def test_small_model_fp32_matches_reference_model():
    """Whole model in fp32 (MedNeXt-S, C=8, 64^3, deep supervision): outputs and
    every gradient vs the model in float64, HIP path vs reference path."""
    print("[model fp32] small C8 64^3", flush=True)
    torch.manual_seed(23)
    ref = mednext_small(in_channels=1, out_channels=3, base_channels=8, deep_supervision=True, optimization="reference")
    cand = mednext_small(in_channels=1, out_channels=3, base_channels=8, deep_supervision=True)
    cand.load_state_dict(ref.state_dict())
    truth = copy.deepcopy(ref).double()
    ref, cand, truth = ref.to(DEV).train(), cand.to(DEV).train(), truth.to(DEV).train()
    x = torch.randn(1, 1, 64, 64, 64, device=DEV)
    with Observe() as seen:
        outs = cand(x)
    want, exact = ref(x), truth(x.double())
    assert seen.ops.count(DW_OP) > 0 and seen.ops.count(GN_OP) > 0
    for i, (a, b, t) in enumerate(zip(outs, want, exact, strict=True)):
        check_against_truth(f"head {i}", a, b, t, 1e-4)
    for model, heads in ((cand, outs), (ref, want), (truth, exact)):
        sum(o.square().mean() for o in heads).backward()
    for (name, p), q, t in zip(cand.named_parameters(), ref.parameters(), truth.parameters(), strict=True):
        check_against_truth(name, p.grad, q.grad, t.grad, 1e-4)


def test_base_training_step_128_bf16_matches_reference():
    """One MedNeXt-Base 128^3 bf16 AdamW step through the
    HIP ops: same loss as the reference model within the bf16 tolerance."""
    print("[model step] base 128^3 bf16", flush=True)
    torch.manual_seed(1234)
    ref = mednext_base(in_channels=1, out_channels=3, deep_supervision=True, optimization="reference").to(DEV).train()
    cand = mednext_base(in_channels=1, out_channels=3, deep_supervision=True).to(DEV).train()
    cand.load_state_dict(ref.state_dict())
    losses = []
    for model in (cand, ref):
        step = make_training_step(model, size=128, device=DEV)
        with Observe() as seen:
            loss = step()
        losses.append(float(loss))
        if model is cand:
            assert DW_OP in seen.ops and DX_OP in seen.ops and DWG_OP in seen.ops and GN_MLP_OP in seen.ops
        del step
    assert abs(losses[0] - losses[1]) / abs(losses[1]) < BF16
    for (name, p), q in zip(cand.named_parameters(), ref.parameters(), strict=True):
        assert torch.isfinite(p).all(), name
    torch.cuda.empty_cache()


def test_large_k5_checkpointed_step_matches_reference():
    """MedNeXt-Large k5 with expansion checkpointing on all stages (BASELINE
    configs[4]) at 64^3: one bf16 AdamW step through the HIP ops (k5 depthwise,
    fused expansions recomputed in backward) gives the reference model's loss
    within the bf16 tolerance and the same gradient norms."""
    print("[model step] large k5 ckpt 64^3 bf16", flush=True)
    from mednext_accel_amd import mednext_large

    torch.manual_seed(4321)
    ckpt = CheckpointConfig(style="expansion", stages=None)
    ref = mednext_large(in_channels=1, out_channels=3, kernel_size=5, deep_supervision=True, checkpointing=ckpt,
                        optimization="reference").to(DEV).train()
    cand = mednext_large(in_channels=1, out_channels=3, kernel_size=5, deep_supervision=True,
                         checkpointing=ckpt).to(DEV).train()
    cand.load_state_dict(ref.state_dict())
    losses, norms = [], []
    for model in (cand, ref):
        step = make_training_step(model, size=64, device=DEV)
        with Observe() as seen:
            loss = step()
        losses.append(float(loss.detach()))
        norms.append(torch.stack([p.grad.float().norm() for p in model.parameters()]))
        if model is cand:
            assert DW_OP in seen.ops and DX_OP in seen.ops and DWG_OP in seen.ops and GN_OP in seen.ops
            # Checkpointed expansions keep GroupNorm unfolded (no second statistics pass).
            assert MLP_OP in seen.ops and MLP_STORED_OP in seen.ops and GN_MLP_OP not in seen.ops
        del step
    assert abs(losses[0] - losses[1]) / abs(losses[1]) < BF16
    assert torch.isfinite(norms[0]).all()
    assert float(((norms[0] - norms[1]).norm() / norms[1].norm())) < 5e-2
    torch.cuda.empty_cache()


def test_groupnorm_fold_is_bit_identical_to_the_unfolded_path():
    """MedNeXt-S (C=8, 32^3, bf16 autocast, no checkpointing) with every
    block's GroupNorm folded into its expand GEMM or run as its own kernels:
    the NORM prologue hands the GEMM the bf16 values the GroupNorm kernel
    writes, so the output and every gradient are bit-identical, except the
    expand weight's, which the folded path takes from the exact map of the raw
    product (no per-element rounding of the normalised operand)."""
    torch.manual_seed(11)
    model = mednext_small(in_channels=1, out_channels=2, base_channels=8).to(DEV).train()
    x = torch.randn(1, 1, 32, 32, 32, device=DEV)
    runs = {}
    try:
        for fold in (True, False):
            AdaptiveExpansion.fold_norm = fold
            model.zero_grad(set_to_none=True)
            with torch.autocast(DEV, dtype=torch.bfloat16), Observe() as seen:
                out = model(x)
            assert (GN_MLP_OP in seen.ops) == fold and (GN_OP in seen.ops) != fold
            out.float().square().mean().backward()
            runs[fold] = (out.detach(), {n: p.grad.detach().clone() for n, p in model.named_parameters()})
    finally:
        AdaptiveExpansion.fold_norm = True
    assert torch.equal(runs[True][0], runs[False][0])
    for name, g in runs[True][1].items():
        other = runs[False][1][name]
        if name.endswith("expand.weight"):
            assert rel_l2(g, other) <= 1e-2, name
        else:
            assert torch.equal(g, other), name


@pytest.mark.parametrize("style", ["expansion", "block"])
def test_checkpointed_model_runs_hip_ops(style):
    """Activation checkpointing recomputes through the HIP ops: bf16 autocast
    outputs and gradients vs float64, no worse than the reference path."""
    torch.manual_seed(3)
    model = mednext_small(in_channels=1, out_channels=2, base_channels=8, checkpointing=CheckpointConfig(style=style))
    ref = mednext_small(in_channels=1, out_channels=2, base_channels=8, optimization="reference")
    ref.load_state_dict(model.state_dict())
    truth = copy.deepcopy(ref).double()
    model, ref, truth = model.to(DEV).train(), ref.to(DEV).train(), truth.to(DEV).train()
    x = torch.randn(1, 1, 32, 32, 32, device=DEV)
    with torch.autocast(DEV, dtype=torch.bfloat16), Observe() as seen:
        a = model(x)
    with torch.autocast(DEV, dtype=torch.bfloat16):
        b = ref(x)
    t = truth(x.double())
    assert DW_OP in seen.ops
    check_against_truth("output", a, b, t, BF16)
    for out in (a, b, t):
        out.float().square().mean().backward() if out is not t else out.square().mean().backward()
    for (name, p), q, r in zip(model.named_parameters(), ref.parameters(), truth.parameters(), strict=True):
        check_against_truth(name, p.grad, q.grad, r.grad, BF16)


def test_wrapped_depthwise_compiles_fullgraph():
    torch.manual_seed(31)
    ref = nn.Conv3d(2, 2, 3, padding=1, groups=2, device=DEV)
    cand = AdaptiveDepthwise3d(copy.deepcopy(ref), PolicyRegistry().resolver(), MC)
    compiled = torch.compile(cand, fullgraph=True, backend="aot_eager")
    x = torch.randn(1, 2, 6, 8, 8, device=DEV, requires_grad=True)
    y = x.detach().clone().requires_grad_()
    got, want = compiled(y), ref(x)
    g = torch.randn_like(want)
    assert max_rel(got, want) <= FP32_OUT
    for a, b in zip(
        torch.autograd.grad(got, (y, *cand.parameters()), g), torch.autograd.grad(want, (x, *ref.parameters()), g),
        strict=True,
    ):
        assert max_rel(a, b) <= FP32_WGRAD


def test_opcheck_custom_ops():
    from mednext_accel_amd import hip_ops

    torch.manual_seed(5)
    x = torch.randn(1, 3, 5, 6, 8, device=DEV, requires_grad=True)
    w = torch.randn(3, 1, 3, 3, 3, device=DEV, requires_grad=True)
    b = torch.randn(3, device=DEV, requires_grad=True)
    recipe = [0, 8, 2]
    torch.library.opcheck(hip_ops.depthwise_conv3d_regular, (x, w, b, 3, recipe, recipe, recipe, True, True, True))
    dy = torch.randn(1, 3, 5, 6, 8, device=DEV)
    torch.library.opcheck(hip_ops.depthwise_input_grad_regular, (dy, w.detach(), 3, recipe))
    torch.library.opcheck(hip_ops.depthwise_weight_grad_regular, (x.detach(), dy, 3, recipe))
    g = torch.rand(3, device=DEV, requires_grad=True)
    torch.library.opcheck(hip_ops.group_norm_channels, (x, g, b, 1e-5, None))
