"""Profiler / policy generator (CPU): workload matrix, component validation
and policy synthesis. The GPU measurement itself is in test_profiling_gpu.py."""

from __future__ import annotations

import dataclasses

import pytest
import torch

from mednext_accel_amd import tiles
from mednext_accel_amd.optimization import parse_policy
from mednext_accel_amd.optimization.descriptors import ExecutionContext, OperatorDescriptor
from mednext_accel_amd.optimization.parameters import validate_parameters
from mednext_accel_amd.optimization.policy_resolver import PolicyResolver
from mednext_accel_amd.profiling import (
    KernelCase,
    Measurement,
    build_workload_cases,
    synthesize_policy,
    validate_components,
)
from mednext_accel_amd.profiling.matrix import stage_shapes


def test_stage_shapes_follow_the_variant_tables():
    assert stage_shapes("base", 128) == [(32, 128, 2), (64, 64, 3), (128, 32, 4), (256, 16, 4), (512, 8, 4)]
    assert stage_shapes("large", 64)[2] == (128, 16, 8)


def test_workload_matrix_candidates_are_valid_recipes():
    cases = build_workload_cases("base", size=128)
    families = {c.family for c in cases}
    assert families == {"depthwise_conv3d", "group_norm3d", "pointwise_conv3d"}
    contexts = {(c.context_key, c.phase) for c in cases}
    for context, phase in contexts:
        impls = {c.implementation for c in cases if (c.context_key, c.phase) == (context, phase)}
        assert "reference" in impls and len(impls) >= 2 or context[0] == "pointwise_conv3d"
    for c in cases:
        if c.parameters:
            validate_parameters(c.implementation, c.parameter_map)
    # The default recipe is among the depthwise candidates of every phase.
    fwd = [c for c in cases if c.family == "depthwise_conv3d" and c.phase == "forward" and c.in_channels == 32]
    default = tiles.depthwise_recipe(1, 32, (128, 128, 128), 3, "bfloat16", "forward")
    assert any(c.parameter_map == dict(zip(("engine", "tile_w", "depth_chunk"), default)) for c in fwd)
    # 4096 hidden channels (Large bottleneck) run the tiled product, so the HIP
    # candidate is offered there too (the limits themselves: test_tiles.py).
    big = [c for c in build_workload_cases("large", size=128) if c.family == "pointwise_conv3d" and 4096 in
           (c.in_channels, c.out_channels)]
    assert big and {c.implementation for c in big} == {"reference", "pointwise_gemm_per_sample", "hip_pointwise_gemm"}
    # Every 1x1x1 context offers the per-sample GEMM; v2 contexts use the v2 widths and ratios.
    pw = [c for c in cases if c.family == "pointwise_conv3d"]
    assert {c.implementation for c in pw} == {"reference", "pointwise_gemm_per_sample", "hip_pointwise_gemm"}
    v2 = {(c.in_channels, c.out_channels) for c in build_workload_cases("v2-base", size=128)
          if c.family == "pointwise_conv3d"}
    assert (32, 96) in v2 and (512, 4096) in v2 and (4096, 512) in v2


def test_validation_accepts_equal_and_rejects_bad_components():
    gen = torch.Generator().manual_seed(0)
    a = torch.randn(3, 1000, generator=gen)
    ok = validate_components({"dX": a.clone(), "output": a * 2}, {"dX": a, "output": a * 2})
    assert ok["valid"] and ok["validation_metrics"]["dX"]["relative_l2"] == 0.0
    noisy = a + 0.05 * torch.randn(a.shape, generator=gen)
    bad = validate_components({"dX": noisy}, {"dX": a})
    assert not bad["valid"] and "relative L2" in bad["rejection_reason"]
    small = validate_components({"dX": a + 1e-3 * torch.randn(a.shape, generator=gen)}, {"dX": a})
    assert small["valid"]
    nan = a.clone()
    nan[0, 0] = float("nan")
    assert "non-finite" in validate_components({"dX": nan}, {"dX": a})["rejection_reason"]
    assert "shape" in validate_components({"dX": a[:2]}, {"dX": a})["rejection_reason"]
    with pytest.raises(ValueError):
        validate_components({"dX": a}, {"dW": a})


def _m(impl, phase, ms, valid=True, params=(), family="depthwise_conv3d", c=32, s=128):
    case = KernelCase(family, phase, c, c, 3 if family == "depthwise_conv3d" else 1, (s, s, s), impl, params)
    return Measurement(case, valid, ms, 1.0)


def test_synthesis_picks_fastest_valid_candidate_and_parses():
    recipe_a = (("depth_chunk", 32), ("engine", 1), ("tile_w", 128))
    recipe_b = (("depth_chunk", 16), ("engine", 1), ("tile_w", 64))
    ms = [
        _m("reference", "forward", 9.0),
        _m("hip_depthwise_fwd", "forward", 0.06, params=recipe_a),
        _m("hip_depthwise_fwd", "forward", 0.05, valid=False, params=recipe_b),  # invalid: never chosen
        _m("reference", "backward_input", 8.0),
        _m("hip_depthwise_dx", "backward_input", 0.07, params=recipe_b),
        _m("reference", "backward_weight", 0.5),
        _m("hip_split_dw", "backward_weight", 0.9, params=recipe_a),  # slower: reference wins
        _m("reference", "training", 0.2, family="group_norm3d"),
        _m("hip_group_norm", "training", 0.1, family="group_norm3d"),
    ]
    doc = synthesize_policy(ms, name="unit", arch="gfx950")
    policy = parse_policy(doc)
    assert len(policy.rules) == 2
    dw = next(r for r in doc["rules"] if r["when"]["family"] == "depthwise_conv3d")
    assert dw["use"]["forward"] == {"implementation": "hip_depthwise_fwd", "parameters": dict(recipe_a)}
    assert dw["use"]["backward_input"]["parameters"] == dict(recipe_b)
    assert dw["use"]["backward_weight"] == {"implementation": "reference"}
    # The synthesized rule resolves for its exact context on a gfx950 device.
    resolver = PolicyResolver(external=policy)
    desc = OperatorDescriptor.convolution(family="depthwise_conv3d", direction="regular", in_channels=32,
                                          out_channels=32, kernel_size=(3, 3, 3), stride=(1, 1, 1),
                                          padding=(1, 1, 1), dilation=(1, 1, 1), groups=32)
    ctx = ExecutionContext(model_family="mednext_v1", variant="base", checkpointing="none", device_type="cuda",
                           sm=(9, 5), total_vram_bytes=288 << 30, dtype="bfloat16", phase="training",
                           batch_size=1, spatial_shape=(128, 128, 128), arch="gfx950")
    fwd = resolver.resolve(desc, ctx, "forward")
    assert fwd.implementation == "hip_depthwise_fwd" and fwd.parameters == dict(recipe_a)
    assert resolver.resolve(desc, ctx, "backward_weight").implementation == "reference"
    other = dataclasses.replace(ctx, spatial_shape=(64, 64, 64))
    assert resolver.resolve(desc, other, "forward").implementation == "reference"
