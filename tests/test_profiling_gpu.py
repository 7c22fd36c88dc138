"""Profiler on the GPU: integrated per-phase measurements validate and time
the HIP candidates against native PyTorch, and a small campaign synthesizes a
policy that the model then runs with."""

from __future__ import annotations

import pytest
import torch

from mednext_accel_amd import mednext_small
from mednext_accel_amd.optimization import parse_policy
from mednext_accel_amd.profiling import KernelCase
from mednext_accel_amd.profiling.api import profile
from mednext_accel_amd.profiling.operator_benchmark import benchmark_operator

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize(
    "case",
    [
        KernelCase("depthwise_conv3d", "forward", 16, 16, 3, (32, 32, 32), "hip_depthwise_fwd",
                   (("depth_chunk", 8), ("engine", 1), ("tile_w", 32))),
        KernelCase("depthwise_conv3d", "backward_input", 16, 16, 3, (32, 32, 32), "hip_depthwise_dx",
                   (("depth_chunk", 8), ("engine", 1), ("tile_w", 32))),
        KernelCase("depthwise_conv3d", "backward_weight", 8, 8, 5, (32, 32, 32), "hip_split_dw",
                   (("depth_chunk", 16), ("engine", 1), ("tile_w", 32))),
        KernelCase("group_norm3d", "training", 8, 8, 1, (15, 15, 15), "hip_group_norm"),
        KernelCase("pointwise_conv3d", "training", 32, 96, 1, (9, 9, 9), "hip_pointwise_gemm"),
        KernelCase("depthwise_conv3d", "forward", 16, 16, 3, (32, 32, 32), "reference"),
    ],
    ids=lambda c: f"{c.family}-{c.phase}-{c.implementation}",
)
def test_benchmark_operator_validates_and_times(case):
    print(f"[profiling] {case.family} {case.phase} {case.implementation}", flush=True)
    result = benchmark_operator(case, repetitions=4, warmup=1)
    assert result["valid"], result["rejection_reason"]
    assert result["candidate_ms"] > 0 and result["reference_ms"] > 0
    for metrics in result["validation_metrics"].values():
        assert metrics["finite"] and metrics["relative_l2"] < 0.02


def test_small_campaign_synthesizes_a_usable_policy(tmp_path):
    print("[profiling] campaign small 32^3", flush=True)
    result = profile("small", size=32, repetitions=3, policy_path=tmp_path / "p.yaml",
                     evidence_path=tmp_path / "e.json", families=("depthwise_conv3d", "group_norm3d"),
                     progress=None)
    policy = parse_policy(result.policy)
    assert policy.rules and policy.target_arch == torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    assert (tmp_path / "p.yaml").exists() and (tmp_path / "e.json").exists()
    assert all(m.valid for m in result.measurements)
    model = mednext_small(in_channels=1, out_channels=2, base_channels=8, optimization=tmp_path / "p.yaml")
    model = model.to(DEV).train()
    with torch.autocast(DEV, dtype=torch.bfloat16):
        out = model(torch.randn(1, 1, 32, 32, 32, device=DEV))
    out.float().square().mean().backward()
    assert all(torch.isfinite(p.grad).all() for p in model.parameters() if p.grad is not None)
