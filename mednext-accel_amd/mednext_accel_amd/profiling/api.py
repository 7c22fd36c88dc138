"""Profiling campaign entry point (reference profiling/api.py:182, ``profile``).

``profile()`` measures every case of the workload matrix on the current GPU
(native module once per context and phase, then each HIP candidate against
it), synthesizes the winners into a policy v2 document for this device and,
when asked, writes the policy (YAML) and the scalar evidence (JSON, whose
SHA-256 the policy records).
"""

from __future__ import annotations

import hashlib
import json
from collections.abc import Callable
from dataclasses import dataclass, field
from pathlib import Path

import yaml

from .matrix import KernelCase, build_workload_cases
from .synthesize import Measurement, synthesize_policy


@dataclass
class ProfilingResult:
    policy: dict[str, object]
    measurements: list[Measurement] = field(default_factory=list)

    def evidence(self) -> dict[str, object]:
        return {"kind": "mednext-accel-evidence", "measurements": [m.to_primitive() for m in self.measurements]}


def profile(
    variant: str = "base",
    *,
    size: int = 128,
    kernel_sizes: tuple[int, ...] = (3,),
    families: tuple[str, ...] = ("depthwise_conv3d", "group_norm3d", "pointwise_conv3d"),
    repetitions: int = 10,
    policy_path: str | Path | None = None,
    evidence_path: str | Path | None = None,
    name: str | None = None,
    progress: Callable[[str], None] | None = print,
) -> ProfilingResult:
    import torch

    from ..adaptive import device_facts
    from .operator_benchmark import benchmark_operator

    _, _, arch = device_facts(torch.cuda.current_device())
    cases = build_workload_cases(variant, size=size, kernel_sizes=kernel_sizes, families=families)
    reference_ms: dict[tuple[tuple[object, ...], str], float] = {}
    measurements: list[Measurement] = []
    for i, case in enumerate(cases):
        key = (case.context_key, case.phase)
        result = benchmark_operator(case, repetitions=repetitions, reference_ms=reference_ms.get(key))
        if case.implementation == "reference" and result.get("reference_ms") is not None:
            reference_ms[key] = result["reference_ms"]
            result["candidate_ms"] = result["reference_ms"]
        m = Measurement.from_result(result)
        measurements.append(m)
        if progress is not None:
            ms = "-" if m.candidate_ms is None else f"{m.candidate_ms * 1000:.1f} us"
            progress(f"[{i + 1}/{len(cases)}] {_describe(case)}: {ms}"
                     + ("" if m.valid else f" rejected ({m.rejection_reason})"))
    result = ProfilingResult(policy={}, measurements=measurements)
    evidence_ref = None
    if evidence_path is not None:
        data = json.dumps(result.evidence(), sort_keys=True, separators=(",", ":")).encode()
        Path(evidence_path).write_bytes(data)
        evidence_ref = [{"id": "integrated-operators", "sha256": hashlib.sha256(data).hexdigest(),
                         "file": Path(evidence_path).name}]
    result.policy = synthesize_policy(measurements, name=name or f"{arch or 'amd'}-{variant}-{size}-generated",
                                      arch=arch, evidence=evidence_ref)
    if policy_path is not None:
        Path(policy_path).write_text(dump_policy(result.policy))
    return result


def dump_policy(policy: dict[str, object]) -> str:
    """YAML text of a synthesized policy (flow style for the leaf mappings)."""
    return yaml.safe_dump(policy, sort_keys=False, default_flow_style=None, width=120)


def _describe(case: KernelCase) -> str:
    d, h, w = case.spatial_shape
    params = ",".join(f"{k}={v}" for k, v in case.parameters)
    return (f"{case.family} {case.in_channels}->{case.out_channels} k{case.kernel_size} {d}x{h}x{w} "
            f"{case.phase} {case.implementation}" + (f"[{params}]" if params else ""))
