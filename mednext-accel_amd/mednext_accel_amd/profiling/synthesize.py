"""Policy synthesis from integrated measurements (reference
profiling/synthesize.py:487, ``synthesize_profile``).

For every measured operator context and phase the fastest *valid* candidate
wins (``reference``, i.e. native PyTorch, is always a candidate, timed the
same way). The winners become exact-context rules of a policy v2 document
for the measuring device: one rule per context, with a phase map for the
depthwise convolution and a ``training`` selection for GroupNorm and the 1x1x1
convolutions, literal launch parameters for recipe-driven implementations,
and confidence ``measured-exact-context``. Contexts that were not measured
are left to the lower policy layers (the bundled gfx950 policy).
"""

from __future__ import annotations

from collections import defaultdict
from collections.abc import Iterable
from dataclasses import dataclass

from ..optimization.parameters import has_parameter_recipe
from .matrix import KernelCase

CONV_FAMILIES = ("depthwise_conv3d", "pointwise_conv3d")


@dataclass(frozen=True, slots=True)
class Measurement:
    case: KernelCase
    valid: bool
    candidate_ms: float | None
    reference_ms: float | None
    rejection_reason: str | None = None

    @classmethod
    def from_result(cls, result: dict[str, object]) -> Measurement:
        case = result["case"]
        cand = result.get("candidate_ms")
        if case.implementation == "reference" and cand is None:
            cand = result.get("reference_ms")
        return cls(case, bool(result.get("valid")), cand, result.get("reference_ms"),
                   result.get("rejection_reason"))

    def to_primitive(self) -> dict[str, object]:
        c = self.case
        return {
            "family": c.family, "direction": c.direction, "phase": c.phase, "in_channels": c.in_channels,
            "out_channels": c.out_channels, "kernel_size": c.kernel_size, "spatial_shape": list(c.spatial_shape),
            "batch": c.batch, "dtype": c.dtype, "implementation": c.implementation,
            "parameters": dict(c.parameters), "valid": self.valid, "candidate_ms": self.candidate_ms,
            "reference_ms": self.reference_ms, "rejection_reason": self.rejection_reason,
        }


def measurements_from_evidence(doc: dict[str, object]) -> list[Measurement]:
    """Measurements back from an evidence document written by ``profile``,
    so a policy can be re-synthesized without re-measuring."""
    if doc.get("kind") != "mednext-accel-evidence":
        raise ValueError("not a mednext-accel evidence document")
    out = []
    for m in doc["measurements"]:
        case = KernelCase(m["family"], m["phase"], m["in_channels"], m["out_channels"], m["kernel_size"],
                          tuple(m["spatial_shape"]), m["implementation"], tuple(sorted(m["parameters"].items())),
                          batch=m["batch"], dtype=m["dtype"], direction=m["direction"])
        out.append(Measurement(case, m["valid"], m["candidate_ms"], m["reference_ms"], m.get("rejection_reason")))
    return out


def best_candidates(measurements: Iterable[Measurement]) -> dict[tuple[tuple[object, ...], str], Measurement]:
    """Fastest valid measurement per (context, phase); ties keep the earlier one."""
    best: dict[tuple[tuple[object, ...], str], Measurement] = {}
    for m in measurements:
        if not m.valid or m.candidate_ms is None:
            continue
        key = (m.case.context_key, m.case.phase)
        if key not in best or m.candidate_ms < best[key].candidate_ms:
            best[key] = m
    return best


def _rule_id(case: KernelCase) -> str:
    d, h, w = case.spatial_shape
    return (f"{case.family}-{case.in_channels}x{case.out_channels}-k{case.kernel_size}-{d}x{h}x{w}"
            f"-n{case.batch}-{case.dtype}")


def synthesize_policy(measurements: Iterable[Measurement], *, name: str = "gfx950-generated",
                      arch: str | None = "gfx950", evidence: list[dict[str, str]] | None = None) -> dict[str, object]:
    """Policy v2 document (plain data, parses with ``parse_policy``)."""
    best = best_candidates(measurements)
    by_context: dict[tuple[object, ...], dict[str, Measurement]] = defaultdict(dict)
    for (context, phase), m in best.items():
        by_context[context][phase] = m
    rules = []
    for context in sorted(by_context, key=repr):
        phases = by_context[context]
        case = next(iter(phases.values())).case
        when: dict[str, object] = {
            "family": case.family,
            "direction": case.direction,
            "dtype": case.dtype,
            "channels": [case.in_channels, case.out_channels],
            "spatial_shape": list(case.spatial_shape),
            "batch": case.batch,
        }
        if case.family in CONV_FAMILIES:
            when["kernel_size"] = [case.kernel_size] * 3
        use: dict[str, object] = {}
        for phase in sorted(phases):
            win = phases[phase].case
            sel: dict[str, object] = {"implementation": win.implementation}
            if win.parameters:
                sel["parameters"] = dict(win.parameters)
            elif has_parameter_recipe(win.implementation):
                sel["parameters"] = "auto"  # measured with the default recipe
            use[phase] = sel
        rules.append({"id": _rule_id(case), "when": when, "use": use, "confidence": "measured-exact-context"})
    target: dict[str, object] = {"vendor": "amd"}
    if arch:
        target["arch"] = arch
    doc: dict[str, object] = {"version": 2, "kind": "mednext-accel-policy", "name": name, "target": target,
                              "rules": rules}
    if evidence:
        doc["evidence"] = evidence
    return doc
