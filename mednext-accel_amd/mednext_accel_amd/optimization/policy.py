"""Policy documents (version 2, kind ``mednext-accel-policy``) and their parser.

The document format is the reference's (optimization/policy.py:59-359) so that
its policy files and tooling stay usable: ``target`` (vendor, optional sm),
``scope`` conditions inherited by every rule, ``rules`` with ``id``, ``when``,
per-phase ``use`` selections and a ``confidence`` label, and descriptive
``evidence`` entries. This build adds one optional target field, ``arch``
(e.g. ``gfx950``), matched against the AMD device's ISA name. A rule with no
selection for a phase falls through; an explicit ``reference`` selection ends
resolution for that phase.
"""

from __future__ import annotations

import math
import re
from collections.abc import Mapping
from dataclasses import dataclass
from pathlib import PurePosixPath
from types import MappingProxyType
from typing import Literal

from .implementations import ImplementationRegistry, default_implementation_registry
from .parameters import has_parameter_recipe, validate_parameters

Confidence = Literal[
    "measured-exact-context",
    "interpolated-bounded",
    "inferred-same-sm",
    "validated-cross-sm",
    "extrapolated",
    "guard",
]
CONFIDENCES = frozenset(Confidence.__args__)  # type: ignore[attr-defined]
PHASES = frozenset(
    {"training", "inference", "export", "forward", "backward_input", "backward_weight", "backward_bias"}
)
STRING_FACTS = frozenset({"family", "direction", "role", "dtype", "model_family", "variant", "checkpointing"})
TUPLE_FACTS = {"kernel_size": 3, "stride": 3, "spatial_shape": 3, "channels": 2}
NUMBER_FACTS = frozenset(
    {"batch", "in_channels", "out_channels", "spatial_volume", "work", "reduction_work", "total_vram_gib"}
)


@dataclass(frozen=True, slots=True)
class NumericRange:
    minimum: int | float | None = None
    maximum: int | float | None = None

    def contains(self, value: int | float) -> bool:
        return (self.minimum is None or value >= self.minimum) and (self.maximum is None or value <= self.maximum)


Condition = str | tuple[int, ...] | NumericRange
Parameters = Mapping[str, str | int | float | bool | None]


@dataclass(frozen=True, slots=True)
class PolicySelection:
    implementation: str
    parameters: Parameters | Literal["auto"] | None = None

    def __post_init__(self) -> None:
        if isinstance(self.parameters, Mapping):
            object.__setattr__(self, "parameters", MappingProxyType(dict(self.parameters)))


@dataclass(frozen=True, slots=True)
class PolicyRule:
    identifier: str
    when: Mapping[str, Condition]
    use: Mapping[str, PolicySelection]
    confidence: Confidence
    declared_when: Mapping[str, Condition]

    def __post_init__(self) -> None:
        for name in ("when", "use", "declared_when"):
            object.__setattr__(self, name, MappingProxyType(dict(getattr(self, name))))


@dataclass(frozen=True, slots=True)
class EvidenceReference:
    identifier: str
    sha256: str
    file: str | None = None


@dataclass(frozen=True, slots=True)
class OptimizationPolicy:
    name: str
    vendor: str
    target_sm: tuple[int, int] | None
    scope: Mapping[str, Condition]
    rules: tuple[PolicyRule, ...]
    evidence: tuple[EvidenceReference, ...] = ()
    version: int = 2
    kind: str = "mednext-accel-policy"
    target_arch: str | None = None

    def __post_init__(self) -> None:
        object.__setattr__(self, "scope", MappingProxyType(dict(self.scope)))
        object.__setattr__(self, "rules", tuple(self.rules))
        object.__setattr__(self, "evidence", tuple(self.evidence))
        if self.target_sm is not None:
            object.__setattr__(self, "target_sm", tuple(self.target_sm))


# ----------------------------------------------------------------- validation


def _as_mapping(value: object, where: str, allowed: frozenset[str] | set[str] | None = None) -> Mapping:
    if not isinstance(value, Mapping) or not all(isinstance(k, str) for k in value):
        raise ValueError(f"{where} must be a mapping with string keys")
    if allowed is not None:
        extra = set(value) - set(allowed)
        if extra:
            raise ValueError(f"{where}: unknown fields {', '.join(sorted(extra))}")
    return value


def _as_string(value: object, where: str) -> str:
    if not isinstance(value, str) or not value.strip():
        raise ValueError(f"{where} must be a non-empty string")
    return value


def _as_ints(value: object, length: int, where: str, minimum: int = 1) -> tuple[int, ...]:
    ok = isinstance(value, (list, tuple)) and len(value) == length
    ok = ok and all(type(v) is int and v >= minimum for v in value)
    if not ok:
        raise ValueError(f"{where} must contain {length} integers >= {minimum}")
    return tuple(value)


def _as_range(value: object, where: str, *, integer: bool) -> NumericRange:
    bounds = dict(_as_mapping(value, where, {"min", "max"})) if isinstance(value, Mapping) else {"min": value, "max": value}
    if not bounds:
        raise ValueError(f"{where} range must supply min or max")
    for key, bound in bounds.items():
        numeric = type(bound) is int if integer else type(bound) in (int, float)
        if not numeric or not math.isfinite(bound) or bound < (1 if integer else 0):
            raise ValueError(f"{where}.{key} must be a finite {'positive integer' if integer else 'nonnegative number'}")
    low, high = bounds.get("min"), bounds.get("max")
    if low is not None and high is not None and low > high:
        raise ValueError(f"{where}: min must not exceed max")
    return NumericRange(low, high)


def _channels_consistent(conditions: Mapping[str, Condition], where: str) -> None:
    exact = conditions.get("channels")
    if exact is None:
        return
    for name, channel in zip(("in_channels", "out_channels"), exact):
        bound = conditions.get(name)
        if isinstance(bound, NumericRange) and not bound.contains(channel):
            raise ValueError(f"{where}.{name} contradicts exact channels")


def _conditions(value: object, where: str) -> dict[str, Condition]:
    data = _as_mapping(value, where, STRING_FACTS | set(TUPLE_FACTS) | NUMBER_FACTS)
    out: dict[str, Condition] = {}
    for name, item in data.items():
        at = f"{where}.{name}"
        if name in STRING_FACTS:
            out[name] = _as_string(item, at)
        elif name in TUPLE_FACTS:
            out[name] = _as_ints(item, TUPLE_FACTS[name], at)
        else:
            out[name] = _as_range(item, at, integer=name != "total_vram_gib")
    _channels_consistent(out, where)
    return out


def _narrow(scope: Mapping[str, Condition], when: Mapping[str, Condition], where: str) -> dict[str, Condition]:
    """A rule's effective condition: the scope, narrowed (never widened) by ``when``."""
    out = dict(scope)
    for name, value in when.items():
        outer = scope.get(name)
        if isinstance(outer, NumericRange) and isinstance(value, NumericRange):
            if (outer.minimum is not None and value.minimum is not None and value.minimum < outer.minimum) or (
                outer.maximum is not None and value.maximum is not None and value.maximum > outer.maximum
            ):
                raise ValueError(f"{where}.{name} cannot widen scope")
            low = outer.minimum if value.minimum is None else value.minimum
            high = outer.maximum if value.maximum is None else value.maximum
            if low is not None and high is not None and low > high:
                raise ValueError(f"{where}.{name} contradicts scope")
            value = NumericRange(low, high)
        elif outer is not None and outer != value:
            raise ValueError(f"{where}.{name} contradicts scope")
        out[name] = value
    _channels_consistent(out, where)
    return out


def _selection(value: object, where: str, registry: ImplementationRegistry) -> PolicySelection:
    data = _as_mapping(value, where, {"implementation", "parameters"})
    implementation = _as_string(data.get("implementation"), f"{where}.implementation")
    try:
        registry.resolve_metadata(implementation)
    except ValueError as error:
        raise ValueError(f"{where}: {error}") from error
    parameters = data.get("parameters")
    if "parameters" in data:
        if parameters == "auto":
            if not has_parameter_recipe(implementation):
                raise ValueError(f"{where}: {implementation!r} has no parameter recipe for auto")
        else:
            parameters = _as_mapping(parameters, f"{where}.parameters")
            try:
                validate_parameters(implementation, parameters)
            except ValueError as error:
                raise ValueError(f"{where}: {error}") from error
    return PolicySelection(implementation, parameters)


def _evidence(value: object, where: str) -> EvidenceReference:
    data = _as_mapping(value, where, {"id", "sha256", "file"})
    identifier = _as_string(data.get("id"), f"{where}.id")
    digest = data.get("sha256")
    if not isinstance(digest, str) or re.fullmatch(r"[0-9a-f]{64}", digest) is None:
        raise ValueError(f"{where}.sha256 must be a lowercase SHA-256 hex digest")
    filename = data.get("file")
    if "file" in data:
        filename = _as_string(filename, f"{where}.file")
        if PurePosixPath(filename).name != filename or filename in (".", "..") or "\\" in filename:
            raise ValueError(f"{where}.file must be a relative evidence filename")
    return EvidenceReference(identifier, digest, filename)


def parse_policy(value: Mapping[str, object], *, registry: ImplementationRegistry | None = None) -> OptimizationPolicy:
    """Validate and normalize one policy document."""
    doc = _as_mapping(value, "policy document")
    if doc.get("kind") == "mednext-accel-evidence":
        raise ValueError("profiling evidence is not a runtime policy; supply its policy YAML")
    if "schema_version" in doc or doc.get("version") == 1:
        raise ValueError("schema-v1 profiles are unsupported; migrate to policy v2")
    _as_mapping(doc, "policy", {"version", "kind", "name", "target", "scope", "evidence", "rules"})
    if type(doc.get("version")) is not int or doc["version"] != 2:
        raise ValueError("policy.version must be 2")
    if doc.get("kind") != "mednext-accel-policy":
        raise ValueError("policy.kind must be mednext-accel-policy")
    name = _as_string(doc.get("name"), "policy.name")
    target = _as_mapping(doc.get("target"), "target", {"vendor", "sm", "arch"})
    vendor = _as_string(target.get("vendor"), "target.vendor")
    sm = _as_ints(target["sm"], 2, "target.sm", minimum=0) if "sm" in target else None
    arch = _as_string(target["arch"], "target.arch") if "arch" in target else None
    scope = _conditions(doc.get("scope", {}), "scope")
    registry = registry or default_implementation_registry()
    raw_rules = doc.get("rules")
    if not isinstance(raw_rules, (list, tuple)):
        raise ValueError("rules must be a sequence")
    rules = []
    for index, raw in enumerate(raw_rules):
        where = f"rules[{index}]"
        data = _as_mapping(raw, where, {"id", "when", "use", "confidence"})
        identifier = _as_string(data.get("id"), f"{where}.id")
        declared = _conditions(data.get("when", {}), f"{where}.when")
        uses = _as_mapping(data.get("use"), f"{where}.use", PHASES)
        if not uses:
            raise ValueError(f"{where}.use must contain a phase selection")
        selections = {phase: _selection(item, f"{where}.use.{phase}", registry) for phase, item in uses.items()}
        confidence = data.get("confidence")
        if confidence not in CONFIDENCES:
            raise ValueError(f"{where}.confidence must be one of {sorted(CONFIDENCES)}")
        rules.append(PolicyRule(identifier, _narrow(scope, declared, f"{where}.when"), selections, confidence, declared))
    if len({rule.identifier for rule in rules}) != len(rules):
        raise ValueError("duplicate rule id")
    raw_evidence = doc.get("evidence", [])
    if not isinstance(raw_evidence, (list, tuple)):
        raise ValueError("evidence must be a sequence")
    evidence = tuple(_evidence(item, f"evidence[{i}]") for i, item in enumerate(raw_evidence))
    if len({item.identifier for item in evidence}) != len(evidence):
        raise ValueError("duplicate evidence id")
    return OptimizationPolicy(name, vendor, sm, scope, tuple(rules), evidence, target_arch=arch)


def policy_to_primitive(policy: OptimizationPolicy) -> dict[str, object]:
    """Portable form of a parsed policy (round-trips through ``parse_policy``)."""

    def conditions(items: Mapping[str, Condition]) -> dict[str, object]:
        out: dict[str, object] = {}
        for name, item in items.items():
            if isinstance(item, NumericRange):
                if item.minimum == item.maximum:
                    out[name] = item.minimum
                else:
                    out[name] = {k: v for k, v in (("min", item.minimum), ("max", item.maximum)) if v is not None}
            else:
                out[name] = list(item) if isinstance(item, tuple) else item
        return out

    def selection(item: PolicySelection) -> dict[str, object]:
        out: dict[str, object] = {"implementation": item.implementation}
        if item.parameters is not None:
            out["parameters"] = dict(item.parameters) if isinstance(item.parameters, Mapping) else item.parameters
        return out

    target: dict[str, object] = {"vendor": policy.vendor}
    if policy.target_sm is not None:
        target["sm"] = list(policy.target_sm)
    if policy.target_arch is not None:
        target["arch"] = policy.target_arch
    doc: dict[str, object] = {"version": 2, "kind": "mednext-accel-policy", "name": policy.name, "target": target}
    if policy.scope:
        doc["scope"] = conditions(policy.scope)
    if policy.evidence:
        doc["evidence"] = [
            {"id": e.identifier, "sha256": e.sha256, **({"file": e.file} if e.file is not None else {})}
            for e in policy.evidence
        ]
    doc["rules"] = [
        {
            "id": rule.identifier,
            "when": conditions(rule.declared_when),
            "use": {phase: selection(sel) for phase, sel in rule.use.items()},
            "confidence": rule.confidence,
        }
        for rule in policy.rules
    ]
    return doc
