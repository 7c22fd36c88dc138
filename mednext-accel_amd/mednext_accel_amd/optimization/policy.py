"""Policy documents: the declarative operator-selection rules, parsed and checked.

The document format is the reference's policy v2 (reference
``optimization/policy.py``), so policy files written for it parse here::

    version: 2
    kind: mednext-accel-policy
    name: <text>
    target: {vendor: amd|nvidia, sm: [major, minor]?, arch: gfx950?}
    scope: {<fact>: <condition>, ...}          # optional, inherited by every rule
    evidence: [{id, sha256, file?}, ...]       # optional, descriptive only
    rules:
      - id: <text>
        when: {<fact>: <condition>, ...}       # narrows the scope, never widens it
        use: {<phase>: {implementation: <id>, parameters: auto | {...}}, ...}
        confidence: <label>

``target.arch`` (the AMD ISA name, e.g. ``gfx950``) is this build's addition.

How this module is organised: ``FACTS`` declares, per condition fact, how its
value is written (text, a fixed-length integer tuple, a positive-integer range
or a non-negative number range); ``_Node`` is a view of one mapping of the
document that knows its own path, so every error names the offending field;
``_Scope`` intersects a rule's ``when`` with the document ``scope``. The parsed
objects (``OptimizationPolicy`` and the dataclasses below) carry the field
names the reference's tooling and reports read.
"""

from __future__ import annotations

import math
import re
from collections.abc import Mapping, Sequence
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

# How each condition fact is written: ("text", 0), ("ints", length),
# ("count", 0) = a positive-integer range, ("amount", 0) = a non-negative
# number range. A range is a bare value (exact) or {min, max} (either optional).
FACTS: Mapping[str, tuple[str, int]] = MappingProxyType(
    {
        **{name: ("text", 0) for name in ("family", "direction", "role", "dtype", "model_family", "variant",
                                          "checkpointing")},
        "kernel_size": ("ints", 3),
        "stride": ("ints", 3),
        "spatial_shape": ("ints", 3),
        "channels": ("ints", 2),
        **{name: ("count", 0) for name in ("batch", "in_channels", "out_channels", "spatial_volume", "work",
                                           "reduction_work")},
        "total_vram_gib": ("amount", 0),
    }
)
# Kept under the reference's names for tooling that groups facts by kind.
STRING_FACTS = frozenset(name for name, (kind, _) in FACTS.items() if kind == "text")
TUPLE_FACTS = {name: n for name, (kind, n) in FACTS.items() if kind == "ints"}
NUMBER_FACTS = frozenset(name for name, (kind, _) in FACTS.items() if kind in ("count", "amount"))

_DOCUMENT_FIELDS = frozenset({"version", "kind", "name", "target", "scope", "evidence", "rules"})
_SHA256 = re.compile(r"[0-9a-f]{64}")


@dataclass(frozen=True, slots=True)
class NumericRange:
    """Closed interval; a missing bound is unbounded."""

    minimum: int | float | None = None
    maximum: int | float | None = None

    def contains(self, value: int | float) -> bool:
        above = self.minimum is None or value >= self.minimum
        below = self.maximum is None or value <= self.maximum
        return above and below


Condition = str | tuple[int, ...] | NumericRange
Parameters = Mapping[str, str | int | float | bool | None]


@dataclass(frozen=True, slots=True)
class PolicySelection:
    """The implementation one rule selects for one phase, with its launch
    parameters: ``None`` (none), ``"auto"`` (the implementation's recipe) or a
    literal mapping."""

    implementation: str
    parameters: Parameters | Literal["auto"] | None = None

    def __post_init__(self) -> None:
        if isinstance(self.parameters, Mapping):
            object.__setattr__(self, "parameters", MappingProxyType(dict(self.parameters)))


@dataclass(frozen=True, slots=True)
class PolicyRule:
    """``when`` is the effective condition (scope narrowed by the rule);
    ``declared_when`` is what the document wrote, kept for round trips."""

    identifier: str
    when: Mapping[str, Condition]
    use: Mapping[str, PolicySelection]
    confidence: Confidence
    declared_when: Mapping[str, Condition]

    def __post_init__(self) -> None:
        for field_name in ("when", "use", "declared_when"):
            object.__setattr__(self, field_name, MappingProxyType(dict(getattr(self, field_name))))


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


# ------------------------------------------------------------------- reading


class _Node:
    """One mapping of the document, with its dotted path for error messages."""

    __slots__ = ("data", "path")

    def __init__(self, value: object, path: str, fields: frozenset[str] | set[str] | None = None) -> None:
        if not isinstance(value, Mapping) or any(not isinstance(key, str) for key in value):
            raise ValueError(f"{path} must be a mapping with string keys")
        if fields is not None:
            unknown = sorted(set(value) - set(fields))
            if unknown:
                raise ValueError(f"{path}: unknown fields {', '.join(unknown)}")
        self.data = value
        self.path = path

    def at(self, key: str) -> str:
        return f"{self.path}.{key}"

    def __contains__(self, key: str) -> bool:
        return key in self.data

    def text(self, key: str) -> str:
        return _text(self.data.get(key), self.at(key))

    def node(self, key: str, fields=None, *, optional: bool = False) -> _Node | None:
        if optional and key not in self.data:
            return None
        return _Node(self.data.get(key), self.at(key), fields)

    def items(self, key: str, *, default=()) -> Sequence[object]:
        value = self.data.get(key, default)
        if not isinstance(value, (list, tuple)):
            raise ValueError(f"{key} must be a sequence")
        return value


def _text(value: object, path: str) -> str:
    if isinstance(value, str) and value.strip():
        return value
    raise ValueError(f"{path} must be a non-empty string")


def _int_tuple(value: object, length: int, path: str, *, least: int) -> tuple[int, ...]:
    if isinstance(value, (list, tuple)) and len(value) == length:
        if all(type(item) is int and item >= least for item in value):
            return tuple(value)
    raise ValueError(f"{path} must contain {length} integers >= {least}")


def _bound(value: object, path: str, kind: str) -> int | float:
    if kind == "count":
        if type(value) is int and value >= 1:
            return value
        raise ValueError(f"{path} must be a finite positive integer")
    if type(value) in (int, float) and math.isfinite(value) and value >= 0:
        return value
    raise ValueError(f"{path} must be a finite nonnegative number")


def _range(value: object, path: str, kind: str) -> NumericRange:
    if not isinstance(value, Mapping):
        exact = _bound(value, path, kind)
        return NumericRange(exact, exact)
    node = _Node(value, path, {"min", "max"})
    if not node.data:
        raise ValueError(f"{path} range must supply min or max")
    low = _bound(node.data["min"], node.at("min"), kind) if "min" in node else None
    high = _bound(node.data["max"], node.at("max"), kind) if "max" in node else None
    if low is not None and high is not None and low > high:
        raise ValueError(f"{path}: min must not exceed max")
    return NumericRange(low, high)


def _condition(name: str, value: object, path: str) -> Condition:
    kind, length = FACTS[name]
    if kind == "text":
        return _text(value, path)
    if kind == "ints":
        return _int_tuple(value, length, path, least=1)
    return _range(value, path, kind)


def _conditions(value: object, path: str) -> dict[str, Condition]:
    node = _Node(value, path, frozenset(FACTS))
    parsed = {name: _condition(name, item, node.at(name)) for name, item in node.data.items()}
    _check_channels(parsed, path)
    return parsed


def _check_channels(conditions: Mapping[str, Condition], path: str) -> None:
    """An exact ``channels`` pair must lie inside any channel-count ranges."""
    pair = conditions.get("channels")
    if pair is None:
        return
    for name, count in (("in_channels", pair[0]), ("out_channels", pair[1])):
        limit = conditions.get(name)
        if isinstance(limit, NumericRange) and not limit.contains(count):
            raise ValueError(f"{path}.{name} contradicts exact channels")


class _Scope:
    """The document scope, which a rule's ``when`` may only narrow."""

    def __init__(self, conditions: Mapping[str, Condition]) -> None:
        self.conditions = dict(conditions)

    def narrowed(self, when: Mapping[str, Condition], path: str) -> dict[str, Condition]:
        effective = dict(self.conditions)
        for name, inner in when.items():
            outer = self.conditions.get(name)
            if outer is None:
                effective[name] = inner
            elif isinstance(outer, NumericRange) and isinstance(inner, NumericRange):
                effective[name] = self._intersect(outer, inner, f"{path}.{name}")
            elif outer == inner:
                effective[name] = inner
            else:
                raise ValueError(f"{path}.{name} contradicts scope")
        _check_channels(effective, path)
        return effective

    @staticmethod
    def _intersect(outer: NumericRange, inner: NumericRange, path: str) -> NumericRange:
        widens_low = inner.minimum is not None and outer.minimum is not None and inner.minimum < outer.minimum
        widens_high = inner.maximum is not None and outer.maximum is not None and inner.maximum > outer.maximum
        if widens_low or widens_high:
            raise ValueError(f"{path} cannot widen scope")
        low = outer.minimum if inner.minimum is None else inner.minimum
        high = outer.maximum if inner.maximum is None else inner.maximum
        if low is not None and high is not None and low > high:
            raise ValueError(f"{path} contradicts scope")
        return NumericRange(low, high)


def _selection(value: object, path: str, registry: ImplementationRegistry) -> PolicySelection:
    node = _Node(value, path, {"implementation", "parameters"})
    implementation = node.text("implementation")
    try:
        registry.resolve_metadata(implementation)
    except ValueError as error:
        raise ValueError(f"{path}: {error}") from error
    if "parameters" not in node:
        return PolicySelection(implementation)
    parameters = node.data["parameters"]
    if parameters == "auto":
        if not has_parameter_recipe(implementation):
            raise ValueError(f"{path}: {implementation!r} has no parameter recipe for auto")
        return PolicySelection(implementation, "auto")
    literal = _Node(parameters, node.at("parameters")).data
    try:
        validate_parameters(implementation, literal)
    except ValueError as error:
        raise ValueError(f"{path}: {error}") from error
    return PolicySelection(implementation, literal)


def _rule(value: object, path: str, scope: _Scope, registry: ImplementationRegistry) -> PolicyRule:
    node = _Node(value, path, {"id", "when", "use", "confidence"})
    identifier = node.text("id")
    declared = _conditions(node.data.get("when", {}), node.at("when"))
    uses = node.node("use", PHASES)
    if not uses.data:
        raise ValueError(f"{uses.path} must contain a phase selection")
    selections = {phase: _selection(item, uses.at(phase), registry) for phase, item in uses.data.items()}
    confidence = node.data.get("confidence")
    if confidence not in CONFIDENCES:
        raise ValueError(f"{node.at('confidence')} must be one of {sorted(CONFIDENCES)}")
    effective = scope.narrowed(declared, node.at("when"))
    return PolicyRule(identifier, effective, selections, confidence, declared)


def _evidence(value: object, path: str) -> EvidenceReference:
    node = _Node(value, path, {"id", "sha256", "file"})
    digest = node.data.get("sha256")
    if not (isinstance(digest, str) and _SHA256.fullmatch(digest)):
        raise ValueError(f"{node.at('sha256')} must be a lowercase SHA-256 hex digest")
    filename = None
    if "file" in node:
        filename = node.text("file")
        plain = PurePosixPath(filename).name == filename and filename not in (".", "..") and "\\" not in filename
        if not plain:
            raise ValueError(f"{node.at('file')} must be a relative evidence filename")
    return EvidenceReference(node.text("id"), digest, filename)


def _unique(items: Sequence[object], key, what: str) -> None:
    seen = [key(item) for item in items]
    if len(set(seen)) != len(seen):
        raise ValueError(f"duplicate {what}")


def _check_header(doc: _Node) -> None:
    """Reject the documents that look like policies but are not v2 policies."""
    data = doc.data
    if data.get("kind") == "mednext-accel-evidence":
        raise ValueError("profiling evidence is not a runtime policy; supply its policy YAML")
    if "schema_version" in data or data.get("version") == 1:
        raise ValueError("schema-v1 profiles are unsupported; migrate to policy v2")
    _Node(data, "policy", _DOCUMENT_FIELDS)
    if type(data.get("version")) is not int or data.get("version") != 2:
        raise ValueError("policy.version must be 2")
    if data.get("kind") != "mednext-accel-policy":
        raise ValueError("policy.kind must be mednext-accel-policy")


def parse_policy(value: Mapping[str, object], *, registry: ImplementationRegistry | None = None) -> OptimizationPolicy:
    """Validate one policy document and return its normalised form."""
    doc = _Node(value, "policy document")
    _check_header(doc)
    registry = registry or default_implementation_registry()
    target = doc.node("target", {"vendor", "sm", "arch"})
    sm = _int_tuple(target.data["sm"], 2, target.at("sm"), least=0) if "sm" in target else None
    arch = target.text("arch") if "arch" in target else None
    scope = _conditions(doc.data.get("scope", {}), "scope")
    narrowing = _Scope(scope)
    rules = tuple(
        _rule(item, f"rules[{i}]", narrowing, registry) for i, item in enumerate(doc.items("rules", default=None))
    )
    _unique(rules, lambda r: r.identifier, "rule id")
    evidence = tuple(_evidence(item, f"evidence[{i}]") for i, item in enumerate(doc.items("evidence")))
    _unique(evidence, lambda e: e.identifier, "evidence id")
    return OptimizationPolicy(
        name=doc.text("name"),
        vendor=_text(target.data.get("vendor"), "target.vendor"),
        target_sm=sm,
        scope=scope,
        rules=rules,
        evidence=evidence,
        target_arch=arch,
    )


# ------------------------------------------------------------------- writing


def _written(condition: Condition) -> object:
    if isinstance(condition, tuple):
        return list(condition)
    if not isinstance(condition, NumericRange):
        return condition
    if condition.minimum == condition.maximum:
        return condition.minimum
    return {key: bound for key, bound in (("min", condition.minimum), ("max", condition.maximum)) if bound is not None}


def _written_selection(selection: PolicySelection) -> dict[str, object]:
    params = selection.parameters
    if params is None:
        return {"implementation": selection.implementation}
    return {"implementation": selection.implementation, "parameters": dict(params) if isinstance(params, Mapping) else params}


def policy_to_primitive(policy: OptimizationPolicy) -> dict[str, object]:
    """The document form of a parsed policy (``parse_policy`` of it gives the
    policy back): plain dicts, lists and scalars, ready for YAML or JSON."""
    target = {"vendor": policy.vendor}
    if policy.target_sm is not None:
        target["sm"] = list(policy.target_sm)
    if policy.target_arch is not None:
        target["arch"] = policy.target_arch
    document: dict[str, object] = {
        "version": policy.version,
        "kind": policy.kind,
        "name": policy.name,
        "target": target,
    }
    if policy.scope:
        document["scope"] = {name: _written(c) for name, c in policy.scope.items()}
    if policy.evidence:
        document["evidence"] = [
            {"id": item.identifier, "sha256": item.sha256} | ({} if item.file is None else {"file": item.file})
            for item in policy.evidence
        ]
    document["rules"] = [
        {
            "id": rule.identifier,
            "when": {name: _written(c) for name, c in rule.declared_when.items()},
            "use": {phase: _written_selection(selection) for phase, selection in rule.use.items()},
            "confidence": rule.confidence,
        }
        for rule in policy.rules
    ]
    return document
