"""Which implementation runs one operator phase in one execution context.

Policies are consulted as layers, in this order:

1. the external policy (``optimization=<file or mapping>``);
2. bundled policies whose target is exactly the device: ``target.arch`` against
   the AMD ISA name (``gfx950``), or ``target.sm`` against an NVIDIA capability;
3. bundled policies of the device's vendor with no target;
4. the built-in ``reference`` (PyTorch's own operator).

Only layers of the device's vendor apply. Within a layer the first rule that
both selects the phase and matches the operator decides for that layer. A
runnable selection, or an explicit ``reference``, is final. A selection whose
eligibility guard fails is kept as the answer (``reference``, with the guard's
reason) only if no later layer gives a runnable one. These semantics are the
reference's (``optimization/policy_resolver.py``), so a policy document means
the same thing here; the vendor/arch layering is this build's.

Mechanics: the layers for one (vendor, target, phase) are compiled once into
``_Candidate`` lists whose rule conditions are predicates over the operator's
facts, and decisions are memoised, because every wrapper resolves on every
forward. Under ``torch.compile`` nothing is cached: the resolution is traced
into the graph once.
"""

from __future__ import annotations

import operator
import warnings
from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass
from functools import partial
from types import MappingProxyType
from typing import Literal

import torch

from .descriptors import ExecutionContext, OperatorDescriptor
from .implementations import ImplementationRegistry, default_implementation_registry
from .parameters import resolve_parameters
from .policy import Confidence, NumericRange, OptimizationPolicy, PolicyRule, PolicySelection


@dataclass(frozen=True, slots=True)
class PolicyDecision:
    """The outcome for one (operator, context, phase), with its provenance:
    which policy and rule decided, how confident that rule is, and why a guard
    turned a selection into ``reference`` (``guard_reason``)."""

    descriptor: OperatorDescriptor
    phase: str
    implementation: str
    parameters: Mapping[str, object]
    policy: str
    rule: str
    confidence: Confidence
    warning: str | None = None
    guard_reason: str | None = None
    execution_guards: tuple[str, ...] = ()
    disposition: Literal["custom", "native", "unwrapped"] = "native"

    def __post_init__(self) -> None:
        object.__setattr__(self, "parameters", MappingProxyType(dict(self.parameters)))
        object.__setattr__(self, "execution_guards", tuple(self.execution_guards))


# Every fact a rule condition may name, read off the operator and the context.
_FACT_SOURCES: dict[str, Callable[[OperatorDescriptor, ExecutionContext], object]] = dict(
    {
        "family": lambda d, c: d.family,
        "direction": lambda d, c: d.direction,
        "role": lambda d, c: d.role,
        "kernel_size": lambda d, c: d.kernel_size,
        "stride": lambda d, c: d.stride,
        "channels": lambda d, c: (d.in_channels, d.out_channels),
        "in_channels": lambda d, c: d.in_channels,
        "out_channels": lambda d, c: d.out_channels,
        "batch": lambda d, c: c.batch_size,
        "spatial_shape": lambda d, c: c.spatial_shape,
        "spatial_volume": lambda d, c: c.spatial_volume,
        # Problem sizes used to bucket launch recipes (reference policy_resolver.py:39-65).
        "work": lambda d, c: c.batch_size * c.spatial_volume * d.in_channels,
        "reduction_work": lambda d, c: c.batch_size * c.spatial_volume,
        "total_vram_gib": lambda d, c: c.total_vram_gib,
        "dtype": lambda d, c: c.dtype,
        "model_family": lambda d, c: c.model_family,
        "variant": lambda d, c: c.variant,
        "checkpointing": lambda d, c: c.checkpointing,
    }
)


def _facts(descriptor: OperatorDescriptor, context: ExecutionContext) -> dict[str, object]:
    """All facts of one (operator, context), built in one expression (no dict
    is mutated, so the resolution also traces under ``torch.compile``)."""
    return {name: source(descriptor, context) for name, source in _FACT_SOURCES.items()}


def _predicate(rule: PolicyRule) -> Callable[[Mapping[str, object]], bool]:
    """The rule's effective condition as one test over the facts; a fact that
    is unknown (None) fails every condition on it."""
    checks = []
    for name, expected in rule.when.items():
        test = expected.contains if isinstance(expected, NumericRange) else partial(operator.eq, expected)
        checks.append((name, test))

    def matches(facts: Mapping[str, object]) -> bool:
        for name, test in checks:
            value = facts.get(name)
            if value is None or not test(value):
                return False
        return True

    return matches


@dataclass(frozen=True, slots=True)
class _Candidate:
    policy: OptimizationPolicy
    rule: PolicyRule
    selection: PolicySelection
    matches: Callable[[Mapping[str, object]], bool]


def _policy_target(policy: OptimizationPolicy) -> object:
    return policy.target_arch if policy.vendor == "amd" else policy.target_sm


def _device_target(context: ExecutionContext) -> object:
    return context.arch if context.vendor == "amd" else context.sm


class PolicyResolver:
    """External -> exact target -> shared (same vendor) -> built-in reference."""

    def __init__(
        self,
        bundled: Sequence[OptimizationPolicy] = (),
        *,
        external: OptimizationPolicy | None = None,
        registry: ImplementationRegistry | None = None,
        triton_available: bool | None = None,
    ) -> None:
        # No Triton backend is part of this build, whatever the caller asks.
        del triton_available
        self.triton_available = False
        self.bundled = tuple(bundled)
        self.external = external
        self.registry = registry or default_implementation_registry()
        self._warned: set[str] = set()
        self._compiled: dict[tuple[str, object, str], tuple[tuple[_Candidate, ...], ...]] = {}
        self._memo: dict[tuple[OperatorDescriptor, ExecutionContext, str], PolicyDecision] = {}

    def __deepcopy__(self, memo):
        # Immutable policies: copies of a wrapped model share one resolver
        # (and its warn-once record).
        return self

    # ------------------------------------------------------------ layers

    def context_layers(self, context: ExecutionContext) -> tuple[OptimizationPolicy, ...]:
        """The policies that apply to ``context``, in consultation order."""
        vendor = context.vendor
        if vendor is None:
            return ()
        device = _device_target(context)
        mine = [p for p in self.bundled if p.vendor == vendor]
        ordered = [self.external] if self.external is not None and self.external.vendor == vendor else []
        ordered += [p for p in mine if _policy_target(p) is not None and _policy_target(p) == device]
        ordered += [p for p in mine if _policy_target(p) is None]
        return tuple(ordered)

    def _layers_for(self, context: ExecutionContext, phase: str) -> tuple[tuple[_Candidate, ...], ...]:
        key = (context.vendor, _device_target(context), phase)
        layers = None if torch.compiler.is_compiling() else self._compiled.get(key)
        if layers is None:
            layers = tuple(
                tuple(
                    _Candidate(policy, rule, rule.use[phase], _predicate(rule))
                    for rule in policy.rules
                    if phase in rule.use
                )
                for policy in self.context_layers(context)
            )
            if not torch.compiler.is_compiling():
                self._compiled[key] = layers
        return layers

    # ------------------------------------------------------------ warnings

    def warn_for_target(self, vendor: str | None, target: object) -> str | None:
        """Warn once (never while the compiler traces) when the external policy
        targets a device other than this one (an ``(major, minor)`` SM for
        NVIDIA, an ISA name such as ``"gfx950"`` for AMD); the policy is
        applied anyway."""
        external = self.external
        if external is None or vendor is None or target is None or vendor != external.vendor:
            return None
        wanted = _policy_target(external)
        if wanted is None or wanted == target:
            return None
        message = f"policy {external.name!r} targets {wanted}, but the current device is {target}; applying it as requested"
        if message not in self._warned and not torch.compiler.is_compiling():
            self._warned.add(message)
            warnings.warn(message, UserWarning, stacklevel=3)
        return message

    def warn_for_sm(self, sm: tuple[int, int] | None) -> str | None:
        """The reference's entry point (an NVIDIA capability tuple)."""
        return self.warn_for_target(None if sm is None else "nvidia", sm)

    # ------------------------------------------------------------ resolution

    def resolve(self, descriptor: OperatorDescriptor, context: ExecutionContext, phase: str) -> PolicyDecision:
        if torch.compiler.is_compiling():
            return self._resolve(descriptor, context, phase)  # traced once into the graph
        key = (descriptor, context, phase)
        decision = self._memo.get(key)
        if decision is None:
            decision = self._resolve(descriptor, context, phase)
            if len(self._memo) < 65536:
                self._memo[key] = decision
        return decision

    def resolve_all(self, descriptors: Sequence[OperatorDescriptor], context: ExecutionContext, phase: str):
        return tuple(self.resolve(d, context, phase) for d in descriptors)

    def _resolve(self, descriptor: OperatorDescriptor, context: ExecutionContext, phase: str) -> PolicyDecision:
        if context.vendor is None:
            return self._reference(descriptor, phase, "reference", "context-guard", None,
                                   "requires a GPU with a known architecture")
        warning = self.warn_for_target(context.vendor, _device_target(context))
        facts = _facts(descriptor, context)
        fallback: PolicyDecision | None = None
        for layer in self._layers_for(context, phase):
            hit = next((c for c in layer if c.matches(facts)), None)
            if hit is None:
                continue
            decision = self._decide(hit, descriptor, context, phase, warning)
            if decision.guard_reason is None or hit.selection.implementation == "reference":
                return decision
            fallback = fallback or decision
        return fallback or self._reference(descriptor, phase, "reference", "fallback", warning, None)

    @staticmethod
    def _reference(descriptor, phase, policy: str, rule: str, warning, reason) -> PolicyDecision:
        return PolicyDecision(descriptor, phase, "reference", {}, policy, rule, "guard", warning, guard_reason=reason)

    def _ineligible(self, selection: PolicySelection, descriptor, context, phase: str) -> str | None:
        """Why ``selection`` cannot run this operator phase (None: it can)."""
        spec = self.registry.resolve_metadata(selection.implementation)
        exporting = context.export or context.phase == "export" or phase == "export"
        reasons = (
            ("*" not in spec.families and descriptor.family not in spec.families,
             "implementation does not support this operator family"),
            (phase not in spec.phases, "implementation does not support this phase"),
            (exporting and not spec.export_safe, "implementation is not export safe"),
            (spec.equivalence == "approximate" and not context.allow_approximate,
             "approximate implementation requires allow_approximate"),
        )
        for failed, reason in reasons:
            if failed:
                return reason
        return self.registry.guard(selection.implementation, descriptor, context, phase)

    def _decide(self, hit: _Candidate, descriptor, context, phase: str, warning) -> PolicyDecision:
        selection = hit.selection
        reason = self._ineligible(selection, descriptor, context, phase)
        parameters: Mapping[str, object] = {}
        if reason is None:
            try:
                parameters = resolve_parameters(selection, descriptor, context)
            except ValueError as error:
                reason = f"invalid launch parameters: {error}"
        if reason is not None:
            return self._reference(descriptor, phase, hit.policy.name, hit.rule.identifier, warning, reason)
        native = selection.implementation == "reference"
        return PolicyDecision(
            descriptor,
            phase,
            selection.implementation,
            parameters,
            hit.policy.name,
            hit.rule.identifier,
            hit.rule.confidence,
            warning,
            execution_guards=self.registry.execution_guards(selection.implementation),
            disposition="native" if native else "custom",
        )
