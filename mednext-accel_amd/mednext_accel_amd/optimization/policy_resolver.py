"""Resolve policy layers against one execution context.

Layer order and decision semantics follow the reference's resolver
(optimization/policy_resolver.py:68-231): external policy, then bundled
policies for the exact target, then bundled shared policies of the same
vendor, then the built-in ``reference``; within a layer the first rule that
matches and selects the phase is authoritative; a selection whose guard fails
is remembered and returned (as ``reference`` with the reason) only if no later
layer yields a runnable selection. The vendor is taken from the context: an
AMD context (``arch`` known) sees only ``vendor: amd`` layers, matched on
``target.arch``; an NVIDIA context sees ``vendor: nvidia`` layers, matched on
``target.sm``, exactly as in the reference.
"""

from __future__ import annotations

import warnings
from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from types import MappingProxyType
from typing import Literal

import torch

from .descriptors import ExecutionContext, OperatorDescriptor
from .implementations import ImplementationRegistry, default_implementation_registry
from .parameters import resolve_parameters
from .policy import Confidence, NumericRange, OptimizationPolicy, PolicyRule, PolicySelection


@dataclass(frozen=True, slots=True)
class PolicyDecision:
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


def _facts(descriptor: OperatorDescriptor, context: ExecutionContext) -> dict[str, object]:
    volume = context.spatial_volume
    return {
        "family": descriptor.family,
        "direction": descriptor.direction,
        "role": descriptor.role,
        "kernel_size": descriptor.kernel_size,
        "stride": descriptor.stride,
        "channels": (descriptor.in_channels, descriptor.out_channels),
        "in_channels": descriptor.in_channels,
        "out_channels": descriptor.out_channels,
        "batch": context.batch_size,
        "spatial_shape": context.spatial_shape,
        "spatial_volume": volume,
        "work": context.batch_size * volume * descriptor.in_channels,
        "reduction_work": context.batch_size * volume,
        "total_vram_gib": context.total_vram_gib,
        "dtype": context.dtype,
        "model_family": context.model_family,
        "variant": context.variant,
        "checkpointing": context.checkpointing,
    }


def _matches(rule: PolicyRule, descriptor: OperatorDescriptor, context: ExecutionContext) -> bool:
    facts = _facts(descriptor, context)
    for name, expected in rule.when.items():
        value = facts.get(name)
        if value is None:
            return False
        if isinstance(expected, NumericRange):
            if not expected.contains(value):
                return False
        elif expected != value:
            return False
    return True


def _target_of(policy: OptimizationPolicy) -> object:
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
        self.triton_available = False
        self.bundled = tuple(bundled)
        self.external = external
        self.registry = registry or default_implementation_registry()
        self._warned: set[str] = set()
        # Decisions are pure functions of (descriptor, context, phase) for a
        # fixed set of layers, so they are memoised: wrappers resolve on every
        # forward and this keeps that off the step's critical path.
        self._memo: dict[tuple[OperatorDescriptor, ExecutionContext, str], PolicyDecision] = {}

    def __deepcopy__(self, memo):
        # Policies are immutable; copies of a wrapped model share the resolver
        # (and its warn-once state).
        return self

    def context_layers(self, context: ExecutionContext) -> tuple[OptimizationPolicy, ...]:
        vendor = context.vendor
        if vendor is None:
            return ()
        target = _device_target(context)
        same_vendor = [p for p in self.bundled if p.vendor == vendor]
        external = (self.external,) if self.external is not None and self.external.vendor == vendor else ()
        exact = tuple(p for p in same_vendor if _target_of(p) is not None and _target_of(p) == target)
        shared = tuple(p for p in same_vendor if _target_of(p) is None)
        return external + exact + shared

    def warn_for_target(self, vendor: str | None, target: object) -> str | None:
        """Warn (once, outside compiler tracing) when the external policy names
        another target than the device's (an ``(major, minor)`` SM for NVIDIA,
        an ISA name such as ``"gfx950"`` for AMD)."""
        if self.external is None or vendor is None or target is None:
            return None
        wanted = _target_of(self.external)
        if vendor != self.external.vendor or wanted is None or wanted == target:
            return None
        message = (
            f"policy {self.external.name!r} targets {wanted}, but the current device is {target}; "
            "applying it as requested"
        )
        if not torch.compiler.is_compiling() and message not in self._warned:
            warnings.warn(message, UserWarning, stacklevel=3)
            self._warned.add(message)
        return message

    def warn_for_sm(self, sm: tuple[int, int] | None) -> str | None:
        """The reference's entry point (an NVIDIA capability tuple)."""
        return self.warn_for_target("nvidia" if sm is not None else None, sm)

    def resolve(self, descriptor: OperatorDescriptor, context: ExecutionContext, phase: str) -> PolicyDecision:
        if torch.compiler.is_compiling():
            # Traced once into the graph; the memo is for eager calls.
            return self._resolve(descriptor, context, phase)
        key = (descriptor, context, phase)
        hit = self._memo.get(key)
        if hit is not None:
            return hit
        decision = self._resolve(descriptor, context, phase)
        if len(self._memo) < 65536:
            self._memo[key] = decision
        return decision

    def _resolve(self, descriptor: OperatorDescriptor, context: ExecutionContext, phase: str) -> PolicyDecision:
        if context.vendor is None:
            return PolicyDecision(
                descriptor, phase, "reference", {}, "reference", "context-guard", "guard",
                guard_reason="requires a GPU with a known architecture",
            )
        warning = self.warn_for_target(context.vendor, _device_target(context))
        guarded: PolicyDecision | None = None
        for policy in self.context_layers(context):
            for rule in policy.rules:
                selection = rule.use.get(phase)
                if selection is None or not _matches(rule, descriptor, context):
                    continue
                decision = self._decision(policy, rule, selection, descriptor, context, phase, warning)
                if selection.implementation == "reference" or decision.guard_reason is None:
                    return decision
                if guarded is None:
                    guarded = decision
                break  # first matching rule decides this layer
        if guarded is not None:
            return guarded
        return PolicyDecision(descriptor, phase, "reference", {}, "reference", "fallback", "guard", warning)

    def _guard_reason(self, selection: PolicySelection, descriptor, context, phase: str) -> str | None:
        spec = self.registry.resolve_metadata(selection.implementation)
        if "*" not in spec.families and descriptor.family not in spec.families:
            return "implementation does not support this operator family"
        if phase not in spec.phases:
            return "implementation does not support this phase"
        if (context.export or context.phase == "export" or phase == "export") and not spec.export_safe:
            return "implementation is not export safe"
        if spec.equivalence == "approximate" and not context.allow_approximate:
            return "approximate implementation requires allow_approximate"
        return self.registry.guard(selection.implementation, descriptor, context, phase)

    def _decision(self, policy, rule, selection, descriptor, context, phase, warning) -> PolicyDecision:
        reason = self._guard_reason(selection, descriptor, context, phase)
        parameters: dict[str, object] = {}
        if reason is None:
            try:
                parameters = resolve_parameters(selection, descriptor, context)
            except ValueError as error:
                reason = f"invalid launch parameters: {error}"
        if reason is not None:
            return PolicyDecision(
                descriptor, phase, "reference", {}, policy.name, rule.identifier, "guard", warning, guard_reason=reason
            )
        return PolicyDecision(
            descriptor,
            phase,
            selection.implementation,
            parameters,
            policy.name,
            rule.identifier,
            rule.confidence,
            warning,
            execution_guards=self.registry.execution_guards(selection.implementation),
            disposition="native" if selection.implementation == "reference" else "custom",
        )

    def resolve_all(self, descriptors: Sequence[OperatorDescriptor], context: ExecutionContext, phase: str):
        return tuple(self.resolve(d, context, phase) for d in descriptors)
