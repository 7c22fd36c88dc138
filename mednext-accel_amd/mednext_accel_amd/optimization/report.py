"""Report of the effective policy layers and per-operator decisions
(reference optimization/report.py)."""

from dataclasses import dataclass

from .descriptors import ExecutionContext
from .policy_resolver import PolicyDecision


@dataclass(frozen=True, slots=True)
class OptimizationReport:
    policies: tuple[str, ...]
    context: ExecutionContext
    decisions: tuple[PolicyDecision, ...]
    warnings: tuple[str, ...] = ()
