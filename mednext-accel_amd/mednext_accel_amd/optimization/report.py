"""What the selection hook decided for a model, in one inspectable object.

``MedNeXtV1.explain_optimization`` / ``MedNeXtV2.explain_optimization`` return
an ``OptimizationReport``: the policy layers that applied (in consultation
order), the execution context the decisions were made for, one
``PolicyDecision`` per (operator, phase) -- including operators that run
PyTorch's own implementation and modules that were never wrapped -- and the
warnings raised on the way. The first four fields are the reference's report
(``optimization/report.py``); the helpers below are this build's.
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass

from .descriptors import ExecutionContext
from .policy_resolver import PolicyDecision


@dataclass(frozen=True, slots=True)
class OptimizationReport:
    policies: tuple[str, ...]
    context: ExecutionContext
    decisions: tuple[PolicyDecision, ...]
    warnings: tuple[str, ...] = ()

    def implementations(self) -> dict[str, int]:
        """How many (operator, phase) decisions chose each implementation."""
        return dict(Counter(d.implementation for d in self.decisions))

    def custom(self) -> tuple[PolicyDecision, ...]:
        """The decisions that run one of this package's kernels."""
        return tuple(d for d in self.decisions if d.disposition == "custom")

    def guarded(self) -> tuple[PolicyDecision, ...]:
        """Selections a guard turned into ``reference``, with their reasons."""
        return tuple(d for d in self.decisions if d.guard_reason is not None)

    def to_primitive(self) -> dict[str, object]:
        """A JSON-ready form (for logs and experiment records)."""
        return {
            "policies": list(self.policies),
            "context": self.context.to_primitive(),
            "decisions": [
                {
                    "operator": d.descriptor.to_primitive(),
                    "phase": d.phase,
                    "implementation": d.implementation,
                    "parameters": dict(d.parameters),
                    "policy": d.policy,
                    "rule": d.rule,
                    "confidence": d.confidence,
                    "disposition": d.disposition,
                    "guard_reason": d.guard_reason,
                }
                for d in self.decisions
            ],
            "warnings": list(self.warnings),
        }
