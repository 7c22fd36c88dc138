"""Implementation selection: descriptors, registry, launch recipes, policies, resolver."""

from .descriptors import ExecutionContext, OperatorDescriptor
from .implementations import ImplementationRegistry, ImplementationSpec, default_implementation_registry
from .policies import PolicyRegistry, load_bundled_policy
from .policy import OptimizationPolicy, PolicyRule, PolicySelection, parse_policy, policy_to_primitive
from .policy_io import load_policy
from .policy_resolver import PolicyDecision, PolicyResolver
from .report import OptimizationReport

__all__ = [
    "ExecutionContext",
    "ImplementationRegistry",
    "ImplementationSpec",
    "OperatorDescriptor",
    "OptimizationPolicy",
    "OptimizationReport",
    "PolicyDecision",
    "PolicyRegistry",
    "PolicyResolver",
    "PolicyRule",
    "PolicySelection",
    "default_implementation_registry",
    "load_bundled_policy",
    "load_policy",
    "parse_policy",
    "policy_to_primitive",
]
