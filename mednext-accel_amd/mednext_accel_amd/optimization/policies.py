"""Bundled policies of this build and the registry that layers them
(reference optimization/policies.py:12-31, with the AMD gfx950 policy in place
of the NVIDIA SM tables)."""

from __future__ import annotations

from functools import cache
from pathlib import Path

import yaml

from .policy import OptimizationPolicy, parse_policy
from .policy_io import PolicySource, load_policy
from .policy_resolver import PolicyResolver

POLICY_DIR = Path(__file__).resolve().parent.parent / "policies"
# Layer order: the measured exact-context gfx950 policy (MedNeXt-Base 128^3,
# written by mednext_accel_amd.profiling) before the formula-driven gfx950
# policy, which covers every other context.
BUNDLED = ("gfx950_base128", "gfx950")


@cache
def load_bundled_policy(name: str) -> OptimizationPolicy:
    if name not in BUNDLED:
        raise ValueError(f"unknown bundled policy {name!r}")
    return parse_policy(yaml.safe_load((POLICY_DIR / f"{name}.yaml").read_text(encoding="utf-8")))


class PolicyRegistry:
    def __init__(self, external: PolicySource | None = None) -> None:
        self.external = None if external is None else load_policy(external)
        self.bundled = tuple(load_bundled_policy(name) for name in BUNDLED)

    def resolver(self, *, triton_available: bool | None = None) -> PolicyResolver:
        return PolicyResolver(self.bundled, external=self.external, triton_available=triton_available)
