"""gfx950 profiler and policy generator.

The method of the reference's ``profiling`` package (integrated per-phase
measurement through the adaptive module interface, relative-L2 validation,
policy synthesis from the measurements), restated for this build's HIP
implementations and launch recipes:

* ``matrix.build_workload_cases``: the operator contexts of a MedNeXt variant
  and the candidate (implementation, recipe) pairs per phase;
* ``operator_benchmark.benchmark_operator``: validate and time one candidate
  against the native module on the GPU;
* ``validation.validate_components``: component relative-L2 check;
* ``synthesize.synthesize_policy``: fastest valid candidate per context ->
  a policy v2 document for the current device;
* ``api.profile``: the whole campaign, optionally written to YAML + JSON.

Run ``python -m mednext_accel_amd.profiling --help`` on a GPU box to
regenerate the bundled gfx950 policy for the installed ROCm / driver stack.
"""

from .matrix import KernelCase, build_workload_cases
from .synthesize import Measurement, synthesize_policy
from .validation import RELATIVE_L2_LIMIT, validate_components

__all__ = [
    "KernelCase",
    "Measurement",
    "RELATIVE_L2_LIMIT",
    "build_workload_cases",
    "synthesize_policy",
    "validate_components",
]
