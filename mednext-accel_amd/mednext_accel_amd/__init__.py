"""MedNeXt operator path for AMD Instinct MI355X (gfx950).

A drop-in backend for the MedNeXt-Accel operator API: the same model factories,
module names, parameters and state-dict keys, the same ``optimization=`` hook
and policy schema, with the hot operators (depthwise Conv3d fwd/dgrad/wgrad,
GroupNorm(C, C), 1x1x1 pointwise GEMMs with fused GELU / residual epilogues)
running as hand-written HIP kernels from ``libmednext_hip.so``.
"""

from __future__ import annotations

__version__ = "0.1.0"

__all__ = ["__version__"]
