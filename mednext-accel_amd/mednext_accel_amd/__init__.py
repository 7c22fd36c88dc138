"""MI355X (gfx950) backend for MedNeXt's operator path.

Hand-written HIP kernels (``csrc/``, built into ``_lib/libmednext_hip.so`` and
called through a C ABI) behind the reference package's operator API: the same
model factories, module wrappers, selection hook and ``torch.library`` ops.
"""

from .adaptive import (
    AdaptiveDepthwise3d,
    AdaptiveGroupNorm3d,
    AdaptivePointwise3d,
    ModelOptimizationContext,
    install_adaptive_operators,
)
from .blocks import EvalModeGELU, MedNeXtBlock, MedNeXtDownBlock, MedNeXtUpBlock, OutputHead
from .checkpointing import CheckpointConfig
from .config import MedNeXtV1Config, get_mednext_v1_config
from .mednext_v1 import MedNeXtV1, mednext_base, mednext_large, mednext_medium, mednext_small
from .optimization import OptimizationReport, PolicyDecision, PolicyRegistry, PolicyResolver

__version__ = "0.1.0"

__all__ = [
    "AdaptiveDepthwise3d",
    "AdaptiveGroupNorm3d",
    "AdaptivePointwise3d",
    "CheckpointConfig",
    "EvalModeGELU",
    "MedNeXtBlock",
    "MedNeXtDownBlock",
    "MedNeXtUpBlock",
    "MedNeXtV1",
    "MedNeXtV1Config",
    "ModelOptimizationContext",
    "OptimizationReport",
    "OutputHead",
    "PolicyDecision",
    "PolicyRegistry",
    "PolicyResolver",
    "get_mednext_v1_config",
    "install_adaptive_operators",
    "mednext_base",
    "mednext_large",
    "mednext_medium",
    "mednext_small",
]
