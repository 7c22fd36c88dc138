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
from .blocks_v2 import MedNeXtV2Block, MedNeXtV2DownBlock, MedNeXtV2UpBlock
from .checkpointing import CheckpointConfig
from .config import MedNeXtV1Config, get_mednext_v1_config
from .config_v2 import MedNeXtV2Config, get_mednext_v2_config
from .grn import (
    AdaptiveGlobalResponseNorm3d,
    GlobalResponseNorm3d,
    global_response_norm3d_reference,
    install_adaptive_grn,
)
from .mednext_v1 import MedNeXtV1, mednext_base, mednext_large, mednext_medium, mednext_small
from .mednext_v2 import MedNeXtV2, mednext_v2_base, mednext_v2_wide
from .optimization import OptimizationReport, PolicyDecision, PolicyRegistry, PolicyResolver

__version__ = "0.1.0"

__all__ = [
    "AdaptiveDepthwise3d",
    "AdaptiveGlobalResponseNorm3d",
    "AdaptiveGroupNorm3d",
    "AdaptivePointwise3d",
    "CheckpointConfig",
    "EvalModeGELU",
    "GlobalResponseNorm3d",
    "MedNeXtBlock",
    "MedNeXtDownBlock",
    "MedNeXtUpBlock",
    "MedNeXtV1",
    "MedNeXtV1Config",
    "MedNeXtV2",
    "MedNeXtV2Block",
    "MedNeXtV2Config",
    "MedNeXtV2DownBlock",
    "MedNeXtV2UpBlock",
    "ModelOptimizationContext",
    "OptimizationReport",
    "OutputHead",
    "PolicyDecision",
    "PolicyRegistry",
    "PolicyResolver",
    "get_mednext_v1_config",
    "get_mednext_v2_config",
    "global_response_norm3d_reference",
    "install_adaptive_grn",
    "install_adaptive_operators",
    "mednext_base",
    "mednext_large",
    "mednext_medium",
    "mednext_small",
    "mednext_v2_base",
    "mednext_v2_wide",
]
