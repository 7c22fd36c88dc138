"""MedNeXt v1 architecture configuration (reference models/config.py:11-98).

The per-variant tables are the published MedNeXt v1 architectures: nine block
stages (4 encoder, bottleneck, 4 decoder) with block counts and expansion
ratios per stage. The downsampling blocks use ratios[1:5] ("official"
checkpoint layout) or ratios[:4] ("monai").
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

MedNeXtVariant = Literal["small", "base", "medium", "large"]
CompatibilityFamily = Literal["official", "monai"]

VARIANTS: dict[str, tuple[tuple[int, ...], tuple[int, ...]]] = {
    # variant: (block counts, expansion ratios), stages 0..8
    "small": ((2,) * 9, (2,) * 9),
    "base": ((2,) * 9, (2, 3, 4, 4, 4, 4, 4, 3, 2)),
    "medium": ((3, 4, 4, 4, 4, 4, 4, 4, 3), (2, 3, 4, 4, 4, 4, 4, 3, 2)),
    "large": ((3, 4, 8, 8, 8, 8, 8, 4, 3), (3, 4, 8, 8, 8, 8, 8, 4, 3)),
}


@dataclass(frozen=True, slots=True)
class MedNeXtV1Config:
    variant: MedNeXtVariant
    spatial_dims: Literal[2, 3]
    in_channels: int
    out_channels: int
    kernel_size: int
    base_channels: int
    block_counts: tuple[int, ...]
    expansion_ratios: tuple[int, ...]
    downsample_expansion_ratios: tuple[int, ...]
    compatibility: CompatibilityFamily
    residual_blocks: bool = True
    residual_resampling: bool = True
    deep_supervision: bool = False

    def __post_init__(self) -> None:
        if self.spatial_dims not in (2, 3):
            raise ValueError("spatial_dims must be 2 or 3")
        if min(self.in_channels, self.out_channels) <= 0:
            raise ValueError("in_channels and out_channels must be positive")
        if self.base_channels <= 0:
            raise ValueError("base_channels must be positive")
        if self.kernel_size <= 0 or self.kernel_size % 2 == 0:
            raise ValueError("kernel_size must be a positive odd integer")
        if len(self.block_counts) != 9 or len(self.expansion_ratios) != 9:
            raise ValueError("MedNeXt v1 requires nine block stages")
        if len(self.downsample_expansion_ratios) != 4:
            raise ValueError("MedNeXt v1 requires four downsample expansion ratios")


def get_mednext_v1_config(
    variant: str,
    *,
    in_channels: int,
    out_channels: int,
    spatial_dims: Literal[2, 3] = 3,
    kernel_size: int = 3,
    base_channels: int = 32,
    deep_supervision: bool = False,
    compatibility: CompatibilityFamily = "official",
) -> MedNeXtV1Config:
    name = variant.lower()
    if name not in VARIANTS:
        raise ValueError(f"unknown MedNeXt v1 variant {variant!r}; expected one of {', '.join(VARIANTS)}")
    if compatibility not in ("official", "monai"):
        raise ValueError("compatibility must be 'official' or 'monai'")
    blocks, ratios = VARIANTS[name]
    down = ratios[1:5] if compatibility == "official" else ratios[:4]
    return MedNeXtV1Config(
        variant=name,  # type: ignore[arg-type]
        spatial_dims=spatial_dims,
        in_channels=in_channels,
        out_channels=out_channels,
        kernel_size=kernel_size,
        base_channels=base_channels,
        block_counts=blocks,
        expansion_ratios=ratios,
        downsample_expansion_ratios=down,
        compatibility=compatibility,
        deep_supervision=deep_supervision,
    )
