"""MedNeXt v2 architecture configuration (reference models/config_v2.py:1-97).

The published Base and Wide networks differ only in width (32 vs 64 base
channels): nine block stages of (3, 4, 8, 8, 8, 8, 8, 4, 3) blocks with the
same expansion ratios, down blocks expanding (4, 8, 8, 8) and up blocks
(8, 8, 4, 3), kernel 3 throughout. The stage tables are the paper's
architecture, so they necessarily equal the reference's.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

MedNeXtV2Variant = Literal["base", "wide"]

STAGE_BLOCKS = (3, 4, 8, 8, 8, 8, 8, 4, 3)
STAGE_RATIOS = (3, 4, 8, 8, 8, 8, 8, 4, 3)
DOWN_RATIOS = (4, 8, 8, 8)
UP_RATIOS = (8, 8, 4, 3)
WIDTHS: dict[str, int] = {"base": 32, "wide": 64}

_SEQUENCES = (
    ("block_counts", 9),
    ("expansion_ratios", 9),
    ("downsample_expansion_ratios", 4),
    ("upsample_expansion_ratios", 4),
)


@dataclass(frozen=True, slots=True)
class MedNeXtV2Config:
    """Validated, immutable MedNeXt v2 description; list fields (as YAML gives
    them) are stored as tuples."""

    variant: MedNeXtV2Variant
    in_channels: int
    out_channels: int
    base_channels: int
    kernel_size: int
    block_counts: tuple[int, ...]
    expansion_ratios: tuple[int, ...]
    downsample_expansion_ratios: tuple[int, ...]
    upsample_expansion_ratios: tuple[int, ...]
    deep_supervision: bool = False

    def __post_init__(self) -> None:
        for name, _ in _SEQUENCES:
            object.__setattr__(self, name, tuple(getattr(self, name)))
        if self.variant not in WIDTHS:
            raise ValueError("variant must be 'base' or 'wide'")
        if self.in_channels <= 0 or self.out_channels <= 0:
            raise ValueError("in_channels and out_channels must be positive")
        if self.base_channels <= 0:
            raise ValueError("base_channels must be positive")
        if self.kernel_size != 3:
            raise ValueError("MedNeXt v2 kernel_size must be 3")
        if len(self.block_counts) != 9 or len(self.expansion_ratios) != 9:
            raise ValueError("MedNeXt v2 requires nine block stages")
        if len(self.downsample_expansion_ratios) != 4 or len(self.upsample_expansion_ratios) != 4:
            raise ValueError("MedNeXt v2 requires four downsample and upsample expansion ratios")
        for name, _ in _SEQUENCES:
            # bool is an int subclass; it is rejected like any non-int entry.
            if any(type(value) is not int or value <= 0 for value in getattr(self, name)):
                raise ValueError(f"{name} entries must be positive integers")


def get_mednext_v2_config(
    variant: str, *, in_channels: int, out_channels: int, deep_supervision: bool = False
) -> MedNeXtV2Config:
    """The published MedNeXt v2 Base or Wide configuration."""
    key = variant.lower()
    if key not in WIDTHS:
        raise ValueError(f"unknown MedNeXt v2 variant {variant!r}; expected 'base' or 'wide'")
    return MedNeXtV2Config(
        variant=key,  # type: ignore[arg-type]
        in_channels=in_channels,
        out_channels=out_channels,
        base_channels=WIDTHS[key],
        kernel_size=3,
        block_counts=STAGE_BLOCKS,
        expansion_ratios=STAGE_RATIOS,
        downsample_expansion_ratios=DOWN_RATIOS,
        upsample_expansion_ratios=UP_RATIOS,
        deep_supervision=deep_supervision,
    )
