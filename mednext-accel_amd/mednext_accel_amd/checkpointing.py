"""Activation-checkpointing selection (reference checkpointing.py:11-48).

``style="expansion"`` recomputes each block's expand -> GELU -> project branch
in backward; ``style="block"`` recomputes whole blocks. ``stages=None`` covers
all five resolution stages, otherwise the given subset of 0..4.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

CheckpointStyle = Literal["expansion", "block"]


@dataclass(frozen=True, slots=True)
class CheckpointConfig:
    style: CheckpointStyle = "expansion"
    stages: tuple[int, ...] | None = None

    def __post_init__(self) -> None:
        if self.style not in ("expansion", "block"):
            raise ValueError("style must be 'expansion' or 'block'")
        if self.stages is None:
            return
        stages = self.stages
        if not stages:
            raise ValueError("stages must be a non-empty tuple or None")
        if not all(type(s) is int for s in stages):
            raise ValueError("stages must contain only integers")
        if len(set(stages)) != len(stages):
            raise ValueError("stages must not contain duplicates")
        if not all(0 <= s <= 4 for s in stages):
            raise ValueError("stages must be between 0 and 4")
        object.__setattr__(self, "stages", tuple(sorted(stages)))

    def includes(self, stage: int) -> bool:
        return self.stages is None or stage in self.stages

    @property
    def checkpoints_expansion(self) -> bool:
        return self.style == "expansion"

    @property
    def checkpoints_blocks(self) -> bool:
        return self.style == "block"
