"""Activation checkpointing: which part of each MedNeXt block is recomputed.

``CheckpointConfig(style, stages)`` (the reference's public configuration,
``checkpointing.py``):

* ``style="expansion"`` recomputes each block's expand -> GELU -> project
  branch during backward (the fused expansion here), keeping only its input;
* ``style="block"`` recomputes whole blocks;
* ``stages`` lists the resolution stages covered, 0 (full resolution) to 4
  (the bottleneck); ``None`` covers all five. Stages are kept sorted.
"""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass
from typing import Literal

CheckpointStyle = Literal["expansion", "block"]
STYLES = ("expansion", "block")
STAGE_COUNT = 5  # MedNeXt resolution stages 0..4


def _stage_set(stages: Iterable[object]) -> tuple[int, ...]:
    """Sorted stage indices, or ValueError naming the first problem found."""
    items = tuple(stages)
    problem = None
    if not items:
        problem = "stages must be a non-empty tuple or None"
    elif any(type(s) is not int for s in items):
        problem = "stages must contain only integers"
    elif len(set(items)) < len(items):
        problem = "stages must not contain duplicates"
    elif not all(0 <= s < STAGE_COUNT for s in items):
        problem = f"stages must be between 0 and {STAGE_COUNT - 1}"
    if problem is not None:
        raise ValueError(problem)
    return tuple(sorted(items))


@dataclass(frozen=True, slots=True)
class CheckpointConfig:
    style: CheckpointStyle = "expansion"
    stages: tuple[int, ...] | None = None

    def __post_init__(self) -> None:
        if self.style not in STYLES:
            raise ValueError(f"style must be one of {STYLES}")
        if self.stages is not None:
            object.__setattr__(self, "stages", _stage_set(self.stages))

    def includes(self, stage: int) -> bool:
        """Whether blocks of resolution stage ``stage`` are checkpointed."""
        return self.stages is None or stage in self.stages

    @property
    def checkpoints_expansion(self) -> bool:
        return self.style == "expansion"

    @property
    def checkpoints_blocks(self) -> bool:
        return self.style == "block"
