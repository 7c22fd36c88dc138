"""Operator identities and execution facts the policy layer resolves against.

Field names and meanings follow the reference's ``OperatorDescriptor`` /
``ExecutionContext`` (optimization/descriptors.py:22-156) so that policies and
reports written for it read the same here. One fact is added: ``arch``, the
GPU's ISA name (``gcnArchName`` without feature suffixes, e.g. ``"gfx950"``),
which is what the AMD policy layer keys on; ``sm`` keeps the value
``torch.cuda.get_device_capability`` reports.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from math import prod
from typing import Literal

ExecutionPhase = Literal["training", "inference", "export"]


def _dims(value, name: str, *, minimum: int = 1) -> tuple[int, ...]:
    out = tuple(value)
    if len(out) not in (2, 3) or not all(isinstance(v, int) for v in out):
        raise ValueError(f"{name} must contain two or three integers")
    if any(v < minimum for v in out):
        raise ValueError(f"{name} values must be >= {minimum}")
    return out


@dataclass(frozen=True, slots=True)
class OperatorDescriptor:
    """Shape-independent identity of one optimizable operator (a module instance)."""

    family: str
    direction: str
    in_channels: int
    out_channels: int
    kernel_size: tuple[int, ...] | None = None
    stride: tuple[int, ...] | None = None
    padding: tuple[int, ...] | None = None
    dilation: tuple[int, ...] | None = None
    groups: int | None = None
    role: str | None = None

    def __post_init__(self) -> None:
        if not self.family or not self.direction:
            raise ValueError("family and direction must be non-empty")
        if self.in_channels <= 0 or self.out_channels <= 0:
            raise ValueError("in_channels and out_channels must be positive")
        geometry = (self.kernel_size, self.stride, self.padding, self.dilation, self.groups)
        given = [g is not None for g in geometry]
        if any(given) and not all(given):
            raise ValueError("convolution geometry fields must be supplied together")
        if not any(given):
            return
        if self.groups <= 0:
            raise ValueError("groups must be positive")
        object.__setattr__(self, "kernel_size", _dims(self.kernel_size, "kernel_size"))
        object.__setattr__(self, "stride", _dims(self.stride, "stride"))
        object.__setattr__(self, "padding", _dims(self.padding, "padding", minimum=0))
        object.__setattr__(self, "dilation", _dims(self.dilation, "dilation"))

    @classmethod
    def normalization(cls, *, family: str, channels: int, role: str | None = None) -> OperatorDescriptor:
        return cls(family, "regular", channels, channels, role=role)

    @classmethod
    def convolution(
        cls,
        *,
        family: str,
        direction: str,
        in_channels: int,
        out_channels: int,
        kernel_size: tuple[int, ...],
        stride: tuple[int, ...],
        padding: tuple[int, ...],
        dilation: tuple[int, ...],
        groups: int,
        role: str | None = None,
    ) -> OperatorDescriptor:
        return cls(family, direction, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, role)

    @property
    def signature(self) -> tuple[object, ...]:
        return (self.family, self.direction, self.in_channels, self.out_channels, self.kernel_size, self.stride)

    def to_primitive(self) -> dict[str, object]:
        data = asdict(self)
        for key in ("kernel_size", "stride", "padding", "dilation"):
            if data[key] is not None:
                data[key] = list(data[key])
        if self.kernel_size is None:
            data = {k: v for k, v in data.items() if v is not None}
        return data


@dataclass(frozen=True, slots=True)
class ExecutionContext:
    """Runtime facts one resolution is made for."""

    phase: ExecutionPhase
    device_type: str
    sm: tuple[int, int] | None
    total_vram_bytes: int
    dtype: str
    batch_size: int
    spatial_shape: tuple[int, ...]
    model_family: str
    variant: str
    checkpointing: str
    export: bool = False
    allow_approximate: bool = False
    arch: str | None = None

    def __post_init__(self) -> None:
        if self.phase not in ("training", "inference", "export"):
            raise ValueError(f"unknown phase {self.phase!r}")
        if self.batch_size <= 0:
            raise ValueError("batch_size must be positive")
        if self.total_vram_bytes < 0:
            raise ValueError("total_vram_bytes must be nonnegative")
        object.__setattr__(self, "spatial_shape", _dims(self.spatial_shape, "spatial_shape"))
        if self.sm is not None:
            sm = tuple(self.sm)
            if len(sm) != 2 or any(v < 0 for v in sm):
                raise ValueError("sm must contain two nonnegative integers")
            object.__setattr__(self, "sm", sm)

    @property
    def vendor(self) -> str | None:
        """``"amd"`` when an ISA name is known, ``"nvidia"`` for an SM-only context."""
        if self.device_type != "cuda":
            return None
        if self.arch is not None:
            return "amd"
        return "nvidia" if self.sm is not None else None

    @property
    def spatial_volume(self) -> int:
        return prod(self.spatial_shape)

    @property
    def total_vram_gib(self) -> float:
        return self.total_vram_bytes / 2**30

    def to_primitive(self) -> dict[str, object]:
        data = asdict(self)
        data["spatial_shape"] = list(self.spatial_shape)
        data["sm"] = None if self.sm is None else list(self.sm)
        return data
