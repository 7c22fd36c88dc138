"""What the policy layer resolves against: an operator and an execution context.

``OperatorDescriptor`` is the shape-independent identity of one wrapped
module; ``ExecutionContext`` the facts of one call (device, dtype, batch,
spatial shape, model). Their field names are the reference's
(``optimization/descriptors.py``), because policy documents and optimization
reports name them. This build adds ``ExecutionContext.arch``: the GPU's ISA
name (``gcnArchName`` without feature flags, e.g. ``"gfx950"``), on which the
AMD policy layers are keyed. ``sm`` keeps what
``torch.cuda.get_device_capability`` reports.

Both are frozen and hashable (the resolver memoises on them) and both
normalise their geometry tuples on construction.
"""

from __future__ import annotations

from dataclasses import dataclass, fields
from math import prod
from typing import Literal

ExecutionPhase = Literal["training", "inference", "export"]
_PHASES = ("training", "inference", "export")
# Geometry fields of a convolution descriptor and the least value each allows.
_GEOMETRY = (("kernel_size", 1), ("stride", 1), ("padding", 0), ("dilation", 1))


def _spatial(value, name: str, least: int) -> tuple[int, ...]:
    """A 2-D or 3-D integer tuple with every entry >= least."""
    items = tuple(value)
    if len(items) not in (2, 3) or any(not isinstance(v, int) for v in items):
        raise ValueError(f"{name} must contain two or three integers")
    if min(items) < least:
        raise ValueError(f"{name} values must be >= {least}")
    return items


def _primitive(instance) -> dict[str, object]:
    """Field values as JSON-ready primitives (tuples become lists)."""
    out = {}
    for f in fields(instance):
        value = getattr(instance, f.name)
        out[f.name] = list(value) if isinstance(value, tuple) else value
    return out


@dataclass(frozen=True, slots=True)
class OperatorDescriptor:
    """One optimizable operator (a module instance), independent of input shape.

    ``family`` (e.g. ``depthwise_conv3d``, ``pointwise_conv3d``,
    ``group_norm3d``) and ``direction`` (``regular``, ``downsample``,
    ``transpose``) name the operator; convolutions also carry their geometry,
    all of it or none; ``role`` is the module's path in the model."""

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
        if not (self.family and self.direction):
            raise ValueError("family and direction must be non-empty")
        if min(self.in_channels, self.out_channels) <= 0:
            raise ValueError("in_channels and out_channels must be positive")
        present = [getattr(self, name) is not None for name, _ in _GEOMETRY] + [self.groups is not None]
        if not any(present):
            return
        if not all(present):
            raise ValueError("convolution geometry fields must be supplied together")
        if self.groups <= 0:
            raise ValueError("groups must be positive")
        for name, least in _GEOMETRY:
            object.__setattr__(self, name, _spatial(getattr(self, name), name, least))

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
        """What identifies the operator's kernel, without its role."""
        return (self.family, self.direction, self.in_channels, self.out_channels, self.kernel_size, self.stride)

    def to_primitive(self) -> dict[str, object]:
        data = _primitive(self)
        if self.kernel_size is None:  # not a convolution: drop the empty fields
            data = {key: value for key, value in data.items() if value is not None}
        return data


@dataclass(frozen=True, slots=True)
class ExecutionContext:
    """The runtime facts of one call that a policy rule may condition on."""

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
        problems = (
            (self.phase not in _PHASES, f"unknown phase {self.phase!r}"),
            (self.batch_size <= 0, "batch_size must be positive"),
            (self.total_vram_bytes < 0, "total_vram_bytes must be nonnegative"),
        )
        for failed, message in problems:
            if failed:
                raise ValueError(message)
        object.__setattr__(self, "spatial_shape", _spatial(self.spatial_shape, "spatial_shape", 1))
        if self.sm is not None:
            sm = tuple(self.sm)
            if len(sm) != 2 or min(sm) < 0:
                raise ValueError("sm must contain two nonnegative integers")
            object.__setattr__(self, "sm", sm)

    @property
    def vendor(self) -> str | None:
        """``"amd"`` when the ISA name is known, ``"nvidia"`` for an SM-only GPU
        context, None off the GPU."""
        if self.device_type != "cuda":
            return None
        if self.arch is not None:
            return "amd"
        return None if self.sm is None else "nvidia"

    @property
    def spatial_volume(self) -> int:
        return prod(self.spatial_shape)

    @property
    def total_vram_gib(self) -> float:
        return self.total_vram_bytes / 2**30

    def to_primitive(self) -> dict[str, object]:
        return _primitive(self)
