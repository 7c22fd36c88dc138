"""Registry of selectable operator implementations (identifier -> metadata + guard).

The registry's shape follows the reference's (optimization/implementations.py:
87-158): an ``ImplementationSpec`` per stable identifier, an optional
eligibility guard returning a reason string, and the execution-time guards the
wrapper checks on the tensor. The HIP implementations of this package are the
``hip_*`` identifiers. The reference's own identifiers stay registered so that
policy documents written for it still parse: ``reference`` and
``pointwise_gemm_per_sample`` run as there (PyTorch ops), and the Triton ones
always resolve to ``reference`` because no Triton backend is part of this build.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from functools import partial
from typing import TYPE_CHECKING, Literal

if TYPE_CHECKING:
    from .descriptors import ExecutionContext, OperatorDescriptor

SemanticEquivalence = Literal["exact", "numerical", "approximate"]
EligibilityGuard = Callable[["OperatorDescriptor", "ExecutionContext", str], "str | None"]

HIP_DEPTHWISE_KERNELS = (1, 3, 5)
HIP_DTYPES = ("bfloat16", "float16", "float32", "float64")
_TENSOR_GUARDS = ("grad_enabled", "rank_5", "contiguous")


@dataclass(frozen=True, slots=True)
class ImplementationSpec:
    identifier: str
    version: int
    families: tuple[str, ...]
    phases: tuple[str, ...]
    equivalence: SemanticEquivalence
    export_safe: bool

    def __post_init__(self) -> None:
        object.__setattr__(self, "families", tuple(self.families))
        object.__setattr__(self, "phases", tuple(self.phases))
        if not self.identifier or self.version <= 0:
            raise ValueError("implementation identifier and version must be valid")
        if not self.families or not self.phases:
            raise ValueError("implementation families and phases must not be empty")
        if self.equivalence not in ("exact", "numerical", "approximate"):
            raise ValueError(f"unknown equivalence {self.equivalence!r}")

    def is_allowed(self, *, allow_approximate: bool, export: bool = False) -> bool:
        approximate_ok = self.equivalence != "approximate" or allow_approximate
        return approximate_ok and (self.export_safe or not export)


class ImplementationRegistry:
    def __init__(self) -> None:
        self._specs: dict[str, ImplementationSpec] = {}
        self._guards: dict[str, EligibilityGuard | None] = {}
        self._execution_guards: dict[str, tuple[str, ...]] = {}

    def register(
        self,
        spec: ImplementationSpec,
        *,
        eligibility: EligibilityGuard | None = None,
        execution_guards: tuple[str, ...] = (),
    ) -> None:
        if spec.identifier in self._specs:
            raise ValueError(f"implementation {spec.identifier!r} is already registered")
        self._specs[spec.identifier] = spec
        self._guards[spec.identifier] = eligibility
        self._execution_guards[spec.identifier] = tuple(execution_guards)

    def resolve_metadata(self, identifier: str) -> ImplementationSpec:
        spec = self._specs.get(identifier)
        if spec is None:
            raise ValueError(f"unknown implementation {identifier!r}")
        return spec

    def guard(self, identifier: str, descriptor, context, phase: str) -> str | None:
        self.resolve_metadata(identifier)
        check = self._guards[identifier]
        return None if check is None else check(descriptor, context, phase)

    def execution_guards(self, identifier: str) -> tuple[str, ...]:
        self.resolve_metadata(identifier)
        return self._execution_guards[identifier]

    def __contains__(self, identifier: object) -> bool:
        return identifier in self._specs

    def __iter__(self):
        return iter(self._specs.values())


def _training_gpu(context, *, amd: bool) -> str | None:
    if context.phase != "training":
        return "implementation requires training"
    if context.device_type != "cuda":
        return "implementation requires a GPU"
    if amd and context.vendor != "amd":
        return "implementation requires an AMD GPU"
    if context.dtype not in HIP_DTYPES:
        return "implementation does not support this dtype"
    return None


def _hip_depthwise(descriptor, context, phase: str) -> str | None:
    reason = _training_gpu(context, amd=True)
    if reason is not None:
        return reason
    k = descriptor.kernel_size
    if (
        k is None
        or descriptor.direction != "regular"
        or k != (k[0],) * 3
        or k[0] not in HIP_DEPTHWISE_KERNELS
        or descriptor.stride != (1, 1, 1)
        or descriptor.padding != (k[0] // 2,) * 3
        or descriptor.dilation != (1, 1, 1)
        or not descriptor.groups == descriptor.in_channels == descriptor.out_channels
    ):
        return "implementation does not support this geometry"
    if len(context.spatial_shape) != 3:
        return "implementation requires a 3D input"
    return None


def _hip_depthwise_stride2(descriptor, context, phase: str, *, direction: str) -> str | None:
    reason = _training_gpu(context, amd=True)
    if reason is not None:
        return reason
    k = descriptor.kernel_size
    if (
        k is None
        or descriptor.direction != direction
        or k != (k[0],) * 3
        or k[0] not in HIP_DEPTHWISE_KERNELS
        or descriptor.stride != (2, 2, 2)
        or descriptor.padding != (k[0] // 2,) * 3
        or descriptor.dilation != (1, 1, 1)
        or not descriptor.groups == descriptor.in_channels == descriptor.out_channels
    ):
        return "implementation does not support this geometry"
    return None


def _hip_group_norm(descriptor, context, phase: str) -> str | None:
    reason = _training_gpu(context, amd=True)
    if reason is not None:
        return reason
    if descriptor.in_channels != descriptor.out_channels:
        return "implementation requires groups == channels"
    return None


def _pointwise_geometry(descriptor) -> bool:
    """1x1x1 convolution: stride 1 (``regular``), stride 2 (``downsample``, the
    GEMM on every second voxel), or a 1x1x1 ConvTranspose3d at stride 1 or 2
    (``transpose``, the same product with the weight read transposed)."""
    stride_ok = descriptor.stride == (1, 1, 1) or (
        descriptor.stride == (2, 2, 2) and descriptor.direction in ("downsample", "transpose")
    )
    return (
        descriptor.direction in ("regular", "downsample", "transpose")
        and descriptor.kernel_size == (1, 1, 1)
        and stride_ok
        and descriptor.padding == (0, 0, 0)
        and descriptor.dilation == (1, 1, 1)
        and descriptor.groups == 1
    )


def _hip_pointwise(descriptor, context, phase: str) -> str | None:
    reason = _training_gpu(context, amd=True)
    if reason is not None:
        return reason
    if context.dtype != "bfloat16":
        return "implementation requires bfloat16"
    if not _pointwise_geometry(descriptor):
        return "implementation does not support this geometry"
    return None


def _hip_expansion(descriptor, context, phase: str) -> str | None:
    reason = _training_gpu(context, amd=True)
    if reason is not None:
        return reason
    if context.dtype != "bfloat16":
        return "implementation requires bfloat16"
    return None


def _hip_grn(descriptor, context, phase: str) -> str | None:
    """Training GRN on an AMD GPU over half-precision activations, the input
    contract of the reference's fused GRN (optimization/implementations.py:18-33)."""
    reason = _training_gpu(context, amd=True)
    if reason is not None:
        return reason
    if phase != "training":
        return "implementation requires training"
    if context.dtype not in ("float16", "bfloat16"):
        return "implementation does not support this dtype"
    return None


def _pointwise_gemm(descriptor, context, phase: str) -> str | None:
    if context.phase != "training":
        return "implementation requires training"
    if context.dtype not in ("bfloat16", "float16", "float32"):
        return "implementation does not support this dtype"
    if (
        descriptor.direction != "regular"
        or descriptor.kernel_size != (1, 1, 1)
        or descriptor.stride != (1, 1, 1)
        or descriptor.padding != (0, 0, 0)
        or descriptor.dilation != (1, 1, 1)
        or descriptor.groups != 1
    ):
        return "implementation does not support this geometry"
    return None


def _no_triton(descriptor, context, phase: str) -> str | None:
    return "Triton backend is not part of this build"


_ALL_PHASES = ("training", "inference", "export", "forward", "backward_input", "backward_weight", "backward_bias")
_DW_GUARDS = (*_TENSOR_GUARDS, "zero_output_padding")


def default_implementation_registry(*, triton_available: bool | None = None) -> ImplementationRegistry:
    """All identifiers this build knows. ``triton_available`` is accepted for
    signature compatibility with the reference and ignored."""
    del triton_available
    registry = ImplementationRegistry()
    table = (
        # identifier, families, phases, equivalence, export_safe, guard, execution guards
        ("reference", ("*",), _ALL_PHASES, "exact", True, None, ()),
        ("hip_depthwise_fwd", ("depthwise_conv3d",), ("forward",), "numerical", False, _hip_depthwise, _DW_GUARDS),
        ("hip_depthwise_dx", ("depthwise_conv3d",), ("backward_input",), "numerical", False, _hip_depthwise, _DW_GUARDS),
        ("hip_split_dw", ("depthwise_conv3d",), ("backward_weight",), "numerical", False, _hip_depthwise, _DW_GUARDS),
        ("hip_depthwise_stride2", ("depthwise_conv3d",), ("forward", "backward_input", "backward_weight"), "numerical", False, partial(_hip_depthwise_stride2, direction="downsample"), _DW_GUARDS),
        ("hip_depthwise_transpose2", ("depthwise_conv_transpose3d",), ("forward", "backward_input", "backward_weight"), "numerical", False, partial(_hip_depthwise_stride2, direction="transpose"), _DW_GUARDS),
        ("hip_group_norm", ("group_norm3d",), ("training",), "numerical", False, _hip_group_norm, _TENSOR_GUARDS),
        ("hip_pointwise_gemm", ("pointwise_conv3d", "conv_transpose3d"), ("training",), "numerical", False, _hip_pointwise, (*_TENSOR_GUARDS, "channels_supported")),
        ("hip_fused_expansion", ("mlp_expansion3d",), ("training",), "numerical", False, _hip_expansion, (*_TENSOR_GUARDS, "channels_supported")),
        ("hip_fused_grn", ("global_response_norm3d",), ("training",), "numerical", False, _hip_grn, _TENSOR_GUARDS),
        ("hip_fused_grn_expansion", ("grn_expansion3d",), ("training",), "numerical", False, _hip_expansion, (*_TENSOR_GUARDS, "channels_supported")),
        ("pointwise_gemm_per_sample", ("pointwise_conv3d",), ("training",), "numerical", False, _pointwise_gemm, _TENSOR_GUARDS),
        ("triton_depthwise_dx", ("depthwise_conv3d",), ("backward_input",), "numerical", False, _no_triton, _DW_GUARDS),
        ("triton_split_dw", ("depthwise_conv3d",), ("backward_weight",), "numerical", False, _no_triton, _DW_GUARDS),
        ("triton_transpose_split_dw", ("depthwise_conv_transpose3d",), ("backward_weight",), "numerical", False, _no_triton, _DW_GUARDS),
        ("triton_downsample_dx", ("depthwise_conv3d",), ("backward_input",), "numerical", False, _no_triton, _DW_GUARDS),
        ("triton_fused_grn", ("global_response_norm3d",), ("training",), "numerical", False, _no_triton, _TENSOR_GUARDS),
        ("gelu_tanh", ("gelu",), ("inference",), "approximate", True, None, ()),
    )
    for identifier, families, phases, equivalence, export_safe, guard, execution in table:
        registry.register(
            ImplementationSpec(identifier, 1, families, phases, equivalence, export_safe),
            eligibility=guard,
            execution_guards=execution,
        )
    return registry
