"""Policy-driven module wrappers that keep the native modules' Parameters and keys.

Mirrors the reference's selection hook (ops/adaptive.py:15-376):
``install_adaptive_operators`` swaps eligible children in place for wrappers
that hold the *same* ``Parameter`` objects, so ``parameters()`` and
``state_dict()`` keys are unchanged; each wrapper resolves, per forward, which
implementation runs from the execution context (phase, device, autocast dtype,
shape) through a ``PolicyResolver``.

Routes:
  * ``AdaptiveDepthwise3d``: forward / dX / dW each resolve independently; any
    HIP selection runs the ``mednext_accel_amd::depthwise_conv3d_odd_regular``
    op with the per-phase launch recipes, with native PyTorch for phases that
    resolve to ``reference``. Stride-2 and transposed depthwise convolutions run
    natively.
  * ``AdaptivePointwise3d``: ``pointwise_gemm_per_sample`` (the reference's
    per-sample ``addmm`` route) or native ``F.conv3d``.
  * ``AdaptiveGroupNorm3d`` (new; the reference has no GroupNorm hook): the HIP
    GroupNorm(C, C) op or native ``F.group_norm``. Under autocast it returns
    float32 like autocast's float32 ``group_norm``.

Unsupported inputs (CPU tensors, evaluation, non-contiguous, ...) take the
native PyTorch route, as in the reference; so does every HIP selection when
``libmednext_hip.so`` cannot be loaded (``_hip_ops``), with one warning.
"""

from __future__ import annotations

import functools
import os
import warnings
from dataclasses import dataclass

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from .optimization.descriptors import ExecutionContext, OperatorDescriptor
from .optimization.policy_resolver import PolicyDecision, PolicyResolver
from .precast import cast_param, precast_or_param
from .tiles import ENGINE_MFMA


@dataclass(frozen=True, slots=True)
class ModelOptimizationContext:
    family: str
    variant: str
    checkpointing: str
    allow_approximate: bool = False


def _dtype_name(dtype: torch.dtype | str) -> str:
    return str(dtype).removeprefix("torch.")


def _query_device(index: int) -> tuple[tuple[int, int], int, str | None]:
    props = torch.cuda.get_device_properties(index)
    arch = getattr(props, "gcnArchName", None) if torch.version.hip else None
    if arch:
        arch = arch.split(":")[0]
    return torch.cuda.get_device_capability(index), int(props.total_memory), arch or None


_cached_device = functools.lru_cache(maxsize=None)(_query_device)


def device_facts(index: int) -> tuple[tuple[int, int], int, str | None]:
    """(capability, total memory, ISA name or None) of one GPU. Cached in eager
    mode (queried once per device); queried directly while torch.compile traces."""
    if torch.compiler.is_compiling():
        return _query_device(index)
    return _cached_device(index)


def execution_context_for_shape(
    model_context: ModelOptimizationContext,
    *,
    batch_size: int,
    spatial_shape: tuple[int, ...],
    dtype: torch.dtype | str,
    device_type: str,
    sm: tuple[int, int] | None,
    total_vram_bytes: int,
    training: bool = True,
    export: bool = False,
    arch: str | None = None,
) -> ExecutionContext:
    return ExecutionContext(
        phase="export" if export else ("training" if training else "inference"),
        device_type=device_type,
        sm=sm,
        total_vram_bytes=total_vram_bytes,
        dtype=_dtype_name(dtype),
        batch_size=batch_size,
        spatial_shape=spatial_shape,
        model_family=model_context.family,
        variant=model_context.variant,
        checkpointing=model_context.checkpointing,
        export=export,
        allow_approximate=model_context.allow_approximate,
        arch=arch,
    )


def _effective_dtype(x: Tensor) -> torch.dtype:
    device = x.device.type
    if torch.is_autocast_enabled(device) and x.dtype != torch.float64:
        return torch.get_autocast_dtype(device)
    return x.dtype


_CONTEXTS: dict[tuple, ExecutionContext] = {}


def _context_from_tensor(x: Tensor, model_context: ModelOptimizationContext, *, training: bool) -> ExecutionContext:
    export = torch.jit.is_tracing() or torch.onnx.is_in_onnx_export()
    if not export and not torch.compiler.is_compiling():
        # Contexts are immutable and depend only on these facts: build each once.
        key = (model_context, tuple(x.shape), x.dtype, x.device, _effective_dtype(x), training)
        hit = _CONTEXTS.get(key)
        if hit is None:
            hit = _build_context(x, model_context, training=training, export=False)
            if len(_CONTEXTS) < 65536:
                _CONTEXTS[key] = hit
        return hit
    return _build_context(x, model_context, training=training, export=export)


def _build_context(x: Tensor, model_context: ModelOptimizationContext, *, training: bool, export: bool) -> ExecutionContext:
    sm, vram, arch = None, 0, None
    if x.device.type == "cuda" and not export:
        sm, vram, arch = device_facts(x.device.index if x.device.index is not None else torch.cuda.current_device())
    return execution_context_for_shape(
        model_context,
        batch_size=1 if x.ndim == 4 else int(x.shape[0]),
        spatial_shape=tuple(int(s) for s in x.shape[-3:]),
        dtype=_effective_dtype(x),
        device_type=x.device.type,
        sm=sm,
        total_vram_bytes=vram,
        training=training,
        export=export,
        arch=arch,
    )


def _conv_descriptor(conv: nn.Module, *, role: str | None) -> OperatorDescriptor:
    """Family naming as in the reference (ops/adaptive.py:80-109)."""
    transpose = isinstance(conv, (nn.ConvTranspose2d, nn.ConvTranspose3d))
    dims = len(conv.kernel_size)
    depthwise = conv.groups == conv.in_channels == conv.out_channels
    if depthwise:
        family = "depthwise_conv_transpose" if transpose else "depthwise_conv"
    elif transpose:
        family = "conv_transpose"
    elif conv.kernel_size == (1,) * dims and conv.groups == 1:
        family = "pointwise_conv"
    else:
        family = "conv"
    direction = "transpose" if transpose else ("downsample" if conv.stride[0] == 2 else "regular")
    return OperatorDescriptor.convolution(
        family=f"{family}{dims}d",
        direction=direction,
        in_channels=conv.in_channels,
        out_channels=conv.out_channels,
        kernel_size=conv.kernel_size,
        stride=conv.stride,
        padding=conv.padding,
        dilation=conv.dilation,
        groups=conv.groups,
        role=role,
    )


def _norm_descriptor(norm: nn.GroupNorm, *, role: str | None = None) -> OperatorDescriptor:
    return OperatorDescriptor.normalization(family="group_norm3d", channels=norm.num_channels, role=role)


def _gemm_guards(x: Tensor, cin: int, cout: int) -> bool:
    """Execution-time guards of the matrix-core pointwise route: grad enabled,
    batched contiguous NCDHW, and channel / voxel counts the kernels take."""
    from .tiles import pointwise_supported

    return (
        torch.is_grad_enabled()
        and x.ndim == 5
        and x.is_contiguous()
        and pointwise_supported(cin, cout, int(x.shape[2] * x.shape[3] * x.shape[4]))
    )


#: Set to 1 to make a HIP selection raise when libmednext_hip.so cannot be
#: loaded, instead of running PyTorch's native operator (the test suites and
#: the benchmark set it, so a result can never come from the fallback).
REQUIRE_HIP_ENV = "MEDNEXT_ACCEL_AMD_REQUIRE_HIP"

_backend_state: list = []  # [hip_ops module] once loaded, [None] once the load failed


def _hip_ops():
    """The HIP operator module, or None when ``libmednext_hip.so`` cannot be
    loaded (not built, stale ABI, no HIP runtime).

    None sends the adaptive modules to PyTorch's native operators, as the
    reference's wrapper does when its kernel backend fails to import (reference
    ``ops/adaptive.py:273-276``): a model built with ``optimization="auto"``
    keeps training, on the GPU, without the custom kernels. The first failure
    is reported once with a ``RuntimeWarning`` naming the cause; with
    ``MEDNEXT_ACCEL_AMD_REQUIRE_HIP=1`` it raises instead. Direct calls of the
    ``hip_ops`` launchers and ops always raise on a missing library.
    """
    if torch.compiler.is_compiling():
        from . import hip_ops

        return hip_ops
    if _backend_state:
        return _backend_state[0]
    from . import _hip

    try:
        _hip.load()
        from . import hip_ops
    except (_hip.HipLibraryError, OSError, ImportError) as error:
        if os.environ.get(REQUIRE_HIP_ENV, "0") not in ("", "0"):
            raise
        warnings.warn(
            f"mednext_accel_amd: the HIP kernels are unavailable ({error}); the adaptive "
            "modules run PyTorch's native operators",
            RuntimeWarning,
            stacklevel=3,
        )
        hip_ops = None
    _backend_state.append(hip_ops)
    return hip_ops


class _AdaptiveModule(nn.Module):
    resolver: PolicyResolver
    model_context: ModelOptimizationContext
    descriptor: OperatorDescriptor

    def _warn_for_device(self) -> None:
        reference = self.weight if getattr(self, "weight", None) is not None else getattr(self, "bias", None)
        if reference is not None and reference.device.type == "cuda":
            sm, _, arch = device_facts(reference.device.index or 0)
            if arch is not None:
                self.resolver.warn_for_target("amd", arch)
            else:
                self.resolver.warn_for_sm(sm)

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        self._warn_for_device()
        return result

    def decision_for_shape(
        self,
        *,
        batch_size: int,
        spatial_shape: tuple[int, int, int],
        dtype: torch.dtype | str,
        device_type: str,
        sm: tuple[int, int] | None,
        total_vram_bytes: int,
        arch: str | None = None,
        phase: str | None = None,
    ) -> PolicyDecision:
        context = execution_context_for_shape(
            self.model_context,
            batch_size=batch_size,
            spatial_shape=spatial_shape,
            dtype=dtype,
            device_type=device_type,
            sm=sm,
            total_vram_bytes=total_vram_bytes,
            training=self.training,
            arch=arch,
        )
        return self.resolver.resolve(self.descriptor, context, phase or context.phase)


class AdaptivePointwise3d(_AdaptiveModule):
    """1x1x1 convolution wrapper (reference ops/adaptive.py:125-200).

    Besides the reference's stride-1 ``nn.Conv3d`` it takes a 1x1x1
    ``nn.ConvTranspose3d`` (the MedNeXt output heads, whose weight is stored
    [Cin, Cout, 1, 1, 1]; ``transposed`` records which one it holds) and the
    stride-2 forms of both, the down / up blocks' residual convolutions: a
    stride-2 1x1 conv is the GEMM on every second voxel of each dimension, a
    stride-2 1x1 transposed conv (output 2s - 1) the GEMM written to the even
    voxels with the bias alone at the odd ones."""

    _mednext_accel_backend_kind = "pointwise_gemm"

    def __init__(
        self,
        conv: nn.Conv3d | nn.ConvTranspose3d,
        resolver: PolicyResolver,
        model_context: ModelOptimizationContext,
        *,
        role: str | None = None,
    ) -> None:
        super().__init__()
        self.weight = conv.weight
        self.bias = conv.bias
        for name in ("in_channels", "out_channels", "kernel_size", "stride", "padding", "dilation", "groups"):
            setattr(self, name, getattr(conv, name))
        self.transposed = isinstance(conv, nn.ConvTranspose3d)
        if self.transposed:
            self.output_padding = conv.output_padding
        self.descriptor = _conv_descriptor(conv, role=role)
        self.resolver = resolver
        self.model_context = model_context
        self.train(conv.training)
        self._warn_for_device()

    def _gemm(self, x: Tensor) -> Tensor:
        """Per-sample ``W @ X[n] + b`` (reference ops/adaptive.py:174-188)."""
        squeeze = x.ndim == 4
        if squeeze:
            x = x.unsqueeze(0)
        spatial = x.shape[2:]
        weight = self.weight.reshape(self.out_channels, self.in_channels)
        rows = []
        for sample in x.reshape(x.shape[0], self.in_channels, -1).unbind(0):
            rows.append(torch.mm(weight, sample) if self.bias is None else torch.addmm(self.bias[:, None], weight, sample))
        out = torch.stack(rows).reshape(x.shape[0], self.out_channels, *spatial)
        return out.squeeze(0) if squeeze else out

    def join_parts(self, x: Tensor) -> tuple[Tensor, Tensor | None] | None:
        """For a stride-2 transposed 1x1x1 conv on the matrix-core route: the
        GEMM output at the input's voxels (bias value included, not tracked)
        and the bf16 bias, which an up block turns into its padded residual sum
        in one pass (``hip_ops.up_block_join`` with ``bias_in_small``: the
        bias's whole gradient comes from the join's one reduction); None when
        this module would not take the HIP route for ``x``."""
        if not (self.transposed and self.stride == (2, 2, 2)):
            return None
        context = _context_from_tensor(x, self.model_context, training=self.training)
        decision = self.resolver.resolve(self.descriptor, context, context.phase)
        if decision.implementation != "hip_pointwise_gemm" or not _gemm_guards(x, self.in_channels, self.out_channels):
            return None
        ops = _hip_ops()
        if ops is None:
            return None
        dt = torch.bfloat16
        bias = cast_param(self.bias, dt) if self.bias is not None else None
        value = bias.detach() if bias is not None else None
        return ops.pointwise_conv_transpose3d(x.to(dt), cast_param(self.weight, dt), value), bias

    def forward(self, x: Tensor) -> Tensor:
        context = _context_from_tensor(x, self.model_context, training=self.training)
        decision = self.resolver.resolve(self.descriptor, context, context.phase)
        strided = self.stride != (1, 1, 1)
        ops = None
        if decision.implementation == "hip_pointwise_gemm" and _gemm_guards(x, self.in_channels, self.out_channels):
            ops = _hip_ops()
        if ops is not None:
            dt = torch.bfloat16
            bias = cast_param(self.bias, dt) if self.bias is not None else None
            weight = cast_param(self.weight, dt)
            if not strided:
                op = ops.pointwise_conv_transpose3d if self.transposed else ops.pointwise_conv3d
                return op(x.to(dt), weight, bias)
            if not self.transposed:
                # Every second voxel, gathered once (autograd scatters its gradient back).
                return ops.pointwise_conv3d(x[:, :, ::2, ::2, ::2].to(dt).contiguous(), weight, bias)
            y = ops.pointwise_conv_transpose3d(x.to(dt), weight, bias)
            full = tuple(2 * s - 1 for s in x.shape[2:])
            if bias is None:
                out = y.new_zeros((x.shape[0], self.out_channels, *full))
            else:
                out = bias.view(1, -1, 1, 1, 1).expand(x.shape[0], self.out_channels, *full).contiguous()
            out[:, :, ::2, ::2, ::2] = y
            return out
        if self.transposed:
            return F.conv_transpose3d(x, precast_or_param(self.weight), precast_or_param(self.bias), stride=self.stride)
        if (
            decision.implementation == "pointwise_gemm_per_sample"
            and not strided
            and torch.is_grad_enabled()
            and x.ndim == 5
            and x.is_contiguous()
        ):
            return self._gemm(x)
        return F.conv3d(x, precast_or_param(self.weight), precast_or_param(self.bias), stride=self.stride)


class AdaptiveDepthwise3d(_AdaptiveModule):
    _mednext_accel_backend_kind = "depthwise"

    def __init__(
        self,
        conv: nn.Conv3d | nn.ConvTranspose3d,
        resolver: PolicyResolver,
        model_context: ModelOptimizationContext,
        *,
        role: str | None = None,
    ) -> None:
        super().__init__()
        self.weight = conv.weight
        self.bias = conv.bias
        for name in ("in_channels", "out_channels", "kernel_size", "stride", "padding", "dilation", "groups"):
            setattr(self, name, getattr(conv, name))
        self.output_padding = getattr(conv, "output_padding", (0, 0, 0))
        self.transpose = isinstance(conv, nn.ConvTranspose3d)
        self.descriptor = _conv_descriptor(conv, role=role)
        self.resolver = resolver
        self.model_context = model_context
        self.train(conv.training)
        self._warn_for_device()

    def _reference(self, x: Tensor) -> Tensor:
        if self.transpose:
            return F.conv_transpose3d(
                x, precast_or_param(self.weight), precast_or_param(self.bias), self.stride, self.padding,
                self.output_padding, self.groups, self.dilation,
            )
        return F.conv3d(x, precast_or_param(self.weight), precast_or_param(self.bias), self.stride, self.padding,
                        self.dilation, self.groups)

    def _forward_stride2(self, x: Tensor, context: ExecutionContext) -> Tensor:
        """Down-block (stride 2) and up-block (transposed, stride 2) routes: the
        HIP op runs all three phases when any phase selects it."""
        if self.stride != (2, 2, 2):
            return self._reference(x)
        impl = "hip_depthwise_transpose2" if self.transpose else "hip_depthwise_stride2"
        if not any(d.implementation == impl for d in self.phase_decisions(context)):
            return self._reference(x)
        hip_ops = _hip_ops()
        if hip_ops is None:
            return self._reference(x)
        dtype = getattr(torch, context.dtype)
        x = x.to(dtype)
        weight = cast_param(self.weight, dtype)
        bias = cast_param(self.bias, dtype) if self.bias is not None else None
        op = hip_ops.depthwise_conv_transpose3d_stride2 if self.transpose else hip_ops.depthwise_conv3d_stride2
        return op(x, weight, bias, self.kernel_size[0])

    def phase_decisions(self, context: ExecutionContext) -> tuple[PolicyDecision, PolicyDecision, PolicyDecision]:
        return tuple(self.resolver.resolve(self.descriptor, context, p) for p in ("forward", "backward_input", "backward_weight"))

    def forward(self, x: Tensor) -> Tensor:
        context = _context_from_tensor(x, self.model_context, training=self.training)
        if (
            context.phase != "training"
            or context.device_type != "cuda"
            or not torch.is_grad_enabled()
            or x.ndim != 5
            or self.output_padding != (0, 0, 0)
            or not x.is_contiguous()
        ):
            return self._reference(x)
        if self.transpose or self.stride == (2, 2, 2):
            return self._forward_stride2(x, context)
        if self.stride != (1, 1, 1):
            return self._reference(x)
        fwd, dx, dw = self.phase_decisions(context)
        custom = [d.implementation != "reference" for d in (fwd, dx, dw)]
        if not any(custom):
            return self._reference(x)
        hip_ops = _hip_ops()
        if hip_ops is None:
            return self._reference(x)
        dtype = getattr(torch, context.dtype)
        x = x.to(dtype)
        weight = cast_param(self.weight, dtype)
        bias = cast_param(self.bias, dtype) if self.bias is not None else None

        def recipe(decision: PolicyDecision) -> list[int]:
            p = decision.parameters
            return [int(p.get("engine", 0)), int(p.get("tile_w", 0)), int(p.get("depth_chunk", 0))] if p else []

        return hip_ops.depthwise_conv3d_regular(
            x, weight, bias, self.kernel_size[0], recipe(fwd), recipe(dx), recipe(dw), *custom
        )

    def forward_tap(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """``(self(x), residual)`` for a block that adds x back at its end: the
        residual is x itself, as a second output of ``DepthwiseResidualTap``
        when every phase takes the HIP route with the matrix-core k = 3 input
        gradient on bf16 x (its gradient is then added inside that kernel),
        x otherwise. The k = 5 kernel supports the same accumulation, but on
        MedNeXt-Large it measured no faster than the separate add (55.96 vs
        55.63 ms per step, alternating steps), so k = 5 blocks keep the add."""
        context = _context_from_tensor(x, self.model_context, training=self.training)
        if (
            context.phase != "training"
            or context.device_type != "cuda"
            or not torch.is_grad_enabled()
            or x.ndim != 5
            or x.dtype != torch.bfloat16
            or not x.is_contiguous()
            or self.transpose
            or self.stride != (1, 1, 1)
            or self.output_padding != (0, 0, 0)
            or self.kernel_size[0] != 3
            or getattr(torch, context.dtype) != torch.bfloat16
        ):
            return self(x), x
        fwd, dx, dw = self.phase_decisions(context)
        if any(d.implementation == "reference" for d in (fwd, dx, dw)):
            return self(x), x

        def recipe(decision: PolicyDecision) -> list[int]:
            p = decision.parameters
            return [int(p.get("engine", 0)), int(p.get("tile_w", 0)), int(p.get("depth_chunk", 0))] if p else []

        hip_ops = _hip_ops()
        if hip_ops is None:
            return self(x), x
        rdx = recipe(dx)
        k = self.kernel_size[0]
        if hip_ops._recipe_for(x, k, rdx or None, "input_grad")[0] != ENGINE_MFMA:
            return self(x), x
        weight = cast_param(self.weight, torch.bfloat16)
        bias = cast_param(self.bias, torch.bfloat16) if self.bias is not None else None
        return hip_ops.DepthwiseResidualTap.apply(x, weight, bias, k, recipe(fwd), rdx, recipe(dw))


class AdaptiveGroupNorm3d(_AdaptiveModule):
    """GroupNorm with groups == channels over 5-D inputs (MedNeXt's ``norm``)."""

    _mednext_accel_backend_kind = "group_norm"

    def __init__(
        self,
        norm: nn.GroupNorm,
        resolver: PolicyResolver,
        model_context: ModelOptimizationContext,
        *,
        role: str | None = None,
    ) -> None:
        super().__init__()
        self.weight = norm.weight
        self.bias = norm.bias
        self.num_groups = norm.num_groups
        self.num_channels = norm.num_channels
        self.eps = norm.eps
        self.affine = norm.affine
        self.descriptor = _norm_descriptor(norm, role=role)
        self.resolver = resolver
        self.model_context = model_context
        self.train(norm.training)
        self._warn_for_device()

    def _reference(self, x: Tensor) -> Tensor:
        return F.group_norm(x, self.num_groups, self.weight, self.bias, self.eps)

    def forward(self, x: Tensor, out_dtype: torch.dtype | None = None) -> Tensor:
        """``out_dtype`` (used by a fused block expansion that consumes the
        result as bf16) overrides the output dtype; the values are the float32
        result rounded once, exactly what the consumer's autocast cast makes."""
        if x.ndim != 5 or not x.is_contiguous() or not torch.is_grad_enabled():
            y = self._reference(x)
            return y if out_dtype is None else y.to(out_dtype)
        context = _context_from_tensor(x, self.model_context, training=self.training)
        decision = self.resolver.resolve(self.descriptor, context, context.phase)
        hip_ops = _hip_ops() if decision.implementation == "hip_group_norm" else None
        if hip_ops is None:
            y = self._reference(x)
            return y if out_dtype is None else y.to(out_dtype)
        autocast = torch.is_autocast_enabled(x.device.type) and x.dtype != torch.float64
        # Autocast runs group_norm in float32 (input cast up, float32 result);
        # the kernel reads the low-precision input directly, which is exact.
        if out_dtype is None:
            out_dtype = torch.float32 if autocast else None
        weight, bias = self.weight, self.bias
        if autocast:
            weight = weight.float() if weight is not None else None
            bias = bias.float() if bias is not None else None
        y, _mean, _rstd = hip_ops.group_norm_channels(x, weight, bias, self.eps, out_dtype)
        return y

    def hip_selected(self, x: Tensor) -> bool:
        """Whether ``forward`` would run the HIP kernels on ``x`` (policy and
        execution guards), for a consumer that folds the normalisation."""
        if x.ndim != 5 or not x.is_contiguous() or not torch.is_grad_enabled():
            return False
        context = _context_from_tensor(x, self.model_context, training=self.training)
        decision = self.resolver.resolve(self.descriptor, context, context.phase)
        return decision.implementation == "hip_group_norm" and _hip_ops() is not None

    def extra_repr(self) -> str:
        return f"{self.num_groups}, {self.num_channels}, eps={self.eps}, affine={self.affine}"


class AdaptiveExpansion:
    """Fused ``project(GELU(expand(h))) [+ residual]`` of one MedNeXt block.

    Deliberately *not* an ``nn.Module``: it holds a reference to its block and
    reads the block's own ``expand`` / ``project`` Parameters at call time, so
    installing it changes neither ``parameters()`` nor the state-dict keys. The
    block consults it (``MedNeXtBlock.forward``) before running its modules;
    when ``applies`` is false the block runs exactly as without it.
    """

    #: Hidden width from which the expansion stores GELU and GELU' of the
    #: expand output (``mlp_expansion_stored``) instead of recomputing GELU in
    #: the project GEMM and its gradients (``mlp_expansion``). Measured on
    #: MI355X, fwd + bwd per block: 64 hidden @128^3 686 vs 721 us (recompute
    #: wins), 192 @64^3 385 vs 351, 512 @32^3 229 vs 190, 2048 @8^3 219 vs 178.
    stored_gelu_from = 128
    #: Project widths up to which GELU is recomputed whatever the hidden width:
    #: a project GEMM this narrow is one row group, so it (and its weight
    #: gradient) evaluates GELU once per element, while storing GELU' writes
    #: another hidden-sized tensor (the up block into stage 0: 128 hidden,
    #: 32 outputs, at 128^3).
    recompute_gelu_up_to = 32

    def stores_gelu(self) -> bool:
        """Whether the expansion stores GELU and GELU' of the expand output."""
        b = self.block
        return b.expand.out_channels >= self.stored_gelu_from and b.project.out_channels > self.recompute_gelu_up_to

    def __init__(self, block: nn.Module, resolver: PolicyResolver, model_context: ModelOptimizationContext,
                 *, role: str | None = None) -> None:
        self.block = block
        self.resolver = resolver
        self.model_context = model_context
        self.descriptor = OperatorDescriptor(
            "mlp_expansion3d", "regular", block.expand.in_channels, block.project.out_channels, role=role
        )

    def applies(self, x: Tensor) -> bool:
        """Decided from the block input: training with grad, bf16 autocast on an
        AMD GPU and the policy selecting the fused kernel. Shapes are checked
        separately (``supports``) on the expansion's own input."""
        b = self.block
        if not (b.training and torch.is_grad_enabled() and x.is_cuda and x.ndim == 5):
            return False
        context = _context_from_tensor(x, self.model_context, training=True)
        if context.dtype != "bfloat16":
            return False
        if self.resolver.resolve(self.descriptor, context, "training").implementation != "hip_fused_expansion":
            return False
        return _hip_ops() is not None

    def supports(self, h: Tensor) -> bool:
        """Shape check on the expansion's input (the depthwise output: halved
        in down blocks, 2s-1 per dimension in up blocks)."""
        from .tiles import pointwise_supported

        b = self.block
        v = int(h.shape[2] * h.shape[3] * h.shape[4])
        return (
            h.is_contiguous()
            and pointwise_supported(b.expand.in_channels, b.expand.out_channels, v)
            and pointwise_supported(b.expand.out_channels, b.project.out_channels, v)
        )

    #: Fold the block's GroupNorm into the expand GEMM (``folds_norm`` /
    #: ``folded``) when its HIP kernels are selected: one statistics pass, and
    #: the expand GEMM normalises as it loads (no normalised tensor).
    fold_norm = True

    def __call__(self, h: Tensor, residual: Tensor | None) -> Tensor:
        b = self.block
        dt = torch.bfloat16
        w1, w2 = cast_param(b.expand.weight, dt), cast_param(b.project.weight, dt)
        b1 = cast_param(b.expand.bias, dt) if b.expand.bias is not None else None
        b2 = cast_param(b.project.bias, dt) if b.project.bias is not None else None
        fuse_residual = residual is not None and residual.dtype == dt and residual.is_contiguous()
        res = residual if fuse_residual else None
        if self.stores_gelu():
            out = _hip_ops().mlp_expansion_stored(h.to(dt), w1, b1, w2, b2, res)[0]
        else:
            out = _hip_ops().mlp_expansion(h.to(dt), w1, b1, w2, b2, res)[0]
        if residual is not None and not fuse_residual:
            out = out + residual
        return out

    def folds_norm(self, d: Tensor) -> bool:
        """Whether ``folded`` applies to the depthwise output ``d``: an affine
        GroupNorm(C, C) wrapped for HIP whose kernels are selected for d, and
        an expand width the AFFINE prologue takes (its coefficients sit in
        LDS: at most 2048 input channels)."""
        norm = self.block.norm
        return (
            self.fold_norm
            and isinstance(norm, AdaptiveGroupNorm3d)
            and norm.affine
            and norm.num_groups == norm.num_channels
            and norm.weight is not None
            and norm.bias is not None
            and self.block.expand.in_channels <= 2048
            and norm.hip_selected(d)
        )

    def folded(self, d: Tensor, residual: Tensor | None) -> Tensor:
        """``project(GELU(expand(GroupNorm(d)))) [+ residual]`` with the
        normalisation inside the expand GEMM (``hip_ops.gn_mlp_expansion``)."""
        b = self.block
        norm = b.norm
        dt = torch.bfloat16
        w1, w2 = cast_param(b.expand.weight, dt), cast_param(b.project.weight, dt)
        b1 = cast_param(b.expand.bias, dt) if b.expand.bias is not None else None
        b2 = cast_param(b.project.bias, dt) if b.project.bias is not None else None
        # Autocast runs group_norm in float32: float32 affine parameters.
        gamma, beta = norm.weight.float(), norm.bias.float()
        fuse_residual = residual is not None and residual.dtype == dt and residual.is_contiguous()
        stored = self.stores_gelu()
        out = _hip_ops().gn_mlp_expansion(
            d.to(dt), gamma, beta, w1, b1, w2, b2, residual if fuse_residual else None, float(norm.eps), stored
        )[0]
        if residual is not None and not fuse_residual:
            out = out + residual
        return out


def _pointwise_eligible(module: nn.Module) -> bool:
    """1x1x1 stride-1 Conv3d (reference ops/adaptive.py:323-332), the same
    geometry as a ConvTranspose3d without output padding (the output heads),
    and both at stride 2 (the down / up blocks' residual convolutions)."""
    if type(module) is nn.ConvTranspose3d and module.output_padding != (0, 0, 0):
        return False
    return (
        type(module) in (nn.Conv3d, nn.ConvTranspose3d)
        and module.kernel_size == (1, 1, 1)
        and module.stride in ((1, 1, 1), (2, 2, 2))
        and module.padding == (0, 0, 0)
        and module.dilation == (1, 1, 1)
        and module.groups == 1
        and module.padding_mode == "zeros"
    )


def _depthwise_eligible(module: nn.Module) -> bool:
    if type(module) not in (nn.Conv3d, nn.ConvTranspose3d):
        return False
    k = module.kernel_size[0]
    return (
        len(set(module.kernel_size)) == 1
        and k % 2 == 1
        and module.in_channels == module.out_channels == module.groups
        and module.stride in ((1, 1, 1), (2, 2, 2))
        and module.padding == (k // 2,) * 3
        and module.dilation == (1, 1, 1)
        and getattr(module, "padding_mode", "zeros") == "zeros"
        and getattr(module, "output_padding", (0, 0, 0)) == (0, 0, 0)
    )


def _group_norm_eligible(module: nn.Module) -> bool:
    return type(module) is nn.GroupNorm and module.num_groups == module.num_channels


def install_adaptive_operators(
    model: nn.Module,
    *,
    resolver: PolicyResolver,
    model_context: ModelOptimizationContext,
    _prefix: str = "",
) -> int:
    """Swap eligible children for wrappers in place and attach a fused expansion
    to each MedNeXt block; returns how many modules were swapped."""
    from .blocks import MedNeXtBlock

    count = 0
    for name, child in list(model.named_children()):
        role = f"{_prefix}.{name}" if _prefix else name
        if _pointwise_eligible(child):
            wrapper: nn.Module = AdaptivePointwise3d(child, resolver, model_context, role=role)
        elif _depthwise_eligible(child):
            wrapper = AdaptiveDepthwise3d(child, resolver, model_context, role=role)
        elif _group_norm_eligible(child):
            wrapper = AdaptiveGroupNorm3d(child, resolver, model_context, role=role)
        else:
            count += install_adaptive_operators(child, resolver=resolver, model_context=model_context, _prefix=role)
            continue
        setattr(model, name, wrapper)
        count += 1
    if isinstance(model, MedNeXtBlock) and _group_norm_wrapped(model):
        # Plain attribute (not a submodule): parameters and keys are unchanged.
        model.__dict__["fused_expansion"] = AdaptiveExpansion(model, resolver, model_context, role=_prefix or None)
    return count


def _group_norm_wrapped(block: nn.Module) -> bool:
    return isinstance(getattr(block, "norm", None), AdaptiveGroupNorm3d)
