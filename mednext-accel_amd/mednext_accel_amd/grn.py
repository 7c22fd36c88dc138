"""Global Response Normalization for MedNeXt v2 (reference src/mednext_accel/ops/grn.py).

Per sample and channel, with ``n_c = ||x_c||_2`` over the spatial volume:

    y = x + gamma * x * n_c / (sum_c n_c + eps) + beta

in float32 for half inputs (the input dtype otherwise), stored in the input's
dtype. ``GlobalResponseNorm3d`` is the plain PyTorch layer the model is built
with (zero-initialised (1, C, 1, 1, 1) parameters, the reference's names);
``AdaptiveGlobalResponseNorm3d`` replaces it after ``install_adaptive_grn`` and
routes training steps to the HIP kernels (``hip_ops.grn_forward_op``) when the
policy selects ``hip_fused_grn``. Evaluation, no-grad and ineligible tensors
run the PyTorch formula, as in the reference (ops/grn.py:50-90).
"""

from __future__ import annotations

import math
from dataclasses import replace

import torch
from torch import Tensor, nn

from .adaptive import ModelOptimizationContext, _context_from_tensor, _hip_ops, device_facts
from .optimization.descriptors import OperatorDescriptor
from .optimization.policy_resolver import PolicyResolver
from .precast import cast_param


def global_response_norm3d_reference(x: Tensor, gamma: Tensor, beta: Tensor, eps: float = 1e-6) -> Tensor:
    """The channel-sum GRN formula in PyTorch operations (reference ops/grn.py:16-30)."""
    if x.ndim != 5:
        raise ValueError("GRN expects an NCDHW tensor")
    work = x.float() if x.dtype in (torch.float16, torch.bfloat16) else x
    norm = torch.linalg.vector_norm(work, dim=(2, 3, 4), keepdim=True)
    ratio = norm / (norm.sum(dim=1, keepdim=True) + eps)
    return (work + gamma.to(work.dtype) * work * ratio + beta.to(work.dtype)).to(x.dtype)


class GlobalResponseNorm3d(nn.Module):
    """GRN layer with zero-initialised affine parameters (reference ops/grn.py:33-47)."""

    def __init__(self, channels: int, eps: float = 1e-6) -> None:
        super().__init__()
        if channels <= 0:
            raise ValueError("channels must be positive")
        if not math.isfinite(eps) or eps <= 0:
            raise ValueError("eps must be finite and positive")
        self.eps = eps
        self.gamma = nn.Parameter(torch.zeros(1, channels, 1, 1, 1))
        self.beta = nn.Parameter(torch.zeros(1, channels, 1, 1, 1))

    def forward(self, x: Tensor) -> Tensor:
        return global_response_norm3d_reference(x, self.gamma, self.beta, self.eps)


class AdaptiveGlobalResponseNorm3d(nn.Module):
    """Policy-selected training GRN (reference ops/grn.py:50-90). Holds the
    wrapped layer's Parameter objects, so parameters and state-dict keys are
    unchanged by installation."""

    _mednext_accel_backend_kind = "global_response_norm"

    def __init__(
        self,
        module: GlobalResponseNorm3d,
        resolver: PolicyResolver,
        model_context: ModelOptimizationContext,
        role: str | None = None,
    ) -> None:
        super().__init__()
        self.gamma = module.gamma
        self.beta = module.beta
        self.eps = module.eps
        self.resolver = resolver
        self.model_context = model_context
        self.descriptor = OperatorDescriptor.normalization(
            family="global_response_norm3d", channels=self.gamma.shape[1], role=role
        )
        self.train(module.training)
        self._warn_for_device()

    def _warn_for_device(self) -> None:
        if self.gamma.device.type == "cuda":
            sm, _, arch = device_facts(self.gamma.device.index or 0)
            if arch is not None:
                self.resolver.warn_for_target("amd", arch)
            else:
                self.resolver.warn_for_sm(sm)

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        self._warn_for_device()
        return result

    def _reference(self, x: Tensor) -> Tensor:
        return global_response_norm3d_reference(x, self.gamma, self.beta, self.eps)

    def forward(self, x: Tensor) -> Tensor:
        if not self.training or not torch.is_grad_enabled() or x.ndim != 5:
            return self._reference(x)
        context = _context_from_tensor(x, self.model_context, training=True)
        # GRN is not an autocast op: the decision keys on the tensor's own dtype.
        context = replace(context, dtype=str(x.dtype).removeprefix("torch."))
        decision = self.resolver.resolve(self.descriptor, context, "training")
        ops = _hip_ops() if decision.implementation == "hip_fused_grn" and x.is_contiguous() else None
        if ops is None:
            return self._reference(x)
        return ops.fused_global_response_norm3d(x, self.gamma, self.beta, self.eps)

    def extra_repr(self) -> str:
        return f"{self.gamma.shape[1]}, eps={self.eps}"


class AdaptiveGRNExpansion:
    """Fused ``project(GRN(GELU(expand(h)))) [+ residual]`` of one MedNeXt v2
    block (``hip_ops.grn_expansion``).

    Like the v1 block's fused expansion it is a plain attribute of the block,
    not a submodule: it reads the block's own ``expand`` / ``grn`` /
    ``project`` Parameters at call time, so installing it changes neither
    ``parameters()`` nor the state-dict keys. ``MedNeXtV2Block.forward``
    consults it; when ``applies`` or ``supports`` is false the block runs its
    modules as without it.
    """

    #: Widest hidden layer the fused path takes; wider expansions (the
    #: MedNeXt v2 Base stage-3/4 blocks: small volumes, K >= 2048) run the
    #: separate operators. Measured on MI355X (v2 Base 128^3 step): 61.4 ms
    #: unfused, 54.0-56.2 ms up to 512, 53.6-54.1 ms up to 1024, 54.3 ms up to 2048.
    max_hidden = 1024

    def __init__(self, block: nn.Module, resolver: PolicyResolver, model_context: ModelOptimizationContext,
                 *, role: str | None = None) -> None:
        self.block = block
        self.resolver = resolver
        self.model_context = model_context
        self.descriptor = OperatorDescriptor(
            "grn_expansion3d", "regular", block.expand.in_channels, block.project.out_channels, role=role
        )

    def applies(self, x: Tensor) -> bool:
        """Training with grad, bf16 autocast on a GPU and the policy selecting
        the fused kernels (decided from the block input)."""
        b = self.block
        if not (b.training and torch.is_grad_enabled() and x.is_cuda and x.ndim == 5):
            return False
        context = _context_from_tensor(x, self.model_context, training=True)
        if context.dtype != "bfloat16":
            return False
        if self.resolver.resolve(self.descriptor, context, "training").implementation != "hip_fused_grn_expansion":
            return False
        return _hip_ops() is not None

    def supports(self, h: Tensor) -> bool:
        """Shape check on the expansion's input (the depthwise output)."""
        from .tiles import pointwise_supported

        b = self.block
        hidden = b.expand.out_channels
        v = int(h.shape[2] * h.shape[3] * h.shape[4])
        return (
            h.is_contiguous()
            and hidden <= self.max_hidden
            and pointwise_supported(b.expand.in_channels, hidden, v)
            and pointwise_supported(hidden, b.project.out_channels, v)
        )

    def __call__(self, h: Tensor, residual: Tensor | None) -> Tensor:
        b = self.block
        dt = torch.bfloat16
        w1, w2 = cast_param(b.expand.weight, dt), cast_param(b.project.weight, dt)
        b1 = cast_param(b.expand.bias, dt) if b.expand.bias is not None else None
        b2 = cast_param(b.project.bias, dt) if b.project.bias is not None else None
        fuse_residual = residual is not None and residual.dtype == dt and residual.is_contiguous()
        out, _a, _dgelu, _coef = _hip_ops().grn_expansion(
            h.to(dt), w1, b1, w2, b2, b.grn.gamma, b.grn.beta, residual if fuse_residual else None, float(b.grn.eps)
        )
        if residual is not None and not fuse_residual:
            out = out + residual
        return out


def install_fused_grn_expansions(
    model: nn.Module,
    *,
    resolver: PolicyResolver,
    model_context: ModelOptimizationContext,
) -> int:
    """Attach an ``AdaptiveGRNExpansion`` to every MedNeXt v2 block whose
    GroupNorm and GRN were wrapped; returns how many were attached."""
    from .adaptive import AdaptiveGroupNorm3d
    from .blocks_v2 import MedNeXtV2Block

    count = 0
    for role, module in model.named_modules():
        if (
            isinstance(module, MedNeXtV2Block)
            and isinstance(module.norm, AdaptiveGroupNorm3d)
            and isinstance(module.grn, AdaptiveGlobalResponseNorm3d)
        ):
            module.__dict__["fused_expansion"] = AdaptiveGRNExpansion(module, resolver, model_context, role=role or None)
            count += 1
    return count


def install_adaptive_grn(
    model: nn.Module,
    *,
    resolver: PolicyResolver,
    model_context: ModelOptimizationContext,
    _prefix: str = "",
) -> int:
    """Replace every ``GlobalResponseNorm3d`` child with the adaptive wrapper,
    keeping its Parameters (reference ops/grn.py:93-112); returns the count."""
    count = 0
    for name, child in list(model.named_children()):
        role = f"{_prefix}.{name}" if _prefix else name
        if type(child) is GlobalResponseNorm3d:
            setattr(model, name, AdaptiveGlobalResponseNorm3d(child, resolver, model_context, role))
            count += 1
        else:
            count += install_adaptive_grn(child, resolver=resolver, model_context=model_context, _prefix=role)
    return count
