"""One-pass bf16 copies of a model's convolution parameters per training forward.

Under bf16 autocast every convolution casts its fp32 weight and bias to bf16
on every forward, and autograd casts each bf16 gradient back: two tiny kernel
launches per parameter per step (several hundred for MedNeXt), each a few
microseconds of launch for a few kilobytes of data. ``install_weight_precast``
replaces them with one concatenation + one cast before the forward and one
concatenation + one cast of all their gradients in the backward
(``_CastMany``). The values are those of the per-parameter casts: the same
bf16 rounding of the same fp32 weights, the same fp32 widening of the same
bf16 gradients.

The adaptive operators fetch their bf16 weights through ``cast_param``, which
returns the pre-cast copy while the model's forward runs and falls back to
``tensor.to(dtype)`` otherwise (evaluation, no autocast, checkpoint
recomputation during the backward).
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

_ACTIVE: dict[int, Tensor] | None = None


def cast_param(p: Tensor, dtype: torch.dtype) -> Tensor:
    """``p.to(dtype)``, served from the current forward's pre-cast copies when
    ``p`` is one of them."""
    if _ACTIVE is not None and p.dtype != dtype:
        t = _ACTIVE.get(id(p))
        if t is not None and t.dtype == dtype:
            return t
    return p.to(dtype)


_ALIGN = 8  # elements: every copy starts 16-byte aligned (the GEMM weight loads need it)
_PADS: dict[tuple[torch.device, torch.dtype], Tensor] = {}


def _pad(device: torch.device, dtype: torch.dtype, n: int) -> Tensor:
    """A view of ``n`` (< 8) zeros of this device and dtype (one buffer per pair)."""
    key = (device, dtype)
    if key not in _PADS:
        _PADS[key] = torch.zeros(_ALIGN, device=device, dtype=dtype)
    return _PADS[key][:n]


def _packed(pieces: list[Tensor], sizes: list[int]) -> list[Tensor]:
    """``pieces`` flattened with zero padding after each to a multiple of 8."""
    out = []
    for t, n in zip(pieces, sizes):
        out.append(t.reshape(-1))
        if n % _ALIGN:
            out.append(_pad(t.device, t.dtype, _ALIGN - n % _ALIGN))
    return out


def _unpacked(flat: Tensor, meta) -> list[Tensor]:
    views, o = [], 0
    for shape, n in meta:
        views.append(flat[o:o + n].view(shape))
        o += -(-n // _ALIGN) * _ALIGN
    return views


def precast_or_param(p: Tensor | None) -> Tensor | None:
    """The current forward's pre-cast copy of ``p`` if there is one, else ``p``
    itself: for operators that leave the casting to autocast (a native
    convolution then finds its weight already in the autocast dtype and casts
    nothing)."""
    if p is None or _ACTIVE is None:
        return p
    return _ACTIVE.get(id(p), p)


class _CastMany(torch.autograd.Function):
    """``tuple(p.to(dtype) for p in params)`` with one concatenation and one
    cast kernel each way. The copies are views of one buffer, each starting on
    a 16-byte boundary."""

    @staticmethod
    def forward(ctx, dtype: torch.dtype, *params: Tensor):
        ctx.meta = [(p.shape, p.numel()) for p in params]
        ctx.src_dtype = params[0].dtype
        ctx.set_materialize_grads(False)
        flat = torch.cat(_packed(list(params), [n for _, n in ctx.meta])).to(dtype)
        return tuple(_unpacked(flat, ctx.meta))

    @staticmethod
    def backward(ctx, *grads: Tensor | None):
        live = [g is not None for g in grads]
        if not any(live):
            return (None,) * (len(grads) + 1)
        ref = next(g for g in grads if g is not None)
        parts = [g if g is not None else ref.new_zeros(n) for g, (_, n) in zip(grads, ctx.meta)]
        flat = torch.cat(_packed(parts, [n for _, n in ctx.meta])).to(ctx.src_dtype)
        views = _unpacked(flat, ctx.meta)
        return (None, *(v if ok else None for v, ok in zip(views, live)))


def precast_parameters(model: nn.Module) -> list[nn.Parameter]:
    """The floating-point parameters the adaptive convolution operators cast
    per forward (depthwise, pointwise and the fused expansions' expand /
    project weights and biases), each once, in module order."""
    from .adaptive import AdaptiveDepthwise3d, AdaptivePointwise3d

    seen: set[int] = set()
    params: list[nn.Parameter] = []
    for module in model.modules():
        if isinstance(module, (AdaptiveDepthwise3d, AdaptivePointwise3d)):
            for p in (module.weight, module.bias):
                if p is not None and p.is_floating_point() and id(p) not in seen:
                    seen.add(id(p))
                    params.append(p)
    return params


def _precast_before(module: nn.Module, args) -> None:
    global _ACTIVE
    # Copies of an earlier forward that did not return (an exception skips the
    # post hook's normal path) must never serve this one.
    _ACTIVE = None
    params = module.__dict__.get("_mednext_precast_params")
    dtype = module.__dict__.get("_mednext_precast_dtype")
    if not params:
        return
    device = params[0].device.type
    if (
        module.training
        and torch.is_grad_enabled()
        and torch.is_autocast_enabled(device)
        and torch.get_autocast_dtype(device) == dtype
        and all(p.dtype != dtype for p in params)
    ):
        copies = _CastMany.apply(dtype, *params)
        _ACTIVE = {id(p): c for p, c in zip(params, copies)}


def _precast_after(module: nn.Module, args, output) -> None:
    global _ACTIVE
    _ACTIVE = None


def install_weight_precast(model: nn.Module, dtype: torch.dtype = torch.bfloat16) -> int:
    """Pre-cast ``precast_parameters(model)`` to ``dtype`` at the start of every
    training forward run under autocast with that dtype (grad enabled), and
    drop the copies when the forward returns. The parameter list lives in the
    model's ``__dict__`` (a deep copy of the model gets its own) and the hooks
    are module-level functions. Returns how many parameters are covered."""
    params = precast_parameters(model)
    if not params:
        return 0
    first = "_mednext_precast_params" not in model.__dict__
    model.__dict__["_mednext_precast_params"] = params
    model.__dict__["_mednext_precast_dtype"] = dtype
    if first:
        model.register_forward_pre_hook(_precast_before)
        model.register_forward_hook(_precast_after, always_call=True)
    return len(params)


__all__ = ["cast_param", "install_weight_precast", "precast_or_param", "precast_parameters"]
