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
returns the pre-cast copy from the forward until that forward's backward has
gone through the copies (so checkpointed branches recomputed during the
backward reuse them instead of casting every weight again), and falls back to
``tensor.to(dtype)`` otherwise (evaluation, no autocast, a parameter changed in
place since the cast).
"""

from __future__ import annotations

import torch
from torch import Tensor, nn

# id(parameter) -> (bf16 copy, the parameter's version counter when cast), and
# the forward that made them (its _CastMany backward drops them).
_ACTIVE: dict[int, tuple[Tensor, int]] | None = None
_OWNER: object | None = None


def _copy_of(p: Tensor, dtype: torch.dtype) -> Tensor | None:
    if _ACTIVE is None:
        return None
    entry = _ACTIVE.get(id(p))
    if entry is None or entry[0].dtype != dtype or entry[1] != p._version:
        return None
    return entry[0]


def _drop(owner: object | None = None) -> None:
    """Forget the copies (only those of ``owner``'s forward, when given)."""
    global _ACTIVE, _OWNER
    if owner is None or owner is _OWNER:
        _ACTIVE, _OWNER = None, None


def cast_param(p: Tensor, dtype: torch.dtype) -> Tensor:
    """``p.to(dtype)``, served from the pre-cast copies when ``p`` is one of
    them and has not changed in place since."""
    if p.dtype != dtype:
        t = _copy_of(p, dtype)
        if t is not None:
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
    entry = _ACTIVE.get(id(p))
    return entry[0] if entry is not None and entry[1] == p._version else p


class _CastMany(torch.autograd.Function):
    """``tuple(p.to(dtype) for p in params)`` with one concatenation and one
    cast kernel each way. The copies are views of one buffer, each starting on
    a 16-byte boundary."""

    @staticmethod
    def forward(ctx, dtype: torch.dtype, owner: object, *params: Tensor):
        ctx.owner = owner
        ctx.meta = [(p.shape, p.numel()) for p in params]
        ctx.src_dtype = params[0].dtype
        ctx.set_materialize_grads(False)
        flat = torch.cat(_packed(list(params), [n for _, n in ctx.meta])).to(dtype)
        return tuple(_unpacked(flat, ctx.meta))

    @staticmethod
    def backward(ctx, *grads: Tensor | None):
        # Every use of the copies, checkpoint recomputation included, has now
        # produced its gradient: the optimizer step may follow.
        _drop(ctx.owner)
        live = [g is not None for g in grads]
        if not any(live):
            return (None,) * (len(grads) + 2)
        ref = next(g for g in grads if g is not None)
        parts = [g if g is not None else ref.new_zeros(n) for g, (_, n) in zip(grads, ctx.meta)]
        flat = torch.cat(_packed(parts, [n for _, n in ctx.meta])).to(ctx.src_dtype)
        views = _unpacked(flat, ctx.meta)
        return (None, None, *(v if ok else None for v, ok in zip(views, live)))


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
    global _ACTIVE, _OWNER
    # Copies of an earlier forward never serve this one.
    _drop()
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
        owner = object()
        copies = _CastMany.apply(dtype, owner, *params)
        _ACTIVE = {id(p): (c, p._version) for p, c in zip(params, copies)}
        _OWNER = owner


def _precast_after(module: nn.Module, args, output) -> None:
    # The copies stay for the backward's checkpoint recomputation; a forward
    # that raised (the hook then sees no output) leaves none behind.
    if output is None:
        _drop()


def install_weight_precast(model: nn.Module, dtype: torch.dtype = torch.bfloat16) -> int:
    """Pre-cast ``precast_parameters(model)`` to ``dtype`` at the start of every
    training forward run under autocast with that dtype (grad enabled), and
    drop the copies when the backward has gone through them (or at the next
    forward, or when the forward raises). The parameter list lives in the
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
