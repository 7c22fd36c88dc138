"""Drop-in replacement for the reference's depthwise backend module.

The reference's ``AdaptiveDepthwise3d`` imports its kernels as a module
(``from ._triton import depthwise as backend``, reference
``ops/adaptive.py:273-276``) and calls three entry points on it; its autograd
glue calls four more ``torch.library`` ops. This module provides all of them
with the reference's names, schemas and argument meaning, backed by the gfx950
HIP kernels of ``libmednext_hip.so``:

======================================================  ==================================
reference (``ops/_triton/depthwise.py``)                here
======================================================  ==================================
``mednext_accel::depthwise_conv3d_odd_regular``         HIP forward, HIP dX / dW (+ dB)
  (:549-563, autograd :583-651)
``mednext_accel::depthwise_input_grad_odd_regular``     HIP dX
  (:486-513)
``mednext_accel::depthwise_weight_grad_odd_regular``    HIP dW (one tensor, as the reference)
  (:445-483)
``mednext_accel::depthwise_conv3d_stride2_regular``     HIP stride-2 forward, dX, dW (+ dB)
  (:654-719)
``mednext_accel::depthwise_input_grad_stride2_regular`` HIP stride-2 dX
  (:516-546)
``mednext_accel::depthwise_conv_transpose3d_odd_regular``  HIP transposed forward, dX, dW
  (:768-850)
``mednext_accel::depthwise_transpose_weight_grad_odd_regular``  HIP transposed dW
  (:722-765)
``depthwise_input_grad`` / ``depthwise_stride2_input_grad`` /   the low-level launchers
``depthwise_weight_grad`` / ``depthwise_transpose_weight_grad``   (:271-442)
======================================================  ==================================

Launch parameters. The reference's ``block`` / ``splits`` / ``dx_block`` /
``dw_block`` / ``dw_splits`` arguments size Triton programs; the CDNA4 kernels
tile differently (matrix-core Toeplitz tiles of 32 rows x 32-128 columns with a
D-run per workgroup, or VALU halo tiles), so the launch recipe is the gfx950 tile
policy's choice for the shape (``tiles.depthwise_recipe``). The reference's
values are still validated by the reference's rules (``block`` a positive power
of two, ``splits`` positive), so an argument the reference rejects is rejected
here. ``channels`` and ``spatial_size`` are checked against the tensors: the
reference's kernels take them on trust as compile-time shape constants.

Results: outputs and input gradients are the reference's, within the tolerance
of the dtype (fp32 accumulation; fp64 for fp64). The bias gradient, which the
reference takes from ATen's ``convolution_backward``, comes out of the same pass
as the weight gradient whenever the weight gradient runs here.

Importing this module registers the ``mednext_accel::`` ops; it is therefore
not imported by the package itself, so that it never collides with the
reference package in one process. Errors follow the reference: the launchers
and ops raise ``ValueError`` for bad arguments, and a missing or stale
``libmednext_hip.so`` raises ``HipLibraryError`` on the first launch.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import hip_ops
from .hip_ops import strided_spatial

__all__ = [
    "depthwise_conv3d_regular",
    "depthwise_conv3d_stride2_regular",
    "depthwise_conv_transpose3d_regular",
    "depthwise_input_grad",
    "depthwise_input_grad_regular",
    "depthwise_input_grad_stride2_regular",
    "depthwise_stride2_input_grad",
    "depthwise_transpose_weight_grad",
    "depthwise_transpose_weight_grad_regular",
    "depthwise_weight_grad",
    "depthwise_weight_grad_regular",
]


# ------------------------------------------------------------------ argument rules


def _power_of_two(value: int) -> bool:
    return value >= 1 and value & (value - 1) == 0


def _check_block(block: int) -> None:
    if not _power_of_two(int(block)):
        raise ValueError("block must be a positive power of two")


def _check_split_launch(splits: int, block: int) -> None:
    if int(splits) < 1 or not _power_of_two(int(block)):
        raise ValueError("splits must be positive and block must be a power of two")


def _check_kernel_size(kernel_size: int) -> None:
    if kernel_size < 1 or kernel_size % 2 == 0:
        raise ValueError("kernel_size must be a positive odd integer")


def _check_static_shape(t: Tensor, channels: int, spatial_size: int, what: str) -> None:
    """The reference compiles ``channels`` and ``spatial_size`` into its kernels
    and trusts them; a mismatch with the tensor would index out of range, so it
    is an error here."""
    if t.ndim != 5 or int(t.shape[1]) != int(channels) or tuple(int(s) for s in t.shape[2:]) != (int(spatial_size),) * 3:
        raise ValueError(
            f"{what} has shape {tuple(t.shape)}, which does not match channels={channels} "
            f"and a cubic spatial_size={spatial_size}"
        )


def _check_weight(weight: Tensor, channels: int, kernel_size: int) -> None:
    if tuple(weight.shape) != (int(channels), 1, int(kernel_size), int(kernel_size), int(kernel_size)):
        raise ValueError("weight must have shape [C, 1, K, K, K]")


# ------------------------------------------------------------- low-level launchers


def depthwise_input_grad(grad_output: Tensor, weight: Tensor, block: int = 256) -> Tensor:
    """Stride-one, same-padding depthwise dX for odd cubic kernels
    (reference ``depthwise.py:271-302``)."""
    hip_ops._check_device(grad_output, weight)
    if grad_output.ndim != 5 or weight.ndim != 5:
        raise ValueError("grad_output and weight must be NCDHW and C1KKK tensors")
    _check_block(block)
    return hip_ops.depthwise_input_grad(grad_output, weight)


def depthwise_stride2_input_grad(grad_output: Tensor, weight: Tensor, input_spatial_size, block: int = 256) -> Tensor:
    """Stride-two, same-padding depthwise Conv3d dX (reference ``depthwise.py:305-348``):
    the input gradient has ``input_spatial_size``; ``grad_output`` must be its
    ``(size + 1) // 2`` image."""
    hip_ops._check_device(grad_output, weight)
    if grad_output.ndim != 5 or weight.ndim != 5:
        raise ValueError("grad_output and weight must be NCDHW and C1KKK tensors")
    if not (grad_output.is_contiguous() and weight.is_contiguous()):
        raise ValueError("contiguous tensors are required")
    if len(input_spatial_size) != 3:
        raise ValueError("input_spatial_size must contain D, H, and W")
    _check_block(block)
    big = [int(s) for s in input_spatial_size]
    if list(grad_output.shape[2:]) != strided_spatial(big):
        raise ValueError("grad_output shape does not match stride-two same padding")
    return hip_ops.depthwise_s2_scatter(grad_output, weight, None, big)


def depthwise_weight_grad(x: Tensor, grad_output: Tensor, splits: int = 64, block: int = 512, kernel_size: int = 3) -> Tensor:
    """Depthwise dW ``[C, 1, k, k, k]`` in x.dtype (reference ``depthwise.py:351-390``)."""
    hip_ops._check_device(x, grad_output)
    _check_split_launch(splits, block)
    _check_kernel_size(kernel_size)
    return hip_ops.depthwise_weight_grad(x, grad_output, kernel_size)[0]


def depthwise_transpose_weight_grad(
    x: Tensor, grad_output: Tensor, splits: int = 64, block: int = 512, kernel_size: int = 3
) -> Tensor:
    """dW of the stride-two, same-padding depthwise ConvTranspose3d: ``x`` is the
    small input, ``grad_output`` its ``2 * size - 1`` image (reference
    ``depthwise.py:393-442``)."""
    hip_ops._check_device(x, grad_output)
    if x.ndim != 5 or grad_output.ndim != 5:
        raise ValueError("x and grad_output must be NCDHW tensors")
    if x.shape[:2] != grad_output.shape[:2]:
        raise ValueError("x and grad_output must have matching batch and channels")
    if not (x.is_contiguous() and grad_output.is_contiguous()):
        raise ValueError("contiguous NCDHW tensors are required")
    _check_split_launch(splits, block)
    _check_kernel_size(kernel_size)
    if tuple(grad_output.shape[2:]) != tuple(2 * int(s) - 1 for s in x.shape[2:]):
        raise ValueError("grad_output must have spatial shape 2 * x.shape[2:] - 1")
    # dW[t] = sum_o x[o] * dy[2o + t - k//2]: the stride-2 reduction with the
    # transposed output as the big operand.
    return hip_ops.depthwise_s2_wgrad(grad_output, x, kernel_size)[0]


# ---------------------------------------------------------------- gradient ops


@torch.library.custom_op("mednext_accel::depthwise_weight_grad_odd_regular", mutates_args=())
def depthwise_weight_grad_regular(
    x: Tensor,
    grad_output: Tensor,
    kernel_size: int,
    channels: int,
    spatial_size: int,
    splits: int,
    block: int,
) -> Tensor:
    """dW of one regular depthwise shape (reference ``depthwise.py:445-483``)."""
    _check_static_shape(x, channels, spatial_size, "x")
    _check_split_launch(splits, block)
    return hip_ops.depthwise_weight_grad(x.contiguous(), grad_output.contiguous(), kernel_size)[0]


@depthwise_weight_grad_regular.register_fake
def _(x, grad_output, kernel_size, channels, spatial_size, splits, block):
    return x.new_empty((channels, 1, kernel_size, kernel_size, kernel_size))


@torch.library.custom_op("mednext_accel::depthwise_input_grad_odd_regular", mutates_args=())
def depthwise_input_grad_regular(
    grad_output: Tensor,
    weight: Tensor,
    kernel_size: int,
    channels: int,
    spatial_size: int,
    block: int,
) -> Tensor:
    """dX of one regular depthwise shape (reference ``depthwise.py:486-513``)."""
    _check_static_shape(grad_output, channels, spatial_size, "grad_output")
    _check_weight(weight, channels, kernel_size)
    _check_block(block)
    return hip_ops.depthwise_input_grad(grad_output.contiguous(), weight.contiguous())


@depthwise_input_grad_regular.register_fake
def _(grad_output, weight, kernel_size, channels, spatial_size, block):
    return torch.empty_like(grad_output, memory_format=torch.contiguous_format)


@torch.library.custom_op("mednext_accel::depthwise_input_grad_stride2_regular", mutates_args=())
def depthwise_input_grad_stride2_regular(
    grad_output: Tensor, weight: Tensor, channels: int, spatial_size: int, block: int
) -> Tensor:
    """dX of one stride-two depthwise shape; ``spatial_size`` is the input's
    (reference ``depthwise.py:516-546``)."""
    if grad_output.ndim != 5 or int(grad_output.shape[1]) != int(channels):
        raise ValueError(f"grad_output has shape {tuple(grad_output.shape)}, which does not match channels={channels}")
    _check_block(block)
    big = [int(spatial_size)] * 3
    if list(grad_output.shape[2:]) != strided_spatial(big):
        raise ValueError("grad_output shape does not match stride-two same padding")
    return hip_ops.depthwise_s2_scatter(grad_output.contiguous(), weight.contiguous(), None, big)


@depthwise_input_grad_stride2_regular.register_fake
def _(grad_output, weight, channels, spatial_size, block):
    return grad_output.new_empty((grad_output.shape[0], channels, spatial_size, spatial_size, spatial_size))


@torch.library.custom_op("mednext_accel::depthwise_transpose_weight_grad_odd_regular", mutates_args=())
def depthwise_transpose_weight_grad_regular(
    x: Tensor,
    grad_output: Tensor,
    kernel_size: int,
    channels: int,
    spatial_size: int,
    splits: int,
    block: int,
) -> Tensor:
    """dW of one stride-two depthwise transpose shape; ``spatial_size`` is the
    input's (reference ``depthwise.py:722-765``)."""
    _check_static_shape(x, channels, spatial_size, "x")
    return depthwise_transpose_weight_grad(x.contiguous(), grad_output.contiguous(), splits, block, kernel_size)


@depthwise_transpose_weight_grad_regular.register_fake
def _(x, grad_output, kernel_size, channels, spatial_size, splits, block):
    return x.new_empty((channels, 1, kernel_size, kernel_size, kernel_size))


# Internal: dW and the fused dB of one pass, for the autograd formulas below
# (the public weight-gradient ops return dW alone, as the reference's do).
@torch.library.custom_op("mednext_accel::_depthwise_weight_bias_grad_odd_regular", mutates_args=())
def _weight_bias_grad(x: Tensor, grad_output: Tensor, kernel_size: int) -> tuple[Tensor, Tensor]:
    return hip_ops.depthwise_weight_grad(x.contiguous(), grad_output.contiguous(), kernel_size)


@_weight_bias_grad.register_fake
def _(x, grad_output, kernel_size):
    c = x.shape[1]
    return x.new_empty((c, 1, kernel_size, kernel_size, kernel_size)), x.new_empty((c,))


@torch.library.custom_op("mednext_accel::_depthwise_stride2_weight_bias_grad", mutates_args=())
def _s2_weight_bias_grad(big: Tensor, small: Tensor, kernel_size: int) -> tuple[Tensor, Tensor]:
    return hip_ops.depthwise_s2_wgrad(big.contiguous(), small.contiguous(), kernel_size)


@_s2_weight_bias_grad.register_fake
def _(big, small, kernel_size):
    c = big.shape[1]
    return big.new_empty((c, 1, kernel_size, kernel_size, kernel_size)), big.new_empty((c,))


# --------------------------------------------------------------- stride one


@torch.library.custom_op("mednext_accel::depthwise_conv3d_odd_regular", mutates_args=())
def depthwise_conv3d_regular(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    kernel_size: int,
    channels: int,
    spatial_size: int,
    dw_splits: int,
    dw_block: int,
    dx_block: int,
    custom_dx: bool = True,
    custom_dw: bool = True,
) -> Tensor:
    """Depthwise Conv3d, stride one, padding k//2 (reference ``depthwise.py:549-563``,
    whose forward is ``F.conv3d``; here the HIP stencil runs it). ``custom_dx`` /
    ``custom_dw`` choose HIP or ATen for the two backward phases, as in the
    reference."""
    _check_static_shape(x, channels, spatial_size, "x")
    _check_weight(weight, channels, kernel_size)
    _check_split_launch(dw_splits, dw_block)
    _check_block(dx_block)
    return hip_ops.depthwise_forward(x.contiguous(), weight.contiguous(), None if bias is None else bias.contiguous())


@depthwise_conv3d_regular.register_fake
def _(x, weight, bias, kernel_size, channels, spatial_size, dw_splits, dw_block, dx_block, custom_dx=True, custom_dw=True):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _save_regular(ctx, inputs, output):
    x, weight, bias, kernel_size, channels, spatial_size, dw_splits, dw_block, dx_block, custom_dx, custom_dw = inputs
    ctx.save_for_backward(x, weight)
    ctx.has_bias = bias is not None
    ctx.launch = (kernel_size, channels, spatial_size, dw_splits, dw_block, dx_block)
    ctx.custom = (custom_dx, custom_dw)


def _native_conv_backward(grad_output, x, weight, has_bias, stride, padding, transposed, mask):
    channels = x.shape[1]
    return torch.ops.aten.convolution_backward(
        grad_output, x, weight, [channels] if has_bias else None, [stride] * 3, [padding] * 3,
        [1, 1, 1], transposed, [0, 0, 0], channels, mask,
    )


def _regular_grads(ctx, grad_output):
    """Per-phase HIP / ATen backward (the mask logic of reference
    ``depthwise.py:609-648``); dB rides on the HIP dW pass when it runs."""
    x, weight = ctx.saved_tensors
    kernel_size, channels, spatial_size, dw_splits, dw_block, dx_block = ctx.launch
    custom_dx, custom_dw = ctx.custom
    grad_output = grad_output.contiguous()
    want_dx, want_dw, want_db = ctx.needs_input_grad[:3]
    want_db = want_db and ctx.has_bias
    fused_db = want_db and custom_dw
    mask = [want_dx and not custom_dx, want_dw and not custom_dw, want_db and not fused_db]
    grads = [None, None, None]
    if any(mask):
        grads = list(_native_conv_backward(grad_output, x, weight, ctx.has_bias, 1, kernel_size // 2, False, mask))
    if want_dx and custom_dx:
        grads[0] = depthwise_input_grad_regular(grad_output, weight, kernel_size, channels, spatial_size, dx_block)
    if custom_dw and (want_dw or fused_db):
        dw, db = _weight_bias_grad(x, grad_output, kernel_size)
        grads[1] = dw if want_dw else None
        if fused_db:
            grads[2] = db
    return (*grads, None, None, None, None, None, None, None, None)


depthwise_conv3d_regular.register_autograd(_regular_grads, setup_context=_save_regular)


# --------------------------------------------------------------- stride two


@torch.library.custom_op("mednext_accel::depthwise_conv3d_stride2_regular", mutates_args=())
def depthwise_conv3d_stride2_regular(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    kernel_size: int,
    channels: int,
    spatial_size: int,
    dx_block: int,
) -> Tensor:
    """Depthwise Conv3d, stride two, padding k//2: the MedNeXt down block
    (reference ``depthwise.py:654-719``; there the forward and dW are ATen's)."""
    _check_static_shape(x, channels, spatial_size, "x")
    _check_weight(weight, channels, kernel_size)
    _check_block(dx_block)
    return hip_ops.depthwise_s2_gather(
        x.contiguous(), weight.contiguous(), None if bias is None else bias.contiguous(), strided_spatial(x.shape[2:])
    )


@depthwise_conv3d_stride2_regular.register_fake
def _(x, weight, bias, kernel_size, channels, spatial_size, dx_block):
    size = (spatial_size + 1) // 2
    return x.new_empty((x.shape[0], channels, size, size, size))


def _save_stride2(ctx, inputs, output):
    x, weight, bias, kernel_size, channels, spatial_size, dx_block = inputs
    ctx.save_for_backward(x, weight)
    ctx.has_bias = bias is not None
    ctx.launch = (kernel_size, channels, spatial_size, dx_block)


def _stride2_grads(ctx, grad_output):
    x, weight = ctx.saved_tensors
    kernel_size, channels, spatial_size, dx_block = ctx.launch
    grad_output = grad_output.contiguous()
    want_dx, want_dw, want_db = ctx.needs_input_grad[:3]
    want_db = want_db and ctx.has_bias
    dx = dw = db = None
    if want_dx:
        dx = depthwise_input_grad_stride2_regular(grad_output, weight, channels, spatial_size, dx_block)
    if want_dw or want_db:
        # dW[t] = sum_o dy[o] x[2o + t - k//2]; the second output is sum(dy) = dB.
        dw_all, db_all = _s2_weight_bias_grad(x, grad_output, kernel_size)
        dw = dw_all if want_dw else None
        db = db_all if want_db else None
    return dx, dw, db, None, None, None, None


depthwise_conv3d_stride2_regular.register_autograd(_stride2_grads, setup_context=_save_stride2)


# ------------------------------------------------------------- transposed


@torch.library.custom_op("mednext_accel::depthwise_conv_transpose3d_odd_regular", mutates_args=())
def depthwise_conv_transpose3d_regular(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    kernel_size: int,
    channels: int,
    spatial_size: int,
    dw_splits: int,
    dw_block: int,
) -> Tensor:
    """Depthwise ConvTranspose3d, stride two, padding k//2, output ``2 * size - 1``:
    the MedNeXt up block (reference ``depthwise.py:768-850``; there the forward
    and dX are ATen's)."""
    _check_static_shape(x, channels, spatial_size, "x")
    _check_weight(weight, channels, kernel_size)
    _check_split_launch(dw_splits, dw_block)
    return hip_ops.depthwise_s2_scatter(
        x.contiguous(), weight.contiguous(), None if bias is None else bias.contiguous(),
        [2 * int(spatial_size) - 1] * 3,
    )


@depthwise_conv_transpose3d_regular.register_fake
def _(x, weight, bias, kernel_size, channels, spatial_size, dw_splits, dw_block):
    size = 2 * spatial_size - 1
    return x.new_empty((x.shape[0], channels, size, size, size))


def _save_transpose(ctx, inputs, output):
    x, weight, bias, kernel_size, channels, spatial_size, dw_splits, dw_block = inputs
    ctx.save_for_backward(x, weight)
    ctx.has_bias = bias is not None
    ctx.launch = (kernel_size, channels, spatial_size, dw_splits, dw_block)


def _transpose_grads(ctx, grad_output):
    x, weight = ctx.saved_tensors
    kernel_size, channels, spatial_size, dw_splits, dw_block = ctx.launch
    grad_output = grad_output.contiguous()
    want_dx, want_dw, want_db = ctx.needs_input_grad[:3]
    dx = dw = db = None
    if want_dx:
        # The transposed conv's input gradient is the stride-two conv of dy.
        dx = hip_ops.depthwise_s2_gather_op(grad_output, weight.contiguous(), list(x.shape[2:]))
    if want_dw:
        dw = depthwise_transpose_weight_grad_regular(
            x, grad_output, kernel_size, channels, spatial_size, dw_splits, dw_block
        )
    if want_db and ctx.has_bias:
        acc = torch.float64 if x.dtype == torch.float64 else torch.float32
        db = grad_output.reshape(grad_output.shape[0], grad_output.shape[1], -1).sum(dim=2, dtype=acc)
        db = db.sum(dim=0).to(x.dtype)
    return dx, dw, db, None, None, None, None, None


depthwise_conv_transpose3d_regular.register_autograd(_transpose_grads, setup_context=_save_transpose)

