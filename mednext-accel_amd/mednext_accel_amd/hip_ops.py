"""PyTorch operators backed by libmednext_hip.so.

Two layers, mirroring the reference's ``ops/_triton/depthwise.py``:

* low-level launchers (``depthwise_forward``, ``depthwise_input_grad``,
  ``depthwise_weight_grad``, ``group_norm_forward``, ``group_norm_backward``) that
  validate tensors and raise ``ValueError`` exactly where the reference's
  launchers do (reference ``ops/_triton/depthwise.py:271-302, 351-390``);
* ``torch.library`` custom ops under the ``mednext_accel_amd`` namespace with
  fake-tensor and autograd registrations, so they trace under
  ``torch.compile(fullgraph=True)`` and pass ``torch.library.opcheck``.

Every kernel runs on PyTorch's current stream; every output and workspace is
allocated by PyTorch. There is no fallback: if the library is missing the
launch raises.
"""

from __future__ import annotations

import functools
import math

import torch
from torch import Tensor

from . import _hip
from .tiles import (
    ENGINE_MFMA,
    ENGINE_VALU,
    ENGINE_VOLUME,
    VOLUME_BAND,
    depthwise_recipe,
    group_norm_splits,
    pointwise_blocks,
    pointwise_wgrad_splits,
)

SUPPORTED_KERNELS = (1, 3, 5)


# --------------------------------------------------------------------------- checks


def _check_device(*tensors: Tensor) -> None:
    if not all(t.is_cuda for t in tensors):
        raise ValueError("CUDA (ROCm) tensors are required")


def _check_recipe(recipe) -> tuple[int, int, int]:
    if recipe is None or len(recipe) != 3:
        raise ValueError("recipe must be [engine, tile_w, depth_chunk]")
    return _checked_recipe(tuple(int(v) for v in recipe))


@functools.lru_cache(maxsize=4096)
def _checked_recipe(recipe: tuple[int, int, int]) -> tuple[int, int, int]:
    if len(recipe) != 3:
        raise ValueError("recipe must be [engine, tile_w, depth_chunk]")
    engine, tile_w, depth_chunk = (int(v) for v in recipe)
    if engine == ENGINE_VALU:
        if tile_w not in (4, 8, 16, 32, 64):
            raise ValueError("VALU tile_w must be 4, 8, 16, 32 or 64")
    elif engine == ENGINE_MFMA:
        if tile_w not in (32, 64, 128):
            raise ValueError("MFMA tile_w must be 32, 64 or 128")
    elif engine == ENGINE_VOLUME:
        if tile_w != VOLUME_BAND:
            raise ValueError(f"volume-engine tile_w must be {VOLUME_BAND}")
    else:
        raise ValueError("engine must be 0 (VALU), 1 (MFMA) or 2 (VOLUME)")
    if depth_chunk < 1:
        raise ValueError("depth_chunk must be >= 1")
    return engine, tile_w, depth_chunk


def _check_depthwise(x: Tensor, weight: Tensor) -> int:
    if x.ndim != 5 or weight.ndim != 5:
        raise ValueError("input and weight must be NCDHW and C1KKK tensors")
    if not (x.is_contiguous() and weight.is_contiguous()):
        raise ValueError("contiguous tensors are required")
    channels = x.shape[1]
    if weight.shape[0] != channels or weight.shape[1] != 1 or len(set(weight.shape[2:])) != 1:
        raise ValueError("weight must have shape [C, 1, K, K, K]")
    kernel_size = int(weight.shape[2])
    if kernel_size < 1 or kernel_size % 2 == 0:
        raise ValueError("kernel_size must be a positive odd integer")
    if kernel_size not in SUPPORTED_KERNELS:
        raise ValueError(f"kernel_size must be one of {SUPPORTED_KERNELS}")
    if weight.dtype != x.dtype:
        raise ValueError("weight must have the input's dtype")
    return kernel_size


def _recipe_for(x: Tensor, kernel_size: int, recipe, phase: str) -> tuple[int, int, int]:
    if recipe is None:
        n, c, d, h, w = (int(v) for v in x.shape)
        dtype = str(x.dtype).removeprefix("torch.")
        recipe = depthwise_recipe(n, c, (d, h, w), kernel_size, dtype, phase)
    return _check_recipe(recipe)


# ------------------------------------------------------------------ low-level launchers


def depthwise_forward(
    x: Tensor, weight: Tensor, bias: Tensor | None = None, recipe=None
) -> Tensor:
    """y = conv3d(x, weight, bias, padding=k//2, groups=C) on the HIP stencil kernel."""
    _check_device(x, weight, *(() if bias is None else (bias,)))
    kernel_size = _check_depthwise(x, weight)
    if bias is not None and (bias.shape != (x.shape[1],) or bias.dtype != x.dtype):
        raise ValueError("bias must be [C] in the input's dtype")
    engine, tile_w, depth_chunk = _recipe_for(x, kernel_size, recipe, "forward")
    y = torch.empty_like(x)
    if x.numel() == 0:
        return y
    n, c, d, h, w = x.shape
    lib = _hip.load()
    _hip.check(
        lib.mednext_depthwise3d_fwd(
            x.data_ptr(), weight.data_ptr(), _hip.ptr(bias.contiguous() if bias is not None else None),
            y.data_ptr(), n, c, d, h, w, kernel_size, _hip.dtype_code(x.dtype), engine, tile_w,
            depth_chunk, _hip.stream_of(x),
        ),
        "mednext_depthwise3d_fwd",
    )
    return y


def depthwise_input_grad(grad_output: Tensor, weight: Tensor, recipe=None) -> Tensor:
    """Stride-one same-padding depthwise dX (reference depthwise.py:271-302)."""
    _check_device(grad_output, weight)
    kernel_size = _check_depthwise(grad_output, weight)
    engine, tile_w, depth_chunk = _recipe_for(grad_output, kernel_size, recipe, "input_grad")
    out = torch.empty_like(grad_output)
    if grad_output.numel() == 0:
        return out
    n, c, d, h, w = grad_output.shape
    lib = _hip.load()
    _hip.check(
        lib.mednext_depthwise3d_dgrad(
            grad_output.data_ptr(), weight.data_ptr(), out.data_ptr(), n, c, d, h, w,
            kernel_size, _hip.dtype_code(grad_output.dtype), engine, tile_w, depth_chunk,
            _hip.stream_of(grad_output),
        ),
        "mednext_depthwise3d_dgrad",
    )
    return out


def depthwise_weight_grad(
    x: Tensor, grad_output: Tensor, kernel_size: int = 3, recipe=None
) -> tuple[Tensor, Tensor]:
    """Depthwise dW [C,1,k,k,k] and fused dB [C], both in x.dtype
    (reference depthwise.py:351-390 computes dW only; dB came from ATen)."""
    _check_device(x, grad_output)
    if x.shape != grad_output.shape or x.ndim != 5:
        raise ValueError("x and grad_output must have the same NCDHW shape")
    if not (x.is_contiguous() and grad_output.is_contiguous()):
        raise ValueError("contiguous NCDHW tensors are required")
    if x.dtype != grad_output.dtype:
        raise ValueError("x and grad_output must share a dtype")
    if kernel_size < 1 or kernel_size % 2 == 0:
        raise ValueError("kernel_size must be a positive odd integer")
    if kernel_size not in SUPPORTED_KERNELS:
        raise ValueError(f"kernel_size must be one of {SUPPORTED_KERNELS}")
    n, c, d, h, w = (int(s) for s in x.shape)
    engine, tile_w, depth_chunk = _recipe_for(x, kernel_size, recipe, "weight_grad")
    grad_weight = torch.empty((c, 1, kernel_size, kernel_size, kernel_size), device=x.device, dtype=x.dtype)
    grad_bias = torch.empty((c,), device=x.device, dtype=x.dtype)
    if x.numel() == 0:
        return grad_weight.zero_(), grad_bias.zero_()
    code = _hip.dtype_code(x.dtype)
    lib = _hip.load()
    nbytes = _wgrad_workspace_bytes(n, c, d, h, w, kernel_size, code, engine, tile_w, depth_chunk)
    if nbytes == 0:
        raise _hip.HipLibraryError(f"wgrad workspace query failed: {_hip.last_error()}")
    workspace = torch.empty((nbytes,), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_depthwise3d_wgrad(
            x.data_ptr(), grad_output.data_ptr(), grad_weight.data_ptr(), grad_bias.data_ptr(),
            workspace.data_ptr(), nbytes, n, c, d, h, w, kernel_size, code, engine, tile_w,
            depth_chunk, _hip.stream_of(x),
        ),
        "mednext_depthwise3d_wgrad",
    )
    return grad_weight, grad_bias


def depthwise_input_grad_acc(grad_output: Tensor, weight: Tensor, accumulate: Tensor, recipe) -> Tensor:
    """``depthwise_input_grad(grad_output, weight) + accumulate`` in one pass
    (bf16, k in {3, 5}, matrix-core recipe): the add rides on the kernel's store."""
    k = _check_depthwise(grad_output, weight)
    if k not in (3, 5) or grad_output.dtype != torch.bfloat16:
        raise ValueError("the accumulating input gradient takes bf16 k = 3 or 5")
    if accumulate.shape != grad_output.shape or accumulate.dtype != torch.bfloat16 or not accumulate.is_contiguous():
        raise ValueError("accumulate must be a contiguous bf16 tensor shaped like grad_output")
    engine, tile_w, depth_chunk = _recipe_for(grad_output, k, recipe, "input_grad")
    if engine != ENGINE_MFMA:
        raise ValueError("the accumulating input gradient runs the matrix-core engine")
    n, c, d, h, w = (int(s) for s in grad_output.shape)
    dx = torch.empty_like(grad_output)
    _hip.check(
        _hip.load().mednext_depthwise3d_dgrad_acc(
            grad_output.data_ptr(), weight.data_ptr(), accumulate.data_ptr(), dx.data_ptr(), n, c, d, h, w, k,
            _hip.dtype_code(grad_output.dtype), engine, tile_w, depth_chunk, _hip.stream_of(grad_output),
        ),
        "mednext_depthwise3d_dgrad_acc",
    )
    return dx


class DepthwiseResidualTap(torch.autograd.Function):
    """``(depthwise(x), x)`` for a block whose input also feeds its residual
    add (reference models/blocks.py:82-91): the residual branch takes the
    second output, so both gradients of x arrive in this function's backward
    and are summed by the input-gradient kernel's store
    (``depthwise_input_grad_acc``) instead of by a separate autograd add.
    HIP recipes for all three phases (bf16, k = 3 or 5, matrix-core input
    gradient)."""

    @staticmethod
    def forward(ctx, x, weight, bias, kernel_size, fwd_recipe, dx_recipe, dw_recipe):
        ctx.save_for_backward(x, weight)
        ctx.kernel_size, ctx.dx_recipe, ctx.dw_recipe = kernel_size, dx_recipe or None, dw_recipe or None
        ctx.has_bias = bias is not None
        return depthwise_forward(x, weight, bias, fwd_recipe or None), x

    @staticmethod
    def backward(ctx, grad_d, grad_x):
        x, weight = ctx.saved_tensors
        need_x, need_w, need_b = ctx.needs_input_grad[:3]
        dx = dw = db = None
        if grad_d is None:
            return grad_x, None, None, None, None, None, None
        grad_d = grad_d.contiguous()
        if need_x:
            if grad_x is not None and grad_x.dtype == grad_d.dtype:
                dx = depthwise_input_grad_acc(grad_d, weight, grad_x.contiguous(), ctx.dx_recipe)
            else:
                dx = depthwise_input_grad(grad_d, weight, ctx.dx_recipe)
                if grad_x is not None:
                    dx = dx + grad_x
        if need_w or (need_b and ctx.has_bias):
            dw, db = depthwise_weight_grad(x, grad_d, ctx.kernel_size, ctx.dw_recipe)
        return dx, dw if need_w else None, db if (need_b and ctx.has_bias) else None, None, None, None, None


@functools.lru_cache(maxsize=4096)
def _wgrad_workspace_bytes(*args: int) -> int:
    return int(_hip.load().mednext_depthwise3d_wgrad_workspace_bytes(*args))


def _stats_dtype(x: Tensor) -> torch.dtype:
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def group_norm_forward(
    x: Tensor,
    weight: Tensor | None,
    bias: Tensor | None,
    eps: float = 1e-5,
    out_dtype: torch.dtype | None = None,
    splits: int | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """GroupNorm(C, C) forward: returns (y, mean [N*C], rstd [N*C])."""
    _check_device(x)
    if x.ndim < 2 or not x.is_contiguous():
        raise ValueError("a contiguous [N, C, ...] input is required")
    n, c = int(x.shape[0]), int(x.shape[1])
    v = x.numel() // max(1, n * c)
    params = [p for p in (weight, bias) if p is not None]
    pdtype = params[0].dtype if params else torch.float32
    for p in params:
        if p.shape != (c,) or p.dtype != pdtype or not p.is_cuda:
            raise ValueError("affine parameters must be [C] CUDA tensors of one dtype")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    y = torch.empty(x.shape, device=x.device, dtype=out_dtype)
    mean = torch.empty((n * c,), device=x.device, dtype=_stats_dtype(x))
    rstd = torch.empty_like(mean)
    if x.numel() == 0:
        return y, mean, rstd
    splits = group_norm_splits(n, c, v) if splits is None else int(splits)
    lib = _hip.load()
    nbytes = lib.mednext_group_norm_workspace_bytes(n, c, v, splits)
    workspace = torch.empty((max(1, nbytes),), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_group_norm_fwd(
            x.data_ptr(), _hip.dtype_code(x.dtype), _hip.ptr(weight), _hip.ptr(bias),
            _hip.dtype_code(pdtype), y.data_ptr(), _hip.dtype_code(out_dtype), mean.data_ptr(),
            rstd.data_ptr(), n, c, v, float(eps), splits, workspace.data_ptr(), nbytes,
            _hip.stream_of(x),
        ),
        "mednext_group_norm_fwd",
    )
    return y, mean, rstd


def group_norm_stats(
    x: Tensor,
    weight: Tensor | None,
    bias: Tensor | None,
    eps: float = 1e-5,
    splits: int | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """GroupNorm(C, C) statistics without the normalised tensor: (coef [N, C, 4]
    float64 = (rstd * gamma, beta, mean, rstd), the NORM prologue's records,
    with which the pointwise kernels reproduce ``group_norm_forward``'s bf16
    output bit for bit; mean [N*C]; rstd [N*C]), mean / rstd bit-identical to
    ``group_norm_forward``'s."""
    _check_device(x)
    if x.ndim < 2 or not x.is_contiguous() or x.numel() == 0:
        raise ValueError("a nonempty contiguous [N, C, ...] input is required")
    n, c = int(x.shape[0]), int(x.shape[1])
    v = x.numel() // (n * c)
    params = [p for p in (weight, bias) if p is not None]
    pdtype = params[0].dtype if params else torch.float32
    for p in params:
        if p.shape != (c,) or p.dtype != pdtype or not p.is_cuda:
            raise ValueError("affine parameters must be [C] CUDA tensors of one dtype")
    coef = torch.empty((n, c, 4), device=x.device, dtype=torch.float64)
    mean = torch.empty((n * c,), device=x.device, dtype=_stats_dtype(x))
    rstd = torch.empty_like(mean)
    splits = group_norm_splits(n, c, v) if splits is None else int(splits)
    lib = _hip.load()
    nbytes = lib.mednext_group_norm_workspace_bytes(n, c, v, splits)
    workspace = torch.empty((max(1, nbytes),), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_group_norm_stats(
            x.data_ptr(), _hip.dtype_code(x.dtype), _hip.ptr(weight), _hip.ptr(bias), _hip.dtype_code(pdtype),
            mean.data_ptr(), rstd.data_ptr(), coef.data_ptr(), n, c, v, float(eps), splits, workspace.data_ptr(),
            nbytes, _hip.stream_of(x),
        ),
        "mednext_group_norm_stats",
    )
    return coef, mean, rstd


def group_norm_backward(
    grad_output: Tensor,
    x: Tensor,
    mean: Tensor,
    rstd: Tensor,
    weight: Tensor | None,
    need_input: bool = True,
    need_weight: bool = True,
    need_bias: bool = True,
    param_dtype: torch.dtype = torch.float32,
    splits: int | None = None,
) -> tuple[Tensor | None, Tensor | None, Tensor | None]:
    """GroupNorm(C, C) backward: (dx in x.dtype, dgamma, dbeta in param_dtype)."""
    _check_device(grad_output, x, mean, rstd)
    if grad_output.shape != x.shape or not (grad_output.is_contiguous() and x.is_contiguous()):
        raise ValueError("grad_output and x must be contiguous with the same shape")
    n, c = int(x.shape[0]), int(x.shape[1])
    v = x.numel() // max(1, n * c)
    if weight is not None:
        param_dtype = weight.dtype
    dx = torch.empty_like(x) if need_input else None
    dgamma = torch.empty((c,), device=x.device, dtype=param_dtype) if need_weight else None
    dbeta = torch.empty((c,), device=x.device, dtype=param_dtype) if need_bias else None
    if x.numel() == 0:
        return dx, (None if dgamma is None else dgamma.zero_()), (None if dbeta is None else dbeta.zero_())
    splits = group_norm_splits(n, c, v) if splits is None else int(splits)
    lib = _hip.load()
    nbytes = lib.mednext_group_norm_workspace_bytes(n, c, v, splits)
    workspace = torch.empty((max(1, nbytes),), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_group_norm_bwd(
            grad_output.data_ptr(), _hip.dtype_code(grad_output.dtype), x.data_ptr(),
            _hip.dtype_code(x.dtype), mean.data_ptr(), rstd.data_ptr(), _hip.ptr(weight),
            _hip.dtype_code(param_dtype), _hip.ptr(dx), _hip.ptr(dgamma), _hip.ptr(dbeta), n, c,
            v, splits, workspace.data_ptr(), nbytes, _hip.stream_of(x),
        ),
        "mednext_group_norm_bwd",
    )
    return dx, dgamma, dbeta


# --------------------------------------------------------------------- pointwise

PW_PROLOGUE_NONE, PW_PROLOGUE_GELU, PW_PROLOGUE_AFFINE, PW_PROLOGUE_NORM = 0, 1, 2, 3
PW_EPILOGUE_BIAS, PW_EPILOGUE_BIAS_GELU, PW_EPILOGUE_BIAS_RESIDUAL, PW_EPILOGUE_GELU_GRAD = 0, 1, 2, 3
PW_EPILOGUE_ROW_REDUCE, PW_EPILOGUE_AFFINE_SCALE, PW_EPILOGUE_BIAS_GELU_PAIR, PW_EPILOGUE_AUX_SCALE = 4, 5, 6, 7
#: Forward kernel family (include/mednext_hip.h ``mednext_pw_kernels``): the
#: library's automatic choice, the streaming kernels only, or the LDS-tiled
#: kernel wherever it applies.
PW_KERNELS_AUTO, PW_KERNELS_STREAMING, PW_KERNELS_TILED, PW_KERNELS_TILED_64 = 0, 1, 2, 3


def set_pointwise_kernels(choice: int) -> None:
    """Process-wide choice of the forward kernel family (``PW_KERNELS_*``)."""
    _hip.check(_hip.load().mednext_pointwise_set_kernels(int(choice)), "mednext_pointwise_set_kernels")
    pointwise_fwd_workspace_bytes.cache_clear()


def pointwise_uses_tiled(n: int, k: int, m: int, v: int, prologue: int = 0, epilogue: int = 0) -> bool:
    """Whether a ``pointwise_conv`` of this shape and mode (automatic launch
    shape) runs the tiled kernel under the current choice."""
    return bool(_hip.load().mednext_pointwise_uses_tiled(n, k, m, v, prologue, epilogue))


def _weight2d(weight: Tensor) -> Tensor:
    if weight.ndim not in (2, 5) or (weight.ndim == 5 and tuple(weight.shape[2:]) != (1, 1, 1)):
        raise ValueError("pointwise weight must be [Cout, Cin] or [Cout, Cin, 1, 1, 1]")
    return weight.reshape(weight.shape[0], weight.shape[1])


def _check_pointwise_tensor(t: Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.ndim < 3:
        raise ValueError(f"{name} must be [N, C, *spatial]")


def pointwise_conv(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None = None,
    *,
    aux: Tensor | None = None,
    prologue: int = PW_PROLOGUE_NONE,
    epilogue: int = PW_EPILOGUE_BIAS,
    transpose: bool = False,
    blocks: int | None = None,
    prologue_coef: Tensor | None = None,
    epilogue_coef: Tensor | None = None,
    row_partial: Tensor | None = None,
    aux2: Tensor | None = None,
) -> Tensor | tuple[Tensor, Tensor] | None:
    """``y = epilogue(W . prologue(x) [+ b])`` per sample on the matrix cores.

    ``weight`` is the conv's [Cout, Cin(, 1, 1, 1)]; with ``transpose=True`` the
    product is ``W^T . x`` (the conv's input gradient). ``aux`` (and ``aux2``
    for AFFINE_SCALE) are per-element operands shaped like ``y``: the residual
    (BIAS_RESIDUAL), the GELU pre-activation (GELU_GRAD), the row-sum weights
    (ROW_REDUCE). ``prologue_coef`` ([N, K, 4] float64) feeds AFFINE / NORM,
    ``epilogue_coef`` ([N, M, 2] float64) AFFINE_SCALE. ROW_REDUCE writes
    ``row_partial`` ([N, M, slots, 2] float64, slots from
    ``pointwise_row_slots``) and returns None; BIAS_GELU_PAIR returns
    ``(GELU(y), GELU'(y))``.
    """
    _check_device(x, weight)
    _check_pointwise_tensor(x, "x")
    w2 = _weight2d(weight)
    if w2.dtype != torch.bfloat16:
        raise ValueError("weight must be bfloat16")
    w2 = w2.contiguous()
    k, m = (w2.shape[0], w2.shape[1]) if transpose else (w2.shape[1], w2.shape[0])
    if x.shape[1] != k:
        raise ValueError(f"x has {x.shape[1]} channels, the weight expects {k}")
    n, v = x.shape[0], x[0, 0].numel()
    out_shape = (n, m, *x.shape[2:])
    y = None if epilogue == PW_EPILOGUE_ROW_REDUCE else x.new_empty(out_shape)
    y2 = x.new_empty(out_shape) if epilogue == PW_EPILOGUE_BIAS_GELU_PAIR else None
    if bias is not None:
        if bias.shape != (m,) or bias.dtype != torch.bfloat16:
            raise ValueError("bias must be a bfloat16 [Cout] tensor")
        bias = bias.contiguous()
    for t, name in ((aux, "aux"), (aux2, "aux2")):
        if t is not None:
            _check_pointwise_tensor(t, name)
            if tuple(t.shape) != out_shape:
                raise ValueError(f"{name} must have the output's shape")
    if blocks is None:
        blocks = pointwise_blocks(n, k, m, v)
    if epilogue == PW_EPILOGUE_ROW_REDUCE:
        slots = pointwise_row_slots(n, k, m, v, int(blocks))
        if row_partial is None or row_partial.dtype != torch.float64 or row_partial.numel() != n * m * slots * 2:
            raise ValueError("ROW_REDUCE needs a float64 row_partial of N * M * slots * 2 values")
    for t, rows, name in ((prologue_coef, k * 4, "prologue_coef"), (epilogue_coef, m * 2, "epilogue_coef")):
        if t is not None and (t.dtype != torch.float64 or not t.is_contiguous() or t.numel() != n * rows):
            raise ValueError(f"{name} must be a contiguous float64 tensor of {n * rows} values")
    lib = _hip.load()
    ws_bytes = pointwise_fwd_workspace_bytes(n, k, m, v, prologue, epilogue) if int(blocks) == 0 else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _hip.check(
        lib.mednext_pointwise_fwd_ws(
            x.data_ptr(), w2.data_ptr(), _hip.ptr(bias), _hip.ptr(aux), _hip.ptr(aux2), _hip.ptr(y), _hip.ptr(y2),
            n, k, m, v, 1 if transpose else 0, prologue, epilogue, _hip.ptr(prologue_coef),
            _hip.ptr(epilogue_coef), _hip.ptr(row_partial), _hip.DTYPE_CODES[torch.bfloat16],
            int(blocks), _hip.ptr(ws), ws_bytes, _hip.stream_of(x),
        ),
        "mednext_pointwise_fwd_ws",
    )
    return (y, y2) if y2 is not None else y


@functools.lru_cache(maxsize=4096)
def pointwise_fwd_workspace_bytes(n: int, k: int, m: int, v: int, prologue: int, epilogue: int) -> int:
    """Bytes of fp32 partials a ``pointwise_conv`` of this shape needs for the
    tiled product's K split (0: the launch splits nothing). Depends on the
    kernel-family choice, so ``set_pointwise_kernels`` clears this cache."""
    return int(_hip.load().mednext_pointwise_fwd_workspace_bytes(n, k, m, v, prologue, epilogue))


@functools.lru_cache(maxsize=4096)
def pointwise_row_slots(n: int, k: int, m: int, v: int, blocks: int = 0) -> int:
    """Row-sum slots per (sample, row) of a ROW_REDUCE launch of this shape."""
    slots = int(_hip.load().mednext_pointwise_row_slots(n, k, m, v, blocks))
    if slots < 1:
        raise ValueError("unsupported ROW_REDUCE shape")
    return slots


def pointwise_weight_grad(
    grad_output: Tensor,
    x: Tensor,
    *,
    prologue: int = PW_PROLOGUE_NONE,
    with_bias: bool = True,
    splits: int | None = None,
    prologue_coef: Tensor | None = None,
) -> tuple[Tensor, Tensor | None]:
    """(dW [Cout, Cin, 1, 1, 1], dB [Cout] or None) of ``y = W . prologue(x) + b``
    (``prologue_coef`` as for ``pointwise_conv``'s AFFINE / NORM; the library
    maps the raw product's per-sample sums exactly instead of rounding
    prologue(x) to bf16)."""
    _check_device(grad_output, x)
    _check_pointwise_tensor(grad_output, "grad_output")
    _check_pointwise_tensor(x, "x")
    if grad_output.shape[0] != x.shape[0] or grad_output.shape[2:] != x.shape[2:]:
        raise ValueError("grad_output and x must share batch and spatial shape")
    n, k, m, v = x.shape[0], x.shape[1], grad_output.shape[1], x[0, 0].numel()
    if splits is None:
        splits = pointwise_wgrad_splits(n, k, m, v)
    lib = _hip.load()
    nbytes = lib.mednext_pointwise_wgrad_workspace_bytes(n, k, m, v, int(splits))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    dw = x.new_empty((m, k, 1, 1, 1))
    db = x.new_empty((m,)) if with_bias else None
    if prologue_coef is not None and (
        prologue_coef.dtype != torch.float64 or not prologue_coef.is_contiguous() or prologue_coef.numel() != n * k * 4
    ):
        raise ValueError(f"prologue_coef must be a contiguous float64 tensor of {n * k * 4} values")
    _hip.check(
        lib.mednext_pointwise_wgrad_ex(
            grad_output.data_ptr(), x.data_ptr(), dw.data_ptr(), _hip.ptr(db), ws.data_ptr(), nbytes,
            n, k, m, v, prologue, _hip.ptr(prologue_coef), _hip.DTYPE_CODES[torch.bfloat16], int(splits),
            _hip.stream_of(x),
        ),
        "mednext_pointwise_wgrad_ex",
    )
    return dw, db


# ------------------------------------------------------------------------ custom ops


@torch.library.custom_op("mednext_accel_amd::depthwise_input_grad_odd_regular", mutates_args=())
def depthwise_input_grad_regular(
    grad_output: Tensor, weight: Tensor, kernel_size: int, recipe: list[int]
) -> Tensor:
    """dX for one regular depthwise shape (reference depthwise.py:486-513)."""
    return depthwise_input_grad(grad_output.contiguous(), weight.contiguous(), recipe)


@depthwise_input_grad_regular.register_fake
def _(grad_output, weight, kernel_size, recipe):
    return torch.empty_like(grad_output, memory_format=torch.contiguous_format)


@torch.library.custom_op("mednext_accel_amd::depthwise_weight_grad_odd_regular", mutates_args=())
def depthwise_weight_grad_regular(
    x: Tensor, grad_output: Tensor, kernel_size: int, recipe: list[int]
) -> tuple[Tensor, Tensor]:
    """(dW, dB) for one regular depthwise shape (reference depthwise.py:445-483)."""
    return depthwise_weight_grad(x.contiguous(), grad_output.contiguous(), kernel_size, recipe)


@depthwise_weight_grad_regular.register_fake
def _(x, grad_output, kernel_size, recipe):
    c = x.shape[1]
    return (
        x.new_empty((c, 1, kernel_size, kernel_size, kernel_size)),
        x.new_empty((c,)),
    )


@torch.library.custom_op("mednext_accel_amd::depthwise_conv3d_odd_regular", mutates_args=())
def depthwise_conv3d_regular(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None,
    kernel_size: int,
    fwd_recipe: list[int],
    dx_recipe: list[int],
    dw_recipe: list[int],
    custom_fwd: bool = True,
    custom_dx: bool = True,
    custom_dw: bool = True,
) -> Tensor:
    """Depthwise Conv3d with per-phase HIP/native selection
    (reference depthwise.py:549-563, which always runs F.conv3d forward)."""
    if custom_fwd:
        return depthwise_forward(x, weight, bias, fwd_recipe)
    return torch.nn.functional.conv3d(x, weight, bias, padding=kernel_size // 2, groups=x.shape[1])


@depthwise_conv3d_regular.register_fake
def _(x, weight, bias, kernel_size, fwd_recipe, dx_recipe, dw_recipe, custom_fwd=True, custom_dx=True, custom_dw=True):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


def _setup_depthwise(ctx, inputs, output):
    x, weight, bias, kernel_size, _fwd, dx_recipe, dw_recipe, _cf, custom_dx, custom_dw = inputs
    ctx.save_for_backward(x, weight)
    ctx.has_bias = bias is not None
    ctx.kernel_size = kernel_size
    ctx.dx_recipe = list(dx_recipe)
    ctx.dw_recipe = list(dw_recipe)
    ctx.custom_dx = custom_dx
    ctx.custom_dw = custom_dw


def _depthwise_backward(ctx, grad_output):
    """Mirror of the reference's per-phase mask (depthwise.py:609-648), except
    that dB is fused into the custom dW pass instead of always going native."""
    x, weight = ctx.saved_tensors
    grad_output = grad_output.contiguous()
    need_dx, need_dw, need_db = ctx.needs_input_grad[:3]
    need_db = need_db and ctx.has_bias
    custom_db = need_db and need_dw and ctx.custom_dw
    native_mask = [need_dx and not ctx.custom_dx, need_dw and not ctx.custom_dw, need_db and not custom_db]
    grad_input = grad_weight = grad_bias = None
    if any(native_mask):
        pad = ctx.kernel_size // 2
        channels = x.shape[1]
        grad_input, grad_weight, grad_bias = torch.ops.aten.convolution_backward(
            grad_output, x, weight, [channels] if ctx.has_bias else None, [1, 1, 1],
            [pad, pad, pad], [1, 1, 1], False, [0, 0, 0], channels, native_mask,
        )
    if need_dx and ctx.custom_dx:
        grad_input = depthwise_input_grad_regular(grad_output, weight, ctx.kernel_size, ctx.dx_recipe)
    if need_dw and ctx.custom_dw:
        grad_weight, fused_bias = depthwise_weight_grad_regular(x, grad_output, ctx.kernel_size, ctx.dw_recipe)
        if custom_db:
            grad_bias = fused_bias
    return grad_input, grad_weight, grad_bias, None, None, None, None, None, None, None


depthwise_conv3d_regular.register_autograd(_depthwise_backward, setup_context=_setup_depthwise)


@torch.library.custom_op("mednext_accel_amd::group_norm_channels", mutates_args=())
def group_norm_channels(
    x: Tensor, weight: Tensor | None, bias: Tensor | None, eps: float, out_dtype: torch.dtype | None
) -> tuple[Tensor, Tensor, Tensor]:
    """GroupNorm(C, C): (y, mean, rstd). ``out_dtype`` lets a bf16 input produce
    the fp32 output the reference gets from autocast's fp32 group_norm."""
    return group_norm_forward(x.contiguous(), weight, bias, eps, out_dtype)


@group_norm_channels.register_fake
def _(x, weight, bias, eps, out_dtype):
    n, c = x.shape[0], x.shape[1]
    stats = torch.float64 if x.dtype == torch.float64 else torch.float32
    return (
        torch.empty(x.shape, dtype=x.dtype if out_dtype is None else out_dtype, device=x.device),
        x.new_empty((n * c,), dtype=stats),
        x.new_empty((n * c,), dtype=stats),
    )


@torch.library.custom_op("mednext_accel_amd::group_norm_channels_backward", mutates_args=())
def group_norm_channels_backward(
    grad_output: Tensor,
    x: Tensor,
    mean: Tensor,
    rstd: Tensor,
    weight: Tensor | None,
    param_dtype: torch.dtype,
) -> tuple[Tensor, Tensor, Tensor]:
    dx, dgamma, dbeta = group_norm_backward(
        grad_output.contiguous(), x.contiguous(), mean, rstd, weight, True, True, True, param_dtype
    )
    return dx, dgamma, dbeta


@group_norm_channels_backward.register_fake
def _(grad_output, x, mean, rstd, weight, param_dtype):
    c = x.shape[1]
    return (
        torch.empty_like(x, memory_format=torch.contiguous_format),
        x.new_empty((c,), dtype=param_dtype),
        x.new_empty((c,), dtype=param_dtype),
    )


def _setup_group_norm(ctx, inputs, output):
    x, weight, bias, _eps, _out_dtype = inputs
    _y, mean, rstd = output
    ctx.mark_non_differentiable(mean, rstd)
    # mean / rstd never receive gradients: do not let autograd build zero tensors for them.
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, mean, rstd, weight)
    ctx.param_dtype = (weight if weight is not None else bias).dtype if (weight is not None or bias is not None) else torch.float32
    ctx.has_weight = weight is not None
    ctx.has_bias = bias is not None


def _group_norm_backward(ctx, grad_y, _grad_mean, _grad_rstd):
    if grad_y is None:
        return None, None, None, None, None
    x, mean, rstd, weight = ctx.saved_tensors
    dx, dgamma, dbeta = group_norm_channels_backward(
        grad_y, x, mean, rstd, weight if ctx.has_weight else None, ctx.param_dtype
    )
    return (
        dx,
        dgamma if ctx.has_weight else None,
        dbeta if ctx.has_bias else None,
        None,
        None,
    )


group_norm_channels.register_autograd(_group_norm_backward, setup_context=_setup_group_norm)


# ---------------------------------------------------------- pointwise custom ops


@torch.library.custom_op("mednext_accel_amd::pointwise_input_grad", mutates_args=())
def pointwise_input_grad_op(grad_output: Tensor, weight: Tensor) -> Tensor:
    """dX = W^T . dY of a 1x1x1 conv (bf16)."""
    return pointwise_conv(grad_output.contiguous(), weight, transpose=True)


@pointwise_input_grad_op.register_fake
def _(grad_output, weight):
    return grad_output.new_empty((grad_output.shape[0], weight.shape[1], *grad_output.shape[2:]))


@torch.library.custom_op("mednext_accel_amd::pointwise_weight_grad", mutates_args=())
def pointwise_weight_grad_op(grad_output: Tensor, x: Tensor, gelu_input: bool) -> tuple[Tensor, Tensor]:
    """(dW, dB) of ``y = W . act(x) + b`` with act = GELU when ``gelu_input``."""
    prologue = PW_PROLOGUE_GELU if gelu_input else PW_PROLOGUE_NONE
    dw, db = pointwise_weight_grad(grad_output.contiguous(), x.contiguous(), prologue=prologue, with_bias=True)
    return dw, db


@pointwise_weight_grad_op.register_fake
def _(grad_output, x, gelu_input):
    m, k = grad_output.shape[1], x.shape[1]
    return x.new_empty((m, k, 1, 1, 1)), x.new_empty((m,))


@torch.library.custom_op("mednext_accel_amd::pointwise_conv3d", mutates_args=())
def pointwise_conv3d(x: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
    """1x1x1 Conv3d (bf16) on the matrix cores: the GEMM route of the reference's
    AdaptivePointwise3d (ops/adaptive.py:174-200)."""
    return pointwise_conv(x.contiguous(), weight, bias)


@pointwise_conv3d.register_fake
def _(x, weight, bias):
    return x.new_empty((x.shape[0], weight.shape[0], *x.shape[2:]))


@torch.library.custom_op("mednext_accel_amd::pointwise_conv_transpose3d", mutates_args=())
def pointwise_conv_transpose3d(x: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
    """1x1x1 stride-1 ConvTranspose3d (bf16): ``Y = W^T . X + b`` with the
    transposed conv's [Cin, Cout, 1, 1, 1] weight (the MedNeXt output heads,
    reference models/blocks.py:185-194)."""
    return pointwise_conv(x.contiguous(), weight, bias, transpose=True)


@pointwise_conv_transpose3d.register_fake
def _(x, weight, bias):
    return x.new_empty((x.shape[0], weight.shape[1], *x.shape[2:]))


def _setup_pointwise(ctx, inputs, output):
    x, weight, bias = inputs
    ctx.save_for_backward(x, weight)
    ctx.has_bias = bias is not None


def _pointwise_backward(ctx, grad_output):
    x, weight = ctx.saved_tensors
    need_x, need_w, need_b = ctx.needs_input_grad
    grad_output = grad_output.contiguous()
    dx = pointwise_input_grad_op(grad_output, weight) if need_x else None
    dw = db = None
    if need_w or (need_b and ctx.has_bias):
        dw, db = pointwise_weight_grad_op(grad_output, x, False)
    return dx, dw if need_w else None, db if (need_b and ctx.has_bias) else None


pointwise_conv3d.register_autograd(_pointwise_backward, setup_context=_setup_pointwise)


def _pointwise_transpose_backward(ctx, grad_output):
    # Y = W^T X + b with W [Cin, Cout]: dX = W dY, dW = X dY^T, dB = sum dY.
    x, weight = ctx.saved_tensors
    need_x, need_w, need_b = ctx.needs_input_grad
    grad_output = grad_output.contiguous()
    dx = pointwise_forward_grad_op(grad_output, weight) if need_x else None
    dw = db = None
    if need_w or (need_b and ctx.has_bias):
        dwt, db = pointwise_weight_grad_op(grad_output, x, False)  # [Cout, Cin]
        dw = dwt.reshape(dwt.shape[0], dwt.shape[1]).t().reshape(weight.shape)
    return dx, dw if need_w else None, db if (need_b and ctx.has_bias) else None


@torch.library.custom_op("mednext_accel_amd::pointwise_forward_grad", mutates_args=())
def pointwise_forward_grad_op(grad_output: Tensor, weight: Tensor) -> Tensor:
    """dX = W . dY of a 1x1x1 transposed conv with weight [Cin, Cout] (bf16)."""
    return pointwise_conv(grad_output.contiguous(), weight)


@pointwise_forward_grad_op.register_fake
def _(grad_output, weight):
    return grad_output.new_empty((grad_output.shape[0], weight.shape[0], *grad_output.shape[2:]))


pointwise_conv_transpose3d.register_autograd(_pointwise_transpose_backward, setup_context=_setup_pointwise)


@torch.library.custom_op("mednext_accel_amd::mlp_expansion", mutates_args=())
def mlp_expansion(
    x: Tensor, w1: Tensor, b1: Tensor | None, w2: Tensor, b2: Tensor | None, residual: Tensor | None
) -> tuple[Tensor, Tensor]:
    """MedNeXt block expansion, fused: ``out = W2 . GELU(W1 . x + b1) + b2 (+ residual)``
    (reference models/blocks.py:79-80 and the residual add :89-90).

    Returns ``(out, h)`` with ``h = W1 . x + b1`` the pre-activation the
    backward needs; GELU(h) is recomputed inside the project GEMM instead of
    being stored."""
    x = x.contiguous()
    h = pointwise_conv(x, w1, b1, epilogue=PW_EPILOGUE_BIAS)
    if residual is None:
        out = pointwise_conv(h, w2, b2, prologue=PW_PROLOGUE_GELU, epilogue=PW_EPILOGUE_BIAS)
    else:
        out = pointwise_conv(
            h, w2, b2, aux=residual.contiguous(), prologue=PW_PROLOGUE_GELU, epilogue=PW_EPILOGUE_BIAS_RESIDUAL
        )
    return out, h


@mlp_expansion.register_fake
def _(x, w1, b1, w2, b2, residual):
    h = x.new_empty((x.shape[0], w1.shape[0], *x.shape[2:]))
    return x.new_empty((x.shape[0], w2.shape[0], *x.shape[2:])), h


@torch.library.custom_op("mednext_accel_amd::mlp_expansion_backward", mutates_args=())
def mlp_expansion_backward(
    grad_out: Tensor, x: Tensor, h: Tensor, w1: Tensor, w2: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dx, dW1, db1, dW2, db2) of ``mlp_expansion``:
    dh = (W2^T . dout) * GELU'(h); dW2 = dout . GELU(h)^T; dW1 = dh . x^T; dx = W1^T . dh."""
    grad_out = grad_out.contiguous()
    dh = pointwise_conv(grad_out, w2, aux=h, epilogue=PW_EPILOGUE_GELU_GRAD, transpose=True)
    dw2, db2 = pointwise_weight_grad(grad_out, h, prologue=PW_PROLOGUE_GELU)
    dw1, db1 = pointwise_weight_grad(dh, x.contiguous())
    dx = pointwise_conv(dh, w1, transpose=True)
    return dx, dw1, db1, dw2, db2


@mlp_expansion_backward.register_fake
def _(grad_out, x, h, w1, w2):
    return (
        torch.empty_like(x),
        w1.new_empty(w1.shape),
        w1.new_empty((w1.shape[0],)),
        w2.new_empty(w2.shape),
        w2.new_empty((w2.shape[0],)),
    )


def _setup_mlp(ctx, inputs, output):
    x, w1, b1, w2, b2, residual = inputs
    _out, h = output
    ctx.mark_non_differentiable(h)
    # h (kept for the backward) never receives a gradient: without this autograd
    # would fill a zero tensor the size of the expanded activation every step.
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, h, w1, w2)
    ctx.has_b1, ctx.has_b2, ctx.has_residual = b1 is not None, b2 is not None, residual is not None


def _mlp_backward(ctx, grad_out, _grad_h):
    if grad_out is None:
        return None, None, None, None, None, None
    x, h, w1, w2 = ctx.saved_tensors
    dx, dw1, db1, dw2, db2 = mlp_expansion_backward(grad_out, x, h, w1, w2)
    return (
        dx,
        dw1,
        db1 if ctx.has_b1 else None,
        dw2,
        db2 if ctx.has_b2 else None,
        grad_out if ctx.has_residual else None,
    )


mlp_expansion.register_autograd(_mlp_backward, setup_context=_setup_mlp)


@torch.library.custom_op("mednext_accel_amd::mlp_expansion_stored", mutates_args=())
def mlp_expansion_stored(
    x: Tensor, w1: Tensor, b1: Tensor | None, w2: Tensor, b2: Tensor | None, residual: Tensor | None
) -> tuple[Tensor, Tensor, Tensor]:
    """``mlp_expansion`` with GELU evaluated once: the expand GEMM writes
    ``a = GELU(h)`` and ``dgelu = GELU'(h)`` (bf16) instead of h, the project
    GEMM reads a as it is, and the backward needs no GELU at all (its input
    gradient multiplies by the stored GELU'). Returns ``(out, a, dgelu)``.
    Pays where the recomputing variant evaluates GELU once per 32-row output
    group of a wide project GEMM."""
    x = x.contiguous()
    a, dgelu = pointwise_conv(x, w1, b1, epilogue=PW_EPILOGUE_BIAS_GELU_PAIR)
    if residual is None:
        out = pointwise_conv(a, w2, b2, epilogue=PW_EPILOGUE_BIAS)
    else:
        out = pointwise_conv(a, w2, b2, aux=residual.contiguous(), epilogue=PW_EPILOGUE_BIAS_RESIDUAL)
    return out, a, dgelu


@mlp_expansion_stored.register_fake
def _(x, w1, b1, w2, b2, residual):
    h = x.new_empty((x.shape[0], w1.shape[0], *x.shape[2:]))
    return x.new_empty((x.shape[0], w2.shape[0], *x.shape[2:])), h, torch.empty_like(h)


@torch.library.custom_op("mednext_accel_amd::mlp_expansion_stored_backward", mutates_args=())
def mlp_expansion_stored_backward(
    grad_out: Tensor, x: Tensor, a: Tensor, dgelu: Tensor, w1: Tensor, w2: Tensor
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dx, dW1, db1, dW2, db2) of ``mlp_expansion_stored``:
    dh = (W2^T . dout) * GELU'(h); dW2 = dout . a^T; dW1 = dh . x^T; dx = W1^T . dh."""
    grad_out = grad_out.contiguous()
    dh = pointwise_conv(grad_out, w2, aux=dgelu, epilogue=PW_EPILOGUE_AUX_SCALE, transpose=True)
    dw2, db2 = pointwise_weight_grad(grad_out, a)
    dw1, db1 = pointwise_weight_grad(dh, x.contiguous())
    dx = pointwise_conv(dh, w1, transpose=True)
    return dx, dw1, db1, dw2, db2


@mlp_expansion_stored_backward.register_fake
def _(grad_out, x, a, dgelu, w1, w2):
    return (
        torch.empty_like(x),
        w1.new_empty(w1.shape),
        w1.new_empty((w1.shape[0],)),
        w2.new_empty(w2.shape),
        w2.new_empty((w2.shape[0],)),
    )


def _setup_mlp_stored(ctx, inputs, output):
    x, w1, b1, w2, b2, residual = inputs
    _out, a, dgelu = output
    ctx.mark_non_differentiable(a, dgelu)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, a, dgelu, w1, w2)
    ctx.has_b1, ctx.has_b2, ctx.has_residual = b1 is not None, b2 is not None, residual is not None


def _mlp_stored_backward(ctx, grad_out, _grad_a, _grad_dgelu):
    if grad_out is None:
        return None, None, None, None, None, None
    x, a, dgelu, w1, w2 = ctx.saved_tensors
    dx, dw1, db1, dw2, db2 = mlp_expansion_stored_backward(grad_out, x, a, dgelu, w1, w2)
    return (
        dx,
        dw1,
        db1 if ctx.has_b1 else None,
        dw2,
        db2 if ctx.has_b2 else None,
        grad_out if ctx.has_residual else None,
    )


mlp_expansion_stored.register_autograd(_mlp_stored_backward, setup_context=_setup_mlp_stored)


@torch.library.custom_op("mednext_accel_amd::gn_mlp_expansion", mutates_args=())
def gn_mlp_expansion(
    d: Tensor,
    gamma: Tensor,
    beta: Tensor,
    w1: Tensor,
    b1: Tensor | None,
    w2: Tensor,
    b2: Tensor | None,
    residual: Tensor | None,
    eps: float,
    stored: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """MedNeXt block ``norm -> expand -> GELU -> project (+ residual)`` with
    the GroupNorm folded into the expand GEMM (reference models/blocks.py:74,
    :84-91): one statistics pass over the depthwise output d gives the
    per-(n, c) records, and the expand GEMM applies GroupNorm through its NORM
    prologue as it loads d (bit for bit the bf16 values ``group_norm_forward``
    writes), so the normalised tensor is never written or read.
    ``stored`` selects the GELU handling of ``mlp_expansion_stored`` (the
    expand GEMM writes GELU(h) and GELU'(h)) or of ``mlp_expansion`` (it
    writes h; the project GEMM and the backward recompute GELU).

    Returns ``(out, act, dgelu, coef, mean, rstd)``: act = GELU(h) (stored)
    or h; dgelu = GELU'(h) (stored) or an empty tensor; coef [N, C, 4] fp64
    (``group_norm_stats``); mean / rstd [N*C] as ``group_norm_forward`` writes
    them."""
    d = d.contiguous()
    coef, mean, rstd = group_norm_stats(d, gamma, beta, eps)
    res = residual.contiguous() if residual is not None else None
    epi_out = PW_EPILOGUE_BIAS if res is None else PW_EPILOGUE_BIAS_RESIDUAL
    if stored:
        act, dgelu = pointwise_conv(d, w1, b1, prologue=PW_PROLOGUE_NORM, epilogue=PW_EPILOGUE_BIAS_GELU_PAIR,
                                    prologue_coef=coef)
        out = pointwise_conv(act, w2, b2, aux=res, epilogue=epi_out)
    else:
        act = pointwise_conv(d, w1, b1, prologue=PW_PROLOGUE_NORM, epilogue=PW_EPILOGUE_BIAS, prologue_coef=coef)
        dgelu = act.new_empty((0,))
        out = pointwise_conv(act, w2, b2, aux=res, prologue=PW_PROLOGUE_GELU, epilogue=epi_out)
    return out, act, dgelu, coef, mean, rstd


@gn_mlp_expansion.register_fake
def _(d, gamma, beta, w1, b1, w2, b2, residual, eps, stored):
    n, c = d.shape[0], d.shape[1]
    h = d.new_empty((n, w1.shape[0], *d.shape[2:]))
    return (
        d.new_empty((n, w2.shape[0], *d.shape[2:])),
        h,
        torch.empty_like(h) if stored else d.new_empty((0,)),
        d.new_empty((n, c, 4), dtype=torch.float64),
        d.new_empty((n * c,), dtype=torch.float32),
        d.new_empty((n * c,), dtype=torch.float32),
    )


@torch.library.custom_op("mednext_accel_amd::gn_mlp_expansion_backward", mutates_args=())
def gn_mlp_expansion_backward(
    grad_out: Tensor,
    d: Tensor,
    act: Tensor,
    dgelu: Tensor,
    coef: Tensor,
    mean: Tensor,
    rstd: Tensor,
    gamma: Tensor,
    w1: Tensor,
    w2: Tensor,
    stored: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dd, dgamma, dbeta, dW1, db1, dW2, db2) of ``gn_mlp_expansion``:
    dh = (W2^T . dout) * GELU'(h); dW2 = dout . GELU(h)^T; dW1 = dh . GN(d)^T
    from the raw product dh . d^T mapped through the NORM records; dz = W1^T . dh; and the
    GroupNorm backward of dz at d."""
    grad_out = grad_out.contiguous()
    if stored:
        dh = pointwise_conv(grad_out, w2, aux=dgelu, epilogue=PW_EPILOGUE_AUX_SCALE, transpose=True)
        dw2, db2 = pointwise_weight_grad(grad_out, act)
    else:
        dh = pointwise_conv(grad_out, w2, aux=act, epilogue=PW_EPILOGUE_GELU_GRAD, transpose=True)
        dw2, db2 = pointwise_weight_grad(grad_out, act, prologue=PW_PROLOGUE_GELU)
    dw1, db1 = pointwise_weight_grad(dh, d, prologue=PW_PROLOGUE_NORM, prologue_coef=coef)
    dz = pointwise_conv(dh, w1, transpose=True)
    dd, dgamma, dbeta = group_norm_backward(dz, d, mean, rstd, gamma)
    return dd, dgamma, dbeta, dw1, db1, dw2, db2


@gn_mlp_expansion_backward.register_fake
def _(grad_out, d, act, dgelu, coef, mean, rstd, gamma, w1, w2, stored):
    return (
        torch.empty_like(d),
        torch.empty_like(gamma),
        torch.empty_like(gamma),
        w1.new_empty(w1.shape),
        w1.new_empty((w1.shape[0],)),
        w2.new_empty(w2.shape),
        w2.new_empty((w2.shape[0],)),
    )


def _setup_gn_mlp(ctx, inputs, output):
    d, gamma, beta, w1, b1, w2, b2, residual, eps, stored = inputs
    _out, act, dgelu, coef, mean, rstd = output
    ctx.mark_non_differentiable(act, dgelu, coef, mean, rstd)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(d, act, dgelu, coef, mean, rstd, gamma, w1, w2)
    ctx.stored = stored
    ctx.has_b1, ctx.has_b2, ctx.has_residual = b1 is not None, b2 is not None, residual is not None


def _gn_mlp_backward(ctx, grad_out, *_unused):
    if grad_out is None:
        return (None,) * 10
    d, act, dgelu, coef, mean, rstd, gamma, w1, w2 = ctx.saved_tensors
    dd, dgamma, dbeta, dw1, db1, dw2, db2 = gn_mlp_expansion_backward(
        grad_out, d, act, dgelu, coef, mean, rstd, gamma, w1, w2, ctx.stored
    )
    return (
        dd,
        dgamma,
        dbeta,
        dw1,
        db1 if ctx.has_b1 else None,
        dw2,
        db2 if ctx.has_b2 else None,
        grad_out if ctx.has_residual else None,
        None,
        None,
    )


gn_mlp_expansion.register_autograd(_gn_mlp_backward, setup_context=_setup_gn_mlp)


# ------------------------------------------------------------ stride-2 depthwise


def _check_s2(big_shape, small_shape, weight: Tensor, *tensors: Tensor) -> int:
    _check_device(weight, *tensors)
    for t in tensors:
        if t.ndim != 5 or not t.is_contiguous():
            raise ValueError("contiguous NCDHW tensors are required")
        if t.dtype != weight.dtype:
            raise ValueError("tensors and weight must share a dtype")
    if weight.ndim != 5 or weight.shape[1] != 1 or len(set(weight.shape[2:])) != 1:
        raise ValueError("weight must have shape [C, 1, K, K, K]")
    k = int(weight.shape[2])
    if k % 2 == 0 or k not in SUPPORTED_KERNELS:
        raise ValueError(f"kernel_size must be one of {SUPPORTED_KERNELS}")
    if big_shape[:2] != small_shape[:2] or big_shape[1] != weight.shape[0]:
        raise ValueError("batch / channel mismatch")
    return k


def _s2_dims(big_shape, small_shape) -> tuple[int, ...]:
    n, c, db, hb, wb = (int(v) for v in big_shape)
    ds, hs, ws = (int(v) for v in small_shape[2:])
    return n, c, db, hb, wb, ds, hs, ws


def depthwise_s2_gather(big: Tensor, weight: Tensor, bias: Tensor | None, small_spatial) -> Tensor:
    """small[o] = bias + sum_t w[t] big[2o + t - k/2]."""
    out = big.new_empty((big.shape[0], big.shape[1], *small_spatial))
    k = _check_s2(big.shape, out.shape, weight, big)
    if bias is not None and (bias.shape != (big.shape[1],) or bias.dtype != big.dtype):
        raise ValueError("bias must be [C] in the input's dtype")
    _hip.check(
        _hip.load().mednext_depthwise3d_s2_gather(
            big.data_ptr(), weight.contiguous().data_ptr(), _hip.ptr(bias.contiguous() if bias is not None else None),
            out.data_ptr(), *_s2_dims(big.shape, out.shape), k, _hip.dtype_code(big.dtype), _hip.stream_of(big),
        ),
        "mednext_depthwise3d_s2_gather",
    )
    return out


def depthwise_s2_scatter(small: Tensor, weight: Tensor, bias: Tensor | None, big_spatial) -> Tensor:
    """big[i] = bias + sum_{o,t: 2o + t - k/2 = i} w[t] small[o]."""
    out = small.new_empty((small.shape[0], small.shape[1], *big_spatial))
    k = _check_s2(out.shape, small.shape, weight, small)
    if bias is not None and (bias.shape != (small.shape[1],) or bias.dtype != small.dtype):
        raise ValueError("bias must be [C] in the input's dtype")
    _hip.check(
        _hip.load().mednext_depthwise3d_s2_scatter(
            small.data_ptr(), weight.contiguous().data_ptr(), _hip.ptr(bias.contiguous() if bias is not None else None),
            out.data_ptr(), *_s2_dims(out.shape, small.shape), k, _hip.dtype_code(small.dtype), _hip.stream_of(small),
        ),
        "mednext_depthwise3d_s2_scatter",
    )
    return out


def depthwise_s2_wgrad(big: Tensor, small: Tensor, kernel_size: int) -> tuple[Tensor, Tensor]:
    """(dW [C,1,k,k,k], sum of ``small`` per channel [C]) with
    dW[t] = sum_{n,o} big[2o + t - k/2] small[o]."""
    if kernel_size % 2 == 0 or kernel_size not in SUPPORTED_KERNELS:
        raise ValueError(f"kernel_size must be one of {SUPPORTED_KERNELS}")
    weight_like = big.new_empty((big.shape[1], 1, kernel_size, kernel_size, kernel_size))
    _check_s2(big.shape, small.shape, weight_like, big, small)
    dims = _s2_dims(big.shape, small.shape)
    code = _hip.dtype_code(big.dtype)
    lib = _hip.load()
    nbytes = int(lib.mednext_depthwise3d_s2_wgrad_workspace_bytes(*dims, kernel_size, code))
    if nbytes == 0:
        raise _hip.HipLibraryError(f"s2 wgrad workspace query failed: {_hip.last_error()}")
    ws = torch.empty((nbytes,), device=big.device, dtype=torch.uint8)
    dw = weight_like
    ds = big.new_empty((big.shape[1],))
    _hip.check(
        lib.mednext_depthwise3d_s2_wgrad(
            big.data_ptr(), small.data_ptr(), dw.data_ptr(), ds.data_ptr(), ws.data_ptr(), nbytes, *dims,
            kernel_size, code, _hip.stream_of(big),
        ),
        "mednext_depthwise3d_s2_wgrad",
    )
    return dw, ds


def strided_spatial(shape) -> list[int]:
    """Output size of the stride-2, padding k//2 conv: (s - 1) // 2 + 1."""
    return [(int(s) - 1) // 2 + 1 for s in shape]


@torch.library.custom_op("mednext_accel_amd::depthwise_s2_gather", mutates_args=())
def depthwise_s2_gather_op(big: Tensor, weight: Tensor, small_spatial: list[int]) -> Tensor:
    return depthwise_s2_gather(big.contiguous(), weight, None, small_spatial)


@depthwise_s2_gather_op.register_fake
def _(big, weight, small_spatial):
    return big.new_empty((big.shape[0], big.shape[1], *small_spatial))


@torch.library.custom_op("mednext_accel_amd::depthwise_s2_scatter", mutates_args=())
def depthwise_s2_scatter_op(small: Tensor, weight: Tensor, big_spatial: list[int]) -> Tensor:
    return depthwise_s2_scatter(small.contiguous(), weight, None, big_spatial)


@depthwise_s2_scatter_op.register_fake
def _(small, weight, big_spatial):
    return small.new_empty((small.shape[0], small.shape[1], *big_spatial))


@torch.library.custom_op("mednext_accel_amd::depthwise_s2_wgrad", mutates_args=())
def depthwise_s2_wgrad_op(big: Tensor, small: Tensor, kernel_size: int) -> tuple[Tensor, Tensor]:
    return depthwise_s2_wgrad(big.contiguous(), small.contiguous(), kernel_size)


@depthwise_s2_wgrad_op.register_fake
def _(big, small, kernel_size):
    c = big.shape[1]
    return big.new_empty((c, 1, kernel_size, kernel_size, kernel_size)), big.new_empty((c,))


@torch.library.custom_op("mednext_accel_amd::depthwise_conv3d_stride2", mutates_args=())
def depthwise_conv3d_stride2(x: Tensor, weight: Tensor, bias: Tensor | None, kernel_size: int) -> Tensor:
    """Depthwise Conv3d, stride 2, padding k//2 (the MedNeXt down block;
    reference ops/_triton/depthwise.py:654-719), all phases in HIP."""
    return depthwise_s2_gather(x.contiguous(), weight, bias, strided_spatial(x.shape[2:]))


@depthwise_conv3d_stride2.register_fake
def _(x, weight, bias, kernel_size):
    return x.new_empty((x.shape[0], x.shape[1], *strided_spatial(x.shape[2:])))


def _setup_s2(ctx, inputs, output):
    x, weight, bias, kernel_size = inputs
    ctx.save_for_backward(x, weight)
    ctx.has_bias = bias is not None
    ctx.kernel_size = kernel_size


def _s2_backward(ctx, grad_output):
    x, weight = ctx.saved_tensors
    grad_output = grad_output.contiguous()
    need_x, need_w, need_b = ctx.needs_input_grad[:3]
    dx = depthwise_s2_scatter_op(grad_output, weight, list(x.shape[2:])) if need_x else None
    dw = db = None
    if need_w or (need_b and ctx.has_bias):
        dw, db = depthwise_s2_wgrad_op(x, grad_output, ctx.kernel_size)
    return dx, dw if need_w else None, db if (need_b and ctx.has_bias) else None, None


depthwise_conv3d_stride2.register_autograd(_s2_backward, setup_context=_setup_s2)


@torch.library.custom_op("mednext_accel_amd::depthwise_conv_transpose3d_stride2", mutates_args=())
def depthwise_conv_transpose3d_stride2(x: Tensor, weight: Tensor, bias: Tensor | None, kernel_size: int) -> Tensor:
    """Depthwise ConvTranspose3d, stride 2, padding k//2, no output padding (the
    MedNeXt up block; reference ops/_triton/depthwise.py:768-850): output 2s - 1
    per dimension, all phases in HIP."""
    return depthwise_s2_scatter(x.contiguous(), weight, bias, [2 * int(s) - 1 for s in x.shape[2:]])


@depthwise_conv_transpose3d_stride2.register_fake
def _(x, weight, bias, kernel_size):
    return x.new_empty((x.shape[0], x.shape[1], *(2 * s - 1 for s in x.shape[2:])))


def _t2_backward(ctx, grad_output):
    x, weight = ctx.saved_tensors
    grad_output = grad_output.contiguous()
    need_x, need_w, need_b = ctx.needs_input_grad[:3]
    dx = depthwise_s2_gather_op(grad_output, weight, list(x.shape[2:])) if need_x else None
    dw = depthwise_s2_wgrad_op(grad_output, x, ctx.kernel_size)[0] if need_w else None
    db = None
    if need_b and ctx.has_bias:
        # Per-(n, c) sums over the contiguous voxels first: a last-dimension
        # reduction runs at memory speed, a reduction over dims (0, 2, 3, 4)
        # of an NCDHW tensor at about a quarter of it.
        acc = torch.float64 if x.dtype == torch.float64 else torch.float32
        db = grad_output.reshape(grad_output.shape[0], grad_output.shape[1], -1).sum(dim=2, dtype=acc)
        db = db.sum(dim=0).to(x.dtype)
    return dx, dw, db, None


depthwise_conv_transpose3d_stride2.register_autograd(_t2_backward, setup_context=_setup_s2)


# ---------------------------------------------------------------- up-block join


def _check_join(main: Tensor, small: Tensor, bias: Tensor | None) -> tuple[int, ...]:
    _check_device(main, small)
    for t, name in ((main, "main"), (small, "small")):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.ndim != 5:
            raise ValueError(f"{name} must be a contiguous bfloat16 NCDHW tensor")
    n, c = main.shape[:2]
    d, h, w = (int(s) + 1 for s in main.shape[2:])
    if tuple(small.shape) != (n, c, d // 2, h // 2, w // 2) or d % 2 or h % 2 or w % 8:
        raise ValueError("main must be [N, C, 2a-1, 2b-1, 2c-1] with 2c % 8 == 0 and small [N, C, a, b, c]")
    if bias is not None and (bias.shape != (c,) or bias.dtype != torch.bfloat16):
        raise ValueError("bias must be a bfloat16 [C] tensor")
    return n, c, d, h, w


def up_join(main: Tensor, small: Tensor, bias: Tensor | None, lead: int) -> Tensor:
    """``pad(main) + pad(residual)`` of a MedNeXt up block in one pass: the
    residual is the stride-2 transposed 1x1x1 conv whose GEMM output (bias
    included) at the even grid points is ``small`` and whose value elsewhere
    is ``bias``; the one-voxel pad is at the start (``lead=1``, v1) or the end
    (``lead=0``, v2)."""
    n, c, d, h, w = _check_join(main, small, bias)
    out = main.new_empty((n, c, d, h, w))
    _hip.check(
        _hip.load().mednext_up_join_fwd(
            main.data_ptr(), small.data_ptr(), _hip.ptr(bias), out.data_ptr(), n, c, d, h, w, int(lead),
            _hip.DTYPE_CODES[torch.bfloat16], _hip.stream_of(main),
        ),
        "mednext_up_join_fwd",
    )
    return out


def up_join_backward(
    grad_out: Tensor, lead: int, with_bias: bool, bias_over_grid: bool = False
) -> tuple[Tensor, Tensor, Tensor | None]:
    """(grad_main, grad_small, grad_bias or None) of ``up_join``; with
    ``bias_over_grid`` grad_bias sums grad_out over the whole (2s - 1)^3 grid,
    all-even points included (the bias's whole gradient when ``small`` was
    computed with an untracked copy of it)."""
    _check_device(grad_out)
    if grad_out.dtype != torch.bfloat16 or not grad_out.is_contiguous() or grad_out.ndim != 5:
        raise ValueError("grad_out must be a contiguous bfloat16 NCDHW tensor")
    n, c, d, h, w = (int(s) for s in grad_out.shape)
    gmain = grad_out.new_empty((n, c, d - 1, h - 1, w - 1))
    gsmall = grad_out.new_empty((n, c, d // 2, h // 2, w // 2))
    gbias = grad_out.new_empty((c,)) if with_bias else None
    lib = _hip.load()
    nbytes = lib.mednext_up_join_bwd_workspace_bytes(n, c, d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=grad_out.device)
    _hip.check(
        lib.mednext_up_join_bwd(
            grad_out.data_ptr(), gmain.data_ptr(), gsmall.data_ptr(), _hip.ptr(gbias), ws.data_ptr(), nbytes,
            n, c, d, h, w, int(lead), int(bool(bias_over_grid)), _hip.DTYPE_CODES[torch.bfloat16],
            _hip.stream_of(grad_out),
        ),
        "mednext_up_join_bwd",
    )
    return gmain, gsmall, gbias


@torch.library.custom_op("mednext_accel_amd::up_block_join", mutates_args=())
def up_block_join(main: Tensor, small: Tensor, bias: Tensor | None, lead: int, bias_in_small: bool = False) -> Tensor:
    """Custom-op form of ``up_join`` (reference models/blocks.py:179-181,
    models/blocks_v2.py:131-133). ``bias_in_small``: the caller computed
    ``small`` with the bias's value but without tracking it, so the bias's
    gradient is the sum over the whole grid (one rounding, as the reference's
    conv_transpose3d bias reduction) instead of over the non-even points."""
    return up_join(main, small, bias, lead)


@up_block_join.register_fake
def _(main, small, bias, lead, bias_in_small=False):
    return main.new_empty((main.shape[0], main.shape[1], *(s + 1 for s in main.shape[2:])))


@torch.library.custom_op("mednext_accel_amd::up_block_join_backward", mutates_args=())
def up_block_join_backward_op(
    grad_out: Tensor, lead: int, with_bias: bool, bias_over_grid: bool
) -> tuple[Tensor, Tensor, Tensor]:
    gmain, gsmall, gbias = up_join_backward(grad_out.contiguous(), lead, with_bias, bias_over_grid)
    return gmain, gsmall, gbias if gbias is not None else grad_out.new_empty((0,))


@up_block_join_backward_op.register_fake
def _(grad_out, lead, with_bias, bias_over_grid):
    n, c, d, h, w = grad_out.shape
    return (grad_out.new_empty((n, c, d - 1, h - 1, w - 1)), grad_out.new_empty((n, c, d // 2, h // 2, w // 2)),
            grad_out.new_empty((c,) if with_bias else (0,)))


def _setup_join(ctx, inputs, output):
    _main, _small, bias, lead, bias_in_small = inputs
    ctx.lead = lead
    ctx.has_bias = bias is not None
    ctx.bias_in_small = bias_in_small


def _join_backward(ctx, grad_out):
    need_main, need_small, need_bias = ctx.needs_input_grad[:3]
    with_bias = ctx.has_bias and need_bias
    gmain, gsmall, gbias = up_block_join_backward_op(grad_out.contiguous(), ctx.lead, with_bias, ctx.bias_in_small)
    return (gmain if need_main else None, gsmall if need_small else None, gbias if with_bias else None, None, None)


up_block_join.register_autograd(_join_backward, setup_context=_setup_join)


# ------------------------------------------------------------------------ GRN


def grn_forward(
    x: Tensor, gamma: Tensor | None, beta: Tensor | None, eps: float = 1e-6, splits: int | None = None
) -> tuple[Tensor, Tensor]:
    """Global Response Normalization forward (reference ops/grn.py:16-30):
    returns ``(y, coef)`` with ``coef`` [N, C, 4] fp64 = (1 + gamma r, beta, r, ||x_c||).
    Accepts f16 / bf16 / f32 / f64 input; parameters are read flat ([C] values)."""
    _check_device(x)
    if x.ndim != 5 or not x.is_contiguous():
        raise ValueError("a contiguous NCDHW input is required")
    n, c = int(x.shape[0]), int(x.shape[1])
    v = x.numel() // max(1, n * c)
    params = [p for p in (gamma, beta) if p is not None]
    pdtype = params[0].dtype if params else torch.float32
    for p in params:
        if p.numel() != c or p.dtype != pdtype or not p.is_cuda or not p.is_contiguous():
            raise ValueError("gamma / beta must be contiguous CUDA tensors of C values and one dtype")
    if x.numel() == 0:
        raise ValueError("GRN requires nonempty input dimensions")
    y = torch.empty_like(x)
    coef = torch.empty((n, c, 4), device=x.device, dtype=torch.float64)
    splits = group_norm_splits(n, c, v) if splits is None else int(splits)
    lib = _hip.load()
    nbytes = lib.mednext_grn_workspace_bytes(n, c, v, splits)
    workspace = torch.empty((max(8, nbytes),), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_grn_fwd(
            x.data_ptr(), _hip.dtype_code(x.dtype), _hip.ptr(gamma), _hip.ptr(beta), _hip.dtype_code(pdtype),
            y.data_ptr(), coef.data_ptr(), n, c, v, float(eps), splits, workspace.data_ptr(), nbytes,
            _hip.stream_of(x),
        ),
        "mednext_grn_fwd",
    )
    return y, coef


def grn_backward(
    grad_output: Tensor,
    x: Tensor,
    coef: Tensor,
    gamma: Tensor | None,
    eps: float = 1e-6,
    need_input: bool = True,
    need_params: bool = True,
    param_dtype: torch.dtype = torch.float32,
    param_shape: tuple[int, ...] | None = None,
    splits: int | None = None,
) -> tuple[Tensor | None, Tensor | None, Tensor | None]:
    """GRN backward: (dx in x.dtype, dgamma, dbeta in ``param_dtype`` and ``param_shape``)."""
    _check_device(grad_output, x, coef)
    if grad_output.shape != x.shape or not (grad_output.is_contiguous() and x.is_contiguous()):
        raise ValueError("grad_output and x must be contiguous with the same shape")
    n, c = int(x.shape[0]), int(x.shape[1])
    v = x.numel() // max(1, n * c)
    if coef.dtype != torch.float64 or coef.numel() != n * c * 4 or not coef.is_contiguous():
        raise ValueError("coef must be the forward's contiguous [N, C, 4] float64 tensor")
    if gamma is not None:
        param_dtype = gamma.dtype
    if grad_output.dtype != x.dtype and not (
        grad_output.dtype == torch.float32 and x.dtype in (torch.bfloat16, torch.float16)
    ):
        grad_output = grad_output.to(x.dtype)
    shape = (c,) if param_shape is None else tuple(param_shape)
    dx = torch.empty_like(x) if need_input else None
    dgamma = torch.empty(shape, device=x.device, dtype=param_dtype) if need_params else None
    dbeta = torch.empty(shape, device=x.device, dtype=param_dtype) if need_params else None
    splits = group_norm_splits(n, c, v) if splits is None else int(splits)
    lib = _hip.load()
    nbytes = lib.mednext_grn_workspace_bytes(n, c, v, splits)
    workspace = torch.empty((max(8, nbytes),), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_grn_bwd(
            grad_output.data_ptr(), _hip.dtype_code(grad_output.dtype), x.data_ptr(), _hip.dtype_code(x.dtype),
            coef.data_ptr(), _hip.ptr(gamma), _hip.dtype_code(param_dtype), _hip.ptr(dx), _hip.ptr(dgamma),
            _hip.ptr(dbeta), n, c, v, float(eps), splits, workspace.data_ptr(), nbytes, _hip.stream_of(x),
        ),
        "mednext_grn_bwd",
    )
    return dx, dgamma, dbeta


@torch.library.custom_op("mednext_accel_amd::grn_forward", mutates_args=())
def grn_forward_op(x: Tensor, gamma: Tensor, beta: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """Fused GRN forward (reference ops/_triton/grn.py:177-229): (y, coef)."""
    return grn_forward(x, gamma, beta, eps)


@grn_forward_op.register_fake
def _(x, gamma, beta, eps):
    return torch.empty_like(x), x.new_empty((x.shape[0], x.shape[1], 4), dtype=torch.float64)


@torch.library.custom_op("mednext_accel_amd::grn_backward", mutates_args=())
def grn_backward_op(
    grad_output: Tensor, x: Tensor, gamma: Tensor, coef: Tensor, eps: float
) -> tuple[Tensor, Tensor, Tensor]:
    """Fused GRN backward (reference ops/_triton/grn.py:242-317): (dx, dgamma, dbeta)."""
    dx, dgamma, dbeta = grn_backward(
        grad_output.contiguous(), x, coef, gamma, eps, param_shape=tuple(gamma.shape)
    )
    return dx, dgamma, dbeta


@grn_backward_op.register_fake
def _(grad_output, x, gamma, coef, eps):
    return torch.empty_like(x), torch.empty_like(gamma), torch.empty_like(gamma)


def _setup_grn(ctx, inputs, output):
    x, gamma, _beta, eps = inputs
    _y, coef = output
    ctx.mark_non_differentiable(coef)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, gamma, coef)
    ctx.eps = eps


def _grn_backward(ctx, grad_output, _grad_coef):
    if grad_output is None:
        return None, None, None, None
    x, gamma, coef = ctx.saved_tensors
    dx, dgamma, dbeta = grn_backward_op(grad_output, x, gamma, coef, ctx.eps)
    need = ctx.needs_input_grad
    return (dx if need[0] else None, dgamma if need[1] else None, dbeta if need[2] else None, None)


grn_forward_op.register_autograd(_grn_backward, setup_context=_setup_grn)


def fused_global_response_norm3d(x: Tensor, gamma: Tensor, beta: Tensor, eps: float = 1e-6) -> Tensor:
    """Fused GRN with the reference's direct-call contract (reference
    ops/_triton/grn.py:404-438): nonempty contiguous NCDHW f16/bf16 GPU input,
    contiguous float32 gamma and beta of shape (1, C, 1, 1, 1) on the same
    device, finite positive eps; anything else raises ``ValueError`` with the
    reference's message instead of silently falling back."""
    if x.ndim != 5:
        raise ValueError("fused GRN expects a rank-5 NCDHW input")
    if not (x.is_cuda and gamma.is_cuda and beta.is_cuda):
        raise ValueError("fused GRN requires CUDA tensors")
    if gamma.device != x.device or beta.device != x.device:
        raise ValueError("fused GRN requires all tensors on the same CUDA device")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("fused GRN requires a float16 or bfloat16 input")
    if not x.is_contiguous():
        raise ValueError("fused GRN requires a contiguous NCDHW input")
    if any(size == 0 for size in x.shape):
        raise ValueError("fused GRN requires nonempty input dimensions")
    if gamma.dtype != torch.float32 or beta.dtype != torch.float32:
        raise ValueError("fused GRN requires float32 gamma and beta")
    expected = (1, x.shape[1], 1, 1, 1)
    if tuple(gamma.shape) != expected or tuple(beta.shape) != expected:
        raise ValueError("fused GRN requires gamma and beta with shape (1, C, 1, 1, 1)")
    if not gamma.is_contiguous() or not beta.is_contiguous():
        raise ValueError("fused GRN requires contiguous gamma and beta")
    if not math.isfinite(eps) or eps <= 0:
        raise ValueError("fused GRN requires eps to be finite and positive")
    return grn_forward_op(x, gamma, beta, float(eps))[0]


def grn_stats(
    x: Tensor, gamma: Tensor | None, beta: Tensor | None, eps: float = 1e-6, *, splits: int | None = None
) -> Tensor:
    """GRN coefficients [N, C, 4] float64 = (1 + gamma r, beta, r, ||x_c||):
    the forward's statistics without its output tensor."""
    _check_device(x)
    if x.ndim != 5 or not x.is_contiguous() or x.numel() == 0:
        raise ValueError("a nonempty contiguous NCDHW input is required")
    n, c = int(x.shape[0]), int(x.shape[1])
    v = x.numel() // (n * c)
    params = [p for p in (gamma, beta) if p is not None]
    pdtype = params[0].dtype if params else torch.float32
    for p in params:
        if p.numel() != c or p.dtype != pdtype or not p.is_cuda or not p.is_contiguous():
            raise ValueError("gamma / beta must be contiguous CUDA tensors of C values and one dtype")
    coef = torch.empty((n, c, 4), device=x.device, dtype=torch.float64)
    splits = group_norm_splits(n, c, v) if splits is None else int(splits)
    lib = _hip.load()
    nbytes = lib.mednext_grn_workspace_bytes(n, c, v, splits)
    workspace = torch.empty((max(8, nbytes),), device=x.device, dtype=torch.uint8)
    _hip.check(
        lib.mednext_grn_stats(
            x.data_ptr(), _hip.dtype_code(x.dtype), _hip.ptr(gamma), _hip.ptr(beta),
            _hip.dtype_code(pdtype), coef.data_ptr(), n, c, v, float(eps), splits, workspace.data_ptr(), nbytes,
            _hip.stream_of(x),
        ),
        "mednext_grn_stats",
    )
    return coef


def grn_backward_from_rows(
    row_partial: Tensor, coef: Tensor, gamma: Tensor, eps: float = 1e-6
) -> tuple[Tensor, Tensor, Tensor]:
    """GRN backward coefficients [N, C, 2] float64 (dy multiplier, y_in
    multiplier) and (dgamma, dbeta) shaped like gamma, from the row sums
    (sum dz * y_in, sum dz) a ROW_REDUCE GEMM epilogue wrote."""
    _check_device(row_partial, coef, gamma)
    n, c = int(coef.shape[0]), int(coef.shape[1])
    if row_partial.dtype != torch.float64 or row_partial.numel() % (n * c * 2):
        raise ValueError("row_partial must be float64 [N, C, slots, 2]")
    slots = row_partial.numel() // (n * c * 2)
    out = torch.empty((n, c, 2), device=coef.device, dtype=torch.float64)
    dgamma = torch.empty_like(gamma)
    dbeta = torch.empty_like(gamma)
    workspace = torch.empty((n * c * 4,), device=coef.device, dtype=torch.float64)
    _hip.check(
        _hip.load().mednext_grn_bwd_rows(
            row_partial.data_ptr(), slots, coef.data_ptr(), gamma.data_ptr(), _hip.dtype_code(gamma.dtype),
            out.data_ptr(), dgamma.data_ptr(), dbeta.data_ptr(), n, c, float(eps), workspace.data_ptr(),
            workspace.numel() * 8, _hip.stream_of(coef),
        ),
        "mednext_grn_bwd_rows",
    )
    return out, dgamma, dbeta


# --------------------------------------------------- MedNeXt v2 fused expansion


@torch.library.custom_op("mednext_accel_amd::grn_expansion", mutates_args=())
def grn_expansion(
    x: Tensor,
    w1: Tensor,
    b1: Tensor | None,
    w2: Tensor,
    b2: Tensor | None,
    gamma: Tensor,
    beta: Tensor,
    residual: Tensor | None,
    eps: float,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """MedNeXt v2 block expansion, fused: ``out = W2 . GRN(GELU(W1 . x + b1)) +
    b2 (+ residual)`` (reference models/blocks_v2.py:44-45 with the GRN of
    ops/grn.py:16-30 and the residual add of :48-55).

    Returns ``(out, a, dgelu, coef)``: the expand GEMM writes a = GELU(u) and
    dgelu = GELU'(u) (u = W1 . x + b1, bf16; the backward needs nothing else of
    u), the GRN statistics of a come from one read of it, and the project GEMM
    applies the GRN affine as it loads a (no GRN output tensor).
    ``coef`` [N, hidden, 4] float64 holds (1 + gamma r, beta, r, norm)."""
    x = x.contiguous()
    a, dgelu = pointwise_conv(x, w1, b1, epilogue=PW_EPILOGUE_BIAS_GELU_PAIR)
    coef = grn_stats(a, gamma, beta, eps)
    if residual is None:
        out = pointwise_conv(a, w2, b2, prologue=PW_PROLOGUE_AFFINE, epilogue=PW_EPILOGUE_BIAS, prologue_coef=coef)
    else:
        out = pointwise_conv(a, w2, b2, aux=residual.contiguous(), prologue=PW_PROLOGUE_AFFINE,
                             epilogue=PW_EPILOGUE_BIAS_RESIDUAL, prologue_coef=coef)
    return out, a, dgelu, coef


@grn_expansion.register_fake
def _(x, w1, b1, w2, b2, gamma, beta, residual, eps):
    shape = (x.shape[0], w1.shape[0], *x.shape[2:])
    return (
        x.new_empty((x.shape[0], w2.shape[0], *x.shape[2:])),
        x.new_empty(shape),
        x.new_empty(shape),
        x.new_empty((x.shape[0], w1.shape[0], 4), dtype=torch.float64),
    )


@torch.library.custom_op("mednext_accel_amd::grn_expansion_backward", mutates_args=())
def grn_expansion_backward(
    grad_out: Tensor, x: Tensor, a: Tensor, dgelu: Tensor, coef: Tensor, w1: Tensor, w2: Tensor, gamma: Tensor,
    eps: float,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dx, dW1, db1, dW2, db2, dgamma, dbeta) of ``grn_expansion``. With
    z = GRN(a) and dz = W2^T . dout (never stored): one transposed GEMM reduces
    the GRN row sums (sum dz * a, sum dz), a small kernel turns them into the
    per-(n, c) GRN backward coefficients (k1, k2) and the gamma / beta
    gradients, a second transposed GEMM writes du = (dz k1 + a k2) * GELU'(u);
    dW2 = dout . z^T reads a through the GRN affine prologue; dW1 = du . x^T
    and dx = W1^T . du as for any conv."""
    grad_out = grad_out.contiguous()
    n, hidden = int(a.shape[0]), int(a.shape[1])
    v = a[0, 0].numel()
    cout = int(grad_out.shape[1])
    blocks = pointwise_blocks(n, cout, hidden, v)
    slots = pointwise_row_slots(n, cout, hidden, v, int(blocks))
    rows = torch.empty((n, hidden, slots, 2), device=a.device, dtype=torch.float64)
    pointwise_conv(grad_out, w2, aux=a, epilogue=PW_EPILOGUE_ROW_REDUCE, transpose=True, blocks=blocks,
                   row_partial=rows)
    bcoef, dgamma, dbeta = grn_backward_from_rows(rows, coef, gamma, eps)
    du = pointwise_conv(grad_out, w2, aux=a, aux2=dgelu, epilogue=PW_EPILOGUE_AFFINE_SCALE, transpose=True,
                        epilogue_coef=bcoef)
    dw2, db2 = pointwise_weight_grad(grad_out, a, prologue=PW_PROLOGUE_AFFINE, prologue_coef=coef)
    dw1, db1 = pointwise_weight_grad(du, x.contiguous())
    dx = pointwise_conv(du, w1, transpose=True)
    return dx, dw1, db1, dw2, db2, dgamma, dbeta


@grn_expansion_backward.register_fake
def _(grad_out, x, a, dgelu, coef, w1, w2, gamma, eps):
    return (
        torch.empty_like(x),
        w1.new_empty(w1.shape),
        w1.new_empty((w1.shape[0],)),
        w2.new_empty(w2.shape),
        w2.new_empty((w2.shape[0],)),
        torch.empty_like(gamma),
        torch.empty_like(gamma),
    )


def _setup_grn_expansion(ctx, inputs, output):
    x, w1, b1, w2, b2, gamma, beta, residual, eps = inputs
    _out, a, dgelu, coef = output
    ctx.mark_non_differentiable(a, dgelu, coef)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, a, dgelu, coef, w1, w2, gamma)
    ctx.eps = eps
    ctx.has_b1, ctx.has_b2, ctx.has_residual = b1 is not None, b2 is not None, residual is not None


def _grn_expansion_backward(ctx, grad_out, _grad_a, _grad_dgelu, _grad_coef):
    if grad_out is None:
        return (None,) * 9
    x, a, dgelu, coef, w1, w2, gamma = ctx.saved_tensors
    dx, dw1, db1, dw2, db2, dgamma, dbeta = grn_expansion_backward(
        grad_out, x, a, dgelu, coef, w1, w2, gamma, ctx.eps
    )
    return (
        dx,
        dw1,
        db1 if ctx.has_b1 else None,
        dw2,
        db2 if ctx.has_b2 else None,
        dgamma,
        dbeta,
        grad_out if ctx.has_residual else None,
        None,
    )


grn_expansion.register_autograd(_grn_expansion_backward, setup_context=_setup_grn_expansion)
