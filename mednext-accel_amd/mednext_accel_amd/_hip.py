"""ctypes binding of libmednext_hip.so (the C ABI declared in include/mednext_hip.h).

The library is loaded after ``torch`` so it shares PyTorch's HIP runtime. A
missing or stale library is an error: nothing here falls back to another
implementation.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_double, c_int32, c_int64, c_size_t, c_void_p

import torch

from ._build import LIB_PATH

DTYPE_CODES = {
    torch.float32: 0,
    torch.float64: 1,
    torch.float16: 2,
    torch.bfloat16: 3,
}

_i64 = c_int64
_i32 = c_int32
_p = c_void_p

# name -> (restype, argtypes); mirrors include/mednext_hip.h.
SIGNATURES: dict[str, tuple[object, tuple[object, ...]]] = {
    "mednext_hip_last_error": (ctypes.c_char_p, ()),
    "mednext_hip_abi_version": (_i32, ()),
    "mednext_depthwise3d_fwd": (
        _i32,
        (_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    ),
    "mednext_depthwise3d_dgrad": (
        _i32,
        (_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    ),
    "mednext_depthwise3d_dgrad_acc": (
        _i32,
        (_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    ),
    "mednext_depthwise3d_wgrad_workspace_bytes": (
        c_size_t,
        (_i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32),
    ),
    "mednext_depthwise3d_wgrad": (
        _i32,
        (_p, _p, _p, _p, _p, c_size_t, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    ),
    "mednext_depthwise3d_wgrad_noalloc_max_bytes": (c_size_t, ()),
    "mednext_depthwise3d_wgrad_noalloc": (
        _i32,
        (_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    ),
    "mednext_group_norm_workspace_bytes": (c_size_t, (_i64, _i64, _i64, _i32)),
    "mednext_group_norm_fwd": (
        _i32,
        (_p, _i32, _p, _p, _i32, _p, _i32, _p, _p, _i64, _i64, _i64, c_double, _i32, _p, c_size_t, _p),
    ),
    "mednext_group_norm_stats": (
        _i32,
        (_p, _i32, _p, _p, _i32, _p, _p, _p, _i64, _i64, _i64, c_double, _i32, _p, c_size_t, _p),
    ),
    "mednext_group_norm_bwd": (
        _i32,
        (_p, _i32, _p, _i32, _p, _p, _p, _i32, _p, _p, _p, _i64, _i64, _i64, _i32, _p, c_size_t, _p),
    ),
    "mednext_pointwise_fwd": (
        _i32,
        (_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _p),
    ),
    "mednext_pointwise_fwd_ex": (
        _i32,
        (_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p, _p, _p, _i32, _i32, _p),
    ),
    "mednext_pointwise_fwd_ws": (
        _i32,
        (_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p, _p, _p, _i32, _i32, _p, c_size_t,
         _p),
    ),
    "mednext_pointwise_fwd_workspace_bytes": (c_size_t, (_i64, _i64, _i64, _i64, _i32, _i32)),
    "mednext_pointwise_row_slots": (_i64, (_i64, _i64, _i64, _i64, _i32)),
    "mednext_pointwise_set_kernels": (_i32, (_i32,)),
    "mednext_pointwise_uses_tiled": (_i32, (_i64, _i64, _i64, _i64, _i32, _i32)),
    "mednext_pointwise_wgrad_workspace_bytes": (c_size_t, (_i64, _i64, _i64, _i64, _i32)),
    "mednext_pointwise_wgrad_ex": (
        _i32,
        (_p, _p, _p, _p, _p, c_size_t, _i64, _i64, _i64, _i64, _i32, _p, _i32, _i32, _p),
    ),
    "mednext_pointwise_wgrad": (
        _i32,
        (_p, _p, _p, _p, _p, c_size_t, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p),
    ),
    "mednext_grn_workspace_bytes": (c_size_t, (_i64, _i64, _i64, _i32)),
    "mednext_grn_fwd": (
        _i32,
        (_p, _i32, _p, _p, _i32, _p, _p, _i64, _i64, _i64, c_double, _i32, _p, c_size_t, _p),
    ),
    "mednext_grn_bwd": (
        _i32,
        (_p, _i32, _p, _i32, _p, _p, _i32, _p, _p, _p, _i64, _i64, _i64, c_double, _i32, _p, c_size_t, _p),
    ),
    "mednext_grn_stats": (
        _i32,
        (_p, _i32, _p, _p, _i32, _p, _i64, _i64, _i64, c_double, _i32, _p, c_size_t, _p),
    ),
    "mednext_grn_bwd_rows": (
        _i32,
        (_p, _i64, _p, _p, _i32, _p, _p, _p, _i64, _i64, c_double, _p, c_size_t, _p),
    ),
    "mednext_up_join_fwd": (_i32, (_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _p)),
    "mednext_up_join_bwd_workspace_bytes": (c_size_t, (_i64, _i64, _i64)),
    "mednext_up_join_bwd": (
        _i32,
        (_p, _p, _p, _p, _p, c_size_t, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p),
    ),
    "mednext_depthwise3d_s2_gather": (_i32, (_p, _p, _p, _p, *(_i64,) * 8, _i32, _i32, _p)),
    "mednext_depthwise3d_s2_scatter": (_i32, (_p, _p, _p, _p, *(_i64,) * 8, _i32, _i32, _p)),
    "mednext_depthwise3d_s2_wgrad_workspace_bytes": (c_size_t, (*(_i64,) * 8, _i32, _i32)),
    "mednext_depthwise3d_s2_wgrad": (
        _i32,
        (_p, _p, _p, _p, _p, c_size_t, *(_i64,) * 8, _i32, _i32, _p),
    ),
}

ABI_VERSION = 14

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class HipLibraryError(RuntimeError):
    """libmednext_hip.so is missing, stale, or a call into it failed."""


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library; raises if it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise HipLibraryError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                "python -m mednext_accel_amd._build"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as error:
                raise HipLibraryError(f"{LIB_PATH} does not export {name}; rebuild it") from error
            fn.restype = restype
            fn.argtypes = list(argtypes)
        version = lib.mednext_hip_abi_version()
        if version != ABI_VERSION:
            raise HipLibraryError(f"ABI version {version} != expected {ABI_VERSION}; rebuild")
        _lib = lib
    return _lib


def last_error() -> str:
    return load().mednext_hip_last_error().decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    if status != 0:
        raise HipLibraryError(f"{what} failed (status {status}): {last_error()}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError as error:
        raise ValueError(f"unsupported dtype {dtype}") from error


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(tensor: torch.Tensor) -> int:
    """hipStream_t of PyTorch's current stream on the tensor's device (the raw
    query avoids building a Stream object on every launch)."""
    if _raw_stream is not None:
        return _raw_stream(tensor.device.index if tensor.device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(tensor.device).cuda_stream


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()
