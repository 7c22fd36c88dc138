"""The C-ABI library loads and exports every symbol include/*.h declares (CPU only:
no compute calls, only symbol lookup and the argument-validation paths that
return before any launch)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from mednext_accel_amd import _build, _hip

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions() -> list[str]:
    names = []
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"\b(mednext_\w+)\s*\(", text)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not _build.LIB_PATH.exists():
        pytest.fail(f"{_build.LIB_PATH} missing: run __graft_entry__.build() first")
    return ctypes.CDLL(str(_build.LIB_PATH))


def test_header_declares_entry_points():
    names = declared_functions()
    for name in ("mednext_depthwise3d_fwd", "mednext_depthwise3d_dgrad", "mednext_depthwise3d_wgrad",
                 "mednext_group_norm_fwd", "mednext_group_norm_bwd", "mednext_hip_last_error"):
        assert name in names


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_every_declared_symbol():
    assert set(declared_functions()) == set(_hip.SIGNATURES)


def test_abi_version_and_error_slot():
    lib = _hip.load()
    assert lib.mednext_hip_abi_version() == _hip.ABI_VERSION
    # Invalid arguments are rejected before any device work.
    status = lib.mednext_depthwise3d_fwd(None, None, None, None, 1, 1, 1, 1, 1, 3, 0, 0, 64, 1, None)
    assert status == 1
    assert "null tensor pointer" in _hip.last_error()
    status = lib.mednext_depthwise3d_fwd(8, 8, None, 8, 1, 1, 1, 1, 1, 7, 0, 0, 64, 1, None)
    assert status == 1 and "kernel_size" in _hip.last_error()
    assert lib.mednext_depthwise3d_wgrad_workspace_bytes(1, 32, 128, 128, 128, 3, 3, 0, 64, 32) > 0
    assert lib.mednext_depthwise3d_wgrad_workspace_bytes(1, 32, 128, 128, 128, 3, 3, 1, 64, 16) > 0
    # MFMA engine rejects fp32 and W not a multiple of 32.
    assert lib.mednext_depthwise3d_wgrad_workspace_bytes(1, 32, 128, 128, 128, 3, 0, 1, 64, 16) == 0
    assert lib.mednext_depthwise3d_wgrad_workspace_bytes(1, 32, 128, 128, 40, 3, 3, 1, 64, 16) == 0
    assert lib.mednext_group_norm_workspace_bytes(1, 32, 128**3, 32) == 1 * 32 * 33 * 2 * 8


def test_pointwise_kernel_choice_is_host_logic():
    """The forward kernel family is chosen on the host from the shape and mode
    alone (no device query): tiled for K >= 256 where the streaming plan would
    re-read X and the tiled grid fills the chip."""
    from mednext_accel_amd import hip_ops as P

    uses = P.pointwise_uses_tiled
    try:
        P.set_pointwise_kernels(P.PW_KERNELS_AUTO)
        assert uses(2, 1024, 128, 32768)                 # GRN project backward: dx = W1^T du
        assert uses(2, 256, 2048, 4096)                  # expand of a 2048-wide hidden layer
        assert uses(2, 256, 64, 64**3, P.PW_PROLOGUE_AFFINE, P.PW_EPILOGUE_BIAS_RESIDUAL)  # GRN project
        assert not uses(2, 128, 1024, 32768, 0, P.PW_EPILOGUE_AFFINE_SCALE)  # K = 128: epilogue-bound
        assert not uses(2, 32, 96, 128**3)               # expand at K = 32: X read twice
        assert not uses(2, 2048, 256, 512)               # too few 128-voxel chunks to fill the chip
        assert not uses(2, 1024, 120, 32768)             # M % 16 != 0
        assert not uses(2, 1000, 128, 32768)             # K % 32 != 0
        assert not uses(2, 1024, 128, 32768, P.PW_PROLOGUE_GELU, 0)
        assert not uses(2, 128, 1024, 32768, 0, P.PW_EPILOGUE_ROW_REDUCE)
        P.set_pointwise_kernels(P.PW_KERNELS_TILED)
        assert uses(2, 32, 96, 128**3) and uses(2, 2048, 256, 512)
        assert not uses(2, 1024, 120, 32768)
        P.set_pointwise_kernels(P.PW_KERNELS_STREAMING)
        assert not uses(2, 1024, 128, 32768)
        P.set_pointwise_kernels(P.PW_KERNELS_TILED_64)
        assert uses(2, 32, 96, 128**3) and not uses(2, 1024, 120, 32768)
        with pytest.raises(_hip.HipLibraryError):
            P.set_pointwise_kernels(4)
    finally:
        P.set_pointwise_kernels(P.PW_KERNELS_AUTO)
