"""The allocation-free weight-gradient entry point against the allocating one.

``mednext_depthwise3d_wgrad_noalloc`` runs the same kernels as
``mednext_depthwise3d_wgrad`` with the partials in the library's per-GPU
scratch array instead of a caller workspace, so its dW and dB must equal the
allocating entry point's bit for bit. Two calls in a row, the second on a
smaller input (the array keeps the first call's contents), for the matrix-core
(bf16) and the VALU (fp32) engines; a shape whose partials exceed the array is
rejected on the host before any launch.
"""

from __future__ import annotations

import pytest
import torch

from mednext_accel_amd import _hip, hip_ops
from mednext_accel_amd.tiles import depthwise_recipe

pytestmark = pytest.mark.gpu

DEV = "cuda"


def noalloc_wgrad(x, dy, k, recipe):
    lib = _hip.load()
    n, c, d, h, w = (int(s) for s in x.shape)
    dw = torch.empty((c, 1, k, k, k), device=x.device, dtype=x.dtype)
    db = torch.empty((c,), device=x.device, dtype=x.dtype)
    engine, tile_w, depth_chunk = recipe
    status = lib.mednext_depthwise3d_wgrad_noalloc(
        x.data_ptr(), dy.data_ptr(), dw.data_ptr(), db.data_ptr(), n, c, d, h, w, k,
        _hip.dtype_code(x.dtype), engine, tile_w, depth_chunk, _hip.stream_of(x),
    )
    _hip.check(status, "mednext_depthwise3d_wgrad_noalloc")
    return dw, db


@pytest.mark.parametrize(
    "dtype,k,shapes",
    [
        (torch.bfloat16, 3, [(1, 32, 64, 64, 64), (1, 8, 32, 32, 64)]),
        (torch.bfloat16, 5, [(2, 16, 48, 64, 64), (1, 4, 33, 32, 32)]),
        (torch.float32, 3, [(1, 16, 40, 40, 40), (2, 3, 9, 11, 13)]),
    ],
)
def test_noalloc_matches_allocating_entry_point(dtype, k, shapes):
    lib = _hip.load()
    limit = int(lib.mednext_depthwise3d_wgrad_noalloc_max_bytes())
    assert limit == 16 << 20
    dtype_name = str(dtype).removeprefix("torch.")
    for i, shape in enumerate(shapes):
        print(f"[wgrad noalloc] call {i} shape={shape} k={k} dtype={dtype}", flush=True)
        gen = torch.Generator(device=DEV).manual_seed(100 + i + k)
        x = torch.randn(shape, generator=gen, device=DEV).to(dtype)
        dy = torch.randn(shape, generator=gen, device=DEV).to(dtype)
        recipe = depthwise_recipe(shape[0], shape[1], tuple(shape[2:]), k, dtype_name, "weight_grad")
        need = int(lib.mednext_depthwise3d_wgrad_workspace_bytes(*shape, k, _hip.dtype_code(dtype), *recipe))
        assert 0 < need <= limit, need
        dw_ref, db_ref = hip_ops.depthwise_weight_grad(x, dy, k, recipe)
        dw, db = noalloc_wgrad(x, dy, k, recipe)
        torch.cuda.synchronize()
        assert torch.equal(dw, dw_ref) and torch.equal(db, db_ref), shape


def test_noalloc_rejects_shapes_beyond_its_scratch():
    """Batch 128 at C32 128^3 bf16 needs about 18 MB of partials: the host
    rejects the call before it launches anything (checked here first from the
    workspace query, so the tensors passed are small)."""
    lib = _hip.load()
    shape, k = (128, 32, 128, 128, 128), 3
    recipe = depthwise_recipe(shape[0], shape[1], tuple(shape[2:]), k, "bfloat16", "weight_grad")
    need = int(lib.mednext_depthwise3d_wgrad_workspace_bytes(*shape, k, _hip.dtype_code(torch.bfloat16), *recipe))
    assert need > int(lib.mednext_depthwise3d_wgrad_noalloc_max_bytes())
    tiny = torch.zeros(16, device=DEV, dtype=torch.bfloat16)
    status = lib.mednext_depthwise3d_wgrad_noalloc(
        tiny.data_ptr(), tiny.data_ptr(), tiny.data_ptr(), tiny.data_ptr(), *shape, k,
        _hip.dtype_code(torch.bfloat16), *recipe, _hip.stream_of(tiny),
    )
    assert status == 1
    assert "scratch" in _hip.last_error()
