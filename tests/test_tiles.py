"""CDNA4 tile-recipe invariants (CPU only): valid launch parameters, LDS within
budget, and enough workgroups to fill 256 CUs wherever the problem allows."""

from __future__ import annotations

import pytest

from mednext_accel_amd import tiles

STAGES = [(32, 128), (64, 64), (128, 32), (256, 16), (512, 8)]


@pytest.mark.parametrize("channels,size", STAGES)
@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32", "float16"])
@pytest.mark.parametrize("phase", tiles.PHASES)
def test_depthwise_recipe_invariants(channels, size, k, dtype, phase):
    engine, tile_w, depth_chunk = tiles.depthwise_recipe(1, channels, (size,) * 3, k, dtype, phase)
    assert 1 <= depth_chunk <= size
    if engine == tiles.ENGINE_MFMA:
        assert dtype == "bfloat16" and tiles.mfma_supported((size,) * 3, k, phase)
        assert tile_w in (32, 64, 128) and tile_w <= max(32, size)
        rows = tiles.mfma_wgrad_rows(k, tile_w) if phase == "weight_grad" else tiles.MFMA_TILE_ROWS
        wgs = channels * -(-size // rows) * -(-size // tile_w) * -(-size // depth_chunk)
        kind = "weight_grad" if phase == "weight_grad" else "stencil"
        target = tiles.MFMA_TARGET_WORKGROUPS[(kind, k)]
        if (kind, k) in tiles.MFMA_ONE_ROUND:
            # One round at most, as close to it as whole D-runs allow.
            assert wgs <= target or depth_chunk == size
            assert depth_chunk == tiles.depth_chunk_floor(size, k) or wgs * 2 > target or depth_chunk == size
            return
    elif engine == tiles.ENGINE_VOLUME:
        assert tiles.volume_supported((size,) * 3) and tile_w == tiles.VOLUME_BAND
        acc = 8 if dtype == "float64" else 4
        plan = tiles.volume_plan(1, channels, (size,) * 3, k, depth_chunk, acc_bytes=acc, wgrad=phase == "weight_grad")
        assert plan.lds_bytes <= tiles.LDS_LIMIT
        wgs = plan.workgroups
        # Fill the chip unless the shortest D-run (the walk's k - 1 planes) forbids it.
        assert wgs >= tiles.VOLUME_TARGET_WORKGROUPS or depth_chunk <= max(2, k - 1)
        return
    else:
        plan = tiles.depthwise_plan(1, channels, (size,) * 3, k, tile_w, depth_chunk)
        assert plan.lds_bytes <= 64 * 1024
        assert plan.threads <= tiles.MAX_THREADS
        wgs = plan.workgroups
        target = tiles.TARGET_WORKGROUPS
    # Fill the chip unless the minimum D-run (halo bound) forbids it.
    assert wgs >= target or depth_chunk == tiles.depth_chunk_floor(size, k)


def test_bf16_stage0_uses_matrix_cores():
    for phase in tiles.PHASES:
        assert tiles.depthwise_recipe(1, 32, (128,) * 3, 3, "bfloat16", phase)[0] == tiles.ENGINE_MFMA


def test_mfma_requires_aligned_planes():
    assert not tiles.mfma_supported((8, 8, 8), 3, "forward")
    assert not tiles.mfma_supported((64, 64, 40), 3, "weight_grad")
    assert tiles.mfma_supported((64, 64, 40), 3, "forward")
    assert not tiles.mfma_supported((64, 64, 64), 1, "forward")


@pytest.mark.parametrize("rows,volume", [(32, 128**3), (512, 8**3), (1, 10), (4096, 16**3)])
def test_group_norm_splits(rows, volume):
    splits = tiles.group_norm_splits(1, rows, volume)
    assert 1 <= splits <= tiles.MAX_GN_SPLITS
    assert splits == 1 or volume // splits >= 4096


def test_mfma_stage0_recipes_match_measured_best():
    """C32 128^3 bf16 (the headline shape): the sweep-best launch shapes."""
    r = tiles.depthwise_recipe
    assert r(1, 32, (128,) * 3, 3, "bfloat16", "forward") == [tiles.ENGINE_MFMA, 128, 32]
    assert r(1, 32, (128,) * 3, 3, "bfloat16", "weight_grad") == [tiles.ENGINE_MFMA, 128, 64]
    assert r(1, 32, (128,) * 3, 5, "bfloat16", "weight_grad") == [tiles.ENGINE_MFMA, 128, 128]
    assert r(1, 64, (64,) * 3, 5, "bfloat16", "weight_grad") == [tiles.ENGINE_MFMA, 64, 32]
    assert r(1, 64, (64,) * 3, 3, "bfloat16", "weight_grad") == [tiles.ENGINE_MFMA, 64, 16]
    assert r(1, 32, (128,) * 3, 5, "bfloat16", "forward") == [tiles.ENGINE_MFMA, 128, 32]
    assert r(1, 64, (64,) * 3, 5, "bfloat16", "input_grad") == [tiles.ENGINE_MFMA, 64, 16]
    assert r(1, 64, (64,) * 3, 3, "bfloat16", "input_grad") == [tiles.ENGINE_MFMA, 64, 16]


def test_small_planes_use_the_volume_engine():
    """16^3 and 8^3 (H * W <= 256) take the volume kernels in every dtype in
    the volume phases; the staged planes fit the LDS limit even in fp64."""
    for channels, size in ((256, 16), (512, 8)):
        for k in (3, 5):
            for dtype in ("bfloat16", "float32", "float64"):
                for phase in tiles.PHASES:
                    engine, tile_w, depth_chunk = tiles.depthwise_recipe(1, channels, (size,) * 3, k, dtype, phase)
                    if phase not in tiles.VOLUME_PHASES:
                        assert engine == tiles.ENGINE_VALU
                        continue
                    assert (engine, tile_w) == (tiles.ENGINE_VOLUME, tiles.VOLUME_BAND)
                    acc = 8 if dtype == "float64" else 4
                    for wgrad in (False, True):
                        plan = tiles.volume_plan(1, channels, (size,) * 3, k, depth_chunk, acc_bytes=acc, wgrad=wgrad)
                        assert plan.lds_bytes <= tiles.LDS_LIMIT
    assert not tiles.volume_supported((32, 32, 32)) and tiles.volume_supported((4, 16, 16))


def test_pointwise_supported_mirrors_the_library_limits():
    """Each direction's reduction K either fits the streaming kernels' weight
    block (<= 2048) or the tiled product (<= 8192, K % 32 == 0, the other side
    % 16 == 0); one sample's tensors stay below 2 GiB."""
    ok = tiles.pointwise_supported
    assert ok(2048, 2048, 512) and ok(1, 3, 127**3) and ok(2048, 3, 8)
    assert ok(512, 4096, 512) and ok(4096, 512, 512)  # MedNeXt-L bottleneck expansion
    assert ok(8192, 16, 8) and not ok(8224, 32, 8)
    assert not ok(4112, 512, 8) and not ok(512, 4112, 8)  # K % 32
    assert not ok(4096, 520, 8) and not ok(520, 4096, 8)  # M % 16 of the wide direction
    assert not ok(0, 32, 8) and not ok(32, 32, 0)
    assert not ok(32, 64, 2**25)  # 64 x 2^25 x 2 bytes = 4 GiB per sample
