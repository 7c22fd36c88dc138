"""CDNA4 (gfx950 / MI355X) launch recipes for the HIP kernels.

Pure integer arithmetic, no torch: the policy layer, the ops and the tests all
call these. The machine model is 256 CUs in 8 XCDs, wave64, 160 KiB LDS per CU
and 256-thread workgroups. Recipes are chosen so that a launch has at least
``TARGET_WORKGROUPS`` workgroups (4 per CU) whenever the problem allows it, while
keeping per-workgroup halo overheads small.
"""

from __future__ import annotations

from dataclasses import dataclass

CU_COUNT = 256
TARGET_WORKGROUPS = 4 * CU_COUNT
LDS_BYTES_PER_CU = 160 * 1024
MAX_THREADS = 256
ROWS_PER_THREAD = 2  # kRH in depthwise.hip
TILE_WIDTHS = (4, 8, 16, 32, 64)
MAX_GN_SPLITS = 4096


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


@dataclass(frozen=True, slots=True)
class DepthwiseTile:
    """Launch shape of one depthwise kernel (mirrors make_plan in depthwise.hip)."""

    tile_w: int
    depth_chunk: int
    threads_w: int
    threads_h: int
    tiles_h: int
    tiles_w: int
    chunks_d: int
    workgroups: int
    threads: int
    lds_bytes: int

    def as_list(self) -> list[int]:
        return [self.tile_w, self.depth_chunk]


def depthwise_plan(
    batch: int,
    channels: int,
    spatial: tuple[int, int, int],
    kernel_size: int,
    tile_w: int,
    depth_chunk: int,
    *,
    acc_bytes: int = 4,
) -> DepthwiseTile:
    """Replicate the kernel-side plan for a given recipe (used by checks and tests)."""
    if tile_w not in TILE_WIDTHS:
        raise ValueError(f"tile_w must be one of {TILE_WIDTHS}")
    if depth_chunk < 1:
        raise ValueError("depth_chunk must be >= 1")
    d, h, w = spatial
    threads_w = tile_w // 4
    threads_h = min(MAX_THREADS // threads_w, _cdiv(h, ROWS_PER_THREAD))
    td = min(depth_chunk, d)
    tiles_h = _cdiv(h, ROWS_PER_THREAD * threads_h)
    tiles_w = _cdiv(w, tile_w)
    chunks_d = _cdiv(d, td)
    used = threads_w * threads_h
    threads = _cdiv(used, 64) * 64
    pad = kernel_size // 2
    lds = (ROWS_PER_THREAD * threads_h + 2 * pad) * (tile_w + 8) * acc_bytes
    return DepthwiseTile(
        tile_w,
        td,
        threads_w,
        threads_h,
        tiles_h,
        tiles_w,
        chunks_d,
        batch * channels * chunks_d * tiles_h * tiles_w,
        threads,
        lds,
    )


def depthwise_recipe(
    batch: int, channels: int, spatial: tuple[int, int, int], kernel_size: int
) -> list[int]:
    """Default ``[tile_w, depth_chunk]`` for fwd / dgrad / wgrad on gfx950.

    The tile is as wide as the plane allows (up to 64 columns, i.e. 128 bytes of
    bf16 per row segment) and as tall as 256 threads reach. The D-run per
    workgroup is the longest that still yields TARGET_WORKGROUPS workgroups, but
    at least 4 planes per halo of k-1 so re-read halo planes stay below ~50%.
    """
    d, h, w = spatial
    tile_w = 4
    while tile_w < 64 and tile_w < w:
        tile_w *= 2
    plan = depthwise_plan(batch, channels, spatial, kernel_size, tile_w, d)
    slabs = plan.workgroups  # workgroups with depth_chunk == D
    wanted_chunks = _cdiv(TARGET_WORKGROUPS, max(1, slabs))
    depth_chunk = max(1, _cdiv(d, wanted_chunks))
    floor = min(d, max(4, 2 * (kernel_size - 1)))
    depth_chunk = max(depth_chunk, floor)
    return [tile_w, depth_chunk]


def group_norm_splits(batch: int, channels: int, spatial_volume: int) -> int:
    """Chunks per (n, c) row: enough workgroups to fill the chip, >= 4096 elements each."""
    rows = max(1, batch * channels)
    by_occupancy = _cdiv(TARGET_WORKGROUPS, rows)
    by_size = max(1, spatial_volume // 4096)
    return max(1, min(by_occupancy, by_size, MAX_GN_SPLITS))
