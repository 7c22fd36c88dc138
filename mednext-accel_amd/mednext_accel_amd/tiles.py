"""CDNA4 (gfx950 / MI355X) launch recipes for the HIP kernels.

Pure integer arithmetic, no torch: the policy layer, the ops and the tests all
call these. The machine model is 256 CUs in 8 XCDs, wave64, 160 KiB LDS per CU
and 256-thread workgroups. Recipes are chosen so that a launch has at least
``TARGET_WORKGROUPS`` workgroups (4 per CU) whenever the problem allows it, while
keeping per-workgroup halo overheads small.
"""

from __future__ import annotations

import functools
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
        return [ENGINE_VALU, self.tile_w, self.depth_chunk]


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


ENGINE_VALU = 0
ENGINE_MFMA = 1
ENGINE_VOLUME = 2
MFMA_TILE_ROWS = 32  # two 16-row MFMA tiles per workgroup
PHASES = ("forward", "input_grad", "weight_grad")


@functools.lru_cache(maxsize=4096)
def mfma_supported(spatial: tuple[int, int, int], kernel_size: int, phase: str) -> bool:
    """Shapes the bf16 matrix-core kernels take (mirrors depthwise_mfma.hip)."""
    d, h, w = spatial
    ok = kernel_size in (3, 5) and w % 8 == 0 and w >= 32 and h >= 32 and d * h * w * 2 < 2**31
    if phase == "weight_grad":
        ok = ok and w % 32 == 0
    return ok


def depth_chunk_floor(d: int, kernel_size: int) -> int:
    """Shortest D-run a recipe uses: k - 1 planes (the re-read halo is then at
    most half the run). Measured on MI355X at the small stage shapes (C256
    16^3, C512 8^3) the k - 1 floor beats longer runs by 6-27%."""
    return min(d, max(2, kernel_size - 1))


def _depth_chunk(d: int, slabs: int, kernel_size: int, target: int = TARGET_WORKGROUPS) -> int:
    wanted_chunks = _cdiv(target, max(1, slabs))
    depth_chunk = max(1, _cdiv(d, wanted_chunks))
    return max(depth_chunk, depth_chunk_floor(d, kernel_size))


# Workgroups a matrix-core depthwise launch aims for, per (phase kind, k). The
# forward / input-grad kernel holds two 16x(tile_w) accumulator rows per wave
# and k rotating output planes, so it wants long D-runs and ~2 workgroups per CU
# (k=5 in its block-Toeplitz form: 2-3 resident per CU). The weight-grad kernel
# (4 waves of 16 - (k-1) grad_output rows x 32 columns each) wants ~2-2.5 per
# CU. Measured on MI355X at the MedNeXt stage shapes (C32 128^3, C64 64^3,
# C128 32^3; k=3 and 5): these targets reproduce the best depth_chunk of a
# sweep over {4..128} within run-to-run noise (k=5 forward at 128^3: tile 128
# / D-run 32 55.5 us, tile 64 / 64 54.1 us, the former target's 128 / 64
# 60.4 us).
MFMA_TARGET_WORKGROUPS = {
    ("stencil", 3): 2 * CU_COUNT,
    ("stencil", 5): 2 * CU_COUNT,
    ("weight_grad", 3): 5 * CU_COUNT // 2,
    ("weight_grad", 5): 2 * CU_COUNT,
}
# Kinds whose grid is kept within one round of the target instead of reaching
# it. The k5 weight-grad kernel holds two workgroups per CU (210 registers),
# and a second, partial round costs about as much as a full one: C64 64^3
# D-run 22 (576 workgroups) 49.6 us against D-run 32 (384) 37.7 us; at C32
# 128^3, 352 to 1536 workgroups all run 108-118 us.
MFMA_ONE_ROUND = {("weight_grad", 5)}


def mfma_wgrad_rows(kernel_size: int, tile_w: int) -> int:
    """grad_output rows per weight-grad workgroup: 4 / (tile_w / 32) waves
    stacked vertically, each covering 16 - (k - 1) rows."""
    return (16 - (kernel_size - 1)) * (4 // (tile_w // 32))


# ----------------------------------------------------------- small planes

VOLUME_BAND = 64  # plane positions per workgroup of the volume kernels (their tile_w)
VOLUME_MAX_PLANE = 4 * VOLUME_BAND  # H * W the volume kernels take
VOLUME_TARGET_WORKGROUPS = 2 * CU_COUNT
# Phases whose default recipe is the volume engine on small planes.
VOLUME_PHASES = ("forward", "input_grad", "weight_grad")
LDS_LIMIT = 64 * 1024  # per-workgroup LDS the kernels request at most


def volume_supported(spatial: tuple[int, int, int]) -> bool:
    """Planes the volume kernels take (mirrors dw_volume_supported)."""
    _d, h, w = spatial
    return 1 <= h * w <= VOLUME_MAX_PLANE


@dataclass(frozen=True, slots=True)
class VolumePlan:
    """Launch shape of the volume kernels (mirrors band_plan in depthwise_volume.hip):
    one workgroup of k waves per (slab, band of 64 plane positions, D-run)."""

    depth_chunk: int
    chunks_d: int
    bands: int
    staged_rows: int
    workgroups: int
    threads: int
    lds_bytes: int


def volume_band_rows(h: int, w: int) -> int:
    """The most plane rows one band of VOLUME_BAND positions spans."""
    most = 1
    for p0 in range(0, h * w, VOLUME_BAND):
        last = min(p0 + VOLUME_BAND, h * w) - 1
        most = max(most, last // w - p0 // w + 1)
    return most


def volume_lds_bytes(depth_chunk: int, spatial, kernel_size: int, acc_bytes: int, wgrad: bool) -> int:
    d, h, w = spatial
    p = kernel_size // 2
    walk = max(min(depth_chunk, d), kernel_size - 1)
    staged = (walk + 2 * p) * (volume_band_rows(h, w) + 2 * p) * (w + 2 * p)
    if not wgrad:
        return (staged + kernel_size * walk * VOLUME_BAND) * acc_bytes
    values = 13 if (acc_bytes == 8 and kernel_size == 5) else kernel_size**2 + 1
    red = kernel_size * VOLUME_BAND * (values | 1)
    return max(staged + walk * VOLUME_BAND, red) * acc_bytes


def volume_plan(batch: int, channels: int, spatial, kernel_size: int, depth_chunk: int, *, acc_bytes: int = 4,
                wgrad: bool = False) -> VolumePlan:
    d, h, w = spatial
    td = min(depth_chunk, d)
    chunks = _cdiv(d, td)
    bands = _cdiv(h * w, VOLUME_BAND)
    return VolumePlan(td, chunks, bands, volume_band_rows(h, w) + 2 * (kernel_size // 2),
                      batch * channels * bands * chunks, VOLUME_BAND * kernel_size,
                      volume_lds_bytes(td, spatial, kernel_size, acc_bytes, wgrad))


def volume_depth_chunk(batch: int, channels: int, spatial, kernel_size: int, acc_bytes: int) -> int:
    """The longest D-run (D, halved) whose grid still has
    VOLUME_TARGET_WORKGROUPS workgroups (down to k - 1 planes, the walk's
    minimum) and whose staged planes fit the LDS limit in both the stencil and
    the weight-gradient kernel."""
    d = spatial[0]
    floor = max(2, kernel_size - 1)

    def fits(td: int) -> bool:
        return all(
            volume_plan(batch, channels, spatial, kernel_size, td, acc_bytes=acc_bytes, wgrad=wgrad).lds_bytes
            <= LDS_LIMIT
            for wgrad in (False, True)
        )

    td = d
    while td > 1 and (
        not fits(td)
        or (td > floor and volume_plan(batch, channels, spatial, kernel_size, td).workgroups < VOLUME_TARGET_WORKGROUPS)
    ):
        td = _cdiv(td, 2)
    return td


@functools.lru_cache(maxsize=4096)
def depthwise_recipe(
    batch: int,
    channels: int,
    spatial: tuple[int, int, int],
    kernel_size: int,
    dtype: str = "float32",
    phase: str = "forward",
) -> list[int]:
    """Default ``[engine, tile_w, depth_chunk]`` for one depthwise phase on gfx950.

    bf16 shapes the matrix-core kernels take use them, with ``tile_w = min(128,
    W)`` columns per workgroup: forward / input-grad tiles are 32 rows high,
    weight-grad tiles ``mfma_wgrad_rows(k, tile_w)``. The D-run per workgroup is
    the longest that still yields ``MFMA_TARGET_WORKGROUPS`` (for the kinds of
    ``MFMA_ONE_ROUND``, the shortest that stays within it).
    Small planes (H * W <= 256: the 16^3 and 8^3 stages) run the volume
    kernels (one workgroup per 64-position band of a plane and D-run) with
    ``tile_w = VOLUME_BAND`` and the D-run of ``volume_depth_chunk``, in the
    phases of ``VOLUME_PHASES``.
    Everything else runs the VALU stencil with the widest tile the plane allows
    (up to 64 columns) and a D-run that yields TARGET_WORKGROUPS workgroups. In
    both cases at least k - 1 planes per workgroup (``depth_chunk_floor``).
    """
    if phase not in PHASES:
        raise ValueError(f"phase must be one of {PHASES}")
    d, h, w = spatial
    if dtype == "bfloat16" and mfma_supported(spatial, kernel_size, phase):
        tile_w = 32
        while tile_w < 128 and tile_w * 2 <= w:
            tile_w *= 2
        if phase == "weight_grad":
            rows, kind = mfma_wgrad_rows(kernel_size, tile_w), "weight_grad"
        else:
            rows, kind = MFMA_TILE_ROWS, "stencil"
        slabs = batch * channels * _cdiv(h, rows) * _cdiv(w, tile_w)
        target = MFMA_TARGET_WORKGROUPS[(kind, kernel_size)]
        if (kind, kernel_size) in MFMA_ONE_ROUND:
            chunks = max(1, target // slabs)
            return [ENGINE_MFMA, tile_w, max(_cdiv(d, chunks), depth_chunk_floor(d, kernel_size))]
        return [ENGINE_MFMA, tile_w, _depth_chunk(d, slabs, kernel_size, target)]
    if volume_supported(spatial) and phase in VOLUME_PHASES:
        acc_bytes = 8 if dtype == "float64" else 4
        return [ENGINE_VOLUME, VOLUME_BAND, volume_depth_chunk(batch, channels, spatial, kernel_size, acc_bytes)]
    return valu_recipe(batch, channels, spatial, kernel_size)


def valu_recipe(batch: int, channels: int, spatial: tuple[int, int, int], kernel_size: int) -> list[int]:
    """The VALU stencil's ``[engine, tile_w, depth_chunk]``: the widest tile the
    plane allows (up to 64 columns) and a D-run that yields TARGET_WORKGROUPS."""
    d, _h, w = spatial
    tile_w = 4
    while tile_w < 64 and tile_w < w:
        tile_w *= 2
    plan = depthwise_plan(batch, channels, spatial, kernel_size, tile_w, d)
    return [ENGINE_VALU, tile_w, _depth_chunk(d, plan.workgroups, kernel_size)]


@functools.lru_cache(maxsize=4096)
def group_norm_splits(batch: int, channels: int, spatial_volume: int) -> int:
    """Chunks per (n, c) row: enough workgroups to fill the chip, >= 4096 elements each."""
    rows = max(1, batch * channels)
    by_occupancy = _cdiv(TARGET_WORKGROUPS, rows)
    by_size = max(1, spatial_volume // 4096)
    return max(1, min(by_occupancy, by_size, MAX_GN_SPLITS))


# ------------------------------------------------------------------ pointwise

PW_CHUNK = 128  # voxels per wave task of pw_fwd_kernel
PW_MAX_K = 2048  # reduction channels the LDS weight block holds (16 x 2048 bf16)
PW_MAX_TILED_K = 8192  # the tiled product streams K in 32-channel slices
PW_WG_VOXELS = 128  # voxels one pw_wgrad workgroup covers per round (4 waves x 32)


@functools.lru_cache(maxsize=4096)
def pointwise_supported(in_channels: int, out_channels: int, voxels: int) -> bool:
    """Shapes the bf16 matrix-core pointwise kernels take (mirrors pointwise.hip).

    Any channel counts and voxel count, as long as the reduction of each
    direction (forward K = in_channels, M = out_channels; input gradient the
    other way round) fits the streaming kernels' weight block (K <= 2048) or
    the tiled product (K <= 8192, K % 32 == 0, M % 16 == 0; no GELU prologue,
    which callers only use below 128 hidden channels), and one sample's tensor
    stays below 2 GiB (32-bit buffer offsets).
    """

    def reduces(k: int, m: int) -> bool:
        return 1 <= k <= PW_MAX_K or (k <= PW_MAX_TILED_K and k % 32 == 0 and m % 16 == 0)

    small = in_channels * voxels * 2 < 2**31 and out_channels * voxels * 2 < 2**31
    return (
        in_channels >= 1 and out_channels >= 1 and voxels >= 1 and small
        and reduces(in_channels, out_channels) and reduces(out_channels, in_channels)
    )


@functools.lru_cache(maxsize=4096)
def pointwise_blocks(batch: int, k: int, m: int, voxels: int) -> int:
    """Workgroups per (sample, row group) for pw_fwd_kernel; 0 lets the library
    pick: at most two resident 4-wave workgroups per CU over the whole grid (the
    kernel is register-bound to two waves per SIMD), at least one 128-voxel
    chunk per wave."""
    del batch, k, m, voxels
    return 0


@functools.lru_cache(maxsize=4096)
def pointwise_wgrad_splits(batch: int, k: int, m: int, voxels: int) -> int:
    """V-splits per sample for pw_wgrad_kernel: about eight workgroups per CU
    over the grid (two rounds at three to four resident), each split at least
    four 128-voxel LDS stages. Measured on MI355X at C32 128^3: 2048 splits run
    the stage-0 weight gradients ~25% faster than 512."""
    def tiles(rows: int) -> int:
        side = 1 if rows <= 16 else 2 if rows <= 32 else 4
        return _cdiv(rows, 16 * side)

    blocks = max(1, batch * tiles(m) * tiles(k))
    wanted = _cdiv(8 * CU_COUNT, blocks)
    return max(1, min(wanted, _cdiv(voxels, 4 * PW_WG_VOXELS), 65535))
