"""Workload matrix: the operator contexts of one MedNeXt variant (v1 small /
base / medium / large, or v2 base / wide as ``v2-base`` / ``v2-wide``) and the
candidate (implementation, launch recipe) pairs measured for each
(reference profiling/matrix.py:154-320, ``build_workload_cases``).

Only the contexts this build accelerates are enumerated: the stride-1
depthwise convolutions of every resolution stage (per phase: forward, input
gradient, weight gradient), GroupNorm(C, C) and the block expansions' 1x1x1
convolutions. Depthwise candidates are the gfx950 default recipe and its
neighbours (the other matrix-core tile widths, half and double the D-run);
every context also carries the ``reference`` (native PyTorch) candidate, and
the 1x1x1 convolutions the per-sample GEMM (``pointwise_gemm_per_sample``,
the reference's own alternative) besides the matrix-core kernels.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from .. import tiles
from ..config import get_mednext_v1_config
from ..config_v2 import get_mednext_v2_config

DEPTHWISE_PHASES = {
    "forward": ("hip_depthwise_fwd", "forward"),
    "backward_input": ("hip_depthwise_dx", "input_grad"),
    "backward_weight": ("hip_split_dw", "weight_grad"),
}


@dataclass(frozen=True, slots=True)
class KernelCase:
    """One measurement: an operator context, a phase and a candidate."""

    family: str  # depthwise_conv3d | group_norm3d | pointwise_conv3d
    phase: str  # forward | backward_input | backward_weight | training
    in_channels: int
    out_channels: int
    kernel_size: int
    spatial_shape: tuple[int, int, int]
    implementation: str
    parameters: tuple[tuple[str, int], ...] = field(default=())
    batch: int = 1
    dtype: str = "bfloat16"
    direction: str = "regular"

    @property
    def context_key(self) -> tuple[object, ...]:
        """Identity of the operator context (everything but the candidate)."""
        return (self.family, self.direction, self.in_channels, self.out_channels, self.kernel_size,
                self.spatial_shape, self.batch, self.dtype)

    @property
    def parameter_map(self) -> dict[str, int]:
        return dict(self.parameters)


def stage_shapes(variant: str = "base", size: int = 128, base_channels: int = 32) -> list[tuple[int, int, int]]:
    """(channels, spatial size, expansion ratio) of the five resolution stages
    (encoder stages 0-3 and the bottleneck) of a MedNeXt v1 variant, or of
    MedNeXt v2 for ``v2-base`` / ``v2-wide`` (whose width the variant fixes)."""
    if variant.startswith("v2-"):
        cfg = get_mednext_v2_config(variant[3:], in_channels=1, out_channels=3)
        base_channels = cfg.base_channels
    else:
        cfg = get_mednext_v1_config(variant, in_channels=1, out_channels=3, base_channels=base_channels)
    out = []
    for stage in range(5):
        s = size >> stage
        if s < 1:
            break
        out.append((base_channels << stage, s, cfg.expansion_ratios[stage]))
    return out


def _depthwise_candidates(batch: int, channels: int, s: int, k: int, dtype: str, phase: str) -> list[dict[str, int]]:
    engine, tile_w, depth_chunk = tiles.depthwise_recipe(batch, channels, (s, s, s), k, dtype, phase)
    seen, out = set(), []

    def add(e: int, tw: int, dc: int) -> None:
        dc = max(1, min(dc, s))
        key = (e, tw, dc)
        if key not in seen:
            seen.add(key)
            out.append({"engine": e, "tile_w": tw, "depth_chunk": dc})

    add(engine, tile_w, depth_chunk)
    if engine == tiles.ENGINE_MFMA:
        for tw in (32, 64, 128):
            if tw <= max(32, s) and tw != tile_w:
                add(engine, tw, depth_chunk)
                add(engine, tw, depth_chunk * tile_w // tw)  # the same workgroup count
    for dc in (depth_chunk // 2, depth_chunk * 2):
        if dc < 1:
            continue
        if engine == tiles.ENGINE_VOLUME:
            acc = 8 if dtype == "float64" else 4
            plan = tiles.volume_plan(batch, channels, (s, s, s), k, dc, acc_bytes=acc, wgrad=phase == "weight_grad")
            if plan.lds_bytes > tiles.LDS_LIMIT:
                continue
        add(engine, tile_w, dc)
    if engine == tiles.ENGINE_VOLUME:
        # The VALU stencil the volume kernels replace, measured beside them.
        add(*tiles.valu_recipe(batch, channels, (s, s, s), k))
    return out


def build_workload_cases(
    variant: str = "base",
    *,
    size: int = 128,
    kernel_sizes: tuple[int, ...] = (3,),
    batch: int = 1,
    dtype: str = "bfloat16",
    families: tuple[str, ...] = ("depthwise_conv3d", "group_norm3d", "pointwise_conv3d"),
) -> tuple[KernelCase, ...]:
    cases: list[KernelCase] = []
    for channels, s, ratio in stage_shapes(variant, size):
        shape = (s, s, s)
        if "depthwise_conv3d" in families:
            for k in kernel_sizes:
                for phase, (impl, tile_phase) in DEPTHWISE_PHASES.items():
                    cases.append(KernelCase("depthwise_conv3d", phase, channels, channels, k, shape, "reference",
                                            batch=batch, dtype=dtype))
                    for params in _depthwise_candidates(batch, channels, s, k, dtype, tile_phase):
                        cases.append(KernelCase("depthwise_conv3d", phase, channels, channels, k, shape, impl,
                                                tuple(sorted(params.items())), batch=batch, dtype=dtype))
        if "group_norm3d" in families:
            for impl in ("reference", "hip_group_norm"):
                cases.append(KernelCase("group_norm3d", "training", channels, channels, 1, shape, impl,
                                        batch=batch, dtype=dtype))
        if "pointwise_conv3d" in families:
            hidden = ratio * channels
            for cin, cout in ((channels, hidden), (hidden, channels)):
                impls = ["reference", "pointwise_gemm_per_sample"]
                if tiles.pointwise_supported(cin, cout, s**3):
                    impls.append("hip_pointwise_gemm")
                for impl in impls:
                    cases.append(KernelCase("pointwise_conv3d", "training", cin, cout, 1, shape, impl,
                                            batch=batch, dtype=dtype))
    return tuple(cases)
