"""Launch recipes for the HIP implementations, as plain integers.

The split between *selecting* an implementation (policy rules) and *computing*
its launch parameters (formulas here) follows the reference
(optimization/parameters.py:52-108): a policy says ``parameters: auto`` or gives
literal overrides, and overrides are validated, never evaluated. The formulas
are this package's gfx950 recipes (``tiles.py``).

Recipe fields:
  hip_depthwise_fwd / hip_depthwise_dx / hip_split_dw:
      engine (0 = VALU stencil, 1 = bf16 matrix cores, 2 = small-plane volume
      kernels), tile_w, depth_chunk
  hip_group_norm: splits (chunks per (n, c) row)
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import TYPE_CHECKING

from .. import tiles
from .descriptors import ExecutionContext, OperatorDescriptor

if TYPE_CHECKING:
    from .policy import PolicySelection

_DEPTHWISE_PHASE = {
    "hip_depthwise_fwd": "forward",
    "hip_depthwise_dx": "input_grad",
    "hip_split_dw": "weight_grad",
}
_HIP_RECIPES = frozenset({*_DEPTHWISE_PHASE, "hip_group_norm"})
# The reference's Triton recipes: accepted by the schema (so its policy files
# parse) but never launched here, since those implementations are always guarded.
_TRITON_RECIPES = {
    "triton_depthwise_dx": {"dx_block"},
    "triton_downsample_dx": {"dx_block"},
    "triton_split_dw": {"dw_block", "dw_splits"},
    "triton_transpose_split_dw": {"dw_block", "dw_splits"},
}
MAX_DEPTH_CHUNK = 1 << 16


def has_parameter_recipe(implementation: str) -> bool:
    return implementation in _HIP_RECIPES or implementation in _TRITON_RECIPES


def _positive_int(name: str, value: object) -> int:
    if type(value) is not int or value <= 0:
        raise ValueError(f"parameters.{name} must be a positive integer")
    return value


def validate_parameters(implementation: str, parameters: Mapping[str, object]) -> None:
    """Check literal launch overrides (types, ranges, combinations)."""
    for name in parameters:
        if not isinstance(name, str):
            raise ValueError("parameters keys must be strings")
    if implementation in _DEPTHWISE_PHASE:
        allowed = {"engine", "tile_w", "depth_chunk"}
    elif implementation == "hip_group_norm":
        allowed = {"splits"}
    elif implementation in _TRITON_RECIPES:
        allowed = _TRITON_RECIPES[implementation]
    else:
        for name, value in parameters.items():
            if value is not None and not isinstance(value, (str, bool, int, float)):
                raise ValueError(f"parameters.{name} must be a literal scalar")
        return
    unknown = set(parameters) - allowed
    if unknown:
        raise ValueError(f"unknown parameters field {sorted(unknown)[0]!r} for {implementation}")
    if implementation in _TRITON_RECIPES:
        for name, value in parameters.items():
            _positive_int(name, value)
            if name == "dw_splits" and value > 512:
                raise ValueError("parameters.dw_splits must be <= 512")
            if name.endswith("_block") and (value & (value - 1) or value > 1024):
                raise ValueError(f"parameters.{name} must be a power of two <= 1024")
        return
    if implementation == "hip_group_norm":
        if "splits" in parameters and _positive_int("splits", parameters["splits"]) > tiles.MAX_GN_SPLITS:
            raise ValueError(f"parameters.splits must be <= {tiles.MAX_GN_SPLITS}")
        return
    engine = parameters.get("engine", tiles.ENGINE_VALU)
    if engine not in (tiles.ENGINE_VALU, tiles.ENGINE_MFMA, tiles.ENGINE_VOLUME) or type(engine) is not int:
        raise ValueError("parameters.engine must be 0 (VALU), 1 (MFMA) or 2 (VOLUME)")
    if "tile_w" in parameters:
        tile_w = _positive_int("tile_w", parameters["tile_w"])
        widths = {tiles.ENGINE_MFMA: (32, 64, 128), tiles.ENGINE_VOLUME: (tiles.VOLUME_BAND,)}.get(
            engine, tiles.TILE_WIDTHS
        )
        if tile_w not in widths:
            raise ValueError(f"parameters.tile_w must be one of {widths} for engine {engine}")
    if "depth_chunk" in parameters and _positive_int("depth_chunk", parameters["depth_chunk"]) > MAX_DEPTH_CHUNK:
        raise ValueError(f"parameters.depth_chunk must be <= {MAX_DEPTH_CHUNK}")


def parameter_defaults(
    implementation: str, descriptor: OperatorDescriptor, context: ExecutionContext
) -> dict[str, int]:
    """gfx950 launch defaults for one (operator, context)."""
    if implementation in _DEPTHWISE_PHASE:
        engine, tile_w, depth_chunk = tiles.depthwise_recipe(
            context.batch_size,
            descriptor.in_channels,
            tuple(context.spatial_shape),
            descriptor.kernel_size[0],
            context.dtype,
            _DEPTHWISE_PHASE[implementation],
        )
        return {"engine": engine, "tile_w": tile_w, "depth_chunk": depth_chunk}
    if implementation == "hip_group_norm":
        return {"splits": tiles.group_norm_splits(context.batch_size, descriptor.in_channels, context.spatial_volume)}
    raise ValueError(f"{implementation!r} has no parameter recipe in this build")


def resolve_parameters(
    selection: PolicySelection, descriptor: OperatorDescriptor, context: ExecutionContext
) -> dict[str, object]:
    """No parameters given -> {}; ``auto`` -> defaults; a mapping overrides the defaults."""
    supplied = selection.parameters
    if supplied is None:
        return {}
    if supplied == "auto":
        return parameter_defaults(selection.implementation, descriptor, context)
    merged = (
        parameter_defaults(selection.implementation, descriptor, context)
        if selection.implementation in _HIP_RECIPES
        else {}
    )
    merged.update(supplied)
    validate_parameters(selection.implementation, merged)
    if selection.implementation in _DEPTHWISE_PHASE:
        _check_engine_fits(selection.implementation, merged, descriptor, context)
    return merged


def _check_engine_fits(implementation, params, descriptor, context) -> None:
    if params["engine"] == tiles.ENGINE_VOLUME:
        spatial = tuple(context.spatial_shape)
        if not tiles.volume_supported(spatial):
            raise ValueError("engine 2 (VOLUME) needs planes of at most 256 elements")
        plan = tiles.volume_plan(context.batch_size, descriptor.in_channels, spatial, descriptor.kernel_size[0],
                                 params["depth_chunk"], acc_bytes=8 if context.dtype == "float64" else 4,
                                 wgrad=implementation == "hip_split_dw")
        if plan.lds_bytes > tiles.LDS_LIMIT:
            raise ValueError("engine 2 (VOLUME): depth_chunk too long for the LDS limit")
        return
    if params["engine"] != tiles.ENGINE_MFMA:
        return
    phase = _DEPTHWISE_PHASE[implementation]
    spatial = tuple(context.spatial_shape)
    if context.dtype != "bfloat16" or not tiles.mfma_supported(spatial, descriptor.kernel_size[0], phase):
        raise ValueError("engine 1 (MFMA) needs bfloat16 and a plane shape the matrix-core kernels take")
