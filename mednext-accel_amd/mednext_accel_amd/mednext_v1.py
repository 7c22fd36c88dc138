"""MedNeXt v1 (reference models/mednext_v1.py:36-512) with the gfx950 selection hook.

Topology: 1x1 stem -> 4 encoder stages (blocks at base*2^s channels), each
followed by a stride-2 down block -> bottleneck -> 4 decoder stages, each
preceded by a transposed up block whose output is added to the encoder skip
-> 1x1 transposed head. With deep supervision, training returns the primary
output plus four auxiliary heads taken before each up block (bottleneck,
stage 3, 2, 1), ordered from the finest to the coarsest.

Parameter names, module order and state-dict keys match the reference, so its
checkpoints load with ``strict=True``. ``optimization="auto"`` (the factories'
default) installs the adaptive wrappers with the bundled gfx950 policy; an
explicit mapping or file path adds an external policy layer; ``"reference"``
keeps the plain PyTorch modules.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import replace
from os import PathLike
from typing import Literal, TypeAlias

import torch
from torch import Tensor, nn
from torch.nn import functional as F
from torch.utils.checkpoint import checkpoint

from .adaptive import (
    AdaptiveDepthwise3d,
    AdaptiveGroupNorm3d,
    AdaptivePointwise3d,
    ModelOptimizationContext,
    _conv_descriptor,
    device_facts,
    execution_context_for_shape,
    install_adaptive_operators,
)
from .blocks import MedNeXtBlock, MedNeXtDownBlock, MedNeXtUpBlock, OutputHead, conv_type
from .checkpointing import CheckpointConfig
from .config import MedNeXtV1Config, get_mednext_v1_config
from .optimization.policies import PolicyRegistry
from .optimization.policy_resolver import PolicyDecision
from .optimization.report import OptimizationReport
from .precast import install_weight_precast

DeepSupervisionOutput = Literal["tuple", "list", "stacked"]
OptimizationSource: TypeAlias = Literal["auto", "reference"] | str | PathLike[str] | Mapping[str, object]


class MedNeXtV1(nn.Module):
    def __init__(
        self,
        config: MedNeXtV1Config,
        *,
        checkpointing: CheckpointConfig | None = None,
        deep_supervision_output: DeepSupervisionOutput = "tuple",
        approximate_gelu_eval: bool = False,
    ) -> None:
        super().__init__()
        if deep_supervision_output not in ("tuple", "list", "stacked"):
            raise ValueError("deep_supervision_output must be 'tuple', 'list', or 'stacked'")
        self.config = config
        self.checkpointing = checkpointing
        self.deep_supervision_output = deep_supervision_output
        self.approximate_gelu_eval = approximate_gelu_eval
        self.optimization_source: OptimizationSource = "reference"

        dims, k = config.spatial_dims, config.kernel_size
        widths = [config.base_channels << s for s in range(5)]
        ratios, counts = config.expansion_ratios, config.block_counts

        def ckpt_expansion(stage: int) -> bool:
            return checkpointing is not None and checkpointing.checkpoints_expansion and checkpointing.includes(stage)

        def blocks(stage: int, index: int) -> nn.Sequential:
            """``counts[index]`` residual blocks at ``widths[stage]`` channels."""
            return nn.Sequential(
                *(
                    MedNeXtBlock(
                        spatial_dims=dims,
                        in_channels=widths[stage],
                        out_channels=widths[stage],
                        expansion_ratio=ratios[index],
                        kernel_size=k,
                        residual=config.residual_blocks,
                        checkpoint_expansion=ckpt_expansion(stage),
                        approximate_gelu_eval=approximate_gelu_eval,
                    )
                    for _ in range(counts[index])
                )
            )

        common = {"spatial_dims": dims, "kernel_size": k, "residual": config.residual_resampling,
                  "approximate_gelu_eval": approximate_gelu_eval}
        self.stem = conv_type(dims)(config.in_channels, config.base_channels, kernel_size=1)
        self.encoder_stages = nn.ModuleList(blocks(s, s) for s in range(4))
        self.downsamples = nn.ModuleList(
            MedNeXtDownBlock(
                in_channels=widths[s],
                out_channels=widths[s + 1],
                expansion_ratio=config.downsample_expansion_ratios[s],
                checkpoint_expansion=ckpt_expansion(s + 1),
                **common,
            )
            for s in range(4)
        )
        self.bottleneck = blocks(4, 4)
        self.upsamples = nn.ModuleList()
        self.decoder_stages = nn.ModuleList()
        for stage, index in zip((3, 2, 1, 0), (5, 6, 7, 8)):
            self.upsamples.append(
                MedNeXtUpBlock(
                    in_channels=widths[stage + 1],
                    out_channels=widths[stage],
                    expansion_ratio=ratios[index],
                    checkpoint_expansion=ckpt_expansion(stage),
                    **common,
                )
            )
            self.decoder_stages.append(blocks(stage, index))
        self.head = OutputHead(spatial_dims=dims, in_channels=widths[0], out_channels=config.out_channels)
        self.deep_supervision_heads = nn.ModuleList()
        if config.deep_supervision:
            self.deep_supervision_heads.extend(
                OutputHead(spatial_dims=dims, in_channels=widths[s], out_channels=config.out_channels)
                for s in (4, 3, 2, 1)
            )

    def _run(self, module: nn.Module, x: Tensor, stage: int) -> Tensor:
        cfg = self.checkpointing
        whole_block = cfg is not None and cfg.checkpoints_blocks and cfg.includes(stage)
        if whole_block and self.training and torch.is_grad_enabled():
            return checkpoint(module, x, use_reentrant=False, preserve_rng_state=False)
        return module(x)

    def _run_stage(self, modules: nn.Sequential, x: Tensor, stage: int) -> Tensor:
        for module in modules:
            x = self._run(module, x, stage)
        return x

    def forward(self, x: Tensor) -> Tensor | tuple[Tensor, ...] | list[Tensor]:
        x = self.stem(x)
        skips = []
        for stage in range(4):
            x = self._run_stage(self.encoder_stages[stage], x, stage)
            skips.append(x)
            x = self._run(self.downsamples[stage], x, stage + 1)
        x = self._run_stage(self.bottleneck, x, 4)
        supervise = self.training and self.config.deep_supervision
        auxiliary = []
        for i in range(4):
            stage = 3 - i
            if supervise:
                auxiliary.append(self.deep_supervision_heads[i](x))
            x = self._run(self.upsamples[i], x, stage) + skips[stage]
            x = self._run_stage(self.decoder_stages[i], x, stage)
        primary = self.head(x)
        if not supervise:
            return primary
        outputs = [primary, *auxiliary[::-1]]
        if self.deep_supervision_output == "tuple":
            return tuple(outputs)
        if self.deep_supervision_output == "list":
            return outputs
        size = primary.shape[2:]
        return torch.stack([o if o.shape[2:] == size else F.interpolate(o, size=size) for o in outputs], dim=1)

    def explain_optimization(
        self,
        *,
        input_shape: tuple[int, ...],
        dtype: str | torch.dtype,
        device: str | torch.device,
    ) -> OptimizationReport:
        """Resolve every operator's implementation for an input shape without running the model."""
        if len(input_shape) != self.config.spatial_dims + 2:
            raise ValueError(
                f"input_shape must have rank {self.config.spatial_dims + 2} for a {self.config.spatial_dims}D model"
            )
        resolver = self.__dict__.get("_optimization_resolver")
        model_context = ModelOptimizationContext(
            "mednext_v1", self.config.variant, checkpoint_name(self.checkpointing), self.approximate_gelu_eval
        )
        target = torch.device(device)
        sm, vram, arch = None, 0, None
        if target.type == "cuda" and torch.cuda.is_available():
            sm, vram, arch = device_facts(target.index if target.index is not None else torch.cuda.current_device())
        context = execution_context_for_shape(
            model_context,
            batch_size=input_shape[0],
            spatial_shape=tuple(input_shape[2:]),
            dtype=dtype,
            device_type=target.type,
            sm=sm,
            total_vram_bytes=vram,
            training=self.training,
            arch=arch,
        )
        decisions: list[PolicyDecision] = []
        for role, module in self.named_modules():
            if isinstance(module, (nn.Conv2d, nn.Conv3d, nn.ConvTranspose2d, nn.ConvTranspose3d)):
                decisions.append(
                    PolicyDecision(
                        _conv_descriptor(module, role=role), context.phase, "reference", {}, "reference",
                        "unwrapped", "guard", disposition="unwrapped",
                    )
                )
                continue
            if not isinstance(module, (AdaptivePointwise3d, AdaptiveDepthwise3d, AdaptiveGroupNorm3d)):
                continue
            local = replace(context, spatial_shape=spatial_shape_for_role(role, context.spatial_shape))
            if isinstance(module, AdaptiveDepthwise3d):
                decisions.extend(resolver.resolve(module.descriptor, local, p) for p in ("forward", "backward_input", "backward_weight"))
            else:
                decisions.append(resolver.resolve(module.descriptor, local, local.phase))
        warnings = tuple(dict.fromkeys(d.warning for d in decisions if d.warning is not None))
        layers = tuple(p.name for p in resolver.context_layers(context)) if resolver is not None else ()
        return OptimizationReport(layers or ("reference",), context, tuple(decisions), warnings)


def checkpoint_name(config: CheckpointConfig | None) -> str:
    if config is None:
        return "none"
    if config.stages is None:
        return "all-expansion" if config.style == "expansion" else "whole-block"
    return f"{config.style}:{','.join(map(str, config.stages))}"


# Resampling-block convs that read the block's input (the rest of the block
# runs at the resampled resolution).
_BLOCK_INPUT_CONVS = ("depthwise", "residual")


def spatial_shape_for_role(role: str | None, input_spatial: tuple[int, ...]) -> tuple[int, ...]:
    """Spatial shape the module named ``role`` sees for a given model input
    (halving per stride-2 step, rounding up; up-block modules after the
    transposed depthwise conv see 2s-1 before padding)."""
    if role is None or role == "stem" or role.startswith("head"):
        return tuple(input_spatial)
    parts = role.split(".")
    top = parts[0]
    if top == "encoder_stages":
        halvings = int(parts[1])
    elif top == "downsamples":
        halvings = int(parts[1]) + (0 if parts[-1] in _BLOCK_INPUT_CONVS else 1)
    elif top == "bottleneck":
        halvings = 4
    elif top == "upsamples":
        halvings = 4 - int(parts[1])
    elif top == "decoder_stages":
        halvings = 3 - int(parts[1])
    elif top == "deep_supervision_heads":
        halvings = 4 - int(parts[1])
    else:
        halvings = 0
    shape = tuple(input_spatial)
    for _ in range(halvings):
        shape = tuple((s + 1) // 2 for s in shape)
    if top == "upsamples" and parts[-1] not in _BLOCK_INPUT_CONVS:
        shape = tuple(2 * s - 1 for s in shape)
    return shape


def configure_optimization(model: MedNeXtV1, optimization: OptimizationSource) -> MedNeXtV1:
    model.optimization_source = optimization
    if isinstance(optimization, str) and optimization == "reference":
        return model
    if isinstance(optimization, str) and optimization in ("torch", "conservative", "autotune"):
        raise ValueError(f"optimization={optimization!r} was removed; use 'auto' or 'reference'")
    external = None if isinstance(optimization, str) and optimization == "auto" else optimization
    resolver = PolicyRegistry(external=external).resolver()
    model_context = ModelOptimizationContext(
        "mednext_v1", model.config.variant, checkpoint_name(model.checkpointing), model.approximate_gelu_eval
    )
    install_adaptive_operators(model, resolver=resolver, model_context=model_context)
    install_weight_precast(model)
    model.__dict__["_optimization_resolver"] = resolver
    model.__dict__["_optimization_model_context"] = model_context
    return model


def _build(
    variant: str,
    *,
    in_channels: int,
    out_channels: int,
    spatial_dims: Literal[2, 3] = 3,
    kernel_size: int = 3,
    base_channels: int = 32,
    deep_supervision: bool = False,
    checkpointing: CheckpointConfig | None = None,
    deep_supervision_output: DeepSupervisionOutput = "tuple",
    approximate_gelu_eval: bool = False,
    optimization: OptimizationSource = "auto",
) -> MedNeXtV1:
    config = get_mednext_v1_config(
        variant,
        in_channels=in_channels,
        out_channels=out_channels,
        spatial_dims=spatial_dims,
        kernel_size=kernel_size,
        base_channels=base_channels,
        deep_supervision=deep_supervision,
    )
    model = MedNeXtV1(
        config,
        checkpointing=checkpointing,
        deep_supervision_output=deep_supervision_output,
        approximate_gelu_eval=approximate_gelu_eval,
    )
    return configure_optimization(model, optimization)


def mednext_small(**kwargs) -> MedNeXtV1:
    """Published MedNeXt Small (keyword arguments as ``mednext_base``)."""
    return _build("small", **kwargs)


def mednext_base(**kwargs) -> MedNeXtV1:
    """Published MedNeXt Base. Keywords: in_channels, out_channels (required);
    spatial_dims=3, kernel_size=3, base_channels=32, deep_supervision=False,
    checkpointing=None, deep_supervision_output="tuple",
    approximate_gelu_eval=False, optimization="auto"."""
    return _build("base", **kwargs)


def mednext_medium(**kwargs) -> MedNeXtV1:
    """Published MedNeXt Medium (keyword arguments as ``mednext_base``)."""
    return _build("medium", **kwargs)


def mednext_large(**kwargs) -> MedNeXtV1:
    """Published MedNeXt Large (keyword arguments as ``mednext_base``)."""
    return _build("large", **kwargs)
