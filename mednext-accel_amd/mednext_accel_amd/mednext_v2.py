"""MedNeXt v2 (reference models/mednext_v2.py:39-382) with the gfx950 selection hook.

Same five-resolution topology as v1 (1x1 stem, four encoder stages each
followed by a down block, bottleneck, four up block + decoder stage pairs,
1x1 transposed head, optional deep-supervision heads), built from the v2
blocks (GRN inside every expansion, kernel 3). Differences from v1 that the
reference fixes and this module keeps:

* up blocks pad at the end of each dimension, and each decoder input is the
  up block's output cropped or zero-padded at the right edges to the encoder
  skip's shape before the add (``reconcile_spatial``), so any input extent
  works;
* a batch-1 input whose volume shrinks to one voxel after four halvings is
  rejected up front (GroupNorm would fail on it with batch size one).

``optimization="auto"`` installs the adaptive operator wrappers and the
adaptive GRN with the bundled gfx950 policy; ``"reference"`` keeps the plain
PyTorch modules; a mapping or path adds an external policy layer.
"""

from __future__ import annotations

from dataclasses import replace

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
from .blocks import OutputHead
from .blocks_v2 import MedNeXtV2Block, MedNeXtV2DownBlock, MedNeXtV2UpBlock
from .checkpointing import CheckpointConfig
from .config_v2 import MedNeXtV2Config, get_mednext_v2_config
from .grn import (
    AdaptiveGlobalResponseNorm3d,
    GlobalResponseNorm3d,
    install_adaptive_grn,
    install_fused_grn_expansions,
)
from .mednext_v1 import DeepSupervisionOutput, OptimizationSource, checkpoint_name, spatial_shape_for_role
from .precast import install_weight_precast
from .optimization.descriptors import OperatorDescriptor
from .optimization.policies import PolicyRegistry
from .optimization.policy_resolver import PolicyDecision
from .optimization.report import OptimizationReport


def reconcile_spatial(x: Tensor, target_shape: tuple[int, ...]) -> Tensor:
    """Crop, then zero-pad, the right edge of each spatial dimension to ``target_shape``."""
    x = x[..., : target_shape[0], : target_shape[1], : target_shape[2]]
    missing = [max(0, want - have) for have, want in zip(x.shape[2:], target_shape)]
    if not any(missing):
        return x
    return F.pad(x, (0, missing[2], 0, missing[1], 0, missing[0]))


_reconcile_spatial = reconcile_spatial  # the reference's private name


class MedNeXtV2(nn.Module):
    def __init__(
        self,
        config: MedNeXtV2Config,
        *,
        checkpointing: CheckpointConfig | None = None,
        deep_supervision_output: DeepSupervisionOutput = "tuple",
    ) -> None:
        super().__init__()
        if deep_supervision_output not in ("tuple", "list", "stacked"):
            raise ValueError("deep_supervision_output must be 'tuple', 'list', or 'stacked'")
        self.config = config
        self.checkpointing = checkpointing
        self.deep_supervision_output = deep_supervision_output
        self.optimization_source: OptimizationSource = "reference"
        widths = [config.base_channels << s for s in range(5)]
        ratios, counts = config.expansion_ratios, config.block_counts

        def ckpt_expansion(stage: int) -> bool:
            return checkpointing is not None and checkpointing.checkpoints_expansion and checkpointing.includes(stage)

        def blocks(stage: int, index: int) -> nn.Sequential:
            return nn.Sequential(
                *(
                    MedNeXtV2Block(
                        in_channels=widths[stage],
                        out_channels=widths[stage],
                        expansion_ratio=ratios[index],
                        checkpoint_expansion=ckpt_expansion(stage),
                    )
                    for _ in range(counts[index])
                )
            )

        self.stem = nn.Conv3d(config.in_channels, widths[0], kernel_size=1)
        self.encoder_stages = nn.ModuleList(blocks(s, s) for s in range(4))
        self.downsamples = nn.ModuleList(
            MedNeXtV2DownBlock(
                in_channels=widths[s],
                out_channels=widths[s + 1],
                expansion_ratio=config.downsample_expansion_ratios[s],
                checkpoint_expansion=ckpt_expansion(s + 1),
            )
            for s in range(4)
        )
        self.bottleneck = blocks(4, 4)
        self.upsamples = nn.ModuleList(
            MedNeXtV2UpBlock(
                in_channels=widths[stage + 1],
                out_channels=widths[stage],
                expansion_ratio=config.upsample_expansion_ratios[i],
                checkpoint_expansion=ckpt_expansion(stage),
            )
            for i, stage in enumerate((3, 2, 1, 0))
        )
        self.decoder_stages = nn.ModuleList(blocks(stage, 5 + i) for i, stage in enumerate((3, 2, 1, 0)))
        self.head = OutputHead(spatial_dims=3, in_channels=widths[0], out_channels=config.out_channels)
        self.deep_supervision_heads = nn.ModuleList()
        if config.deep_supervision:
            self.deep_supervision_heads.extend(
                OutputHead(spatial_dims=3, in_channels=widths[s], out_channels=config.out_channels)
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
        # ceil(s / 16) == 1 for every extent <= 16: one bottleneck voxel.
        if x.shape[0] == 1 and all(-(-int(s) // 16) == 1 for s in x.shape[2:]):
            raise ValueError(
                "GroupNorm requires more than one value per channel for batch size one; "
                "the spatial volume after four downsamplings must exceed one"
            )
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
            skip = skips[stage]
            x = reconcile_spatial(self._run(self.upsamples[i], x, stage), tuple(skip.shape[2:]))
            x = self._run_stage(self.decoder_stages[i], x + skip, stage)
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
        """Resolve every operator, GRN included, at its own input resolution
        without running the model (reference models/mednext_v2.py:181-282)."""
        if len(input_shape) != 5:
            raise ValueError("input_shape must have rank 5 for a 3D model")
        resolver = self.__dict__.get("_optimization_resolver")
        model_context = ModelOptimizationContext("mednext_v2", self.config.variant, checkpoint_name(self.checkpointing))
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
            if isinstance(module, (nn.Conv3d, nn.ConvTranspose3d, GlobalResponseNorm3d)):
                descriptor = (
                    OperatorDescriptor.normalization(
                        family="global_response_norm3d", channels=module.gamma.shape[1], role=role
                    )
                    if isinstance(module, GlobalResponseNorm3d)
                    else _conv_descriptor(module, role=role)
                )
                decisions.append(
                    PolicyDecision(
                        descriptor, context.phase, "reference", {}, "reference", "unwrapped", "guard",
                        disposition="unwrapped",
                    )
                )
                continue
            adaptive = (AdaptivePointwise3d, AdaptiveDepthwise3d, AdaptiveGroupNorm3d, AdaptiveGlobalResponseNorm3d)
            if not isinstance(module, adaptive):
                continue
            local = replace(context, spatial_shape=spatial_shape_for_role(role, context.spatial_shape))
            if isinstance(module, AdaptiveGlobalResponseNorm3d):
                if not module.training:
                    decisions.append(
                        PolicyDecision(
                            module.descriptor, "inference", "reference", {}, "reference", "context-guard", "guard",
                            guard_reason="GRN evaluation uses reference",
                        )
                    )
                else:
                    decisions.append(resolver.resolve(module.descriptor, local, "training"))
            elif isinstance(module, AdaptiveDepthwise3d):
                decisions.extend(
                    resolver.resolve(module.descriptor, local, p) for p in ("forward", "backward_input", "backward_weight")
                )
            else:
                decisions.append(resolver.resolve(module.descriptor, local, local.phase))
        warnings = tuple(dict.fromkeys(d.warning for d in decisions if d.warning is not None))
        layers = tuple(p.name for p in resolver.context_layers(context)) if resolver is not None else ()
        return OptimizationReport(layers or ("reference",), context, tuple(decisions), warnings)


def configure_optimization(model: MedNeXtV2, optimization: OptimizationSource) -> MedNeXtV2:
    """Install the adaptive operators and GRN (keeping every Parameter object)."""
    model.optimization_source = optimization
    if isinstance(optimization, str) and optimization == "reference":
        return model
    if isinstance(optimization, str) and optimization in ("torch", "conservative", "autotune"):
        raise ValueError(f"optimization={optimization!r} was removed; use 'auto' or 'reference'")
    external = None if isinstance(optimization, str) and optimization == "auto" else optimization
    resolver = PolicyRegistry(external=external).resolver()
    model_context = ModelOptimizationContext("mednext_v2", model.config.variant, checkpoint_name(model.checkpointing))
    install_adaptive_operators(model, resolver=resolver, model_context=model_context)
    install_adaptive_grn(model, resolver=resolver, model_context=model_context)
    install_fused_grn_expansions(model, resolver=resolver, model_context=model_context)
    install_weight_precast(model)
    model.__dict__["_optimization_resolver"] = resolver
    model.__dict__["_optimization_model_context"] = model_context
    return model


_configure_optimization = configure_optimization  # the reference's private name


def _build(
    variant: str,
    *,
    in_channels: int,
    out_channels: int,
    deep_supervision: bool = False,
    deep_supervision_output: DeepSupervisionOutput = "tuple",
    checkpointing: CheckpointConfig | None = None,
    optimization: OptimizationSource = "auto",
) -> MedNeXtV2:
    config = get_mednext_v2_config(
        variant, in_channels=in_channels, out_channels=out_channels, deep_supervision=deep_supervision
    )
    model = MedNeXtV2(config, checkpointing=checkpointing, deep_supervision_output=deep_supervision_output)
    return configure_optimization(model, optimization)


def mednext_v2_base(**kwargs) -> MedNeXtV2:
    """Published MedNeXt v2 Base (61,969,507 parameters at 1 -> 3 channels).
    Keywords: in_channels, out_channels (required); deep_supervision=False,
    deep_supervision_output="tuple", checkpointing=None, optimization="auto"."""
    return _build("base", **kwargs)


def mednext_v2_wide(**kwargs) -> MedNeXtV2:
    """Published MedNeXt v2 Wide (base width 64; keyword arguments as ``mednext_v2_base``)."""
    return _build("wide", **kwargs)
