"""MedNeXt v2 blocks (reference models/blocks_v2.py:13-137).

A v2 block inserts Global Response Normalization between the expansion's GELU
and its projection, and fixes the kernel at 3:

    y = project(GRN(GELU(expand(GroupNorm_C(depthwise(x)))))) [+ x]

The down block uses a stride-2 depthwise conv and a stride-2 1x1 residual
conv; the up block uses stride-2 transposed convs (output 2s - 1 per
dimension) and pads one voxel at the END of each spatial dimension to 2s
(v1 pads at the start). Attribute names (``depthwise``, ``norm``, ``expand``,
``activation``, ``grn``, ``project``, ``residual``) are the reference's, so the
state-dict keys are the same.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.nn import functional as F
from torch.utils.checkpoint import checkpoint

from .blocks import EvalModeGELU, join_up_residual
from .grn import GlobalResponseNorm3d


class MedNeXtV2Block(nn.Module):
    def __init__(
        self,
        *,
        in_channels: int,
        out_channels: int,
        expansion_ratio: int,
        residual: bool = True,
        checkpoint_expansion: bool = False,
    ) -> None:
        super().__init__()
        hidden = in_channels * expansion_ratio
        self.use_residual = residual
        self.checkpoint_expansion = checkpoint_expansion
        self.depthwise = nn.Conv3d(in_channels, in_channels, 3, stride=1, padding=1, groups=in_channels)
        self.norm = nn.GroupNorm(in_channels, in_channels)
        self.expand = nn.Conv3d(in_channels, hidden, kernel_size=1)
        self.activation = EvalModeGELU(approximate_eval=False)
        self.grn = GlobalResponseNorm3d(hidden)
        self.project = nn.Conv3d(hidden, out_channels, kernel_size=1)

    def _expansion_forward(self, h: Tensor) -> Tensor:
        return self.project(self.grn(self.activation(self.expand(h))))

    def forward(self, x: Tensor) -> Tensor:
        # A fused expansion (attached by the model's optimization setup; a plain
        # attribute, not a submodule) replaces expand -> GELU -> GRN -> project
        # and the residual add with matrix-core kernels when it applies.
        fused = self.__dict__.get("fused_expansion")
        if fused is not None and fused.applies(x):
            d, res = self._depthwise_and_residual(x)
            if fused.supports(d):
                h = self.norm(d, out_dtype=torch.bfloat16)
                residual = res if self.use_residual else None
                if self.checkpoint_expansion and self.training and torch.is_grad_enabled():
                    return checkpoint(fused, h, residual, use_reentrant=False, preserve_rng_state=False)
                return fused(h, residual)
            return self._finish(self.norm(d), res)
        d, res = self._depthwise_and_residual(x)
        return self._finish(self.norm(d), res)

    def _depthwise_and_residual(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """The depthwise output and the tensor the residual add uses (x; from
        an adaptive depthwise its tap, so the two gradients of x are summed in
        the depthwise input-gradient kernel)."""
        tap = getattr(self.depthwise, "forward_tap", None)
        if self.use_residual and tap is not None:
            return tap(x)
        return self.depthwise(x), x

    def _finish(self, h: Tensor, x: Tensor) -> Tensor:
        if self.checkpoint_expansion and self.training and torch.is_grad_enabled():
            h = checkpoint(self._expansion_forward, h, use_reentrant=False, preserve_rng_state=False)
        else:
            h = self._expansion_forward(h)
        return h + x if self.use_residual else h


class MedNeXtV2DownBlock(MedNeXtV2Block):
    def __init__(
        self,
        *,
        in_channels: int,
        out_channels: int,
        expansion_ratio: int,
        residual: bool = True,
        checkpoint_expansion: bool = False,
    ) -> None:
        super().__init__(
            in_channels=in_channels,
            out_channels=out_channels,
            expansion_ratio=expansion_ratio,
            residual=False,
            checkpoint_expansion=checkpoint_expansion,
        )
        self.depthwise = nn.Conv3d(in_channels, in_channels, 3, stride=2, padding=1, groups=in_channels)
        self.residual = nn.Conv3d(in_channels, out_channels, kernel_size=1, stride=2) if residual else None

    def forward(self, x: Tensor) -> Tensor:
        out = super().forward(x)
        return out if self.residual is None else out + self.residual(x)


class MedNeXtV2UpBlock(MedNeXtV2Block):
    def __init__(
        self,
        *,
        in_channels: int,
        out_channels: int,
        expansion_ratio: int,
        residual: bool = True,
        checkpoint_expansion: bool = False,
    ) -> None:
        super().__init__(
            in_channels=in_channels,
            out_channels=out_channels,
            expansion_ratio=expansion_ratio,
            residual=False,
            checkpoint_expansion=checkpoint_expansion,
        )
        self.depthwise = nn.ConvTranspose3d(in_channels, in_channels, 3, stride=2, padding=1, groups=in_channels)
        self.residual = (
            nn.ConvTranspose3d(in_channels, out_channels, kernel_size=1, stride=2) if residual else None
        )
        self._pad = (0, 1) * 3  # one trailing voxel per dim: 2s-1 -> 2s

    def forward(self, x: Tensor) -> Tensor:
        main = super().forward(x)
        if self.residual is not None:
            joined = join_up_residual(self.residual, x, main, lead=0)
            if joined is not None:
                return joined
        out = F.pad(main, self._pad)
        return out if self.residual is None else out + F.pad(self.residual(x), self._pad)


__all__ = ["MedNeXtV2Block", "MedNeXtV2DownBlock", "MedNeXtV2UpBlock"]
