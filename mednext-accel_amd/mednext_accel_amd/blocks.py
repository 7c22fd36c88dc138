"""MedNeXt v1 building blocks (reference models/blocks.py:32-194).

Module attribute names (``depthwise``, ``norm``, ``expand``, ``activation``,
``project``, ``residual``, ``conv``) are the reference's, so state dicts and
the official checkpoint layout carry over unchanged. A block computes

    y = project(GELU(expand(GroupNorm_C(depthwise(x))))) [+ x]

with a stride-2 depthwise conv and a stride-2 1x1 residual conv in the down
block, and transposed convs padded by one leading voxel per dimension in the
up block.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.nn import functional as F
from torch.utils.checkpoint import checkpoint


def conv_type(spatial_dims: int) -> type[nn.Module]:
    if spatial_dims not in (2, 3):
        raise ValueError("spatial_dims must be 2 or 3")
    return nn.Conv2d if spatial_dims == 2 else nn.Conv3d


def conv_transpose_type(spatial_dims: int) -> type[nn.Module]:
    if spatial_dims not in (2, 3):
        raise ValueError("spatial_dims must be 2 or 3")
    return nn.ConvTranspose2d if spatial_dims == 2 else nn.ConvTranspose3d


class EvalModeGELU(nn.Module):
    """Exact (erf) GELU; tanh approximation only in eval mode when opted in."""

    def __init__(self, approximate_eval: bool = False) -> None:
        super().__init__()
        self.approximate_eval = approximate_eval

    def forward(self, x: Tensor) -> Tensor:
        use_tanh = self.approximate_eval and not self.training
        return F.gelu(x, approximate="tanh" if use_tanh else "none")

    def extra_repr(self) -> str:
        return f"approximate_eval={self.approximate_eval}"


class MedNeXtBlock(nn.Module):
    def __init__(
        self,
        *,
        spatial_dims: int,
        in_channels: int,
        out_channels: int,
        expansion_ratio: int,
        kernel_size: int,
        residual: bool = True,
        checkpoint_expansion: bool = False,
        approximate_gelu_eval: bool = False,
    ) -> None:
        super().__init__()
        conv = conv_type(spatial_dims)
        hidden = in_channels * expansion_ratio
        self.use_residual = residual
        self.checkpoint_expansion = checkpoint_expansion
        self.depthwise = conv(in_channels, in_channels, kernel_size, stride=1, padding=kernel_size // 2, groups=in_channels)
        self.norm = nn.GroupNorm(in_channels, in_channels)
        self.expand = conv(in_channels, hidden, kernel_size=1)
        self.activation = EvalModeGELU(approximate_eval=approximate_gelu_eval)
        self.project = conv(hidden, out_channels, kernel_size=1)

    def _expansion_forward(self, x: Tensor) -> Tensor:
        return self.project(self.activation(self.expand(x)))

    def forward(self, x: Tensor) -> Tensor:
        # A fused expansion (attached by install_adaptive_operators; a plain
        # attribute, not a submodule) replaces expand -> GELU -> project and the
        # residual add with two matrix-core kernels when it applies.
        fused = self.__dict__.get("fused_expansion")
        if fused is not None and fused.applies(x):
            d, res = self._depthwise_and_residual(x)
            if fused.supports(d):
                residual = res if self.use_residual else None
                recompute = self.checkpoint_expansion and self.training and torch.is_grad_enabled()
                # The GroupNorm folds into the expand GEMM when its HIP kernels
                # are selected and the branch is not recomputed (a recompute
                # would repeat the statistics pass); otherwise it runs here and
                # the expansion takes its bf16 output.
                if not recompute and fused.folds_norm(d):
                    return fused.folded(d, residual)
                h = self.norm(d, out_dtype=torch.bfloat16)
                if recompute:
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
        # The recomputed branches draw no random numbers (MedNeXt has no
        # dropout), so checkpoints stash no RNG state: cheaper, and valid
        # inside a captured step.
        if self.checkpoint_expansion and self.training and torch.is_grad_enabled():
            h = checkpoint(self._expansion_forward, h, use_reentrant=False, preserve_rng_state=False)
        else:
            h = self._expansion_forward(h)
        return h + x if self.use_residual else h


class MedNeXtDownBlock(MedNeXtBlock):
    def __init__(
        self,
        *,
        spatial_dims: int,
        in_channels: int,
        out_channels: int,
        expansion_ratio: int,
        kernel_size: int,
        residual: bool = True,
        checkpoint_expansion: bool = False,
        approximate_gelu_eval: bool = False,
    ) -> None:
        super().__init__(
            spatial_dims=spatial_dims,
            in_channels=in_channels,
            out_channels=out_channels,
            expansion_ratio=expansion_ratio,
            kernel_size=kernel_size,
            residual=False,
            checkpoint_expansion=checkpoint_expansion,
            approximate_gelu_eval=approximate_gelu_eval,
        )
        conv = conv_type(spatial_dims)
        self.depthwise = conv(in_channels, in_channels, kernel_size, stride=2, padding=kernel_size // 2, groups=in_channels)
        self.residual = conv(in_channels, out_channels, kernel_size=1, stride=2) if residual else None

    def forward(self, x: Tensor) -> Tensor:
        out = super().forward(x)
        return out if self.residual is None else out + self.residual(x)


class MedNeXtUpBlock(MedNeXtBlock):
    def __init__(
        self,
        *,
        spatial_dims: int,
        in_channels: int,
        out_channels: int,
        expansion_ratio: int,
        kernel_size: int,
        residual: bool = True,
        checkpoint_expansion: bool = False,
        approximate_gelu_eval: bool = False,
    ) -> None:
        super().__init__(
            spatial_dims=spatial_dims,
            in_channels=in_channels,
            out_channels=out_channels,
            expansion_ratio=expansion_ratio,
            kernel_size=kernel_size,
            residual=False,
            checkpoint_expansion=checkpoint_expansion,
            approximate_gelu_eval=approximate_gelu_eval,
        )
        deconv = conv_transpose_type(spatial_dims)
        self.depthwise = deconv(in_channels, in_channels, kernel_size, stride=2, padding=kernel_size // 2, groups=in_channels)
        self.residual = deconv(in_channels, out_channels, kernel_size=1, stride=2) if residual else None
        self._pad = (1, 0) * spatial_dims  # one leading voxel per dim: 2s-1 -> 2s

    def forward(self, x: Tensor) -> Tensor:
        main = super().forward(x)
        if self.residual is not None:
            joined = join_up_residual(self.residual, x, main, lead=1)
            if joined is not None:
                return joined
        out = F.pad(main, self._pad)
        return out if self.residual is None else out + F.pad(self.residual(x), self._pad)


def join_up_residual(residual: nn.Module, x: Tensor, main: Tensor, *, lead: int) -> Tensor | None:
    """``pad(main) + pad(residual(x))`` of an up block in one HIP pass
    (``hip_ops.up_block_join``) when the residual's stride-2 transposed 1x1x1
    conv takes the matrix-core route and the shapes fit (bf16, main
    contiguous at 2s - 1 per dimension, the padded width a multiple of 8);
    None otherwise, and the caller pads and adds as usual. ``lead`` 1 pads at
    the start (v1), 0 at the end (v2)."""
    parts_of = getattr(residual, "join_parts", None)
    if (
        parts_of is None
        or not main.is_cuda
        or main.dtype != torch.bfloat16
        or main.ndim != 5
        or not main.is_contiguous()
        or tuple(main.shape[2:]) != tuple(2 * s - 1 for s in x.shape[2:])
        or (main.shape[-1] + 1) % 8 != 0
    ):
        return None
    parts = parts_of(x)
    if parts is None:
        return None
    from . import hip_ops

    small, bias = parts
    return hip_ops.up_block_join(main, small, bias, lead, True)


class OutputHead(nn.Module):
    """1x1 transposed conv (the official checkpoints store heads this way)."""

    def __init__(self, *, spatial_dims: int, in_channels: int, out_channels: int) -> None:
        super().__init__()
        self.conv = conv_transpose_type(spatial_dims)(in_channels, out_channels, kernel_size=1)

    def forward(self, x: Tensor) -> Tensor:
        return self.conv(x)
