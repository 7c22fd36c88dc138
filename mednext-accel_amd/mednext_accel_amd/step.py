"""One MedNeXt training step, as the reference's benchmarks define it
(benchmarks/implementations.py:133-168).

Inputs: ``x ~ N(0, 1)`` of shape (B, C_in, S, S, S) and integer labels uniform
in ``[0, classes)``; for deep supervision the labels are nearest-resized to
every head's resolution. Loss: mean over heads of the mean cross-entropy, in
bf16 autocast. Optimizer: AdamW(lr=1e-3). One step = zero_grad, forward,
loss, backward, optimizer step.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import Tensor, nn
from torch.nn import functional as F


@dataclass
class TrainingStep:
    model: nn.Module
    optimizer: torch.optim.Optimizer
    sample: Tensor
    targets: dict[tuple[int, ...], Tensor]
    autocast_dtype: torch.dtype | None = torch.bfloat16
    last_loss: Tensor | None = field(default=None, init=False)

    def loss(self, outputs) -> Tensor:
        heads = (outputs,) if isinstance(outputs, Tensor) else tuple(outputs)
        total = sum(F.cross_entropy(h, self.targets[tuple(h.shape[2:])]) for h in heads)
        return total / len(heads)

    def __call__(self) -> Tensor:
        self.optimizer.zero_grad(set_to_none=True)
        device = self.sample.device.type
        enabled = self.autocast_dtype is not None
        with torch.autocast(device, dtype=self.autocast_dtype or torch.bfloat16, enabled=enabled):
            loss = self.loss(self.model(self.sample))
        loss.backward()
        self.optimizer.step()
        self.last_loss = loss
        return loss


def make_training_step(
    model: nn.Module,
    *,
    batch: int = 1,
    in_channels: int = 1,
    classes: int = 3,
    size: int = 128,
    seed: int = 1234,
    lr: float = 1e-3,
    autocast_dtype: torch.dtype | None = torch.bfloat16,
    device: torch.device | str | None = None,
) -> TrainingStep:
    """Synthetic inputs (seeded on the CPU generator, then moved) and AdamW."""
    device = torch.device(device) if device is not None else next(model.parameters()).device
    gen = torch.Generator().manual_seed(seed)
    sample = torch.randn(batch, in_channels, size, size, size, generator=gen).to(device)
    labels = torch.randint(classes, (batch, size, size, size), generator=gen).to(device)
    targets = {}
    s = size
    while s >= 1:
        shape = (s, s, s)
        if s == size:
            targets[shape] = labels
        else:
            targets[shape] = F.interpolate(labels[:, None].float(), size=shape, mode="nearest")[:, 0].long()
        if s % 2:
            break
        s //= 2
    optimizer = torch.optim.AdamW(model.parameters(), lr=lr)
    return TrainingStep(model, optimizer, sample, targets, autocast_dtype)
