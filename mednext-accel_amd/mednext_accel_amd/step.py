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
    #: Autocast's cast cache (reuses a weight's bf16 copy within a forward).
    #: A captured step disables it: cached casts would be graph-pool tensors
    #: held across the capture boundary.
    autocast_cache: bool = True
    last_loss: Tensor | None = field(default=None, init=False)

    def loss(self, outputs) -> Tensor:
        heads = (outputs,) if isinstance(outputs, Tensor) else tuple(outputs)
        total = sum(F.cross_entropy(h, self.targets[tuple(h.shape[2:])]) for h in heads)
        return total / len(heads)

    def __call__(self) -> Tensor:
        self.optimizer.zero_grad(set_to_none=True)
        device = self.sample.device.type
        enabled = self.autocast_dtype is not None
        with torch.autocast(device, dtype=self.autocast_dtype or torch.bfloat16, enabled=enabled,
                            cache_enabled=self.autocast_cache):
            loss = self.loss(self.model(self.sample))
        loss.backward()
        self.optimizer.step()
        # Detached: a kept loss must not hold the step's autograd graph (and
        # its gradient-accumulation nodes) alive into the next step.
        self.last_loss = loss.detach()
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
    capturable: bool = False,
    fused_optimizer: bool | None = None,
) -> TrainingStep:
    """Synthetic inputs (seeded on the CPU generator, then moved) and AdamW
    (``capturable=True``: its step counters live on the device, as a captured
    step needs). ``fused_optimizer`` (default: on for GPU parameters) selects
    PyTorch's single-pass AdamW kernel over its multi-tensor form: the same
    update, one read and write of parameters, gradients and moments instead
    of one per elementwise stage."""
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
    if fused_optimizer is None:
        fused_optimizer = device.type == "cuda"
    optimizer = torch.optim.AdamW(model.parameters(), lr=lr, capturable=capturable, fused=fused_optimizer or None)
    return TrainingStep(model, optimizer, sample, targets, autocast_dtype)


class GraphedTrainingStep:
    """A ``TrainingStep`` captured once as a HIP graph and replayed.

    Every replay runs the whole step's kernels (zero-free gradient writes,
    forward, loss, backward, AdamW) from one host call, so the step no longer
    waits on Python and per-launch host work. The inputs, the targets and
    every intermediate are fixed device buffers (the graph's private pool);
    the parameters and optimizer state are updated in place as in eager
    mode. Capture needs a capturable optimizer (``make_training_step(...,
    capturable=True)``) and a step without host synchronisation.
    """

    def __init__(self, step: TrainingStep, *, warmup: int = 3) -> None:
        device = step.sample.device
        if device.type != "cuda":
            raise ValueError("a captured training step needs a GPU")
        for group in step.optimizer.param_groups:
            if not group.get("capturable", False):
                raise ValueError("capture needs an optimizer built with capturable=True")
        step.autocast_cache = False
        self.step = step
        # Eager warm-up on a side stream (default priority): lazily created
        # state (optimizer moments, library handles, cached plans) exists
        # before capture and the capture stream starts from a quiet device.
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                step()
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
        step.optimizer.zero_grad(set_to_none=True)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.loss = step().detach()

    @property
    def last_loss(self) -> Tensor:
        """The loss buffer the graph writes (valid after a replay)."""
        return self.loss

    def __call__(self) -> Tensor:
        self.graph.replay()
        return self.loss
