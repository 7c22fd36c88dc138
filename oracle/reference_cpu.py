"""The reference's CPU execution of the depthwise path, used only as bench.py's
``cpu_baseline`` (timed, never shipped).

On a CPU tensor the reference's wrapper takes its ``_reference`` branch
(reference src/mednext_accel/ops/adaptive.py:257-268, :247-255): ``F.conv3d``
with padding k//2 and groups=C, and autograd's ``aten.convolution_backward``
for dX, dW and dB (the native mask the reference requests at
ops/_triton/depthwise.py:612-633). This module restates that call sequence.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def depthwise_phases(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, dy: torch.Tensor):
    """Run fwd, then dX / dW+dB, each as its own call, returning the outputs."""
    k = w.shape[-1]
    c = x.shape[1]
    y = F.conv3d(x, w, b, padding=k // 2, groups=c)
    dx, _, _ = torch.ops.aten.convolution_backward(
        dy, x, w, [c], [1, 1, 1], [k // 2] * 3, [1, 1, 1], False, [0, 0, 0], c, [True, False, False]
    )
    _, dw, db = torch.ops.aten.convolution_backward(
        dy, x, w, [c], [1, 1, 1], [k // 2] * 3, [1, 1, 1], False, [0, 0, 0], c, [False, True, True]
    )
    return y, dx, dw, db
