"""Comparison metrics used by the parity tests.

``max_rel`` is the normwise max relative error max|a - b| / max|b| — the
"max relative error" bound of the target (fp32: 1e-5 outputs / input grads,
1e-4 weight grads; bf16 autocast: 2e-2). ``rel_l2`` is the reference
profiler's relative L2 metric (reference profiling/validation.py:30-93).
"""

from __future__ import annotations

import numpy as np
import torch

FP32_OUT = 1e-5
FP32_WGRAD = 1e-4
BF16 = 2e-2


def _np(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        return a.detach().to("cpu", torch.float64).numpy()
    return np.asarray(a, dtype=np.float64)


def max_rel(actual, expected) -> float:
    a, e = _np(actual), _np(expected)
    assert a.shape == e.shape, (a.shape, e.shape)
    scale = np.abs(e).max()
    if scale == 0:
        return float(np.abs(a).max())
    return float(np.abs(a - e).max() / scale)


def rel_l2(actual, expected) -> float:
    a, e = _np(actual), _np(expected)
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))
