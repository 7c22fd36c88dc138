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


def check_against_truth(name, hip, reference, truth, tol):
    """``hip`` must be within ``tol`` (rel-L2) of the float64 ``truth`` or no
    worse than 2x the reference path's error (both paths round at different
    points under autocast, so their errors fluctuate independently). A gradient that is zero in
    exact arithmetic (the depthwise bias in front of GroupNorm(C, C), which
    removes any per-channel constant) carries only rounding noise in both
    paths: there the HIP noise must stay within 4x the reference's."""
    e_hip, e_ref = rel_l2(hip, truth), rel_l2(reference, truth)
    print(f"  {name:34s} hip {e_hip:.2e}  reference {e_ref:.2e}", flush=True)
    if e_ref > 1.0:  # truth is ~0: the reference's own result is pure noise
        assert hip.double().norm() <= 4 * reference.double().norm() + 1e-30, name
    else:
        assert e_hip < tol or e_hip <= 2.0 * e_ref, name
