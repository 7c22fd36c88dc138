"""Component numerical validation (reference profiling/validation.py:67-93).

A candidate implementation is accepted for a context only if every component
it produces (output, dX, dW, dB) is finite and within relative L2 error
``RELATIVE_L2_LIMIT`` of the native module's on the same inputs. The criterion
and its 2% bound are the reference's (bf16 operators reduce in different
orders; a normwise bound tolerates that near zero without letting one bad
component hide behind a larger one). Norms accumulate in fp64 over bounded
chunks so multi-GiB activations need no full-size scratch.
"""

from __future__ import annotations

import math
from collections.abc import Mapping

import torch
from torch import Tensor

RELATIVE_L2_LIMIT = 0.02
_CHUNK = 1 << 20


def _metrics(name: str, actual: Tensor, expected: Tensor) -> tuple[dict[str, object], str | None]:
    if actual.shape != expected.shape:
        return {"finite": False, "relative_l2": None, "max_absolute": None}, f"{name}: shape mismatch"
    a, e = actual.detach().reshape(-1), expected.detach().reshape(-1)
    err_sq = torch.zeros((), dtype=torch.float64, device=a.device)
    ref_sq = torch.zeros((), dtype=torch.float64, device=a.device)
    peak = torch.zeros((), dtype=torch.float32, device=a.device)
    finite = torch.ones((), dtype=torch.bool, device=a.device)
    for start in range(0, a.numel(), _CHUNK):
        got, want = a[start : start + _CHUNK].float(), e[start : start + _CHUNK].float()
        finite &= torch.isfinite(got).all() & torch.isfinite(want).all()
        diff = got - want
        err_sq += torch.linalg.vector_norm(diff, dtype=torch.float64).square()
        ref_sq += torch.linalg.vector_norm(want, dtype=torch.float64).square()
        peak = torch.maximum(peak, diff.abs().max() if diff.numel() else peak)
    if not bool(finite):
        return {"finite": False, "relative_l2": None, "max_absolute": None}, f"{name}: non-finite values"
    rel = float(err_sq.sqrt() / ref_sq.sqrt().clamp_min(1e-12))
    mx = float(peak)
    reason = None
    if not (math.isfinite(rel) and math.isfinite(mx)):
        reason = f"{name}: non-finite error metrics"
    elif rel >= RELATIVE_L2_LIMIT:
        reason = f"{name}: relative L2 error {rel:.3g} is not below {RELATIVE_L2_LIMIT}"
    return {"finite": True, "relative_l2": rel, "max_absolute": mx}, reason


def validate_components(actual: Mapping[str, Tensor], expected: Mapping[str, Tensor]) -> dict[str, object]:
    """Scalar verdict for matching component maps: ``valid``, per-component
    metrics and the first rejection reason (components in sorted order)."""
    if not actual or actual.keys() != expected.keys():
        raise ValueError("validation requires the same non-empty component names")
    metrics: dict[str, object] = {}
    reason = None
    with torch.no_grad():
        for name in sorted(expected):
            metrics[name], why = _metrics(name, actual[name], expected[name])
            reason = reason or why
    return {
        "valid": reason is None,
        "validator": "component-relative-l2",
        "validation_metrics": metrics,
        "rejection_reason": reason,
    }
