"""Depthwise Conv3d oracle (float64 numpy), stride 1, odd cubic k, zero padding k//2.

Follows the reference's formulas:
  forward  y[n,c,i] = b[c] + sum_t w[c,t] x[n,c,i+t-p]
           reference src/mednext_accel/ops/_triton/depthwise.py:563 (F.conv3d with
           padding=k//2, groups=C) and ops/adaptive.py:247-255.
  dX       dx[n,c,i] = sum_t dy[n,c,i-t+p] w[c,t]   (masked)
           reference ops/_triton/depthwise.py:191-202 (_depthwise_input_grad_kernel).
  dW       dW[c,t] = sum_{n,i} x[n,c,i+t-p] dy[n,c,i]  (masked)
           reference ops/_triton/depthwise.py:56-74 (_partial_dw_kernel) and the
           fixed-order finish :77-83.
  dB       db[c] = sum_{n,i} dy[n,c,i]
           reference ops/_triton/depthwise.py:612-633 (native mask bit 2).
"""

from __future__ import annotations

import numpy as np


def _shifted(a: np.ndarray, sd: int, sh: int, sw: int) -> np.ndarray:
    """out[..., d, h, w] = a[..., d+sd, h+sh, w+sw] with zeros outside."""
    out = np.zeros_like(a)
    d, h, w = a.shape[-3:]

    def rng(n: int, s: int) -> tuple[slice, slice]:
        lo, hi = max(0, -s), min(n, n - s)
        if lo >= hi:
            return slice(0, 0), slice(0, 0)
        return slice(lo, hi), slice(lo + s, hi + s)

    (od, idd), (oh, ih), (ow, iw) = rng(d, sd), rng(h, sh), rng(w, sw)
    out[..., od, oh, ow] = a[..., idd, ih, iw]
    return out


def _taps(k: int):
    p = k // 2
    for kd in range(k):
        for kh in range(k):
            for kw in range(k):
                yield kd, kh, kw, kd - p, kh - p, kw - p


def forward(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    k = w.shape[-1]
    y = np.zeros_like(x)
    for kd, kh, kw, sd, sh, sw in _taps(k):
        y += w[None, :, 0, kd, kh, kw, None, None, None] * _shifted(x, sd, sh, sw)
    if b is not None:
        y += np.asarray(b, dtype=np.float64)[None, :, None, None, None]
    return y


def input_grad(dy: np.ndarray, w: np.ndarray) -> np.ndarray:
    dy = np.asarray(dy, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    k = w.shape[-1]
    dx = np.zeros_like(dy)
    for kd, kh, kw, sd, sh, sw in _taps(k):
        # dy[i - t + p] = dy shifted by -(t - p)
        dx += w[None, :, 0, kd, kh, kw, None, None, None] * _shifted(dy, -sd, -sh, -sw)
    return dx


def weight_grad(x: np.ndarray, dy: np.ndarray, k: int) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    c = x.shape[1]
    dw = np.zeros((c, 1, k, k, k), dtype=np.float64)
    for kd, kh, kw, sd, sh, sw in _taps(k):
        dw[:, 0, kd, kh, kw] = np.einsum("ncdhw,ncdhw->c", _shifted(x, sd, sh, sw), dy)
    return dw


def bias_grad(dy: np.ndarray) -> np.ndarray:
    return np.asarray(dy, dtype=np.float64).sum(axis=(0, 2, 3, 4))


def forward_loops(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """Brute-force scalar loops (tiny shapes only) — an independent formulation."""
    n_, c_, d_, h_, w_ = x.shape
    k = w.shape[-1]
    p = k // 2
    y = np.zeros((n_, c_, d_, h_, w_), dtype=np.float64)
    for n in range(n_):
        for c in range(c_):
            for d in range(d_):
                for h in range(h_):
                    for ww in range(w_):
                        s = 0.0 if b is None else float(b[c])
                        for kd in range(k):
                            for kh in range(k):
                                for kw in range(k):
                                    i, j, l = d + kd - p, h + kh - p, ww + kw - p
                                    if 0 <= i < d_ and 0 <= j < h_ and 0 <= l < w_:
                                        s += float(w[c, 0, kd, kh, kw]) * float(x[n, c, i, j, l])
                        y[n, c, d, h, ww] = s
    return y
