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


# ----------------------------------------------------------------- stride 2
#
# MedNeXt's down block uses a stride-2, padding k//2 depthwise Conv3d and its up
# block the matching ConvTranspose3d (reference models/blocks.py:120-127 and
# :165-172; ops/_triton/depthwise.py:654-667 and :768-782 call F.conv3d /
# F.conv_transpose3d with stride=2, padding=k//2, groups=C).


def strided_output_shape(shape):
    """Spatial output of the stride-2, padding k//2 conv: (s - 1) // 2 + 1 per dim."""
    return tuple((s - 1) // 2 + 1 for s in shape)


def strided_forward(x, w, b=None):
    """y[o] = b + sum_t w[t] x[2o + t - p] (zero padding)."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    n, c = x.shape[:2]
    k = w.shape[-1]
    p = k // 2
    od, oh, ow = strided_output_shape(x.shape[2:])
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p), (p, p)))
    y = np.zeros((n, c, od, oh, ow))
    for kd, kh, kw, *_ in _taps(k):
        y += w[None, :, 0, kd, kh, kw, None, None, None] * xp[
            :, :, kd : kd + 2 * od : 2, kh : kh + 2 * oh : 2, kw : kw + 2 * ow : 2
        ]
    if b is not None:
        y += np.asarray(b, dtype=np.float64)[None, :, None, None, None]
    return y


def strided_input_grad(dy, w, input_spatial):
    """Adjoint of ``strided_forward`` (no bias): dx[i] = sum_{o,t: 2o+t-p=i} w[t] dy[o]."""
    dy = np.asarray(dy, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    n, c, od, oh, ow = dy.shape
    k = w.shape[-1]
    p = k // 2
    d, h, wd = input_spatial
    dxp = np.zeros((n, c, d + 2 * p + 1, h + 2 * p + 1, wd + 2 * p + 1))
    for kd, kh, kw, *_ in _taps(k):
        dxp[:, :, kd : kd + 2 * od : 2, kh : kh + 2 * oh : 2, kw : kw + 2 * ow : 2] += (
            w[None, :, 0, kd, kh, kw, None, None, None] * dy
        )
    return dxp[:, :, p : p + d, p : p + h, p : p + wd]


def strided_weight_grad(x, dy, k):
    """dW[c, t] = sum_{n,o} x[2o + t - p] dy[o]; returns (dW [C,1,k,k,k], dB [C])."""
    x = np.asarray(x, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    c = x.shape[1]
    p = k // 2
    od, oh, ow = dy.shape[2:]
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p), (p, p)))
    dw = np.zeros((c, 1, k, k, k))
    for kd, kh, kw, *_ in _taps(k):
        win = xp[:, :, kd : kd + 2 * od : 2, kh : kh + 2 * oh : 2, kw : kw + 2 * ow : 2]
        dw[:, 0, kd, kh, kw] = (win * dy).sum(axis=(0, 2, 3, 4))
    return dw, dy.sum(axis=(0, 2, 3, 4))


def transposed_forward(x, w, b=None):
    """ConvTranspose3d(stride 2, padding k//2, no output padding): output 2s - 1
    per dim, y = strided_input_grad(x) + b."""
    x = np.asarray(x, dtype=np.float64)
    out = tuple(2 * s - 1 for s in x.shape[2:])
    y = strided_input_grad(x, w, out)
    if b is not None:
        y = y + np.asarray(b, dtype=np.float64)[None, :, None, None, None]
    return y


def strided_forward_loops(x, w, b=None):
    """Brute-force restatement of ``strided_forward`` (tiny shapes only)."""
    x = np.asarray(x, dtype=np.float64)
    n, c, d, h, wd = x.shape
    k = w.shape[-1]
    p = k // 2
    od, oh, ow = strided_output_shape((d, h, wd))
    y = np.zeros((n, c, od, oh, ow))
    for ni in range(n):
        for ci in range(c):
            for a in range(od):
                for bb in range(oh):
                    for e in range(ow):
                        s = 0.0 if b is None else float(b[ci])
                        for kd, kh, kw, *_ in _taps(k):
                            i, j, l = 2 * a + kd - p, 2 * bb + kh - p, 2 * e + kw - p
                            if 0 <= i < d and 0 <= j < h and 0 <= l < wd:
                                s += w[ci, 0, kd, kh, kw] * x[ni, ci, i, j, l]
                        y[ni, ci, a, bb, e] = s
    return y
