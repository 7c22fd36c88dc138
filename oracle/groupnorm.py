"""GroupNorm(C, C) oracle (float64 numpy).

The reference uses ``nn.GroupNorm(in_channels, in_channels)`` with PyTorch's
default eps=1e-5 and affine weight/bias (reference src/mednext_accel/models/
blocks.py:74, applied at :84). With groups == channels it normalises each
(n, c) over the spatial volume with the biased variance:
  y = (x - mean) / sqrt(var + eps) * gamma + beta
Backward (closed form, g = dy * gamma, x̂ = (x - mean) * rstd, V = volume):
  dx     = rstd * (g - mean_V(g) - x̂ * mean_V(g * x̂))
  dgamma = sum_{n, V} dy * x̂,   dbeta = sum_{n, V} dy
"""

from __future__ import annotations

import numpy as np

EPS = 1e-5


def forward(x, gamma=None, beta=None, eps: float = EPS):
    x = np.asarray(x, dtype=np.float64)
    n, c = x.shape[:2]
    flat = x.reshape(n, c, -1)
    mean = flat.mean(axis=2)
    var = ((flat - mean[..., None]) ** 2).mean(axis=2)
    rstd = 1.0 / np.sqrt(var + eps)
    xhat = (flat - mean[..., None]) * rstd[..., None]
    g = np.ones(c) if gamma is None else np.asarray(gamma, dtype=np.float64)
    b = np.zeros(c) if beta is None else np.asarray(beta, dtype=np.float64)
    y = xhat * g[None, :, None] + b[None, :, None]
    return y.reshape(x.shape), mean, rstd


def backward(dy, x, gamma=None, eps: float = EPS):
    dy = np.asarray(dy, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    n, c = x.shape[:2]
    _, mean, rstd = forward(x, None, None, eps)
    flat = x.reshape(n, c, -1)
    g_flat = dy.reshape(n, c, -1)
    xhat = (flat - mean[..., None]) * rstd[..., None]
    gam = np.ones(c) if gamma is None else np.asarray(gamma, dtype=np.float64)
    g = g_flat * gam[None, :, None]
    dx = rstd[..., None] * (g - g.mean(axis=2, keepdims=True) - xhat * (g * xhat).mean(axis=2, keepdims=True))
    dgamma = (g_flat * xhat).sum(axis=(0, 2))
    dbeta = g_flat.sum(axis=(0, 2))
    return dx.reshape(x.shape), dgamma, dbeta
