"""Global Response Normalization oracle (float64 numpy) — test infrastructure only.

The reference's GRN (src/mednext_accel/ops/grn.py:16-30) normalises each
sample's channel norms by their channel SUM:
  n_c = ||x_c||_2 over the spatial volume,  S = sum_c n_c,  r_c = n_c / (S + eps)
  y   = x + gamma_c * x * r_c + beta_c
Backward (the derivative its fused kernels implement, ops/_triton/grn.py:110-175,
with the cross-channel term through S and a zero subgradient where n_c = 0):
  g_c      = sum_V dy * x,         T = sum_c gamma_c * g_c * n_c
  dx       = dy * (1 + gamma_c r_c) + x * (gamma_c g_c / (S + eps) - T / (S + eps)^2) / n_c
  dgamma_c = sum_n g_c * r_c,      dbeta_c = sum_{n, V} dy
The backward is derived here, not taken from autograd; the tests pin it against
torch float64 autograd of the forward formula, finite differences and the
reference tests' closed-form coupling case.
"""

from __future__ import annotations

import numpy as np

EPS = 1e-6


def _params(c: int, gamma, beta):
    g = np.zeros(c) if gamma is None else np.asarray(gamma, dtype=np.float64).reshape(c)
    b = np.zeros(c) if beta is None else np.asarray(beta, dtype=np.float64).reshape(c)
    return g, b


def norms(x, eps: float = EPS):
    """(n_c [N, C], r_c [N, C])."""
    x = np.asarray(x, dtype=np.float64)
    flat = x.reshape(x.shape[0], x.shape[1], -1)
    n = np.sqrt((flat * flat).sum(axis=2))
    r = n / (n.sum(axis=1, keepdims=True) + eps)
    return n, r


def forward(x, gamma=None, beta=None, eps: float = EPS):
    x = np.asarray(x, dtype=np.float64)
    c = x.shape[1]
    g, b = _params(c, gamma, beta)
    _, r = norms(x, eps)
    shape = (x.shape[0], c) + (1,) * (x.ndim - 2)
    scale = (1.0 + g[None, :] * r).reshape(shape)
    return x * scale + b.reshape((1, c) + (1,) * (x.ndim - 2))


def backward(dy, x, gamma=None, eps: float = EPS):
    """(dx, dgamma [C], dbeta [C])."""
    dy = np.asarray(dy, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    nb, c = x.shape[:2]
    g, _ = _params(c, gamma, None)
    n, r = norms(x, eps)
    flat_x = x.reshape(nb, c, -1)
    flat_dy = dy.reshape(nb, c, -1)
    gc = (flat_dy * flat_x).sum(axis=2)  # [N, C]
    denom = n.sum(axis=1, keepdims=True) + eps  # [N, 1]
    t = (g[None, :] * gc * n).sum(axis=1, keepdims=True)  # [N, 1]
    with np.errstate(divide="ignore", invalid="ignore"):
        k2 = np.where(n > 0, (g[None, :] * gc / denom - t / denom**2) / n, 0.0)
    k1 = 1.0 + g[None, :] * r
    dx = flat_dy * k1[..., None] + flat_x * k2[..., None]
    dgamma = (gc * r).sum(axis=0)
    dbeta = flat_dy.sum(axis=(0, 2))
    return dx.reshape(x.shape), dgamma, dbeta
