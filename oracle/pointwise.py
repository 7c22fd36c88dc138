"""Pointwise (1x1x1) convolution, exact GELU and residual oracle (float64 numpy).

  conv     Y[n] = W X[n] + b with X[n] = x[n].reshape(Cin, V)
           reference src/mednext_accel/ops/adaptive.py:174-188 (_gemm: per-sample
           torch.addmm(bias, W, X)) and :200 (F.conv3d 1x1x1).
  GELU     gelu(a) = a * Phi(a) = 0.5 a (1 + erf(a / sqrt 2)) in training
           reference src/mednext_accel/models/blocks.py:39-41 (approximate="none").
  block    project(gelu(expand(h))) + residual
           reference models/blocks.py:79-80, 89-90.
Backward: dX = W^T dY, dW = sum_n dY X^T, db = sum_{n,V} dY,
          gelu'(a) = Phi(a) + a phi(a).
"""

from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

SQRT1_2 = 1.0 / math.sqrt(2.0)
INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


def conv1x1(x, w, b=None):
    x = np.asarray(x, dtype=np.float64)
    w2 = np.asarray(w, dtype=np.float64).reshape(w.shape[0], -1)
    n, cin = x.shape[:2]
    y = np.einsum("oi,niv->nov", w2, x.reshape(n, cin, -1))
    if b is not None:
        y += np.asarray(b, dtype=np.float64)[None, :, None]
    return y.reshape((n, w2.shape[0]) + x.shape[2:])


def conv1x1_backward(dy, x, w):
    dy = np.asarray(dy, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    w2 = np.asarray(w, dtype=np.float64).reshape(w.shape[0], -1)
    n, cin = x.shape[:2]
    cout = w2.shape[0]
    dyf = dy.reshape(n, cout, -1)
    xf = x.reshape(n, cin, -1)
    dx = np.einsum("oi,nov->niv", w2, dyf).reshape(x.shape)
    dw = np.einsum("nov,niv->oi", dyf, xf).reshape(w.shape)
    db = dyf.sum(axis=(0, 2))
    return dx, dw, db


def gelu(a):
    a = np.asarray(a, dtype=np.float64)
    return 0.5 * a * (1.0 + erf(a * SQRT1_2))


def gelu_grad(a):
    a = np.asarray(a, dtype=np.float64)
    return 0.5 * (1.0 + erf(a * SQRT1_2)) + a * INV_SQRT_2PI * np.exp(-0.5 * a * a)
