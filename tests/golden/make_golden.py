"""Write the small float64 golden fixtures in this folder.

The reference commits no numeric tensor fixtures: its parity tests compare
against PyTorch float64 at run time (reference tests/ops/test_depthwise.py:31-62,
tests/ops/test_adaptive.py:76-96). These fixtures freeze that same library
routine — torch float64 ``F.conv3d`` / ``F.group_norm`` / ``F.gelu`` and
autograd on CPU — at the reference test's shapes and seeds, so the oracle and
the HIP kernels are checked against identical stored vectors on every machine.

Run:  python tests/golden/make_golden.py   (writes golden_ops.npz)
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).with_name("golden_ops.npz")


def depthwise_case(k: int) -> dict[str, np.ndarray]:
    # Shape and seed of the reference's low-level gradient test (17 + k).
    torch.manual_seed(17 + k)
    x = torch.randn(2, 3, 5, 6, 7, dtype=torch.float64, requires_grad=True)
    w = torch.randn(3, 1, k, k, k, dtype=torch.float64, requires_grad=True)
    b = torch.randn(3, dtype=torch.float64, requires_grad=True)
    y = F.conv3d(x, w, b, padding=k // 2, groups=3)
    dy = torch.randn_like(y)
    dx, dw, db = torch.autograd.grad(y, (x, w, b), dy)
    p = f"dw_k{k}_"
    return {p + n: t.detach().numpy() for n, t in (("x", x), ("w", w), ("b", b), ("y", y), ("dy", dy), ("dx", dx), ("dw", dw), ("db", db))}


def group_norm_case() -> dict[str, np.ndarray]:
    torch.manual_seed(5)
    x = (torch.randn(2, 4, 3, 5, 6, dtype=torch.float64) * 3 + 7).requires_grad_()
    g = torch.randn(4, dtype=torch.float64, requires_grad=True)
    b = torch.randn(4, dtype=torch.float64, requires_grad=True)
    y = F.group_norm(x, 4, g, b, eps=1e-5)
    dy = torch.randn_like(y)
    dx, dg, dbb = torch.autograd.grad(y, (x, g, b), dy)
    return {"gn_" + n: t.detach().numpy() for n, t in (("x", x), ("g", g), ("b", b), ("y", y), ("dy", dy), ("dx", dx), ("dg", dg), ("db", dbb))}


def pointwise_case() -> dict[str, np.ndarray]:
    torch.manual_seed(37)  # seed of the reference's _gemm test
    x = torch.randn(3, 4, 3, 4, 5, dtype=torch.float64, requires_grad=True)
    w1 = torch.randn(8, 4, 1, 1, 1, dtype=torch.float64, requires_grad=True)
    b1 = torch.randn(8, dtype=torch.float64, requires_grad=True)
    w2 = torch.randn(4, 8, 1, 1, 1, dtype=torch.float64, requires_grad=True)
    b2 = torch.randn(4, dtype=torch.float64, requires_grad=True)
    a = F.conv3d(x, w1, b1)
    h = F.gelu(a, approximate="none")
    y = F.conv3d(h, w2, b2) + x
    dy = torch.randn_like(y)
    grads = torch.autograd.grad(y, (x, w1, b1, w2, b2), dy)
    names = ("x", "w1", "b1", "w2", "b2", "a", "h", "y", "dy", "dx", "dw1", "db1", "dw2", "db2")
    tensors = (x, w1, b1, w2, b2, a, h, y, dy, *grads)
    return {"pw_" + n: t.detach().numpy() for n, t in zip(names, tensors)}


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    for k in (1, 3, 5):
        arrays.update(depthwise_case(k))
    arrays.update(group_norm_case())
    arrays.update(pointwise_case())
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(arrays)} arrays)")


if __name__ == "__main__":
    main()
