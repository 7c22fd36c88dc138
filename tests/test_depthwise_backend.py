"""The reference-schema depthwise backend on the CPU: op schemas, fake-tensor
shapes and argument checks (no kernel launches).

The expected schemas are the reference's, read off the type annotations of its
ops in ``ops/_triton/depthwise.py`` (``torch.library`` turns ``int`` into
``SymInt`` and ``torch.Tensor | None`` into ``Tensor?``):
``:445-454`` (weight grad), ``:486-493`` (input grad), ``:516-519`` (stride-2
input grad), ``:549-563`` (regular conv), ``:654-664`` (stride-2 conv),
``:722-731`` (transpose weight grad), ``:768-778`` (transposed conv).
"""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import mednext_accel_amd.depthwise_backend as backend

EXPECTED_SCHEMAS = {
    "depthwise_weight_grad_odd_regular": (
        "(Tensor x, Tensor grad_output, SymInt kernel_size, SymInt channels, SymInt spatial_size, "
        "SymInt splits, SymInt block) -> Tensor"
    ),
    "depthwise_input_grad_odd_regular": (
        "(Tensor grad_output, Tensor weight, SymInt kernel_size, SymInt channels, SymInt spatial_size, "
        "SymInt block) -> Tensor"
    ),
    "depthwise_input_grad_stride2_regular": (
        "(Tensor grad_output, Tensor weight, SymInt channels, SymInt spatial_size, SymInt block) -> Tensor"
    ),
    "depthwise_conv3d_odd_regular": (
        "(Tensor x, Tensor weight, Tensor? bias, SymInt kernel_size, SymInt channels, SymInt spatial_size, "
        "SymInt dw_splits, SymInt dw_block, SymInt dx_block, bool custom_dx=True, bool custom_dw=True) -> Tensor"
    ),
    "depthwise_conv3d_stride2_regular": (
        "(Tensor x, Tensor weight, Tensor? bias, SymInt kernel_size, SymInt channels, SymInt spatial_size, "
        "SymInt dx_block) -> Tensor"
    ),
    "depthwise_transpose_weight_grad_odd_regular": (
        "(Tensor x, Tensor grad_output, SymInt kernel_size, SymInt channels, SymInt spatial_size, "
        "SymInt splits, SymInt block) -> Tensor"
    ),
    "depthwise_conv_transpose3d_odd_regular": (
        "(Tensor x, Tensor weight, Tensor? bias, SymInt kernel_size, SymInt channels, SymInt spatial_size, "
        "SymInt dw_splits, SymInt dw_block) -> Tensor"
    ),
}


@pytest.mark.parametrize("name", sorted(EXPECTED_SCHEMAS))
def test_op_schema_is_the_references(name):
    schema = str(getattr(torch.ops.mednext_accel, name).default._schema)
    assert schema == f"mednext_accel::{name}{EXPECTED_SCHEMAS[name]}"


def test_module_exposes_the_reference_backend_entry_points():
    """The names the reference's wrapper and tests call on its backend module
    (reference ops/adaptive.py:281-320, tests/ops/test_depthwise.py)."""
    for name in (
        "depthwise_conv3d_regular",
        "depthwise_conv3d_stride2_regular",
        "depthwise_conv_transpose3d_regular",
        "depthwise_input_grad",
        "depthwise_stride2_input_grad",
        "depthwise_weight_grad",
        "depthwise_transpose_weight_grad",
        "depthwise_input_grad_regular",
        "depthwise_weight_grad_regular",
        "depthwise_input_grad_stride2_regular",
        "depthwise_transpose_weight_grad_regular",
    ):
        assert callable(getattr(backend, name)), name


def test_fake_shapes_follow_the_reference():
    with FakeTensorMode():
        x = torch.empty(2, 8, 16, 16, 16, dtype=torch.bfloat16)
        w = torch.empty(8, 1, 3, 3, 3, dtype=torch.bfloat16)
        b = torch.empty(8, dtype=torch.bfloat16)
        ops = torch.ops.mednext_accel
        y = ops.depthwise_conv3d_odd_regular(x, w, b, 3, 8, 16, 8, 512, 128)
        assert y.shape == x.shape and y.dtype == x.dtype
        assert ops.depthwise_input_grad_odd_regular(x, w, 3, 8, 16, 128).shape == x.shape
        assert ops.depthwise_weight_grad_odd_regular(x, x, 3, 8, 16, 8, 512).shape == (8, 1, 3, 3, 3)
        small = ops.depthwise_conv3d_stride2_regular(x, w, b, 3, 8, 16, 128)
        assert small.shape == (2, 8, 8, 8, 8)
        assert ops.depthwise_input_grad_stride2_regular(small, w, 8, 16, 128).shape == x.shape
        big = ops.depthwise_conv_transpose3d_odd_regular(x, w, b, 3, 8, 16, 8, 256)
        assert big.shape == (2, 8, 31, 31, 31)
        assert ops.depthwise_transpose_weight_grad_odd_regular(x, big, 3, 8, 16, 8, 256).shape == (8, 1, 3, 3, 3)


def test_odd_spatial_size_fake_shapes():
    """Stride-two output (size + 1) // 2 at an odd size (reference :671-672)."""
    with FakeTensorMode():
        x = torch.empty(1, 4, 15, 15, 15)
        w = torch.empty(4, 1, 5, 5, 5)
        small = torch.ops.mednext_accel.depthwise_conv3d_stride2_regular(x, w, None, 5, 4, 15, 64)
        assert small.shape == (1, 4, 8, 8, 8)


def _cpu(*shape):
    return torch.zeros(*shape)


@pytest.mark.parametrize(
    "call,message",
    [
        (lambda: backend.depthwise_input_grad(_cpu(1, 2, 4, 4, 4), _cpu(2, 1, 3, 3, 3)), "CUDA"),
        (lambda: backend.depthwise_weight_grad(_cpu(1, 2, 4, 4, 4), _cpu(1, 2, 4, 4, 4)), "CUDA"),
        (lambda: backend.depthwise_input_grad_regular(_cpu(1, 2, 4, 4, 4), _cpu(2, 1, 3, 3, 3), 3, 2, 4, 100), "power of two"),
        (lambda: backend.depthwise_weight_grad_regular(_cpu(1, 2, 4, 4, 4), _cpu(1, 2, 4, 4, 4), 3, 2, 4, 0, 64), "splits"),
        (lambda: backend.depthwise_weight_grad_regular(_cpu(1, 2, 4, 4, 4), _cpu(1, 2, 4, 4, 4), 3, 3, 4, 8, 64), "channels=3"),
        (lambda: backend.depthwise_conv3d_regular(_cpu(1, 2, 4, 4, 4), _cpu(2, 1, 3, 3, 3), None, 3, 2, 5, 8, 64, 64), "spatial_size=5"),
        (lambda: backend.depthwise_conv3d_regular(_cpu(1, 2, 4, 4, 4), _cpu(2, 1, 5, 5, 5), None, 3, 2, 4, 8, 64, 64), r"\[C, 1, K, K, K\]"),
        (lambda: backend.depthwise_conv3d_regular(_cpu(1, 2, 4, 4, 4), _cpu(2, 1, 3, 3, 3), None, 3, 2, 4, 8, 64, 96), "power of two"),
        (lambda: backend.depthwise_stride2_input_grad(_cpu(1, 2, 2, 2, 2), _cpu(2, 1, 3, 3, 3), (5, 5, 5)), "CUDA"),
        (lambda: backend.depthwise_transpose_weight_grad(_cpu(1, 2, 4, 4, 4), _cpu(1, 2, 8, 8, 8)), "CUDA"),
    ],
)
def test_argument_errors_raise_value_error(call, message):
    with pytest.raises(ValueError, match=message):
        call()
