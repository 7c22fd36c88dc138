"""Shared pytest setup: import paths, the ``gpu`` marker and comparison helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "mednext-accel_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


# A HIP selection whose library cannot be loaded must fail the test, never run
# PyTorch's operators in its place (the adaptive wrappers' fallback).
os.environ.setdefault("MEDNEXT_ACCEL_AMD_REQUIRE_HIP", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
