"""Pytest configuration: repo root on sys.path and the `gpu` marker.

Tests marked `gpu` run the HIP kernels through the C ABI and are skipped on a
machine without a GPU; everything else runs on the CPU.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible (gpu tests run on an MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
