"""Shared test setup: the `gpu` marker and import paths."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); runs the native kernels")


def _hip_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


HIP = _hip_available()


def pytest_collection_modifyitems(config, items):
    if HIP:
        return
    skip = pytest.mark.skip(reason="no HIP GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
