"""Shared pytest configuration.

Marker ``gpu``: needs an AMD GPU (MI355X).  Without a visible GPU those tests
are skipped, as in the reference's conftest (tests/conftest.py:16-23); on a
GPU box they run against the in-tree HIP library and fail loudly if it is
missing.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an AMD GPU (gfx950)")


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
