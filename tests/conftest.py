"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (they call the HIP library through its C
ABI); everything else runs on the CPU.  GPU tests are skipped, not faked, when
no device is visible.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP library calls)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _has_gpu():
    """A GPU is visible to the HIP runtime (asked through the library's own
    mtx_device_count; False when the library is not built)."""
    try:
        import ctypes

        from minitorch_amd import _lib

        n = ctypes.c_int(0)
        return _lib.lib().mtx_device_count(ctypes.byref(n)) == 0 and n.value > 0
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    """GPU 0, initialised through the library (loud failure if it is not
    built or no GPU is visible)."""
    from minitorch_amd import device

    return device.device()
