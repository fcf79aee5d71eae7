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


def _keep_host_memory_mapped():
    """The oracle's full-size checks allocate and free hundreds of MB of
    float64 arrays per step.  On hosts where a fresh page costs a slow fault
    (virtual machines with transparent huge pages) that dominates their run
    time, so freed memory stays in the process (glibc: no mmap for large
    blocks, no trimming) and NumPy stops asking for huge pages.  Run-time
    settings only; results are unchanged."""
    import ctypes

    import numpy as np

    try:
        np._core.multiarray._set_madvise_hugepage(False)
    except AttributeError:
        pass
    try:
        libc = ctypes.CDLL("libc.so.6")
        M_TRIM_THRESHOLD, M_TOP_PAD, M_MMAP_MAX = -1, -2, -4
        libc.mallopt(M_MMAP_MAX, 0)
        libc.mallopt(M_TRIM_THRESHOLD, 1 << 30)
        libc.mallopt(M_TOP_PAD, 256 << 20)
    except OSError:
        pass


_keep_host_memory_mapped()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP library calls)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def _has_gpu():
    """A GPU is visible to the HIP runtime (asked through the library's own
    mtx_device_count).  On a machine with a GPU driver (/dev/kfd) a library
    that does not load or a failing device query is an error, never a reason
    to skip: the GPU tests must run there."""
    import ctypes

    from minitorch_amd import _lib

    gpu_machine = os.path.exists("/dev/kfd")
    try:
        lib = _lib.lib()
    except Exception:
        if gpu_machine:
            raise
        return False
    n = ctypes.c_int(0)
    rc = lib.mtx_device_count(ctypes.byref(n))
    if rc != 0:
        if gpu_machine:
            raise RuntimeError(f"mtx_device_count failed: {lib.mtx_last_error().decode()}")
        return False
    if gpu_machine and n.value < 1:
        raise RuntimeError("/dev/kfd exists but the HIP runtime sees no GPU")
    return n.value > 0


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
