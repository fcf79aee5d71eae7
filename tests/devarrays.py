"""Device arrays for the GPU tests, made with the package's own runtime
(libmtx_hip's allocator and copies; no other GPU framework)."""
import numpy as np

from minitorch_amd import device as dev


def T(x, dtype="float32"):
    """Host array -> device (a DevBuf; bfloat16 rounds to nearest even)."""
    return dev.from_host(np.asarray(x), dtype).t


def H(t):
    """Device array (DevBuf or DeviceArray) -> host NumPy (waits for the
    device; bfloat16 comes back as float32 values)."""
    return t.numpy()


def empty(shape, dtype="float32"):
    return dev.empty_buf(tuple(shape), dtype)


def full(shape, value, dtype="float32"):
    return dev.full(tuple(shape), value, dtype).t


def sync():
    dev.synchronize()
