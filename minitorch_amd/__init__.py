"""minitorch_amd -- MI355X-native causal-attention hot path for minitorch.

Kernels live in libmtx_hip.so (HIP, gfx950), reached through the C ABI in
include/mtx.h via ctypes (``minitorch_amd._lib``).
"""
__version__ = "0.1.0"
