"""Device arrays: the storage behind ``Tensor.data`` on the GPU.

A ``DeviceArray`` wraps a torch CUDA tensor that is used strictly as a device
memory handle: torch allocates (through its caching allocator), copies between
host and device, and builds metadata-only views (view / expand / transpose /
slicing).  Every arithmetic operation on the contents runs in libmtx_hip.so,
via ``minitorch_amd.kernels``.

``DeviceArray`` exposes the small NumPy-like surface the reference's code reads
from ``Tensor.data`` (``shape``, ``ndim``, ``size``, ``dtype``, ``copy()``,
indexing to host values, ``np.asarray``); reading values synchronises with the
device.
"""
from __future__ import annotations

import numpy as np
import torch

_DEV = None


def device() -> torch.device:
    global _DEV
    if _DEV is None:
        if not torch.cuda.is_available():
            raise RuntimeError("minitorch_amd needs a GPU (MI355X); none is visible and there is "
                               "no CPU fallback")
        _DEV = torch.device("cuda", torch.cuda.current_device())
    return _DEV


_NP = {torch.float32: np.dtype(np.float32), torch.int64: np.dtype(np.int64),
       torch.bfloat16: np.dtype("V2"), torch.uint8: np.dtype(np.uint8)}


class DeviceArray:
    """An n-d array in GPU memory (float32 unless stated)."""

    __slots__ = ("t",)

    def __init__(self, t: torch.Tensor):
        self.t = t

    # -- numpy-like metadata ------------------------------------------------
    @property
    def shape(self):
        return tuple(self.t.shape)

    @property
    def ndim(self):
        return self.t.dim()

    @property
    def size(self):
        return self.t.numel()

    @property
    def dtype(self):
        return _NP.get(self.t.dtype, self.t.dtype)

    @property
    def strides(self):
        """Element strides (NumPy reports bytes; kernels take elements)."""
        return tuple(self.t.stride())

    def is_contiguous(self):
        return self.t.is_contiguous()

    # -- host access ----------------------------------------------------------
    def numpy(self) -> np.ndarray:
        return self.t.detach().cpu().numpy()

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a.astype(dtype) if dtype is not None else a

    def __getitem__(self, key):
        return self.numpy()[key]

    def __float__(self):
        return float(self.numpy())

    def __len__(self):
        return self.shape[0]

    def __repr__(self):
        return f"DeviceArray({self.numpy()!r})"

    def copy(self) -> "DeviceArray":
        from . import kernels as K

        out = empty(self.shape)
        K.ewise("COPY", out.t, self.t)
        return out

    # -- metadata-only views -------------------------------------------------
    def view_as_shape(self, shape):
        return DeviceArray(self.t.view(*shape))

    def reshape(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        try:
            return DeviceArray(self.t.view(*shape))
        except RuntimeError:
            return self.contiguous().reshape(*shape)

    def contiguous(self) -> "DeviceArray":
        if self.t.is_contiguous():
            return self
        return self.copy()

    def transpose(self, axes):
        return DeviceArray(self.t.permute(*axes))

    def swapaxes(self, a, b):
        return DeviceArray(self.t.transpose(a, b))

    def broadcast_to(self, shape):
        return DeviceArray(self.t.expand(*shape))


def empty(shape, dtype=torch.float32) -> DeviceArray:
    return DeviceArray(torch.empty(tuple(shape), dtype=dtype, device=device()))


def full(shape, value: float) -> DeviceArray:
    from . import kernels as K

    out = empty(shape)
    K.fill(out.t, float(value))
    return out


def zeros(shape) -> DeviceArray:
    return full(shape, 0.0)


def from_host(a, dtype=np.float32) -> DeviceArray:
    """Copy a host array (or scalar / nested list) to the device."""
    arr = np.ascontiguousarray(np.asarray(a, dtype=dtype))
    return DeviceArray(torch.from_numpy(arr).to(device()))


def index_array(idx) -> DeviceArray:
    """Token ids (any integer array) as a contiguous int64 device array."""
    if isinstance(idx, DeviceArray):
        return idx if idx.t.dtype == torch.int64 else DeviceArray(idx.t.long())
    return from_host(np.asarray(idx), dtype=np.int64)


_CONST = {}


def const(value: float) -> DeviceArray:
    """A cached 0-d device constant (Python scalars in Tensor arithmetic)."""
    key = float(value)
    d = _CONST.get(key)
    if d is None:
        d = from_host(np.float32(key))
        _CONST[key] = d
    return d
