"""Device arrays: the storage behind ``Tensor.data`` on the GPU.

Memory comes from libmtx_hip's own caching allocator (``mtx_malloc`` /
``mtx_free``); host <-> device copies, fills, streams and graphs are library
calls too, so the package needs no other GPU framework.  Two layers:

* ``DevBuf`` -- a strided view (pointer, element offset, shape, element
  strides, dtype) of a reference-counted allocation.  It offers the small
  tensor-like surface the kernel wrappers use (``data_ptr()``, ``stride()``,
  ``view``, ``transpose``, ``expand``, basic slicing, ``copy_``, ...); views
  share memory and never copy.
* ``DeviceArray`` -- what ``Tensor.data`` holds: the NumPy-like surface the
  reference's code reads from ``.data`` (``shape``, ``ndim``, ``size``,
  ``dtype``, ``copy()``, indexing to host values, ``np.asarray``).  Reading
  values synchronises with the device.

The reference keeps each Tensor's data in a NumPy array it owns
(tensor.py:50-61); a DeviceArray owns its device memory the same way and frees
it (back to the library's cache) when the last view goes away.
"""
from __future__ import annotations

import ctypes as C
from functools import reduce
from operator import mul

import numpy as np

from . import _lib as L

ITEMSIZE = {"float32": 4, "bfloat16": 2, "int64": 8, "int32": 4, "uint8": 1}
_HOST = {"float32": np.dtype(np.float32), "int64": np.dtype(np.int64), "int32": np.dtype(np.int32),
         "uint8": np.dtype(np.uint8), "bfloat16": np.dtype(np.uint16)}


def dtype_name(x) -> str:
    """Canonical dtype name ('float32', 'bfloat16', 'int64', 'int32', 'uint8')
    of a DevBuf / DeviceArray, a NumPy dtype or type, a name, or any array
    object whose ``dtype`` prints like one (e.g. a framework tensor a test
    passes in)."""
    d = x if isinstance(x, (str, type, np.dtype)) else getattr(x, "dtype", x)
    if isinstance(d, str):
        name = d
    else:
        try:
            name = np.dtype(d).name
        except TypeError:
            name = str(d).rsplit(".", 1)[-1]
    if name not in ITEMSIZE:
        raise ValueError(f"unsupported dtype {d!r}")
    return name


_READY = False


def device() -> int:
    """Initialise the library on GPU 0 (once) and return its index.  Raises
    when no GPU is visible: there is no CPU fallback."""
    global _READY
    if not _READY:
        n = C.c_int(0)
        L.call("mtx_device_count", C.byref(n))
        if n.value < 1:
            raise RuntimeError("minitorch_amd needs a GPU (MI355X); none is visible and there is "
                               "no CPU fallback")
        L.call("mtx_device_init", 0)
        _READY = True
    return 0


def synchronize() -> None:
    """Wait for all work issued on the device."""
    L.call("mtx_device_sync")


class _Storage:
    """One mtx_malloc allocation; freed to the library's cache with the last
    reference."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes: int):
        device()
        p = C.c_void_p()
        L.call("mtx_malloc", C.byref(p), max(1, int(nbytes)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    def __del__(self):
        try:
            if self.ptr:
                L.lib().mtx_free(C.c_void_p(self.ptr))
                self.ptr = 0
        except Exception:  # interpreter shutdown: the process frees everything
            pass


def _prod(shape):
    return reduce(mul, shape, 1)


def _contig_strides(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= max(int(s), 1)
    return tuple(reversed(st))


def _norm_shape(shape, numel=None):
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    shape = tuple(int(s) for s in shape)
    if shape.count(-1) > 1:
        raise ValueError("only one dimension can be inferred")
    if -1 in shape:
        if numel is None:
            raise ValueError("cannot infer a dimension here")
        rest = _prod([s for s in shape if s != -1])
        if rest == 0 or numel % rest:
            raise ValueError(f"cannot reshape {numel} elements into {shape}")
        shape = tuple(numel // rest if s == -1 else s for s in shape)
    return shape


def _view_strides(old_shape, old_strides, new_shape):
    """Strides that present the same elements in `new_shape` without a copy
    (C order), or None when the old layout does not allow it (NumPy's
    no-copy reshape rule)."""
    if _prod(old_shape) != _prod(new_shape):
        return None
    if _prod(new_shape) == 0:
        return _contig_strides(new_shape)
    od = [(s, st) for s, st in zip(old_shape, old_strides) if s != 1]
    oldd = [s for s, _ in od]
    olds = [st for _, st in od]
    newd = list(new_shape)
    news = [0] * len(newd)
    oi, oj, ni, nj = 0, 1, 0, 1
    while ni < len(newd) and oi < len(oldd):
        np_, op = newd[ni], oldd[oi]
        while np_ != op:
            if np_ < op:
                np_ *= newd[nj]
                nj += 1
            else:
                op *= oldd[oj]
                oj += 1
        for ok in range(oi, oj - 1):
            if olds[ok] != oldd[ok + 1] * olds[ok + 1]:
                return None
        news[nj - 1] = olds[oj - 1]
        for nk in range(nj - 1, ni, -1):
            news[nk - 1] = news[nk] * newd[nk]
        ni, nj, oi, oj = nj, nj + 1, oj, oj + 1
    last = news[ni - 1] if ni >= 1 else 1
    for nk in range(ni, len(newd)):
        news[nk] = last
    return tuple(news)


class DevBuf:
    """A strided view of library-allocated device memory (see module doc)."""

    __slots__ = ("_st", "_off", "shape", "_strides", "dtype")
    is_cuda = True

    def __init__(self, st: _Storage, off: int, shape, strides, dtype: str):
        self._st = st
        self._off = int(off)
        self.shape = tuple(int(s) for s in shape)
        self._strides = tuple(int(s) for s in strides)
        self.dtype = dtype

    # -- metadata -------------------------------------------------------------
    def data_ptr(self) -> int:
        return self._st.ptr + self._off * ITEMSIZE[self.dtype]

    def stride(self, d=None):
        return self._strides if d is None else self._strides[d]

    def size(self, d=None):
        return self.shape if d is None else self.shape[d]

    def dim(self) -> int:
        return len(self.shape)

    def numel(self) -> int:
        return _prod(self.shape)

    def element_size(self) -> int:
        return ITEMSIZE[self.dtype]

    def is_contiguous(self) -> bool:
        acc = 1
        for s, st in zip(reversed(self.shape), reversed(self._strides)):
            if s != 1 and st != acc:
                return False
            acc *= s
        return True

    def __len__(self):
        return self.shape[0]

    def __repr__(self):
        return f"DevBuf(shape={self.shape}, strides={self._strides}, dtype={self.dtype})"

    def _with(self, off, shape, strides):
        return DevBuf(self._st, off, shape, strides, self.dtype)

    # -- views (no copies) ------------------------------------------------------
    def view(self, *shape):
        shape = _norm_shape(shape, self.numel())
        st = _view_strides(self.shape, self._strides, shape)
        if st is None:
            raise RuntimeError(f"view of shape {shape} needs a copy (strides {self._strides}); use reshape")
        return self._with(self._off, shape, st)

    def reshape(self, *shape):
        shape = _norm_shape(shape, self.numel())
        st = _view_strides(self.shape, self._strides, shape)
        if st is None:
            return self.contiguous().view(*shape)
        return self._with(self._off, shape, st)

    def permute(self, *axes):
        if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            axes = tuple(axes[0])
        nd = self.dim()
        axes = tuple(a % nd for a in axes)
        if sorted(axes) != list(range(nd)):
            raise ValueError(f"bad permutation {axes}")
        return self._with(self._off, [self.shape[a] for a in axes], [self._strides[a] for a in axes])

    def transpose(self, a: int, b: int):
        nd = self.dim()
        a, b = a % nd, b % nd
        axes = list(range(nd))
        axes[a], axes[b] = axes[b], axes[a]
        return self.permute(*axes)

    def t(self):
        if self.dim() != 2:
            raise ValueError("t() needs a 2-d array")
        return self.transpose(0, 1)

    def unsqueeze(self, d: int):
        nd = self.dim() + 1
        d = d % nd
        shape = list(self.shape)
        strides = list(self._strides)
        inner = strides[d] * shape[d] if d < len(shape) else 1
        shape.insert(d, 1)
        strides.insert(d, inner)
        return self._with(self._off, shape, strides)

    def as_strided(self, shape, strides, offset=None):
        """The same memory seen with explicit shape / element strides (and
        element offset from the allocation's start)."""
        return self._with(self._off if offset is None else offset, shape, strides)

    def squeeze(self, d: int):
        d = d % self.dim()
        if self.shape[d] != 1:
            return self
        return self._with(self._off, self.shape[:d] + self.shape[d + 1:], self._strides[:d] + self._strides[d + 1:])

    def unflatten(self, d: int, sizes):
        """Split dimension d into `sizes` (a view)."""
        d = d % self.dim()
        sizes = tuple(int(x) for x in sizes)
        if _prod(sizes) != self.shape[d]:
            raise ValueError(f"cannot unflatten size {self.shape[d]} into {sizes}")
        st = self._strides[d]
        inner = list(_contig_strides(sizes))
        return self._with(self._off, self.shape[:d] + sizes + self.shape[d + 1:],
                          self._strides[:d] + tuple(st * x for x in inner) + self._strides[d + 1:])

    def expand(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = shape[0]
        shape = tuple(int(s) for s in shape)
        pad = len(shape) - self.dim()
        if pad < 0:
            raise ValueError(f"cannot expand {self.shape} to {shape}")
        new_shape, new_strides = [], []
        for d, s in enumerate(shape):
            if d < pad:
                if s < 0:
                    raise ValueError("-1 only for existing dims")
                new_shape.append(s)
                new_strides.append(0)
                continue
            cur, cst = self.shape[d - pad], self._strides[d - pad]
            if s == -1 or s == cur:
                new_shape.append(cur)
                new_strides.append(cst)
            elif cur == 1:
                new_shape.append(s)
                new_strides.append(0)
            else:
                raise ValueError(f"cannot expand {self.shape} to {shape}")
        return self._with(self._off, new_shape, new_strides)

    def __getitem__(self, key):
        if not isinstance(key, tuple):
            key = (key,)
        n_real = sum(1 for k in key if k is not None and k is not Ellipsis)
        if any(k is Ellipsis for k in key):
            i = next(j for j, k in enumerate(key) if k is Ellipsis)
            key = key[:i] + (slice(None),) * (self.dim() - n_real) + key[i + 1:]
        key = key + (slice(None),) * (self.dim() - sum(1 for k in key if k is not None))
        off = self._off
        shape, strides = [], []
        d = 0
        for k in key:
            if k is None:
                shape.append(1)
                strides.append(0)
                continue
            size, st = self.shape[d], self._strides[d]
            if isinstance(k, (int, np.integer)):
                i = int(k)
                if i < 0:
                    i += size
                if not 0 <= i < size:
                    raise IndexError(f"index {k} out of range for size {size}")
                off += i * st
            elif isinstance(k, slice):
                start, stop, step = k.indices(size)
                if step < 1:
                    raise ValueError("slices need a positive step")
                n = len(range(start, stop, step))
                off += start * st if n else 0
                shape.append(n)
                strides.append(st * step)
            else:
                raise TypeError(f"unsupported index {k!r} (ints and slices only)")
            d += 1
        return self._with(off, shape, strides)

    # -- data movement ------------------------------------------------------------
    def copy_(self, src):
        """Copy `src` (a DevBuf of the same dtype, broadcastable to this
        shape, or a host array) into this view."""
        from . import kernels as K

        if isinstance(src, np.ndarray):
            if not self.is_contiguous():
                raise ValueError("host copies need a contiguous destination")
            host = host_array(src, self.dtype)
            if host.size != self.numel():
                raise ValueError(f"host array of {host.size} elements into {self.numel()}")
            L.call("mtx_memcpy_h2d", C.c_void_p(self.data_ptr()), host.ctypes.data_as(C.c_void_p),
                   host.nbytes, L.stream_handle())
            return self
        if dtype_name(src) != self.dtype:
            raise ValueError(f"copy_ from {dtype_name(src)} into {self.dtype}")
        if self.dtype == "float32":
            K.ewise("COPY", self, src)
        elif self.is_contiguous() and src.is_contiguous() and tuple(src.shape) == self.shape:
            L.call("mtx_memcpy_d2d", C.c_void_p(self.data_ptr()), C.c_void_p(src.data_ptr()),
                   self.numel() * self.element_size(), L.stream_handle())
        else:
            raise ValueError(f"{self.dtype} copies need contiguous arrays of one shape")
        return self

    def clone(self) -> "DevBuf":
        out = empty_buf(self.shape, self.dtype)
        if self.numel():
            out.copy_(self)
        return out

    def contiguous(self) -> "DevBuf":
        return self if self.is_contiguous() else self.clone()

    def fill_(self, value):
        """Set every element to `value` (float32: any strides; others:
        contiguous)."""
        from . import kernels as K

        if self.dtype == "float32":
            K.fill(self, float(value))
            return self
        if not self.is_contiguous():
            raise ValueError("fill_ of non-float arrays needs a contiguous array")
        word = np.zeros(1, np.uint64)
        word.view(_HOST[self.dtype])[0] = value
        L.call("mtx_fill", C.c_void_p(self.data_ptr()), self.numel(), int(word[0]), self.element_size(),
               L.stream_handle())
        return self

    def numpy(self) -> np.ndarray:
        """A host copy (waits for the device).  bfloat16 comes back as
        float32 values."""
        src = self.contiguous()
        host = np.empty(self.shape, dtype=_HOST[self.dtype])
        if host.size:
            L.call("mtx_memcpy_d2h", host.ctypes.data_as(C.c_void_p), C.c_void_p(src.data_ptr()),
                   host.nbytes, L.stream_handle())
        if self.dtype == "bfloat16":
            return (host.astype(np.uint32) << 16).view(np.float32)
        return host


def host_array(a, dtype: str) -> np.ndarray:
    """A contiguous host array in the device layout of `dtype` (bfloat16:
    round-to-nearest-even to uint16 bit patterns; a NaN stays a NaN of the
    same sign -- the quiet NaN 0x7FC0 / 0xFFC0, as the rounding add would
    otherwise carry a payload into the exponent)."""
    if dtype == "bfloat16":
        x = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
        u = x.view(np.uint32).astype(np.uint64)
        r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)
        nan = np.isnan(x)
        if nan.any():
            r[nan] = (0x7FC0 | ((u[nan] >> 16) & 0x8000)).astype(np.uint16)
        return r
    return np.ascontiguousarray(np.asarray(a, dtype=_HOST[dtype]))


def empty_buf(shape, dtype="float32") -> DevBuf:
    dtype = dtype_name(dtype)
    shape = tuple(int(s) for s in shape)
    st = _Storage(_prod(shape) * ITEMSIZE[dtype])
    return DevBuf(st, 0, shape, _contig_strides(shape), dtype)


def empty_like_layout(t, dtype="float32") -> DevBuf:
    """An uninitialised buffer of t's shape whose memory order follows t's
    strides (dims laid out from the largest stride to the smallest), so a
    gradient of a transposed view has the view's physical layout and the
    inverse transpose + reshape stays a view."""
    nd = t.dim()
    order = sorted(range(nd), key=lambda d: (-t.stride(d), d))
    base = empty_buf([t.shape[d] for d in order], dtype)
    inv = [0] * nd
    for i, d in enumerate(order):
        inv[d] = i
    return base.permute(*inv)


class DeviceArray:
    """An n-d array in GPU memory (float32 unless stated); ``t`` is its
    DevBuf."""

    __slots__ = ("t",)

    def __init__(self, t: DevBuf):
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
        d = self.t.dtype
        return np.dtype(d) if d != "bfloat16" else d

    @property
    def strides(self):
        """Element strides (NumPy reports bytes; kernels take elements)."""
        return tuple(self.t.stride())

    def is_contiguous(self):
        return self.t.is_contiguous()

    # -- host access ----------------------------------------------------------
    def numpy(self) -> np.ndarray:
        return self.t.numpy()

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
        return DeviceArray(self.t.clone())

    # -- metadata-only views -------------------------------------------------
    def view_as_shape(self, shape):
        return DeviceArray(self.t.view(*shape))

    def reshape(self, *shape):
        return DeviceArray(self.t.reshape(*shape))

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


def empty(shape, dtype="float32") -> DeviceArray:
    return DeviceArray(empty_buf(shape, dtype))


def full(shape, value, dtype="float32") -> DeviceArray:
    out = empty(shape, dtype)
    out.t.fill_(value)
    return out


def zeros(shape, dtype="float32") -> DeviceArray:
    return full(shape, 0, dtype)


def from_host(a, dtype=np.float32) -> DeviceArray:
    """Copy a host array (or scalar / nested list) to the device
    (dtype 'bfloat16': rounded to nearest even)."""
    name = dtype_name(dtype)
    host = host_array(a, name)
    out = empty(host.shape, name)
    if host.size:
        L.call("mtx_memcpy_h2d", C.c_void_p(out.t.data_ptr()), host.ctypes.data_as(C.c_void_p),
               host.nbytes, L.stream_handle())
    return out


def index_array(idx) -> DeviceArray:
    """Token ids (any integer array) as a contiguous int64 device array."""
    if isinstance(idx, DeviceArray):
        if idx.t.dtype != "int64":
            raise ValueError("device token ids must be int64")
        return idx
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


def memory_stats():
    """(bytes in use, bytes cached) of the library's allocator."""
    a, b = C.c_size_t(0), C.c_size_t(0)
    L.call("mtx_memory_stats", C.byref(a), C.byref(b))
    return a.value, b.value


def empty_cache() -> None:
    L.call("mtx_empty_cache")


__all__ = ["DevBuf", "DeviceArray", "device", "synchronize", "empty", "empty_buf", "empty_like_layout", "full", "zeros",
           "from_host", "host_array", "index_array", "const", "dtype_name", "memory_stats", "empty_cache",
           "ITEMSIZE"]
