"""Host-side logic of the package's device arrays and runtime entry points
that needs no GPU: DevBuf views (view / reshape / transpose / expand /
slicing / unflatten) against NumPy's own stride arithmetic on the same
shapes, dtype names, the bf16 host rounding, and the runtime's argument
checks (which return before any HIP call)."""
import ctypes as C
import itertools

import numpy as np
import pytest

from minitorch_amd import _lib as L
from minitorch_amd import device as dev


class _FakeStorage:
    """Stands in for an allocation: views only do pointer arithmetic."""

    def __init__(self, ptr=1 << 20):
        self.ptr = ptr


def _buf(a: np.ndarray) -> dev.DevBuf:
    """A DevBuf with the element strides of NumPy array `a` (no memory)."""
    st = tuple(s // a.itemsize for s in a.strides)
    return dev.DevBuf(_FakeStorage(), 0, a.shape, st, "float32")


def _same(b: dev.DevBuf, a: np.ndarray, base: np.ndarray):
    assert tuple(b.shape) == a.shape
    assert tuple(b.stride()) == tuple(s // a.itemsize for s in a.strides) or a.size <= 1
    off = (a.__array_interface__["data"][0] - base.__array_interface__["data"][0]) // a.itemsize
    assert b.data_ptr() == (1 << 20) + 4 * off


def test_views_match_numpy_strides():
    base = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    for perm in itertools.permutations(range(4)):
        a = base.transpose(perm)
        b = _buf(base).permute(*perm)
        _same(b, a, base)
        for new in [(-1,), (a.shape[0], -1), (a.shape[0] * a.shape[1], a.shape[2], a.shape[3]),
                    (a.shape[0], a.shape[1], 1, a.shape[2] * a.shape[3]), (1,) + a.shape]:
            try:
                v = a.view()
                v.shape = tuple(new) if -1 not in new else np.empty(a.size).reshape(new).shape
                view_ok = True
            except AttributeError:
                view_ok = False
            shape = np.empty(a.size).reshape(new).shape
            if view_ok:
                _same(b.view(*new), a.reshape(shape), base)
            else:
                with pytest.raises(RuntimeError):
                    b.view(*new)


def test_slicing_expand_unflatten():
    base = np.arange(6 * 7 * 8, dtype=np.float32).reshape(6, 7, 8)
    b = _buf(base)
    for key in [(slice(1, 5), 3), (Ellipsis, slice(2, 8, 3)), (2, slice(None), slice(1, 2)), (-1,),
                (slice(0, 0),), (None, 1)]:
        _same(b[key], base[key], base)
    e = _buf(base[:, :1, :]).expand(6, 7, 8)
    assert e.shape == (6, 7, 8) and e.stride() == (56, 0, 1)
    e = _buf(np.zeros(8, np.float32)).expand(3, -1)
    assert e.shape == (3, 8) and e.stride() == (0, 1)
    u = b.transpose(0, 1).unflatten(2, (2, 4))
    _same(u, base.transpose(1, 0, 2).reshape(7, 6, 2, 4), base)
    assert b.unsqueeze(1).shape == (6, 1, 7, 8)
    _same(_buf(base[0]).t(), base[0].T, base)
    with pytest.raises(ValueError):
        b.expand(6, 3, 8)


def test_contiguity():
    base = np.zeros((4, 5, 6), np.float32)
    assert _buf(base).is_contiguous()
    assert not _buf(base).transpose(0, 2).is_contiguous()
    assert not _buf(base[:, :2]).is_contiguous()
    assert _buf(base[:1]).is_contiguous()


def test_dtype_names_and_bf16_host_rounding():
    assert dev.dtype_name(np.float32) == "float32"
    assert dev.dtype_name(np.dtype(np.int64)) == "int64"
    assert dev.dtype_name("bfloat16") == "bfloat16"
    with pytest.raises(ValueError):
        dev.dtype_name(np.float16)
    from oracle.attention import bf16_round

    x = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    bits = dev.host_array(x, "bfloat16")
    assert bits.dtype == np.uint16
    back = (bits.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(back, bf16_round(x))
    # NaNs with payloads (which round-to-nearest would carry into +-Inf or
    # +-0) stay NaNs of their sign; Inf and the largest finite values round
    # as IEEE rounding does (to Inf past the bf16 maximum)
    pats = np.array([0x7F800001, 0x7FFFFFFF, 0xFFFFFFFF, 0xFF800001, 0x7FC00000, 0x7F800000, 0xFF800000,
                     0x7F7FFFFF, 0x7F7F0000, 0x00000001, 0x80000000], dtype=np.uint32)
    got = dev.host_array(pats.view(np.float32), "bfloat16")
    want = np.array([0x7FC0, 0x7FC0, 0xFFC0, 0xFFC0, 0x7FC0, 0x7F80, 0xFF80, 0x7F80, 0x7F7F, 0x0000, 0x8000],
                    dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


def test_runtime_argument_checks_without_gpu():
    lib = L.lib()
    n = C.c_int(-1)
    assert lib.mtx_device_count(C.byref(n)) == 0 and n.value >= 0
    assert lib.mtx_fill(C.c_void_p(256), 4, 0, 3, None) == L.MTX_ERR_ARG
    assert "width" in lib.mtx_last_error().decode()
    assert lib.mtx_fill(C.c_void_p(258), 4, 0, 4, None) == L.MTX_ERR_ARG
    assert lib.mtx_free(C.c_void_p(12345)) == L.MTX_ERR_ARG
    assert "not a live" in lib.mtx_last_error().decode()
    assert lib.mtx_free(None) == 0
    assert lib.mtx_graph_begin(None) == L.MTX_ERR_ARG
    h = C.c_void_p()
    assert lib.mtx_graph_end(C.c_void_p(64), C.byref(h)) == L.MTX_ERR_ARG
    assert lib.mtx_memcpy_h2d(None, None, 0, None) == 0  # empty copies are no-ops
    a, c = C.c_size_t(1), C.c_size_t(1)
    assert lib.mtx_memory_stats(C.byref(a), C.byref(c)) == 0


def test_noalloc_rejects_oversize_before_any_hip_call():
    s = (C.c_int64 * 4)(64, 64, 64, 1)
    p = C.c_void_p(256)
    Tq = L.ATTN_SCRATCH_BYTES // 4 + 1
    rc = L.lib().mtx_attn_bwd_noalloc(L.MTX_F32, 1, 1, Tq, Tq, 64, p, s, p, s, p, s, p, s, p, s, p,
                                      p, s, p, s, p, s, 0.125, 1, 0, None)
    assert rc == L.MTX_ERR_SHAPE and "scratch" in L.lib().mtx_last_error().decode()
