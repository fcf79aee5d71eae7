"""mtx_attn_bwd_noalloc (the backward entry point that allocates nothing:
delta lives in the library's fixed per-GPU device array) against
mtx_attn_bwd with a caller workspace.  Same kernels, so the results must be
identical bit for bit; checked on two calls in a row, the second with a
smaller input (the array keeps the first call's contents), for fp32 and
bf16, plus the host-side rejection of inputs beyond the array's size."""
import ctypes as C
import sys

import numpy as np
import pytest

from devarrays import T, full, sync
from oracle.attention import bf16_round

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(rng, shp_q, shp_k, bf16):
    arrs = [rng.standard_normal(s, dtype=np.float32) for s in (shp_q, shp_k, shp_k, shp_q)]
    if bf16:
        arrs = [bf16_round(0.5 * a) for a in arrs]
    return [T(a, "bfloat16" if bf16 else "float32") for a in arrs]


@pytest.mark.parametrize("bf16", [False, True])
def test_noalloc_matches_workspace_entry_point(dev, bf16):
    from minitorch_amd import kernels as K

    rng = np.random.default_rng(77)
    # second call smaller than the first: rows of the first call stay behind
    # in the scratch array and must not leak into the second
    for (B, H, Tq, Tk, D) in [(4, 6, 300, 300, 64), (2, 3, 129, 200, 64)]:
        _say(f"[noalloc] bf16={bf16} B={B} H={H} Tq={Tq} Tk={Tk} D={D}")
        q, k, v, do = _inputs(rng, (B, H, Tq, D), (B, H, Tk, D), bf16)
        o, lse = K.attn_fwd(q, k, v, 0.125, True)
        ref = K.attn_bwd(q, k, v, o, do, lse, 0.125, True)
        got = [full((B, H, t, D), float("nan")) for t in (Tq, Tk, Tk)]
        K.attn_bwd_noalloc(q, k, v, o, do, lse, 0.125, True, *got)
        sync()
        for name, a, b in zip(("dq", "dk", "dv"), ref, got):
            a, b = a.numpy(), b.numpy()
            assert np.all(np.isfinite(b)), name
            assert np.array_equal(a, b), (name, float(np.abs(a - b).max()))


def test_noalloc_rejects_oversize(dev):
    from minitorch_amd import _lib as L

    rows_max = L.ATTN_SCRATCH_BYTES // 4
    s = (C.c_int64 * 4)(64, 64, 64, 1)
    p = C.c_void_p(256)
    B, H, Tq = 1, 1, rows_max + 1
    rc = L.lib().mtx_attn_bwd_noalloc(L.MTX_F32, B, H, Tq, Tq, 64, p, s, p, s, p, s, p, s, p, s, p,
                                      p, s, p, s, p, s, 0.125, 1, 0, None)
    assert rc == L.MTX_ERR_SHAPE
    assert "scratch" in L.lib().mtx_last_error().decode()
