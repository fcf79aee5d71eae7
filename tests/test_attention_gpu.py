"""GPU parity of the fused attention kernels against the CPU oracle.

Bars (the parity tolerances of the hot path):
  * fp32 inputs: elementwise |gpu - ref| <= 1e-5 + 1e-4 * |ref|
  * bf16 inputs ("rel 2e-2"): max|gpu - ref| <= 2e-2 * max|ref| and
    ||gpu - ref||_F <= 2e-2 * ||ref||_F, against the fp32/fp64 NumPy reference
    run on the bf16-rounded inputs.  (An elementwise relative bar against the
    reference is not meaningful here: the flash backward rounds P and dS to
    bf16 before the MFMA products, so near-cancelled gradient entries carry
    absolute errors of ~0.5% of max|ref|.)  In addition every bf16 result is
    compared elementwise with oracle.attention.attention_bf16_emulated, which
    makes exactly the kernels' roundings (_emu_bar: a much tighter bar).
The oracle is oracle.attention.reference_attention (the reference's own dtype
flow, transformer.py:36-44).  Full-size bf16 (C3) runs are checked on a subset
of (b, h) slices against the oracle and in full through identities that hold
for any size: sum_j dV_j = sum_i dO_i and sum_j dK_j = 0 per (b, h).
"""
import ctypes
import math
import sys

import numpy as np
import pytest

from devarrays import T as _T, empty, full, sync
from oracle.attention import attention_bf16_emulated, bf16_round, reference_attention

pytestmark = pytest.mark.gpu
C_i64 = ctypes.c_int64


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _worst(err, lim):
    """max of err/lim over elements, with 0/0 counted as 0."""
    ratio = np.divide(err, lim, out=np.zeros_like(err), where=lim > 0)
    ratio[(lim == 0) & (err > 0)] = np.inf
    return float(ratio.max()) if ratio.size else 0.0


def _fp32_bar(got, ref, name):
    err = np.abs(got.astype(np.float64) - ref)
    lim = 1e-5 + 1e-4 * np.abs(ref)
    worst = _worst(err, lim)
    assert np.all(err <= lim), f"{name}: max err {err.max():.3e}, worst err/limit {worst:.3f}"
    return worst


def _bf16_bar(got, ref, name):
    ref = ref.astype(np.float64)
    diff = got.astype(np.float64) - ref
    amax = float(np.abs(ref).max())
    nmax = float(np.abs(diff).max()) / amax if amax > 0 else float(np.abs(diff).max())
    fro = float(np.linalg.norm(ref))
    rfro = float(np.linalg.norm(diff)) / fro if fro > 0 else float(np.linalg.norm(diff))
    assert nmax <= 2e-2 and rfro <= 2e-2, (
        f"{name}: max err / max|ref| = {nmax:.3e}, relative Frobenius error {rfro:.3e} (bar 2e-2)")
    return max(nmax, rfro) / 2e-2


# Elementwise bar against attention_bf16_emulated (the kernels' own bf16
# rounding points restated in float64): what is left is fp32 accumulation
# order and the rare bf16 rounding that a last-bit difference of a score
# flips.  |gpu - emu| <= EMU_ATOL * max|emu| + EMU_RTOL * |emu| + EMU_FLOOR
# per (b, h) slice and tensor (the floor covers gradients that are exactly 0
# in exact arithmetic, e.g. dq at T = 1, where fp32 leaves ~1e-8); a wrong
# row, column or tile is off by O(max|emu|).
EMU_ATOL, EMU_RTOL, EMU_FLOOR = 2e-3, 8e-3, 1e-6


def _emu_bar(got, emu, name):
    got = got.astype(np.float64)
    err = np.abs(got - emu)
    amax = max(float(np.abs(emu).max()), EMU_FLOOR)
    lim = EMU_ATOL * amax + EMU_RTOL * np.abs(emu) + EMU_FLOOR
    worst = _worst(err, lim)
    assert np.all(err <= lim), (f"{name}: max err {err.max():.3e} (= {err.max() / amax:.3e} of max|emu|), "
                                f"worst err/limit {worst:.3f}")
    return float(err.max()) / amax


def _to_dev(x, dev, dtype):
    return _T(x, dtype)


def _onepass(dtype, D):
    """Whether attn_bwd runs the one-pass backward for these inputs (its dQ
    is then emulated from the key-outer pass's dS: attention_bf16_emulated
    onepass=True)."""
    from minitorch_amd import kernels as K

    return K.attn_bwd_onepass_used(dtype, D)


@pytest.fixture(params=["onepass", "twopass"])
def bwd_mode(request, dev):
    """bf16 backward tests run under both structures: the deterministic two
    passes (the default) and the one-pass kernel (dQ by atomics)."""
    from minitorch_amd import kernels as K

    prev = K.set_attn_bwd_mode(K.ATTN_BWD_ONEPASS if request.param == "onepass" else K.ATTN_BWD_TWOPASS)
    yield request.param
    K.set_attn_bwd_mode(prev)


def _run(dev, q, k, v, do, scale, causal, dtype, views=None):
    """Run fwd+bwd on the device; returns numpy (o, dq, dk, dv, lse)."""
    from minitorch_amd import kernels as K

    tq, tk, tv, tdo = (_to_dev(x, dev, dtype) for x in (q, k, v, do))
    if views is not None:
        tq, tk, tv, tdo = (views(t) for t in (tq, tk, tv, tdo))
    o, lse = K.attn_fwd(tq, tk, tv, scale, causal)
    dq, dk, dv = K.attn_bwd(tq, tk, tv, o, tdo, lse, scale, causal)
    sync()
    f = lambda t: t.numpy()
    return f(o), f(dq), f(dk), f(dv), f(lse)


@pytest.fixture(params=["bf16x3", "fp32"])
def attn_mode(request, dev):
    """fp32 attention tests run under both product kernels (they differ for
    64-wide heads): the three-piece bf16 split (the default) and fp32 MFMA."""
    from minitorch_amd import kernels as Kn

    prev = Kn.set_attn_mode(Kn.GEMM_BF16X3 if request.param == "bf16x3" else Kn.GEMM_FP32)
    yield request.param
    Kn.set_attn_mode(prev)


CASES = [
    # (B, H, Tq, Tk, D, causal)
    (1, 1, 1, 1, 64, True),
    (2, 3, 7, 7, 16, True),
    (1, 2, 63, 63, 64, True),
    (1, 2, 64, 64, 32, True),
    (2, 2, 65, 65, 64, True),
    (1, 3, 130, 130, 128, True),
    (2, 2, 200, 200, 64, False),
    (1, 2, 17, 100, 64, True),   # Tq < Tk: bottom-right causal alignment
    (1, 2, 33, 70, 16, False),
    (2, 4, 256, 256, 16, True),
]


@pytest.mark.parametrize("B,H,Tq,Tk,D,causal", CASES)
def test_fp32_small(dev, attn_mode, B, H, Tq, Tk, D, causal):
    _say(f"[attn fp32 {attn_mode}] B={B} H={H} Tq={Tq} Tk={Tk} D={D} causal={causal}")
    rng = np.random.default_rng(1000 + Tq + 7 * Tk + D)
    q = rng.standard_normal((B, H, Tq, D), dtype=np.float32)
    k = rng.standard_normal((B, H, Tk, D), dtype=np.float32)
    v = rng.standard_normal((B, H, Tk, D), dtype=np.float32)
    do = rng.standard_normal((B, H, Tq, D), dtype=np.float32)
    scale = 1.0 / math.sqrt(D)
    o, dq, dk, dv, lse = _run(dev, q, k, v, do, scale, causal, "float32")
    ro, rdq, rdk, rdv = reference_attention(q, k, v, do, scale, causal)
    _fp32_bar(o, ro, "o")
    _fp32_bar(dq, rdq, "dq")
    _fp32_bar(dk, rdk, "dk")
    _fp32_bar(dv, rdv, "dv")
    # lse against log-sum-exp of the float64 scores
    s = (q.astype(np.float64) @ np.swapaxes(k, -1, -2).astype(np.float64)) * scale
    if causal:
        from oracle.attention import causal_mask

        s = np.where(causal_mask(Tq, Tk), -np.inf, s)
    m = s.max(-1, keepdims=True)
    rlse = (m + np.log(np.exp(s - m).sum(-1, keepdims=True)))[..., 0]
    assert np.max(np.abs(lse - rlse)) < 1e-4


@pytest.mark.parametrize("B,H,Tq,Tk,D,causal", [c for c in CASES if c[4] != 128] + [(1, 2, 100, 100, 128, True)])
def test_bf16_small(dev, bwd_mode, B, H, Tq, Tk, D, causal):
    _say(f"[attn bf16 {bwd_mode}] B={B} H={H} Tq={Tq} Tk={Tk} D={D} causal={causal}")
    rng = np.random.default_rng(2000 + Tq + 7 * Tk + D)
    q = bf16_round(0.5 * rng.standard_normal((B, H, Tq, D), dtype=np.float32))
    k = bf16_round(0.5 * rng.standard_normal((B, H, Tk, D), dtype=np.float32))
    v = bf16_round(0.5 * rng.standard_normal((B, H, Tk, D), dtype=np.float32))
    do = bf16_round(rng.standard_normal((B, H, Tq, D), dtype=np.float32))
    scale = 1.0 / math.sqrt(D)
    o, dq, dk, dv, lse = _run(dev, q, k, v, do, scale, causal, "bfloat16")
    ro, rdq, rdk, rdv = reference_attention(q, k, v, do, scale, causal)
    _bf16_bar(o, ro, "o")
    _bf16_bar(dq, rdq, "dq")
    _bf16_bar(dk, rdk, "dk")
    _bf16_bar(dv, rdv, "dv")
    emu = attention_bf16_emulated(q, k, v, do, scale, causal, onepass=_onepass("bfloat16", D))
    for b in range(B):
        for h in range(H):
            for name, got, e in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv), emu):
                _emu_bar(got[b, h], e[b, h], f"{name}[{b},{h}]")


def test_fp32_strided_split_heads(dev, attn_mode):
    """q/k/v as the (B,H,T,D) strided views _split_heads makes of a (B,T,C)
    projection (transformer.py:26-28): strides (T*C, D, C, 1), no copies."""
    B, T, H, D = 2, 96, 6, 64
    C = H * D
    _say(f"[attn fp32 views] B={B} T={T} H={H} D={D}")
    rng = np.random.default_rng(7)
    xs = [rng.standard_normal((B, T, C), dtype=np.float32) for _ in range(4)]
    split = lambda t: t.view(B, T, H, D).transpose(1, 2)
    o, dq, dk, dv, _ = _run(dev, *xs, 1 / 8, True, "float32", views=split)
    q, k, v, do = (x.reshape(B, T, H, D).transpose(0, 2, 1, 3) for x in xs)
    ro, rdq, rdk, rdv = reference_attention(q, k, v, do, 1 / 8, True)
    _fp32_bar(o, ro, "o")
    _fp32_bar(dq, rdq, "dq")
    _fp32_bar(dk, rdk, "dk")
    _fp32_bar(dv, rdv, "dv")


def test_accumulate_flag(dev, attn_mode):
    """accumulate=1 adds into existing gradients (_accum_grad, tensor.py:29-33)."""
    from minitorch_amd import kernels as K

    _say("[attn accumulate]")
    rng = np.random.default_rng(3)
    shp = (1, 2, 50, 64)
    q, k, v, do = (_to_dev(rng.standard_normal(shp, dtype=np.float32), dev, "float32") for _ in range(4))
    o, lse = K.attn_fwd(q, k, v, 0.125, True)
    dq, dk, dv = K.attn_bwd(q, k, v, o, do, lse, 0.125, True)
    base = [t.clone() for t in (dq, dk, dv)]
    K.attn_bwd(q, k, v, o, do, lse, 0.125, True, dq=dq, dk=dk, dv=dv, accumulate=True)
    sync()
    for a, b in zip((dq, dk, dv), base):
        np.testing.assert_allclose(a.numpy(), 2 * b.numpy(), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dtype_name", ["float32", "bfloat16"])
def test_phases_split_match_fused(dev, attn_mode, dtype_name):
    """mtx_attn_bwd_phase run as three calls (standalone delta kernel, then
    dQ, then dK/dV) gives the oracle's gradients and agrees with the fused
    DELTA|DQ path of mtx_attn_bwd (two-pass mode) up to the summation order
    of delta."""
    from minitorch_amd import _lib as L
    from minitorch_amd import kernels as K

    dtype = dtype_name
    _say(f"[attn phases split vs fused] {dtype_name}")
    prev = K.set_attn_bwd_mode(K.ATTN_BWD_TWOPASS)
    try:
        _phases_split(L, K, dtype)
    finally:
        K.set_attn_bwd_mode(prev)


def _phases_split(L, K, dtype):
    rng = np.random.default_rng(17)
    B, H, Tq, Tk, D = 2, 3, 150, 190, 64
    arrs = [rng.standard_normal((B, H, T, D), dtype=np.float32) for T in (Tq, Tk, Tk, Tq)]
    if dtype == "bfloat16":
        arrs = [bf16_round(0.5 * x) for x in arrs]
    q, k, v, do = (_to_dev(x, None, dtype) for x in arrs)
    o, lse = K.attn_fwd(q, k, v, 0.125, True)
    fused = K.attn_bwd(q, k, v, o, do, lse, 0.125, True)
    split = [full(t.shape, float("nan")) for t in fused]
    ws = empty((L.lib().mtx_attn_bwd_workspace_bytes(B, H, Tq),), "uint8")
    for ph in (L.ATTN_BWD_DELTA, L.ATTN_BWD_DQ, L.ATTN_BWD_DKDV):
        K.attn_bwd(q, k, v, o, do, lse, 0.125, True, dq=split[0], dk=split[1], dv=split[2],
                   workspace=ws, phases=ph)
    sync()
    refs = reference_attention(*arrs, 0.125, True)[1:]
    for name, a, b, r in zip(("dq", "dk", "dv"), fused, split, refs):
        a, b = a.numpy(), b.numpy()
        assert np.all(np.isfinite(b)), name
        scale = float(np.abs(r).max())
        assert np.abs(a - b).max() <= 1e-5 * scale, (name, float(np.abs(a - b).max()), scale)
        (_fp32_bar if dtype == "float32" else _bf16_bar)(b, r, name)


ONEPASS_CASES = [
    # (B, H, Tq, Tk, D, causal)
    (1, 1, 1, 1, 64, True),
    (2, 3, 150, 190, 64, True),    # Tq < Tk, ragged key block
    (1, 2, 1000, 1000, 64, True),  # ragged last query tile and key block
    (2, 2, 200, 200, 64, False),
    (2, 2, 65, 70, 64, False),     # non-causal, ragged key block
    (1, 2, 17, 100, 64, True),
    (2, 4, 256, 256, 16, True),
    (1, 2, 64, 64, 32, True),
    (1, 2, 130, 130, 32, False),
]


@pytest.mark.parametrize("B,H,Tq,Tk,D,causal", ONEPASS_CASES)
def test_onepass_matches_twopass_and_emulation(dev, B, H, Tq, Tk, D, causal):
    """bf16 one-pass backward (dK/dV written, dQ added with fp32 atomics by
    the key-outer kernel): dK and dV bit-identical to the two-pass kernels'
    (the same products in the same order), dQ elementwise against the
    rounding emulation of the one-pass form and within the bf16 bar of the
    reference."""
    from minitorch_amd import kernels as K

    _say(f"[attn bf16 one-pass vs two-pass] B={B} H={H} Tq={Tq} Tk={Tk} D={D} causal={causal}")
    rng = np.random.default_rng(3000 + Tq + 7 * Tk + D)
    q = bf16_round(0.5 * rng.standard_normal((B, H, Tq, D), dtype=np.float32))
    k = bf16_round(0.5 * rng.standard_normal((B, H, Tk, D), dtype=np.float32))
    v = bf16_round(0.5 * rng.standard_normal((B, H, Tk, D), dtype=np.float32))
    do = bf16_round(rng.standard_normal((B, H, Tq, D), dtype=np.float32))
    scale = 1.0 / math.sqrt(D)
    prev = K.set_attn_bwd_mode(K.ATTN_BWD_ONEPASS)
    try:
        o1, dq1, dk1, dv1, lse = _run(dev, q, k, v, do, scale, causal, "bfloat16")
        K.set_attn_bwd_mode(K.ATTN_BWD_TWOPASS)
        o2, dq2, dk2, dv2, _ = _run(dev, q, k, v, do, scale, causal, "bfloat16")
    finally:
        K.set_attn_bwd_mode(prev)
    assert np.array_equal(o1, o2)
    assert np.array_equal(dk1, dk2), float(np.abs(dk1 - dk2).max())
    assert np.array_equal(dv1, dv2), float(np.abs(dv1 - dv2).max())
    assert np.all(np.isfinite(dq1))
    _, rdq, _, _ = reference_attention(q, k, v, do, scale, causal)
    _bf16_bar(dq1, rdq, "dq one-pass")
    emu = attention_bf16_emulated(q, k, v, do, scale, causal, onepass=True)
    for b in range(B):
        for h in range(H):
            _emu_bar(dq1[b, h], emu[2][b, h], f"dq[{b},{h}]")


def test_onepass_phases_and_accumulate(dev):
    """The one-pass kernels through explicit phases (ONEPASS|DELTA: delta and
    dq zeroed; ONEPASS|DQ|DKDV: the key-outer kernel) equal mtx_attn_bwd in
    one-pass mode; with accumulate=1 the gradients are added (dq starts from
    the given values: the delta kernel leaves it alone); two runs agree up to
    the atomics' summation order (dK/dV bit for bit)."""
    from minitorch_amd import _lib as L
    from minitorch_amd import kernels as K

    _say("[attn bf16 one-pass phases / accumulate]")
    rng = np.random.default_rng(41)
    B, H, Tq, Tk, D = 2, 3, 300, 300, 64
    arrs = [bf16_round(0.5 * rng.standard_normal((B, H, T, D), dtype=np.float32)) for T in (Tq, Tk, Tk, Tq)]
    q, k, v, do = (_to_dev(x, None, "bfloat16") for x in arrs)
    prev = K.set_attn_bwd_mode(K.ATTN_BWD_ONEPASS)
    try:
        o, lse = K.attn_fwd(q, k, v, 0.125, True)
        ref = [t.numpy() for t in K.attn_bwd(q, k, v, o, do, lse, 0.125, True)]
        again = [t.numpy() for t in K.attn_bwd(q, k, v, o, do, lse, 0.125, True)]
        ws = empty((L.lib().mtx_attn_bwd_workspace_bytes(B, H, Tq),), "uint8")
        got = [full((B, H, t, D), float("nan")) for t in (Tq, Tk, Tk)]
        for ph in (L.ATTN_BWD_ONEPASS | L.ATTN_BWD_DELTA, L.ATTN_BWD_ONEPASS | L.ATTN_BWD_DQ | L.ATTN_BWD_DKDV):
            K.attn_bwd(q, k, v, o, do, lse, 0.125, True, dq=got[0], dk=got[1], dv=got[2], workspace=ws, phases=ph)
        sync()
        got = [t.numpy() for t in got]
        acc = [_to_dev(x, None, "float32") for x in ref]
        K.attn_bwd(q, k, v, o, do, lse, 0.125, True, dq=acc[0], dk=acc[1], dv=acc[2], accumulate=True)
        sync()
        acc = [t.numpy() for t in acc]
    finally:
        K.set_attn_bwd_mode(prev)
    for name, r, a, g, c in zip(("dq", "dk", "dv"), ref, again, got, acc):
        amax = float(np.abs(r).max())
        if name == "dq":
            assert np.abs(a - r).max() <= 1e-6 * amax, (name, float(np.abs(a - r).max()), amax)
            assert np.abs(g - r).max() <= 1e-6 * amax, (name, float(np.abs(g - r).max()), amax)
        else:
            assert np.array_equal(a, r) and np.array_equal(g, r), name
        assert np.abs(c - 2 * r).max() <= 2e-6 * amax, (name, float(np.abs(c - 2 * r).max()), amax)


def test_onepass_phase_rejections(dev):
    """The one-pass phase bit is refused, before any device work, for fp32
    inputs and for DQ without DKDV."""
    from minitorch_amd import _lib as L

    s = (C_i64 * 4)(64, 64, 64, 1)
    lib = L.lib()
    for dtype, phases in ((L.MTX_F32, L.ATTN_BWD_ONEPASS | L.ATTN_BWD_ALL),
                          (L.MTX_BF16, L.ATTN_BWD_ONEPASS | L.ATTN_BWD_DQ)):
        rc = lib.mtx_attn_bwd_phase(phases, dtype, 1, 1, 64, 64, 64, None, s, None, s, None, s, None, s,
                                    None, s, None, None, s, None, s, None, s, None, 0, 0.125, 1, 0, None)
        assert rc != 0
        assert "ONEPASS" in lib.mtx_last_error().decode() or "one-pass" in lib.mtx_last_error().decode()


def test_c1_full(dev, attn_mode):
    """Config C1: B=32, H=8, T=256, D=64 fp32, q,k,v,dO ~ N(0,1) drawn in that
    order from default_rng(1); scale 1/8.  Full tensors vs the oracle."""
    _say(f"[attn C1 full {attn_mode}] B=32 H=8 T=256 D=64 fp32")
    rng = np.random.default_rng(1)
    shp = (32, 8, 256, 64)
    q, k, v, do = (rng.standard_normal(shp, dtype=np.float32) for _ in range(4))
    o, dq, dk, dv, _ = _run(dev, q, k, v, do, 0.125, True, "float32")
    ro, rdq, rdk, rdv = reference_attention(q, k, v, do, 0.125, True)
    w = [_fp32_bar(o, ro, "o"), _fp32_bar(dq, rdq, "dq"), _fp32_bar(dk, rdk, "dk"), _fp32_bar(dv, rdv, "dv")]
    _say(f"  worst err/limit o,dq,dk,dv = {[round(x, 4) for x in w]}")


def _emu_slices(tag, q, k, v, do, scale, outs, slices, group=4):
    """Every (b, h) of `slices` elementwise against the rounding emulation
    (each slice to its own bar); consecutive heads of one b go through the
    emulation together, `group` at a time."""
    onepass = _onepass("bfloat16", q.shape[-1])
    worst = {}
    runs = []
    for b, h in slices:
        if runs and runs[-1][0] == b and runs[-1][2] == h and runs[-1][2] - runs[-1][1] < group:
            runs[-1][2] = h + 1
        else:
            runs.append([b, h, h + 1])
    for b, h0, h1 in runs:
        sl = (slice(b, b + 1), slice(h0, h1))
        emu = attention_bf16_emulated(q[sl], k[sl], v[sl], do[sl], scale, True, onepass=onepass)
        for name, got, e in zip(("o", "lse", "dq", "dk", "dv"), outs, emu):
            g = got[sl]
            for j in range(h1 - h0):
                r = _emu_bar(g[:, j], e[:, j], f"{tag} {name}[{b},{h0 + j}]")
                worst[name] = max(worst.get(name, 0.0), r)
    _say(f"  {tag}: max |gpu - emu| / max|emu| over {len(slices)} slices: "
         + ", ".join(f"{n} {w:.2e}" for n, w in worst.items()))


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_forward_reference_moves(dev, dtype):
    """Scores that grow along the keys (q = 1, k_j = j/16: 0.72 log2 units
    per key at D = 64): every key tile's max exceeds the row's reference by
    more than 8, so the forward moves the reference on every tile (the
    rescale branch, which random inputs take only on the first tile).  bf16
    against the rounding emulation (which models where the reference moves),
    fp32 against the oracle: the forward outputs and dV.
    (dQ and dK are only checked finite: with scores up to ~180 log2 units
    the bf16 rounding of the pre-scaled operand moves P by tens of percent
    and dS cancels, so the emulation itself is 47% / 24% away from float64
    there and last-bit differences are amplified past any elementwise bar.)"""
    from oracle.attention import _lazy_reference, causal_mask, LOG2E

    _say(f"[attn moving reference] {dtype}")
    B, H, T, D = 1, 2, 256, 64
    rng = np.random.default_rng(57)
    q = np.ones((B, H, T, D), np.float32)
    k = np.broadcast_to((np.arange(T, dtype=np.float32) / 16)[:, None], (B, H, T, D)).copy()
    v = bf16_round(rng.standard_normal((B, H, T, D), dtype=np.float32))
    do = bf16_round(rng.standard_normal((B, H, T, D), dtype=np.float32))
    s2 = np.where(causal_mask(T, T), -np.inf, (q[0, 0].astype(np.float64) * (0.125 * LOG2E)) @ k[0, 0].T)
    mt = _lazy_reference(s2, 64, 8.0)
    assert len(np.unique(mt[-1])) == 4  # the last row's reference moves on every tile
    o, dq, dk, dv, lse = _run(dev, q, k, v, do, 0.125, True, dtype)
    assert np.all(np.isfinite(dq)) and np.all(np.isfinite(dk))
    if dtype == "bfloat16":
        emu = attention_bf16_emulated(q, k, v, do, 0.125, True, onepass=_onepass(dtype, D))
        for b in range(B):
            for h in range(H):
                for name, got, e in zip(("o", "lse", "dv"), (o, lse, dv), (emu[0], emu[1], emu[4])):
                    _emu_bar(got[b, h], e[b, h], f"{name}[{b},{h}]")
    else:
        # fp32 scores of up to ~127 (natural units) carry rounding of about
        # |s| 2^-22, which exp turns into that relative error in P: beyond
        # the 1e-4 elementwise bar for any fp32 implementation, so 1e-3 of
        # the largest entry here (a wrongly moved reference is off by O(1))
        ro, _, _, rdv = reference_attention(q, k, v, do, 0.125, True)
        for name, got, r in (("o", o, ro), ("dv", dv, rdv)):
            err = float(np.abs(got - r).max())
            assert err <= 1e-3 * float(np.abs(r).max()), (name, err)


def test_bf16_elementwise_ragged_t(dev):
    """bf16 kernels elementwise against the rounding emulation at a T that is
    not a multiple of the 64-row tiles (ragged last query and key tiles,
    diagonal tiles in every slice): all B*H = 16 slices."""
    B, H, T, D = 2, 8, 1000, 64
    _say(f"[attn bf16 elementwise] B={B} H={H} T={T} D={D}")
    rng = np.random.default_rng(31)
    q, k, v = (bf16_round(0.5 * rng.standard_normal((B, H, T, D), dtype=np.float32)) for _ in range(3))
    do = bf16_round(rng.standard_normal((B, H, T, D), dtype=np.float32))
    o, dq, dk, dv, lse = _run(dev, q, k, v, do, 0.125, True, "bfloat16")
    _emu_slices("T=1000", q, k, v, do, 0.125, (o, lse, dq, dk, dv),
                [(b, h) for b in range(B) for h in range(H)])


def test_c3_full(dev):
    """Config C3: B=8, H=16, T=2048, D=64; q,k,v = 0.5*N(0,1), dO = N(0,1), all
    rounded to bf16, drawn in that order from default_rng(3).  All 128 (b,h)
    slices elementwise against the bf16 rounding emulation; six slices vs
    the fp32/fp64 oracle at the bf16 bar; every slice through the dV / dK
    sum identities."""
    _say("[attn C3 full] B=8 H=16 T=2048 D=64 bf16")
    rng = np.random.default_rng(3)
    shp = (8, 16, 2048, 64)
    q = bf16_round(0.5 * rng.standard_normal(shp, dtype=np.float32))
    k = bf16_round(0.5 * rng.standard_normal(shp, dtype=np.float32))
    v = bf16_round(0.5 * rng.standard_normal(shp, dtype=np.float32))
    do = bf16_round(rng.standard_normal(shp, dtype=np.float32))
    o, dq, dk, dv, lse = _run(dev, q, k, v, do, 0.125, True, "bfloat16")
    assert np.all(np.isfinite(o)) and np.all(np.isfinite(dq))
    # every slice elementwise against the bf16 rounding emulation
    import time

    t0 = time.time()
    _emu_slices("C3", q, k, v, do, 0.125, (o, lse, dq, dk, dv), [(b, h) for b in range(8) for h in range(16)])
    _say(f"  C3 emulation of 128 slices: {time.time() - t0:.1f}s")
    for b, h in [(0, 0), (0, 15), (3, 7), (5, 2), (7, 0), (7, 15)]:
        sl = (slice(b, b + 1), slice(h, h + 1))
        ro, rdq, rdk, rdv = reference_attention(q[sl], k[sl], v[sl], do[sl], 0.125, True)
        _bf16_bar(o[sl], ro, f"o[{b},{h}]")
        _bf16_bar(dq[sl], rdq, f"dq[{b},{h}]")
        _bf16_bar(dk[sl], rdk, f"dk[{b},{h}]")
        _bf16_bar(dv[sl], rdv, f"dv[{b},{h}]")
    # identities: sum over keys of dV equals sum over queries of dO; sum of dK is 0
    sdv = dv.astype(np.float64).sum(axis=2)
    sdo = do.astype(np.float64).sum(axis=2)
    scale_ref = np.abs(dv).astype(np.float64).sum(axis=2) + 1.0
    assert np.max(np.abs(sdv - sdo) / scale_ref) < 2e-2
    sdk = dk.astype(np.float64).sum(axis=2)
    assert np.max(np.abs(sdk) / (np.abs(dk).astype(np.float64).sum(axis=2) + 1.0)) < 2e-2


@pytest.mark.parametrize("B,H,T,D", [(32, 8, 256, 64), (16, 4, 32, 16)])
def test_unfused_reference_composition(dev, B, H, T, D):
    """transformer.py:36-44 written out literally on minitorch_amd Tensors
    (the unfused path the reference's own op set takes): q @ k^T through
    Tensor.__matmul__, * (1.0 / np.sqrt(D)) with its np.float64 scale, +
    Tensor(np.triu(ones, 1) * -1e9), F.softmax, @ v, then .backward() with
    upstream gradient dO.  At the C1 shape and at C0's head shape (D = 16).
    out/dq/dk/dv against the oracle at the fp32 bar, and against the fused
    attention node (functional.causal_attention) on the same inputs."""
    import minitorch_amd as mt
    from minitorch_amd import functional as F

    _say(f"[attn unfused composition] B={B} H={H} T={T} D={D}")
    rng = np.random.default_rng(400 + D)
    q, k, v, do = (rng.standard_normal((B, H, T, D), dtype=np.float32) for _ in range(4))

    def run(fused):
        tq, tk, tv = (mt.Tensor(a, requires_grad=True) for a in (q, k, v))
        if fused:
            out = F.causal_attention(tq, tk, tv, scale=1.0 / np.sqrt(D))
        else:
            scores = (tq @ tk.transpose(-2, -1)) * (1.0 / np.sqrt(D))
            mask = np.triu(np.ones((T, T), dtype=np.float32), k=1) * -1e9
            scores = scores + mt.Tensor(mask)
            attn = F.softmax(scores, axis=-1)
            out = attn @ tv
        (out * mt.Tensor(do)).sum().backward()
        return out.numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()

    unf = run(False)
    fus = run(True)
    ref = reference_attention(q, k, v, do, 1.0 / np.sqrt(D), True)
    for name, a, b, r in zip(("out", "dq", "dk", "dv"), unf, fus, ref):
        _fp32_bar(a, r, f"unfused {name}")
        _fp32_bar(b, r, f"fused {name}")
        scale = float(np.abs(r).max())
        assert np.abs(a - b).max() <= 2e-5 * scale, (name, float(np.abs(a - b).max()), scale)
