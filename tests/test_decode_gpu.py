"""GPU parity of the decode-step attention (mtx_attn_decode) and the device
greedy pick (mtx_argmax_f32).

Decode attention is the reference's attention sub-graph (transformer.py:36-44)
at one query position against L cached keys; the oracle is
oracle.attention.flash_forward (float64 softmax(scale q k^T) v and its
log-sum-exp) on the same keys.  Bars as for the fused kernels: fp32
|gpu - ref| <= 1e-5 + 1e-4 |ref|; bf16 inputs max err <= 2e-2 max|ref| and
relative Frobenius error <= 2e-2.  The greedy pick must equal np.argmax (first
maximum) exactly, and the margin the top-2 difference of np.sort.
"""
import sys

import numpy as np
import pytest
from devarrays import T, T as _T, empty, full

from oracle.attention import bf16_round, flash_forward

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _cache(rng, B, H, Lmax, D, dtype):
    """q (B,H,1,D) and (B,Lmax,H*D) key/value caches with their head views."""

    q = rng.standard_normal((B, H, 1, D), dtype=np.float32)
    kc = rng.standard_normal((B, Lmax, H * D), dtype=np.float32)
    vc = rng.standard_normal((B, Lmax, H * D), dtype=np.float32)
    if dtype == "bfloat16":
        q, kc, vc = (bf16_round(0.5 * x) for x in (q, kc, vc))
    heads = lambda t: t.view(B, Lmax, H, D).transpose(1, 2)
    tq, tk, tv = (T(x, dtype) for x in (q, kc, vc))
    host = lambda x: x.reshape(B, Lmax, H, D).transpose(0, 2, 1, 3)
    return (tq, heads(tk), heads(tv)), (q, host(kc), host(vc))


def _check(got, ref, dtype, name):

    got = got.astype(np.float64)
    if dtype == "float32":
        err = np.abs(got - ref)
        assert np.all(err <= 1e-5 + 1e-4 * np.abs(ref)), (name, float(err.max()))
    else:
        amax = np.abs(ref).max()
        assert np.abs(got - ref).max() <= 2e-2 * amax, (name, float(np.abs(got - ref).max()), amax)
        assert np.linalg.norm(got - ref) <= 2e-2 * np.linalg.norm(ref), name


@pytest.mark.parametrize("dtype_name", ["float32", "bfloat16"])
@pytest.mark.parametrize("D", [16, 64, 128])
def test_decode_matches_oracle_ragged(dev, dtype_name, D):
    from minitorch_amd import kernels as K

    dtype = dtype_name
    B, H, Lmax = 4, 3, 300
    lengths = [1, 137, 256, 300]
    _say(f"[decode] {dtype_name} D={D} B={B} H={H} lengths={lengths}")
    rng = np.random.default_rng(40 + D)
    (tq, tk, tv), (q, k, v) = _cache(rng, B, H, Lmax, D, dtype)
    lens = T(np.array(lengths), "int32")
    lse = empty((B, H))
    o, _ = K.attn_decode(tq, tk, tv, D ** -0.5, lse=lse, lengths=lens)
    o = o.numpy()
    lse = lse.numpy()
    for b, Lb in enumerate(lengths):
        ro, rl = flash_forward(q[b:b + 1], k[b:b + 1, :, :Lb], v[b:b + 1, :, :Lb], D ** -0.5, causal=False)
        _check(o[b:b + 1], ro, dtype, f"o b={b}")
        np.testing.assert_allclose(lse[b], rl[0, :, 0], rtol=1e-4 if dtype == "float32" else 2e-2,
                                   atol=1e-5 if dtype == "float32" else 2e-2)


def test_decode_full_cache_and_empty(dev):
    """No lengths: every sequence uses all L keys (L = 8192, the maximum);
    length 0 gives o = 0 and lse = -inf."""
    from minitorch_amd import kernels as K

    _say("[decode] L=8192 fp32, and a zero length")
    rng = np.random.default_rng(7)
    (tq, tk, tv), (q, k, v) = _cache(rng, 1, 2, 8192, 64, "float32")
    lse = empty((1, 2))
    o, _ = K.attn_decode(tq, tk, tv, 0.125, lse=lse)
    ro, rl = flash_forward(q, k, v, 0.125, causal=False)
    _check(o.numpy(), ro, "float32", "o")
    np.testing.assert_allclose(lse.numpy(), rl[..., 0], rtol=1e-5, atol=1e-5)
    zero = full((1,), 0, "int32")
    o, _ = K.attn_decode(tq, tk, tv, 0.125, lse=lse, lengths=zero)
    assert np.all(o.numpy() == 0) and np.all(np.isneginf(lse.numpy()))


def test_decode_matches_fused_forward_at_last_position(dev):
    """A decode step equals the fused causal forward's last query row."""
    from minitorch_amd import kernels as K

    _say("[decode] vs fused forward, last row")
    rng = np.random.default_rng(11)
    B, H, T, D = 2, 6, 97, 64
    q, k, v = (_T(rng.standard_normal((B, H, T, D), dtype=np.float32)) for _ in range(3))
    o_full, lse_full = K.attn_fwd(q, k, v, 0.125, True)
    lse = empty((B, H))
    o, _ = K.attn_decode(q[:, :, T - 1:T], k, v, 0.125, lse=lse)
    np.testing.assert_allclose(o.numpy(), o_full[:, :, T - 1:T].numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(lse.numpy(), lse_full[:, :, T - 1].numpy(), rtol=1e-5, atol=1e-5)


def test_argmax_matches_numpy(dev):
    from minitorch_amd import kernels as K

    _say("[argmax] rows of 65 and 200 columns, with ties")
    rng = np.random.default_rng(5)
    for cols in (65, 200):
        x = rng.standard_normal((70, cols)).astype(np.float32)
        x[0, 3] = x[0, 40] = 9.0          # tie: first index wins, margin 0
        x[1, -1] = 50.0                   # maximum in the last column
        x[2, :] = 1.0                     # all equal
        x[3, 64 % cols] = x[3, 0] = 7.0   # tie across lanes
        # np.argmax's order past the numbers: the first NaN wins (above
        # +Inf), a row of -Inf picks index 0; margins come out NaN there
        x[4, 10] = x[4, 50] = np.nan
        x[5, :] = -np.inf
        x[6, 7] = np.inf
        x[6, 30] = np.nan
        x[7, 63] = np.inf                 # +Inf in one lane, numbers elsewhere
        t = T(x)
        margin = empty((70,))
        idx, _ = K.argmax_rows(t, margin=margin)
        np.testing.assert_array_equal(idx.numpy(), np.argmax(x, axis=1))
        top2 = np.sort(x, axis=1)[:, -2:]
        with np.errstate(invalid="ignore"):  # -Inf - -Inf and NaN rows: NaN margins
            want = top2[:, 1] - top2[:, 0]
        np.testing.assert_array_equal(margin.numpy(), want)


def _gelu64(x):
    c0, c1 = np.float64(np.float32(np.sqrt(2 / np.pi))), np.float64(np.float32(0.044715))
    return 0.5 * x * (1.0 + np.tanh(c0 * (x + c1 * x ** 3)))


@pytest.mark.parametrize("M,K,N,act,beta", [(64, 384, 1536, 1, 0.0), (37, 384, 384, 0, 1.0),
                                            (5, 100, 70, 1, 0.5), (64, 512, 16, 0, 0.0)])
def test_gemm_step_matches_float64(dev, M, K, N, act, beta):
    """mtx_gemm_step_f32 without cache columns: C = act(A @ B + bias + beta*C)."""
    from minitorch_amd import kernels as Kn

    _say(f"[gemm_step] M={M} K={K} N={N} act={act} beta={beta}")
    rng = np.random.default_rng(M + K + N)
    a = rng.standard_normal((M, K), dtype=np.float32)
    b = (0.05 * rng.standard_normal((K, N))).astype(np.float32)
    bias = rng.standard_normal(N, dtype=np.float32)
    c0 = rng.standard_normal((M, N), dtype=np.float32)
    ta, tb, tbias, tc = (T(x) for x in (a, b, bias, c0))
    Kn.gemm_step(ta, tb, bias=tbias, c=tc, beta=beta, act=act)
    ref = a.astype(np.float64) @ b + bias + beta * c0
    if act:
        ref = _gelu64(ref)
    got = tc.numpy()
    err = np.abs(got - ref)
    assert np.all(err <= 1e-5 + 1e-4 * np.abs(ref)), f"max err {err.max():.3e}"


def test_gemm_step_writes_kv_cache_rows(dev):
    """The q/k/v step projection: q columns to c, k and v columns to cache row
    lengths[m] - 1; rows of sequences with lengths 0 or past T untouched."""
    from minitorch_amd import kernels as Kn

    _say("[gemm_step] kv scatter")
    rng = np.random.default_rng(77)
    B, C, T = 64, 384, 40
    a = rng.standard_normal((B, C), dtype=np.float32)
    w = (0.05 * rng.standard_normal((C, 3 * C))).astype(np.float32)
    bias = rng.standard_normal(3 * C, dtype=np.float32)
    lengths = rng.integers(1, T + 1, B).astype(np.int32)
    lengths[3], lengths[10] = 0, T + 1  # skipped
    kc0 = rng.standard_normal((B, T, C), dtype=np.float32)
    vc0 = rng.standard_normal((B, T, C), dtype=np.float32)
    ta, tw, tb = (_T(x) for x in (a, w, bias))
    tk, tv, tl = _T(kc0), _T(vc0), _T(lengths, "int32")
    q = empty((B, C))
    Kn.gemm_step(ta, tw, bias=tb, c=q, kv=(tk, tv, tl))
    P = a.astype(np.float64) @ w + bias
    tol = lambda r: 1e-5 + 1e-4 * np.abs(r)
    assert np.all(np.abs(q.numpy() - P[:, :C]) <= tol(P[:, :C]))
    kg, vg = tk.numpy(), tv.numpy()
    kref, vref = kc0.copy(), vc0.copy()
    for m in range(B):
        t = lengths[m] - 1
        if 0 <= t < T:
            assert np.all(np.abs(kg[m, t] - P[m, C:2 * C]) <= tol(P[m, C:2 * C])), m
            assert np.all(np.abs(vg[m, t] - P[m, 2 * C:]) <= tol(P[m, 2 * C:])), m
            kref[m, t], vref[m, t] = kg[m, t], vg[m, t]
    assert np.array_equal(kg, kref) and np.array_equal(vg, vref), "rows other than lengths-1 changed"


def test_greedy_pick_matches_argmax_advance_and_records(dev):
    """mtx_greedy_pick_f32 against mtx_argmax_f32 + mtx_decode_advance and
    the host-side record of the pick: cur, the id row lengths[b], the margin
    row lengths[b] - t_base, lengths + 1, pos + 1; rows whose length falls
    outside the buffers skip the record."""
    from minitorch_amd import kernels as Kn

    _say("[greedy_pick]")
    rng = np.random.default_rng(9)
    rows, cols, Tmax, T0, n = 64, 65, 40, 10, 30
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[5, 3] = x[5, 9] = 10.0  # tie: first index
    x[6, 20] = x[6, 2] = np.nan  # a NaN logit: the first NaN (np.argmax), never an out-of-range id
    lengths = rng.integers(T0 + 1, Tmax, rows).astype(np.int32)
    lengths[7] = Tmax + 3     # past the id buffer: no record
    ids0 = rng.integers(0, 65, (Tmax, rows)).astype(np.int64)
    m0 = rng.standard_normal((n, rows)).astype(np.float32)
    tx, cur, ids, mg, tl, pos = _T(x), _T(np.zeros(rows, np.int64), "int64"), _T(ids0, "int64"), _T(m0), \
        _T(lengths, "int32"), _T(np.array([17], np.int64), "int64")
    Kn.greedy_pick(tx, cur, ids, tl, pos, mg, t_base=T0)
    ref_idx, ref_m = np.argmax(x, axis=1), np.sort(x, axis=1)
    ref_m = ref_m[:, -1] - ref_m[:, -2]
    np.testing.assert_array_equal(cur.numpy(), ref_idx)
    want_ids, want_m = ids0.copy(), m0.copy()
    for b in range(rows):
        L = lengths[b]
        if 0 <= L < Tmax:
            want_ids[L, b] = ref_idx[b]
        if 0 <= L - T0 < n:
            want_m[L - T0, b] = ref_m[b]
    np.testing.assert_array_equal(ids.numpy(), want_ids)
    np.testing.assert_array_equal(mg.numpy(), want_m)
    np.testing.assert_array_equal(tl.numpy(), lengths + 1)
    assert int(pos.numpy()[0]) == 18


def test_embedding2_matches_gathers_plus_add(dev):
    """mtx_embedding2_fwd_f32: token rows + position rows in one pass, equal
    bit for bit to the two gathers and the add (one fp32 addition each);
    ib_stride 0 broadcasts one position."""
    from minitorch_amd import kernels as Kn

    _say("[embedding2]")
    rng = np.random.default_rng(10)
    Wt = rng.standard_normal((65, 384)).astype(np.float32)
    Wp = rng.standard_normal((256, 384)).astype(np.float32)
    ia = rng.integers(0, 65, 64)
    ib = rng.integers(0, 256, 64)
    out = empty((64, 384))
    Kn.embedding2_fwd(_T(Wt), _T(ia, "int64"), _T(Wp), _T(ib, "int64"), out)
    np.testing.assert_array_equal(out.numpy(), Wt[ia] + Wp[ib])
    Kn.embedding2_fwd(_T(Wt), _T(ia, "int64"), _T(Wp), _T(np.array([37]), "int64"), out, ib_stride=0)
    np.testing.assert_array_equal(out.numpy(), Wt[ia] + Wp[37])


@pytest.mark.parametrize("C", [384, 64, 1000])
def test_embedding2_ln_matches_embedding2_then_layernorm(dev, C):
    """mtx_embedding2_ln_fwd_f32: the embedding sum and the first LayerNorm
    of a decode step in one launch, bit for bit the two launches'
    (mtx_embedding2_fwd_f32, mtx_layernorm_fwd_f32), and the LayerNorm
    against float64."""
    from minitorch_amd import kernels as Kn
    from oracle.gpt import ln_fwd

    _say(f"[embedding2_ln] C={C}")
    rng = np.random.default_rng(11 + C)
    Wt = rng.standard_normal((65, C)).astype(np.float32)
    Wp = rng.standard_normal((256, C)).astype(np.float32)
    gam = rng.standard_normal(C).astype(np.float32)
    bet = rng.standard_normal(C).astype(np.float32)
    ia = rng.integers(0, 65, 64)
    eps = float(np.float32(1e-5))
    pos = _T(np.array([37]), "int64")
    out, y = empty((64, C)), empty((64, C))
    Kn.embedding2_ln_fwd(_T(Wt), _T(ia, "int64"), _T(Wp), pos, out, _T(gam), _T(bet), eps, y, ib_stride=0)
    out2, y2 = empty((64, C)), empty((64, C))
    Kn.embedding2_fwd(_T(Wt), _T(ia, "int64"), _T(Wp), pos, out2, ib_stride=0)
    Kn.layernorm_fwd(out2, _T(gam), _T(bet), y2, empty((64,)), empty((64,)), eps)
    np.testing.assert_array_equal(out.numpy(), Wt[ia] + Wp[37])
    np.testing.assert_array_equal(y.numpy(), y2.numpy())
    ref = ln_fwd((Wt[ia] + Wp[37]).astype(np.float64), gam.astype(np.float64), bet.astype(np.float64), 1e-5)[0]
    assert np.max(np.abs(y.numpy() - ref)) <= 1e-4 * (1 + np.abs(ref).max())


@pytest.mark.parametrize("rows,K,V", [(64, 384, 65), (5, 64, 65), (64, 1000, 200), (3, 17, 1)])
def test_head_pick_matches_product_then_pick(dev, rows, K, V):
    """mtx_head_pick_f32: the head product and the greedy pick of a decode
    step in one launch.  Logits against float64 (each an fp32 fused
    multiply-add chain); the pick and its bookkeeping against the same
    records computed on the host from float64 logits (the
    rows whose top two float64 logits are within 1e-3 are not compared)."""
    from minitorch_amd import kernels as Kn

    _say(f"[head_pick] rows={rows} K={K} V={V}")
    rng = np.random.default_rng(12 + K)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    w = (rng.standard_normal((K, V)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(V).astype(np.float32)
    logits = x.astype(np.float64) @ w + b
    top = np.argmax(logits, axis=1)
    Tmax, T0, n = 40, 10, 30
    lengths = rng.integers(T0 + 1, Tmax, rows).astype(np.int32)
    ids0 = rng.integers(0, 65, (Tmax, rows)).astype(np.int64)
    m0 = rng.standard_normal((n, rows)).astype(np.float32)
    cur, ids, mg, tl, pos = _T(np.zeros(rows, np.int64), "int64"), _T(ids0, "int64"), _T(m0), \
        _T(lengths, "int32"), _T(np.array([17], np.int64), "int64")
    Kn.head_pick(_T(x), _T(w), _T(b), cur, ids, tl, pos, mg, t_base=T0)
    srt = np.sort(logits, axis=1)
    marg = srt[:, -1] - (srt[:, -2] if V > 1 else -np.inf)
    clear = marg > 1e-3 if V > 1 else np.ones(rows, bool)
    got = cur.numpy()
    np.testing.assert_array_equal(got[clear], top[clear])
    for r in range(rows):
        L = lengths[r]
        if 0 <= L < Tmax:
            assert ids.numpy()[L, r] == got[r]
        if V > 1 and 0 <= L - T0 < n and clear[r]:
            assert abs(mg.numpy()[L - T0, r] - marg[r]) <= 1e-4 * (1 + abs(logits[r]).max())
    np.testing.assert_array_equal(tl.numpy(), lengths + 1)
    assert int(pos.numpy()[0]) == 18


@pytest.mark.parametrize("B,H,D,T,with_bias", [(64, 6, 64, 256, True), (5, 4, 128, 40, True),
                                               (3, 16, 64, 17, False), (7, 8, 128, 300, True)])
def test_qkv_attn_step_matches_projection_then_attention(dev, B, H, D, T, with_bias):
    """mtx_decode_qkv_attn_f32: a decode step's q/k/v projection and
    attention in one launch.  Against float64: the projection P = x @ W + b,
    k and v rows at cache row lengths[b] - 1 (other rows untouched; lengths 0
    and T + 1 write nothing), and softmax(scale q k^T) v over the first
    min(lengths[b], T) rows of the updated cache (fp32 bar 1e-5 + 1e-4|ref|).
    The same step through mtx_gemm_step_f32 + mtx_attn_decode agrees to the
    same bar."""
    from minitorch_amd import kernels as Kn

    _say(f"[qkv_attn] B={B} H={H} D={D} T={T} bias={with_bias}")
    rng = np.random.default_rng(1000 + B + D + T)
    C = H * D
    x = rng.standard_normal((B, C), dtype=np.float32)
    w = (rng.standard_normal((C, 3 * C)) / np.sqrt(C)).astype(np.float32)
    bias = rng.standard_normal(3 * C).astype(np.float32) if with_bias else None
    lengths = rng.integers(1, T + 1, B).astype(np.int32)
    lengths[0] = T
    if B > 2:
        lengths[1], lengths[2] = 0, T + 1
    kc0 = rng.standard_normal((B, T, C), dtype=np.float32)
    vc0 = rng.standard_normal((B, T, C), dtype=np.float32)
    scale = 1.0 / np.sqrt(D)
    tk, tv, tl = _T(kc0), _T(vc0), _T(lengths, "int32")
    out = empty((B, C))
    Kn.qkv_attn_step(_T(x), _T(w), _T(bias) if with_bias else None, tk, tv, tl, H, scale, out)

    P = x.astype(np.float64) @ w + (bias if with_bias else 0.0)
    tol = lambda r: 1e-5 + 1e-4 * np.abs(r)
    kg, vg = tk.numpy(), tv.numpy()
    kref, vref = kc0.astype(np.float64), vc0.astype(np.float64)
    for b in range(B):
        t = lengths[b] - 1
        if 0 <= t < T:
            assert np.all(np.abs(kg[b, t] - P[b, C:2 * C]) <= tol(P[b, C:2 * C])), b
            assert np.all(np.abs(vg[b, t] - P[b, 2 * C:]) <= tol(P[b, 2 * C:])), b
            kref[b, t], vref[b, t] = P[b, C:2 * C], P[b, 2 * C:]
            kc0[b, t], vc0[b, t] = kg[b, t], vg[b, t]
    assert np.array_equal(kg, kc0) and np.array_equal(vg, vc0), "rows other than lengths-1 changed"
    ref = np.zeros((B, C))
    for b in range(B):
        Lb = min(max(int(lengths[b]), 0), T)
        for h in range(H):
            sl = slice(h * D, (h + 1) * D)
            if Lb == 0:
                continue
            s = (kref[b, :Lb, sl] @ P[b, sl]) * scale
            p = np.exp(s - s.max())
            ref[b, sl] = (p / p.sum()) @ vref[b, :Lb, sl]
    got = out.numpy()
    err = np.abs(got - ref)
    assert np.all(err <= tol(ref)), f"max err {err.max():.3e}"

    # the two-launch form of the same step (where mtx_gemm_step_f32 takes it)
    if not Kn.step_fits(B, C):
        return
    tk2, tv2 = _T(tk.numpy()), _T(tv.numpy())
    q = empty((B, C))
    Kn.gemm_step(_T(x), _T(w), bias=_T(bias) if with_bias else None, c=q, kv=(tk2, tv2, tl))
    heads = lambda a: a.view(B, T, H, D).transpose(1, 2)
    o2 = empty((B, 1, H, D))
    Kn.attn_decode(q.view(B, 1, H, D).transpose(1, 2), heads(tk2), heads(tv2), scale,
                   out=o2.transpose(1, 2), lengths=tl)
    got2 = o2.numpy().reshape(B, C)
    assert np.all(np.abs(got - got2) <= tol(got2)), f"vs two launches: {np.abs(got - got2).max():.3e}"


@pytest.mark.parametrize("B,H,D,Khid,T", [(64, 6, 64, 1536, 64), (5, 2, 128, 300, 20), (3, 3, 64, 16, 9)])
def test_pending_update_modes_match_reduce_ln(dev, B, H, D, Khid, T):
    """The deferred second residual add of a decode step: the partial
    products of mtx_gemm_partials_f32, summed with bias and residual inside
    mtx_decode_qkv_attn_f32 (rows written to x_out) and mtx_head_pick_f32,
    then normalised there, give bit for bit what mtx_gemm_ln_f32 (reduce +
    LayerNorm launch) and the normalised-input forms of the two entry points
    give on the same inputs; the partials summed in order on the host match
    float64 within the fp32 dot bound."""
    from minitorch_amd import kernels as Kn

    _say(f"[pending] B={B} H={H} D={D} K={Khid} T={T}")
    rng = np.random.default_rng(5000 + B + Khid)
    C = H * D
    hmid = rng.standard_normal((B, Khid), dtype=np.float32)
    w2 = (rng.standard_normal((Khid, C)) / np.sqrt(Khid)).astype(np.float32)
    b2 = rng.standard_normal(C, dtype=np.float32)
    x0 = rng.standard_normal((B, C), dtype=np.float32)
    gam = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    bet = (0.1 * rng.standard_normal(C)).astype(np.float32)
    eps = float(np.float32(1e-5))
    ws, ks = Kn.gemm_partials(_T(hmid), _T(w2))
    parts = ws.numpy()[:ks * B * C].reshape(ks, B, C)
    ref = hmid.astype(np.float64) @ w2
    assert np.abs(parts.sum(0) - ref).max() <= 1e-5 * np.sqrt(Khid) * (1 + np.abs(ref).max())
    # reference: the reduce + LayerNorm launch on the same product
    xr, yr = _T(x0), empty((B, C))
    Kn.gemm_ln(_T(hmid), _T(w2), xr, _T(gam), _T(bet), eps, yr, bias=_T(b2))

    wq = (rng.standard_normal((C, 3 * C)) / np.sqrt(C)).astype(np.float32)
    bq = rng.standard_normal(3 * C, dtype=np.float32)
    lengths = rng.integers(1, T + 1, B).astype(np.int32)
    kc0 = rng.standard_normal((B, T, C), dtype=np.float32)
    vc0 = rng.standard_normal((B, T, C), dtype=np.float32)
    tl = _T(lengths, "int32")
    scale = 1.0 / np.sqrt(D)
    lnp = (_T(gam), _T(bet), eps)
    # pending mode
    tk1, tv1, o1, xo = _T(kc0), _T(vc0), empty((B, C)), empty((B, C))
    Kn.qkv_attn_step(_T(x0), _T(wq), _T(bq), tk1, tv1, tl, H, scale, o1, pending=(ws, ks, _T(b2)), x_out=xo, ln=lnp)
    # normalised-input mode on gemm_ln's y
    tk2, tv2, o2 = _T(kc0), _T(vc0), empty((B, C))
    Kn.qkv_attn_step(yr, _T(wq), _T(bq), tk2, tv2, tl, H, scale, o2)
    np.testing.assert_array_equal(xo.numpy(), xr.numpy())
    np.testing.assert_array_equal(o1.numpy(), o2.numpy())
    np.testing.assert_array_equal(tk1.numpy(), tk2.numpy())
    np.testing.assert_array_equal(tv1.numpy(), tv2.numpy())
    # raw-row mode without pending partials: LayerNorm of x itself
    o3 = empty((B, C))
    Kn.qkv_attn_step(xr, _T(wq), _T(bq), _T(kc0), _T(vc0), tl, H, scale, o3, ln=lnp)
    np.testing.assert_array_equal(o3.numpy(), o2.numpy())

    # the head with the pick
    V = 65
    wh = (rng.standard_normal((C, V)) / np.sqrt(C)).astype(np.float32)
    bh = rng.standard_normal(V, dtype=np.float32)
    Tm = 40
    res = []
    for mode in ("pending", "normalised"):
        cur = _T(np.zeros(B, np.int64), "int64")
        ids = _T(np.zeros((Tm, B), np.int64), "int64")
        mg = _T(np.zeros((Tm, B), np.float32))
        tl2 = _T(np.full(B, 5, np.int32), "int32")
        if mode == "pending":
            Kn.head_pick(_T(x0), _T(wh), _T(bh), cur, ids, tl2, None, mg, pending=(ws, ks, _T(b2)), ln=lnp)
        else:
            Kn.head_pick(yr, _T(wh), _T(bh), cur, ids, tl2, None, mg)
        res.append((cur.numpy(), ids.numpy(), mg.numpy()))
    for a, b in zip(*res):
        np.testing.assert_array_equal(a, b)
