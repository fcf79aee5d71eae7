"""Attention dropout: the oracle's Philox restatement and dropout attention
(CPU), and the device generator / fused kernels against them (GPU).

Bars:
  * Philox4x32-10: the published known-answer vectors (Random123's
    kat_vectors for philox4x32 with 10 rounds), bit-exact.
  * device keep-mask (mtx_dropout_keep_philox) vs the oracle's restatement:
    bit-exact, including ragged row lengths, counter offsets that carry into
    the counter's second word, and untouched padding bytes.
  * dropout attention, fp32: |gpu - ref| <= 1e-5 + 1e-4 |ref| against the
    oracle's restatement of the reference sub-graph with attn_drop
    (transformer.py:36-44, layers.py:115-126) on the same mask; bf16: the
    2e-2 bars of the attention tests.
  * MultiHeadAttention in training mode draws its mask where the reference
    does (host RNG): outputs and gradients vs the oracle with the mask
    redrawn from the same seed.
  * C0 GPT training with dropout 0.1 in every Dropout vs the reference's own
    10-step loss curve (tests/golden/c0_train_dropout.npz): the masks of the
    embedding, attention and MLP dropouts come from the same np.random stream
    in the same order; |dloss| <= 1e-4 * loss per step (the C0 curve's bar).
"""
import math
import sys
from pathlib import Path

import numpy as np
import pytest
from devarrays import T, T as _T, full

from oracle import attention as A
from oracle.philox import keep_mask, philox4x32_10

GOLD = Path(__file__).resolve().parent / "golden"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------------------
# CPU: oracle pinning
# ---------------------------------------------------------------------------

KATS = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", KATS)
def test_philox_known_answers(ctr, key, expect):
    got = philox4x32_10([ctr], key)[0]
    assert [int(x) for x in got] == list(expect)


def test_keep_mask_rate_and_stream_continuation():
    m = keep_mask(1000, 1000, 0.1, seed=7)
    rate = m.mean()
    # 1e6 Bernoulli(0.9) draws: sd 3e-4
    assert abs(rate - 0.9) < 2e-3, rate
    # a mask drawn at offset n/4 continues the stream of a longer draw
    a = keep_mask(8, 12, 0.3, seed=9)
    b = keep_mask(4, 12, 0.3, seed=9, offset=4 * 12 // 4)
    np.testing.assert_array_equal(a[4:], b)
    # p = 0 keeps every element except those whose uniform is exactly 0
    assert keep_mask(64, 64, 0.0, seed=1).mean() > 0.999


def test_dropout_attention_oracle_grads_finite_differences():
    rng = np.random.default_rng(31)
    q, k, v, do = (rng.standard_normal((1, 2, 5, 4)) for _ in range(4))
    keep = rng.random((1, 2, 5, 5)) > 0.3
    _, _, dq, dk, dv, _ = A.attention_f64(q, k, v, do, 0.5, True, keep=keep, p_drop=0.3)
    f = lambda: float((A.attention_f64(q, k, v, None, 0.5, True, keep=keep, p_drop=0.3)[0] * do).sum())
    nq, nk, nv = A.numerical_gradient(f, [q, k, v])
    for a, n in ((dq, nq), (dk, nk), (dv, nv)):
        np.testing.assert_allclose(a, n, atol=1e-4, rtol=1e-3)


def test_dropout_reference_flow_matches_f64_and_no_dropout():
    rng = np.random.default_rng(32)
    q, k, v, do = (rng.standard_normal((2, 2, 24, 16), dtype=np.float32) for _ in range(4))
    keep = rng.random((2, 2, 24, 24)) > 0.2
    r = A.reference_attention(q, k, v, do, 0.25, True, keep=keep, p=0.2)
    e = A.attention_f64(q, k, v, do, 0.25, True, keep=keep, p_drop=0.2)
    np.testing.assert_allclose(r[0], e[0], rtol=1e-5, atol=1e-6)
    for a, b in zip(r[1:], (e[2], e[3], e[4])):
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-5)
    # an all-ones mask with p = 0 is the plain sub-graph
    ones = np.ones((2, 2, 24, 24), dtype=np.uint8)
    for a, b in zip(A.reference_attention(q, k, v, do, 0.25, True, keep=ones, p=0.0),
                    A.reference_attention(q, k, v, do, 0.25, True)):
        np.testing.assert_array_equal(a, b)
    # dropped entries carry no gradient to v: zeroing the mask zeroes dV
    zero = np.zeros_like(ones)
    assert not np.any(A.reference_attention(q, k, v, do, 0.25, True, keep=zero, p=0.2)[3])


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,p,seed,offset", [
    (1, 1, 0.5, 0, 0),
    (3, 5, 0.1, 1, 0),
    (7, 33, 0.5, 2**40 + 3, 2**32 - 5),  # counter carries into its second word
    (2 * 4 * 63, 63, 0.9, 99, 17),
    (64 * 6 * 256, 256, 0.1, 12345, 0),  # one C2 layer's attention matrix
])
def test_device_keep_mask_matches_oracle(dev, rows, cols, p, seed, offset):

    from minitorch_amd import _lib as L
    from minitorch_amd import kernels as K

    _say(f"[dropout] philox mask rows={rows} cols={cols} p={p} seed={seed} offset={offset}")
    ld = K.keep_ld(cols) + 4
    out = full((rows, ld), 0xAB, "uint8")
    L.call("mtx_dropout_keep_philox", L.ptr(out), rows, cols, ld, float(p), seed, offset,
           L.stream_handle())
    got = out.numpy()
    np.testing.assert_array_equal(got[:, :cols], keep_mask(rows, cols, p, seed, offset))
    assert np.all(got[:, cols:] == 0xAB), "padding bytes were written"


def _host_keep(rng, B, H, Tq, Tk, p):
    from minitorch_amd import kernels as K

    ld = K.keep_ld(Tk)
    keep = np.zeros((B, H, Tq, ld), dtype=np.uint8)
    keep[..., :Tk] = rng.random((B, H, Tq, Tk)) > p
    return keep


DROP_CASES = [
    # (B, H, Tq, Tk, D, p)
    (1, 1, 1, 1, 64, 0.5),
    (2, 3, 17, 17, 16, 0.1),
    (1, 2, 63, 63, 64, 0.2),
    (2, 2, 130, 130, 32, 0.5),
    (1, 2, 100, 100, 128, 0.1),
    (1, 2, 17, 100, 64, 0.3),  # Tq < Tk: bottom-right causal alignment
]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype_name", ["fp32", "bf16"])
@pytest.mark.parametrize("B,H,Tq,Tk,D,p", DROP_CASES)
def test_fused_dropout_attention_matches_oracle(dev, dtype_name, B, H, Tq, Tk, D, p):

    from minitorch_amd import kernels as K

    _say(f"[dropout] attention {dtype_name} B={B} H={H} Tq={Tq} Tk={Tk} D={D} p={p}")
    rng = np.random.default_rng(4000 + Tq + 7 * Tk + D)
    bf = dtype_name == "bf16"
    sc = 0.5 if bf else 1.0
    q, k, v = (sc * rng.standard_normal((B, H, t, D), dtype=np.float32) for t in (Tq, Tk, Tk))
    do = rng.standard_normal((B, H, Tq, D), dtype=np.float32)
    if bf:
        q, k, v, do = (A.bf16_round(x) for x in (q, k, v, do))
    keep = _host_keep(rng, B, H, Tq, Tk, p)
    tdt = "bfloat16" if bf else "float32"
    tq, tk, tv, tdo = (T(x, tdt) for x in (q, k, v, do))
    tkeep = T(keep, "uint8")
    ks = float(np.float32(1.0 / (1.0 - p)))
    scale = 1.0 / math.sqrt(D)
    o, lse = K.attn_fwd(tq, tk, tv, scale, True, keep=tkeep, keep_scale=ks)
    dq, dk, dv = K.attn_bwd(tq, tk, tv, o, tdo, lse, scale, True, keep=tkeep, keep_scale=ks)
    ref = A.reference_attention(q, k, v, do, scale, True, keep=keep[..., :Tk], p=p)
    for name, got, r in zip(("o", "dq", "dk", "dv"), (o, dq, dk, dv), ref):
        g = got.numpy().astype(np.float64)
        if bf:
            amax = max(float(np.abs(r).max()), 1e-30)
            nmax = float(np.abs(g - r).max()) / amax
            rfro = float(np.linalg.norm(g - r)) / max(float(np.linalg.norm(r)), 1e-30)
            assert nmax <= 2e-2 and rfro <= 2e-2, (name, nmax, rfro)
        else:
            err = np.abs(g - r)
            assert np.all(err <= 1e-5 + 1e-4 * np.abs(r)), (name, float(err.max()))


@pytest.mark.gpu
def test_all_kept_dropout_equals_plain_attention_fp32(dev):
    """keep everything, scale 1: the dropout forward computes the plain
    kernels' values bit for bit (same row-sum order, same products); the
    backward forms dS = P ((dP - delta) + delta - delta) with one extra
    rounding, so its gradients agree to the fp32 bar."""

    from minitorch_amd import kernels as K

    rng = np.random.default_rng(77)
    B, H, T, D = 2, 2, 96, 64
    q, k, v, do = (_T(rng.standard_normal((B, H, T, D), dtype=np.float32)) for _ in range(4))
    ones = full((B, H, T, K.keep_ld(T)), 1, "uint8")
    o1, l1 = K.attn_fwd(q, k, v, 0.125, True)
    o2, l2 = K.attn_fwd(q, k, v, 0.125, True, keep=ones, keep_scale=1.0)
    g1 = K.attn_bwd(q, k, v, o1, do, l1, 0.125, True)
    g2 = K.attn_bwd(q, k, v, o2, do, l2, 0.125, True, keep=ones, keep_scale=1.0)
    assert np.array_equal(o1.numpy(), o2.numpy()) and np.array_equal(l1.numpy(), l2.numpy())
    for a, b in zip(g1, g2):
        a, b = a.numpy(), b.numpy()
        assert np.all(np.abs(a - b) <= 1e-5 + 1e-4 * np.abs(a)), float(np.abs(a - b).max())


@pytest.mark.gpu
def test_mha_training_mode_draws_reference_mask(dev):
    """MultiHeadAttention(dropout=p) in training mode: the host mask is
    np.random.rand(B, H, T, T) > p drawn at the reference's point, so a
    reseeded draw reproduces it; y and all gradients vs the oracle."""
    import minitorch_amd as mt
    from minitorch_amd import functional as F

    F.set_attention_dropout_rng("host")
    rng = np.random.default_rng(51)
    B, T, C, H, p = 3, 29, 48, 3, 0.25
    mha = mt.MultiHeadAttention(C, H, dropout=p)
    mha.train()
    W = {n: (0.2 * rng.standard_normal(t.shape)).astype(np.float32) for n, t in mha.state_dict().items()}
    mha.load_state_dict(W)
    x = rng.standard_normal((B, T, C), dtype=np.float32)
    gy = rng.standard_normal((B, T, C), dtype=np.float32)
    np.random.seed(2024)
    xt = mt.Tensor(x, requires_grad=True)
    y = mha(xt)
    (y * mt.Tensor(gy)).sum().backward()
    np.random.seed(2024)
    keep = np.random.rand(B, H, T, T) > p
    # oracle: projections, attention with the mask, out_proj, in float64
    D = C // H
    lin = lambda a, n: a @ W[f"{n}.weight"].astype(np.float64) + W[f"{n}.bias"]
    heads = lambda a: a.reshape(B, T, H, D).transpose(0, 2, 1, 3)
    x64 = x.astype(np.float64)
    qh, kh, vh = (heads(lin(x64, n)) for n in ("q_proj", "k_proj", "v_proj"))
    do_merged = gy.astype(np.float64) @ W["out_proj.weight"].astype(np.float64).T
    dO = do_merged.reshape(B, T, H, D).transpose(0, 2, 1, 3)
    o, _, dq, dk, dv, _ = A.attention_f64(qh, kh, vh, dO, 1.0 / math.sqrt(D), True, keep=keep, p_drop=p)
    y_ref = lin(o.transpose(0, 2, 1, 3).reshape(B, T, C), "out_proj")
    merge = lambda a: a.transpose(0, 2, 1, 3).reshape(B, T, C)
    dx_ref = sum(merge(g) @ W[f"{n}.weight"].astype(np.float64).T
                 for g, n in ((dq, "q_proj"), (dk, "k_proj"), (dv, "v_proj")))
    yg = y.numpy()
    assert np.all(np.abs(yg - y_ref) <= 1e-5 + 1e-4 * np.abs(y_ref)), np.abs(yg - y_ref).max()
    dxg = xt.grad.numpy()
    assert np.all(np.abs(dxg - dx_ref) <= 1e-5 + 1e-4 * np.abs(dx_ref)), np.abs(dxg - dx_ref).max()


@pytest.mark.gpu
def test_c0_dropout_training_matches_reference_curve(dev):
    import minitorch_amd as mt
    from minitorch_amd import functional as F
    from oracle.gpt import C0, draw_batch, init_params

    g = np.load(GOLD / "c0_train_dropout.npz", allow_pickle=False)
    p, steps = float(g["p"]), int(g["steps"])
    _say(f"[dropout] C0 {steps}-step loss curve with dropout {p} vs reference golden")
    F.set_attention_dropout_rng("host")
    rng = np.random.default_rng(int(g["seed"]))
    model = mt.GPT(C0.vocab, C0.block, C0.n_embd, C0.n_head, C0.n_layer, dropout=p)
    model.load_state_dict(init_params(C0, rng))
    opt = mt.Adam(model.parameters(), lr=3e-4)
    model.train()
    np.random.seed(int(g["dseed"]))
    losses = []
    for _ in range(steps):
        x, y = draw_batch(rng, C0.vocab, int(g["B"]), C0.block)
        logits = model(x)
        Bb, Tt, V = logits.shape
        loss = mt.cross_entropy_loss(logits.reshape(Bb * Tt, V), mt.Tensor(y.reshape(-1)))
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(float(loss))
    rel = np.abs(np.array(losses) - g["losses"]) / g["losses"]
    _say(f"  max relative loss difference {rel.max():.2e}")
    assert np.all(rel <= 1e-4), rel


@pytest.mark.gpu
def test_device_rng_training_is_reproducible(dev):
    """Device-drawn attention masks: a seeded run repeats exactly, and the
    masks change from step to step (the counter offset advances)."""
    import minitorch_amd as mt
    from minitorch_amd import functional as F
    from oracle.gpt import C0, draw_batch, init_params

    def run():
        F.set_attention_dropout_rng("device", seed=5)
        rng = np.random.default_rng(0)
        model = mt.GPT(C0.vocab, C0.block, C0.n_embd, C0.n_head, C0.n_layer, dropout=0.1)
        model.load_state_dict(init_params(C0, rng))
        opt = mt.Adam(model.parameters(), lr=3e-4)
        model.train()
        np.random.seed(3)
        out = []
        for _ in range(3):
            x, y = draw_batch(rng, C0.vocab, 16, C0.block)
            logits = model(x)
            Bb, Tt, V = logits.shape
            loss = mt.cross_entropy_loss(logits.reshape(Bb * Tt, V), mt.Tensor(y.reshape(-1)))
            opt.zero_grad()
            loss.backward()
            opt.step()
            out.append(float(loss))
        return out

    try:
        a, b = run(), run()
        assert a == b
        assert np.all(np.isfinite(a))
    finally:
        F.set_attention_dropout_rng("host")
