"""Pinning the CPU oracle (no GPU).

Each oracle function is checked against something other than itself:
  * golden vectors written by the reference itself (tests/golden/*.npz, made
    by tests/golden/make_golden.py);
  * float64 central differences -- the reference's grad_check method
    (grad_check.py:5-38, atol 1e-4 / rtol 1e-3);
  * an independent library: torch CPU in float64 (scaled_dot_product_attention,
    layer_norm, tanh-GELU, cross_entropy);
  * invariants / closed forms: softmax rows sum to 1, exact zeros above the
    causal diagonal, causality, T=1 gives O=V, identical keys give uniform
    weights, sum_j dS_ij = 0, Adam's first step = -lr*g/(|g|+eps).
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as A
from oracle import gpt as G

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


# ---------------------------------------------------------------------------
# attention sub-graph
# ---------------------------------------------------------------------------

def test_attention_matches_reference_golden():
    g = load("attn_subgraph.npz")
    out, dq, dk, dv = A.reference_attention(g["q"], g["k"], g["v"], g["do"], None, True)
    assert out.dtype == np.float64 and str(g["out_dtype"]) == "float64"
    assert dq.dtype == np.float32 and str(g["dq_dtype"]) == "float32"
    np.testing.assert_allclose(out, g["out"], rtol=1e-13, atol=1e-15)
    for got, ref in ((dq, g["dq"]), (dk, g["dk"]), (dv, g["dv"])):
        np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)


def test_attention_f64_matches_torch_sdpa():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    q, k, v, do = (rng.standard_normal((2, 3, 19, 8)) for _ in range(4))
    out, p, dq, dk, dv, ds = A.attention_f64(q, k, v, do, 0.3, True)
    tq, tk, tv = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    to = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True, scale=0.3)
    to.backward(torch.tensor(do))
    np.testing.assert_allclose(out, to.detach().numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dq, tq.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dk, tk.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv, tv.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_attention_f64_finite_differences():
    rng = np.random.default_rng(12)
    q, k, v = (rng.standard_normal((1, 2, 5, 4)) for _ in range(3))
    do = rng.standard_normal((1, 2, 5, 4))
    _, _, dq, dk, dv, _ = A.attention_f64(q, k, v, do, 0.5, True)
    f = lambda: float((A.attention_f64(q, k, v, None, 0.5, True)[0] * do).sum())
    nq, nk, nv = A.numerical_gradient(f, [q, k, v])
    for a, n in ((dq, nq), (dk, nk), (dv, nv)):
        np.testing.assert_allclose(a, n, atol=1e-4, rtol=1e-3)


def test_reference_flow_close_to_f64():
    rng = np.random.default_rng(13)
    q, k, v, do = (rng.standard_normal((2, 2, 40, 16), dtype=np.float32) for _ in range(4))
    r = A.reference_attention(q, k, v, do, 0.25, True)
    e = A.attention_f64(q, k, v, do, 0.25, True)
    np.testing.assert_allclose(r[0], e[0], rtol=1e-5, atol=1e-6)
    for a, b in zip(r[1:], (e[2], e[3], e[4])):
        np.testing.assert_allclose(a, b, rtol=1e-4, atol=1e-5)


def test_flash_form_equals_direct_form():
    rng = np.random.default_rng(14)
    q, k, v, do = (rng.standard_normal((2, 3, 33, 8)) for _ in range(4))
    o, p, dq, dk, dv, _ = A.attention_f64(q, k, v, do, 0.35, True)
    fo, lse = A.flash_forward(q, k, v, 0.35, True)
    np.testing.assert_allclose(fo, o, rtol=1e-13, atol=1e-14)
    s = (q @ np.swapaxes(k, -1, -2)) * 0.35
    s = np.where(A.causal_mask(33, 33), -np.inf, s)
    np.testing.assert_allclose(lse, np.log(np.exp(s).sum(-1)), rtol=1e-13)
    fq, fk, fv = A.flash_backward(q, k, v, fo, do, lse, 0.35, True)
    for a, b in ((fq, dq), (fk, dk), (fv, dv)):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


def test_attention_invariants():
    rng = np.random.default_rng(15)
    B, H, T, D = 2, 2, 12, 4
    q, k, v, do = (rng.standard_normal((B, H, T, D)) for _ in range(4))
    o, p, dq, dk, dv, ds = A.attention_f64(q, k, v, do, 0.5, True)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-14)
    assert np.all(p[..., A.causal_mask(T, T)] == 0.0)
    np.testing.assert_allclose(ds.sum(-1), 0.0, atol=1e-13)
    # causality: changing inputs at positions > t leaves O[:t+1] unchanged
    t = 5
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    q2[..., t + 1:, :] += 1.0
    k2[..., t + 1:, :] -= 2.0
    v2[..., t + 1:, :] *= 3.0
    o2 = A.attention_f64(q2, k2, v2, None, 0.5, True)[0]
    np.testing.assert_array_equal(o2[..., : t + 1, :], o[..., : t + 1, :])
    # T=1 gives O = V
    o1 = A.attention_f64(q[..., :1, :], k[..., :1, :], v[..., :1, :], None, 0.5, True)[0]
    np.testing.assert_allclose(o1, v[..., :1, :], rtol=1e-15)
    # identical keys: uniform weights over the visible prefix
    kk = np.broadcast_to(k[..., :1, :], k.shape).copy()
    pu = A.attention_f64(q, kk, v, None, 0.5, True)[1]
    expect = np.tril(np.ones((T, T))) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(pu[0, 0], expect, rtol=1e-13)
    # the reference's -1e9 additive mask gives exact zeros too
    _, _, _, _ = A.reference_attention(q.astype(np.float32), k.astype(np.float32),
                                       v.astype(np.float32), None, 0.5, True)


def test_bottom_right_causal_rule():
    m = A.causal_mask(3, 5)
    assert m.tolist() == [[False, False, False, True, True],
                          [False, False, False, False, True],
                          [False, False, False, False, False]]
    assert np.array_equal(A.causal_mask(4, 4), np.triu(np.ones((4, 4)), 1) != 0)


def test_bf16_round_is_rne():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e-3], dtype=np.float32)
    r = A.bf16_round(x)
    torch = pytest.importorskip("torch")
    np.testing.assert_array_equal(r, torch.tensor(x).to(torch.bfloat16).float().numpy())


# ---------------------------------------------------------------------------
# GPT pieces vs torch float64 and finite differences
# ---------------------------------------------------------------------------

def test_bf16_emulation_pinned():
    """attention_bf16_emulated (the bf16 kernels' rounding points): without
    rounding it is attention_f64 to float64 precision for causal, non-causal
    and Tq < Tk, so its structure (every product, the lazy reference and its
    tile weights, delta, the scale) is the reference mathematics; with
    rounding the error against float64 is nonzero and within the size bf16
    rounding of P, dS and the pre-scaled operand gives (2^-9 relative per
    rounding)."""
    rng = np.random.default_rng(21)
    for (B, H, Tq, Tk, D, causal) in [(1, 2, 150, 150, 64, True), (2, 1, 70, 70, 16, False),
                                      (1, 1, 40, 130, 32, True)]:
        q = A.bf16_round(0.5 * rng.standard_normal((B, H, Tq, D), dtype=np.float32))
        k, v = (A.bf16_round(0.5 * rng.standard_normal((B, H, Tk, D), dtype=np.float32)) for _ in range(2))
        do = A.bf16_round(rng.standard_normal((B, H, Tq, D), dtype=np.float32))
        ref = A.attention_f64(q, k, v, do, 1 / np.sqrt(D), causal)
        _, lse = A.flash_forward(q, k, v, 1 / np.sqrt(D), causal)
        refs = (ref[0], lse, ref[2], ref[3], ref[4])
        for onepass in (False, True):
            exact = A.attention_bf16_emulated(q, k, v, do, 1 / np.sqrt(D), causal, rounding=False,
                                              onepass=onepass)
            rounded = A.attention_bf16_emulated(q, k, v, do, 1 / np.sqrt(D), causal, onepass=onepass)
            for name, e, r, b in zip(("out", "lse", "dq", "dk", "dv"), exact, refs, rounded):
                amax = np.abs(r).max()
                assert np.abs(e - r).max() <= 1e-12 * amax, (name, onepass)
                rel = np.linalg.norm(b - r) / np.linalg.norm(r)
                assert 1e-6 < rel < 1e-2, (name, onepass, rel)
        # the two dQ forms round different scores (K*c vs Q*c): their dQ
        # differ by a bf16-rounding-sized amount, not by a structural one
        two = A.attention_bf16_emulated(q, k, v, do, 1 / np.sqrt(D), causal)[2]
        one = A.attention_bf16_emulated(q, k, v, do, 1 / np.sqrt(D), causal, onepass=True)[2]
        d = np.linalg.norm(one - two) / np.linalg.norm(refs[2])
        assert 0 < d < 1e-2, d
    # a tile reference that moves (scores growing along the keys) still
    # reproduces the exact softmax: the tile weights exp2(m_t - m_final)
    T = 200
    q = np.ones((1, 1, T, 16), np.float32)
    k = (np.arange(T, dtype=np.float32)[:, None] * np.ones((1, 16), np.float32) / 8)[None, None]
    v = A.bf16_round(rng.standard_normal((1, 1, T, 16), dtype=np.float32))
    do = A.bf16_round(rng.standard_normal((1, 1, T, 16), dtype=np.float32))
    mt = A._lazy_reference(np.where(A.causal_mask(T, T), -np.inf,
                                    (q[0, 0].astype(np.float64) * 0.25 * A.LOG2E) @ k[0, 0].T.astype(np.float64)),
                           64, 8.0)
    assert len(np.unique(mt[-1])) > 1  # the last row's reference moved
    e = A.attention_bf16_emulated(q, k, v, do, 0.25, True, rounding=False)
    r = A.attention_f64(q, k, v, do, 0.25, True)
    assert np.abs(e[0] - r[0]).max() <= 1e-12 * np.abs(r[0]).max()


def test_layernorm_gelu_ce_match_torch_f64():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    x = rng.standard_normal((3, 5, 16))
    gam = rng.standard_normal(16).astype(np.float32)
    bet = rng.standard_normal(16).astype(np.float32)
    y, _ = G.ln_fwd(x, gam, bet)
    ty = torch.nn.functional.layer_norm(torch.tensor(x), (16,), torch.tensor(gam, dtype=torch.float64),
                                        torch.tensor(bet, dtype=torch.float64), eps=float(np.float32(1e-5)))
    np.testing.assert_allclose(y, ty.numpy(), rtol=1e-12, atol=1e-12)
    gl, _ = G.gelu_fwd(x)
    tg = torch.nn.functional.gelu(torch.tensor(x), approximate="tanh")
    np.testing.assert_allclose(gl, tg.numpy(), rtol=1e-6, atol=1e-7)  # float32-rounded constants
    logits = rng.standard_normal((10, 7))
    labels = rng.integers(0, 7, 10)
    loss, _ = G.cross_entropy(logits, labels)
    tl = torch.nn.functional.cross_entropy(torch.tensor(logits), torch.tensor(labels))
    assert abs(float(loss) - float(tl)) < 1e-13


def _tiny_cfg():
    return G.GPTConfig(vocab=7, block=4, n_embd=8, n_head=2, n_layer=1)


def test_gpt_grads_finite_differences():
    cfg = _tiny_cfg()
    rng = np.random.default_rng(22)
    P32 = G.init_params(cfg, rng)
    # non-trivial LayerNorm params and biases so every gradient path is exercised
    P = {k: (v.astype(np.float64) + 0.1 * rng.standard_normal(v.shape)) for k, v in P32.items()}
    x, y = G.draw_batch(rng, cfg.vocab, 2, cfg.block)
    _, _, grads = G.gpt_loss_and_grads(P, x, y, cfg)
    names = list(P)
    f = lambda: float(G.cross_entropy(G.gpt_forward(P, x, cfg).reshape(-1, cfg.vocab), y.reshape(-1))[0])
    num = A.numerical_gradient(f, [P[n] for n in names])
    for n, ng in zip(names, num):
        np.testing.assert_allclose(grads[n], ng, atol=1e-4, rtol=1e-3, err_msg=n)


def test_adam_first_step_closed_form():
    rng = np.random.default_rng(23)
    p = {"w": rng.standard_normal(50).astype(np.float32)}
    g = {"w": rng.standard_normal(50).astype(np.float32)}
    p0 = p["w"].copy()
    opt = G.Adam(p, lr=3e-4)
    opt.step(p, g)
    expect = p0 - 3e-4 * g["w"] / (np.abs(g["w"]) + 1e-8)
    np.testing.assert_allclose(p["w"], expect, rtol=0, atol=2e-7)


# ---------------------------------------------------------------------------
# whole-model golden vectors from the reference
# ---------------------------------------------------------------------------

def test_mha_module_matches_reference_golden():
    g = load("mha_module.npz")
    cfg = G.GPTConfig(vocab=1, block=17, n_embd=48, n_head=3, n_layer=1)
    P = {"attn." + k[len("param."):]: g[k] for k in g.files if k.startswith("param.")}
    y, cache = G.mha_fwd(g["x"], P, "attn.", cfg)
    assert y.dtype == np.float64
    np.testing.assert_allclose(y, g["y"], rtol=1e-10, atol=1e-12)
    hx = G.Holder(g["x"].shape, np.float32)
    GR = {k: G.Holder(v.shape, np.float32) for k, v in P.items()}
    G.mha_bwd(g["dy"].astype(np.float64), cache, hx, GR, "attn.", cfg)
    np.testing.assert_allclose(hx.g, g["dx"], rtol=1e-5, atol=1e-6)
    for k in P:
        np.testing.assert_allclose(GR[k].g, g["grad." + k[len("attn."):]], rtol=1e-5, atol=1e-6, err_msg=k)


def test_c0_step0_matches_reference_golden():
    g = load("c0_train.npz")
    cfg = G.C0
    rng = np.random.default_rng(int(g["seed"]))
    P = G.init_params(cfg, rng)
    x, y = G.draw_batch(rng, cfg.vocab, int(g["B"]), cfg.block)
    loss, logits, grads = G.gpt_loss_and_grads(P, x, y, cfg)
    assert str(g["logits_dtype"]) == str(logits.dtype) == "float64"
    np.testing.assert_allclose(logits[0], g["logits0_row0"], rtol=1e-9, atol=1e-12)
    assert abs(loss - g["losses"][0]) < 1e-12
    names = list(g["names"])
    norms = np.array([np.sqrt((grads[n].astype(np.float64) ** 2).sum()) for n in names])
    # k_proj biases have mathematically zero gradients (softmax shift invariance):
    # their norms are roundoff (~1e-11..1e-20), hence the absolute floor
    np.testing.assert_allclose(norms, g["grad_norms"], rtol=1e-6, atol=1e-10)
    for n in names:
        if f"grad.{n}" in g.files:
            np.testing.assert_allclose(grads[n], g[f"grad.{n}"], rtol=1e-5, atol=1e-8, err_msg=n)
        else:
            ix = g[f"gidx.{n}"]
            np.testing.assert_allclose(grads[n][tuple(ix.T)], g[f"gval.{n}"], rtol=1e-5, atol=1e-8, err_msg=n)


def test_c0_loss_curve_matches_reference_golden():
    g = load("c0_train.npz")
    losses, _, _ = G.train(G.C0, int(g["seed"]), int(g["B"]), int(g["steps"]), record_grads_at=())
    np.testing.assert_allclose(losses, g["losses"], rtol=1e-9, atol=0)


def test_greedy_matches_reference_golden():
    g = load("greedy_c0.npz")
    rng = np.random.default_rng(int(g["seed"]))
    P = G.init_params(G.C0, rng)
    prompts = rng.integers(0, G.C0.vocab, g["prompts"].shape)
    np.testing.assert_array_equal(prompts, g["prompts"])
    toks, margins = G.greedy_generate(P, G.C0, prompts, g["tokens"].shape[1] - prompts.shape[1])
    np.testing.assert_array_equal(toks, g["tokens"])
    np.testing.assert_allclose(margins, g["margins"], rtol=1e-6, atol=1e-12)


@pytest.mark.skipif(not (GOLD / "c2_train.npz").exists(), reason="C2 golden curve not generated")
def test_c2_step0_matches_reference_golden():
    g = load("c2_train.npz")
    cfg = G.C2
    rng = np.random.default_rng(int(g["seed"]))
    P = G.init_params(cfg, rng)
    x, y = G.draw_batch(rng, cfg.vocab, int(g["B"]), cfg.block)
    loss, logits, grads = G.gpt_loss_and_grads(P, x, y, cfg)
    np.testing.assert_allclose(logits[0], g["logits0_row0"], rtol=1e-9, atol=1e-12)
    assert abs(loss - g["losses"][0]) < 1e-11
    names = list(g["names"])
    norms = np.array([np.sqrt((grads[n].astype(np.float64) ** 2).sum()) for n in names])
    np.testing.assert_allclose(norms, g["grad_norms"], rtol=1e-5, atol=1e-10)


def test_cached_greedy_matches_reference_golden():
    """The KV-cache form of greedy decoding gives the reference's tokens."""
    g = load("greedy_c0.npz")
    rng = np.random.default_rng(int(g["seed"]))
    P = G.init_params(G.C0, rng)
    prompts = rng.integers(0, G.C0.vocab, g["prompts"].shape)
    toks, margins = G.greedy_generate_cached(P, G.C0, prompts, g["tokens"].shape[1] - prompts.shape[1])
    np.testing.assert_array_equal(toks, g["tokens"])
    # block 0 runs in float32 (the reference's dtype flow); a (B*T, C) product
    # and a (B, 1, C) product round differently, so margins agree to ~1e-7
    np.testing.assert_allclose(margins, g["margins"], rtol=0, atol=2e-6)


def test_c4_oracle_fixture_matches_reference_fixture():
    """Config C4 at full size (the C2 model, 64 prompts x 32 ids, +224
    greedy tokens): the oracle's cached decoding (c4_greedy.npz,
    make_c4_fixture.py) gives the tokens the reference's own GPT.forward +
    argmax loop wrote (c4_greedy_ref.npz, make_golden.py --only-c4), all
    224 steps; margins agree to float32 rounding."""
    r = load("c4_greedy_ref.npz")
    o = load("c4_greedy.npz")
    assert int(r["steps"]) == 224 and r["tokens"].shape == (64, 256)
    np.testing.assert_array_equal(o["prompts"], r["prompts"])
    np.testing.assert_array_equal(o["tokens"], r["tokens"])
    np.testing.assert_allclose(o["margins"], r["margins"], rtol=0, atol=2e-6)


def test_cached_greedy_equals_recompute_on_larger_model():
    cfg = G.GPTConfig(vocab=65, block=48, n_embd=96, n_head=6, n_layer=3)
    rng = np.random.default_rng(31)
    P = G.init_params(cfg, rng)
    prompts = rng.integers(0, cfg.vocab, (3, 8))
    a, ma = G.greedy_generate(P, cfg, prompts, 20)
    b, mb = G.greedy_generate_cached(P, cfg, prompts, 20)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_allclose(ma, mb, rtol=0, atol=2e-6)
