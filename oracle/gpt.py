"""NumPy restatement of the reference GPT training step and greedy decoding.

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; never by the product.

The reference builds the GPT (transformer.py:49-104) from autograd Tensor ops
and differentiates it with a generic closure walk (tensor.py:453-477).  This
module computes the same forward and the same gradients with an explicit,
hand-derived backward pass, keeping the reference's dtype behaviour under
NumPy 2, which it pins (uv.lock):

  * Python scalars that become Tensors are float32 0-d arrays
    (tensor.py:55-56): the 2 of ``diff ** 2``, LayerNorm's eps, GELU's
    constants, CE's ``-1`` and ``/ N``.  They do not promote.
  * The attention scale ``1.0 / np.sqrt(D)`` is an np.float64 scalar kept at
    float64 (tensor.py:53-54), so from the first attention score on every
    activation is float64 (float32 * float64 0-d array -> float64).
  * Gradient holders take the dtype of their tensor (``_accum_grad``,
    tensor.py:29-33), so a float64 gradient reaching a float32 node is rounded
    to float32 there; all parameter gradients are float32.
  * Broadcast gradients are reduced with the reference's _sum_to_shape order
    (tensor.py:20-26).

Where one tensor feeds several ops the reference adds the contributions in
the iteration order of a Python set (tensor.py:472), which is not fixed; here
the order is fixed, so results agree with the reference to rounding, not bit
for bit.  Pinned by tests/golden/ fixtures written by the reference itself.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np

F32 = np.float32
F64 = np.float64


def c32(x):
    """A Python scalar as the reference turns it into a Tensor: a float32 0-d
    array (tensor.py:55-56)."""
    return np.array(x, dtype=F32)


def sum_to_shape(g, shape):
    """tensor.py:20-26: reduce a broadcast gradient to `shape` (leading axes
    first, then size-1 axes)."""
    while g.ndim > len(shape):
        g = g.sum(axis=0)
    for i, (gd, sd) in enumerate(zip(g.shape, shape)):
        if sd == 1 and gd != 1:
            g = g.sum(axis=i, keepdims=True)
    return g.reshape(shape)


class Holder:
    """A gradient accumulator with the reference's _accum_grad semantics
    (tensor.py:29-33): zero-initialised in the tensor's dtype, then += ."""

    __slots__ = ("g", "dtype", "shape")

    def __init__(self, shape, dtype):
        self.g = None
        self.shape = tuple(shape)
        self.dtype = dtype

    def add(self, grad):
        if self.g is None:
            self.g = np.zeros(self.shape, dtype=self.dtype)
        self.g += grad
        return self


@dataclass(frozen=True)
class GPTConfig:
    vocab: int
    block: int
    n_embd: int
    n_head: int
    n_layer: int

    @property
    def head_dim(self):
        return self.n_embd // self.n_head


C0 = GPTConfig(65, 32, 64, 4, 2)
C2 = GPTConfig(65, 256, 384, 6, 6)


# ---------------------------------------------------------------------------
# parameters: names and order of Module.state_dict (module.py:81-94)
# ---------------------------------------------------------------------------

def param_spec(cfg: GPTConfig):
    """[(name, shape, kind)] in the reference's state_dict()/parameters() order
    (GPT.__init__ attribute order, transformer.py:70-78; block 52-61; MHA
    18-24; Linear weight (in, out) then bias, layers.py:22-26; LayerNorm gamma
    then beta, layers.py:77-78).  kind: 'w' (N(0,0.02) init), 'b' (zeros),
    'g' (ones)."""
    C, V = cfg.n_embd, cfg.vocab
    spec = [("tok_emb.weight", (V, C), "w"), ("pos_emb.weight", (cfg.block, C), "w")]
    for i in range(cfg.n_layer):
        p = f"blocks.{i}."
        spec += [(p + "ln1.gamma", (C,), "g"), (p + "ln1.beta", (C,), "b")]
        for proj in ("q_proj", "k_proj", "v_proj", "out_proj"):
            spec += [(p + f"attn.{proj}.weight", (C, C), "w"), (p + f"attn.{proj}.bias", (C,), "b")]
        spec += [(p + "ln2.gamma", (C,), "g"), (p + "ln2.beta", (C,), "b")]
        spec += [(p + "mlp.layers.0.weight", (C, 4 * C), "w"), (p + "mlp.layers.0.bias", (4 * C,), "b"),
                 (p + "mlp.layers.2.weight", (4 * C, C), "w"), (p + "mlp.layers.2.bias", (C,), "b")]
    spec += [("ln_f.gamma", (C,), "g"), ("ln_f.beta", (C,), "b"),
             ("lm_head.weight", (C, V), "w"), ("lm_head.bias", (V,), "b")]
    return spec


def init_params(cfg: GPTConfig, rng: np.random.Generator):
    """The harness initialisation: in state_dict order, every Linear weight and
    Embedding table ~ N(0, 0.02) (drawn as float64 standard normals * 0.02,
    then cast to float32), biases 0, LayerNorm gamma 1 / beta 0."""
    out = OrderedDict()
    for name, shape, kind in param_spec(cfg):
        if kind == "w":
            out[name] = (rng.standard_normal(shape) * 0.02).astype(F32)
        elif kind == "b":
            out[name] = np.zeros(shape, dtype=F32)
        else:
            out[name] = np.ones(shape, dtype=F32)
    return out


def draw_batch(rng: np.random.Generator, vocab: int, B: int, T: int):
    """One training batch: ids ~ U[0, vocab) of shape (B, T+1); x = ids[:, :-1],
    y = ids[:, 1:]."""
    ids = rng.integers(0, vocab, (B, T + 1))
    return ids[:, :-1], ids[:, 1:]


# ---------------------------------------------------------------------------
# forward pieces (each returns output and a cache for its backward)
# ---------------------------------------------------------------------------

def ln_fwd(x, gamma, beta, eps=1e-5):
    """LayerNorm composite, layers.py:82-86."""
    mean = x.mean(axis=-1, keepdims=True)
    diff = x - mean
    sq = diff ** c32(2)
    var = sq.mean(axis=-1, keepdims=True)
    ve = var + c32(eps)
    std = ve ** c32(0.5)
    xh = diff / std
    y1 = xh * gamma
    y = y1 + beta
    return y, (x, diff, ve, std, xh, y1, gamma, beta)


def ln_bwd(gy, cache, gx: Holder, ggamma: Holder, gbeta: Holder):
    """Backward of ln_fwd: the closures of add, mul, div, pow, add, mean, pow,
    sub, mean (tensor.py) in reverse order."""
    x, diff, ve, std, xh, y1, gamma, beta = cache
    C = x.shape[-1]
    gbeta.add(sum_to_shape(gy, beta.shape))
    g_y1 = Holder(y1.shape, y1.dtype).add(sum_to_shape(gy, y1.shape)).g
    ggamma.add(sum_to_shape(xh * g_y1, gamma.shape))
    g_xh = Holder(xh.shape, xh.dtype).add(sum_to_shape(gamma * g_y1, xh.shape)).g
    h_diff = Holder(diff.shape, diff.dtype)
    h_diff.add(sum_to_shape(g_xh / std, diff.shape))
    g_std = Holder(std.shape, std.dtype).add(sum_to_shape(-diff / (std ** 2) * g_xh, std.shape)).g
    half = c32(0.5)
    g_ve = Holder(ve.shape, ve.dtype).add(sum_to_shape(half * (ve ** (half - c32(1.0))) * g_std, ve.shape)).g
    g_var = g_ve  # var + eps: identity into var's holder (same dtype)
    g_sq = np.broadcast_to(g_var, diff.shape) / C
    two = c32(2)
    h_diff.add(sum_to_shape(two * (diff ** (two - c32(1))) * g_sq, diff.shape))
    g_diff = h_diff.g
    gx.add(sum_to_shape(g_diff, x.shape))
    g_mean = Holder(diff.shape[:-1] + (1,), x.dtype).add(sum_to_shape(-g_diff, diff.shape[:-1] + (1,))).g
    gx.add(np.broadcast_to(g_mean, x.shape) / C)


GELU_C = math.sqrt(2.0 / math.pi)


def gelu_fwd(x):
    """functional.py:54-59 (tanh approximation, constants as float32 Tensors)."""
    x3 = x ** c32(3)
    t1 = x3 * c32(0.044715)
    t2 = x + t1
    inner = t2 * c32(GELU_C)
    th = np.tanh(inner)
    t3 = th + c32(1.0)
    h = x * c32(0.5)
    return h * t3, (x, th, t3, h)


def gelu_bwd(gy, cache, gx: Holder):
    x, th, t3, h = cache
    g_h = t3 * gy
    g_t3 = h * gy
    g_inner = (1.0 - th ** 2) * g_t3  # functional.py:46
    g_t2 = c32(GELU_C) * g_inner
    g_x3 = c32(0.044715) * g_t2
    three = c32(3)
    gx.add(g_t2)
    gx.add(three * (x ** (three - c32(1))) * g_x3)
    gx.add(c32(0.5) * g_h)


def linear_fwd(x, W, b):
    """layers.py:31-37: x @ W + b, W stored (in, out)."""
    t = x @ W
    return t + b, (x, t, W, b)


def linear_bwd(gy, cache, gx: Holder, gW: Holder, gb: Holder):
    x, t, W, b = cache
    gb.add(sum_to_shape(gy, b.shape))
    g_t = Holder(t.shape, t.dtype).add(sum_to_shape(gy, t.shape)).g
    gx.add(sum_to_shape(g_t @ W.swapaxes(-1, -2), x.shape))
    gW.add(sum_to_shape(x.swapaxes(-1, -2) @ g_t, W.shape))


def attn_core_fwd(qh, kh, vh):
    """transformer.py:36-44: scores, scale (np.float64), -1e9 mask, softmax,
    attn @ v.  qh/kh/vh: (B, H, T, D) in the projection dtype."""
    D, T = qh.shape[-1], qh.shape[-2]
    sc = np.asarray(np.float64(1.0 / np.sqrt(D)))
    kt = kh.swapaxes(-1, -2)
    qk = qh @ kt
    s = qk * sc
    mask = (np.triu(np.ones((T, T), dtype=F32), k=1) * -1e9).astype(F32)
    s2 = s + mask
    shifted = s2 - s2.max(axis=-1, keepdims=True)
    e = np.exp(shifted)
    p = e / e.sum(axis=-1, keepdims=True)
    o = p @ vh
    return o, (qh, kh, vh, qk, sc, p)


def attn_core_bwd(go, cache, gq: Holder, gk: Holder, gv: Holder):
    qh, kh, vh, qk, sc, p = cache
    g_p = go @ vh.swapaxes(-1, -2)
    gv.add(sum_to_shape(p.swapaxes(-1, -2) @ go, vh.shape))
    g = g_p * p
    g_s2 = g - p * g.sum(axis=-1, keepdims=True)  # functional.py:69-73
    g_qk = Holder(qk.shape, qk.dtype).add(sum_to_shape(sc * g_s2, qk.shape)).g
    gq.add(sum_to_shape(g_qk @ kh, qh.shape))
    g_kt = qh.swapaxes(-1, -2) @ g_qk
    gk.add(g_kt.swapaxes(-1, -2))


def mha_fwd(x, P, pre, cfg):
    B, T, C = x.shape
    H, D = cfg.n_head, cfg.head_dim
    q, cq = linear_fwd(x, P[pre + "q_proj.weight"], P[pre + "q_proj.bias"])
    k, ck = linear_fwd(x, P[pre + "k_proj.weight"], P[pre + "k_proj.bias"])
    v, cv = linear_fwd(x, P[pre + "v_proj.weight"], P[pre + "v_proj.bias"])
    split = lambda t: t.reshape(B, T, H, D).transpose(0, 2, 1, 3)
    o, ca = attn_core_fwd(split(q), split(k), split(v))
    om = o.transpose(0, 2, 1, 3).reshape(B, T, C)
    y, co = linear_fwd(om, P[pre + "out_proj.weight"], P[pre + "out_proj.bias"])
    return y, (cq, ck, cv, ca, co, q.dtype, o.dtype)


def mha_bwd(gy, cache, gx: Holder, G, pre, cfg):
    cq, ck, cv, ca, co, qdt, odt = cache
    B, T, C = gy.shape
    H, D = cfg.n_head, cfg.head_dim
    h_om = Holder((B, T, C), odt)
    linear_bwd(gy, co, h_om, G[pre + "out_proj.weight"], G[pre + "out_proj.bias"])
    go = h_om.g.reshape(B, T, H, D).transpose(0, 2, 1, 3)
    hq, hk, hv = (Holder((B, H, T, D), qdt) for _ in range(3))
    attn_core_bwd(go, ca, hq, hk, hv)
    merge = lambda g: g.transpose(0, 2, 1, 3).reshape(B, T, C)
    for h_, c_, name in ((hq, cq, "q_proj"), (hk, ck, "k_proj"), (hv, cv, "v_proj")):
        g_lin = Holder((B, T, C), qdt).add(merge(h_.g)).g
        linear_bwd(g_lin, c_, gx, G[pre + name + ".weight"], G[pre + name + ".bias"])


# ---------------------------------------------------------------------------
# model
# ---------------------------------------------------------------------------

def gpt_forward(P, idx, cfg: GPTConfig, keep=False):
    """GPT.forward, transformer.py:80-91 (dropout p=0 -> identity,
    layers.py:118-119).  Returns logits (B, T, V) and, if keep, the caches."""
    idx = np.asarray(idx)
    B, T = idx.shape
    assert T <= cfg.block
    tok = P["tok_emb.weight"][idx]
    pos = P["pos_emb.weight"][np.arange(T)]
    x = tok + pos
    caches = []
    for i in range(cfg.n_layer):
        pre = f"blocks.{i}."
        h, c1 = ln_fwd(x, P[pre + "ln1.gamma"], P[pre + "ln1.beta"])
        a, cm = mha_fwd(h, P, pre + "attn.", cfg)
        x_mid = x + a
        h2, c2 = ln_fwd(x_mid, P[pre + "ln2.gamma"], P[pre + "ln2.beta"])
        f1, cf1 = linear_fwd(h2, P[pre + "mlp.layers.0.weight"], P[pre + "mlp.layers.0.bias"])
        gl, cg = gelu_fwd(f1)
        f2, cf2 = linear_fwd(gl, P[pre + "mlp.layers.2.weight"], P[pre + "mlp.layers.2.bias"])
        x_out = x_mid + f2
        if keep:
            caches.append((x.dtype, x.shape, c1, cm, x_mid.dtype, c2, cf1, cg, cf2, x_out.dtype))
        x = x_out
    xf, cfn = ln_fwd(x, P["ln_f.gamma"], P["ln_f.beta"])
    logits, clm = linear_fwd(xf, P["lm_head.weight"], P["lm_head.bias"])
    if keep:
        return logits, (idx, tok.dtype, caches, cfn, clm, x.dtype)
    return logits


def cross_entropy(logits2d, labels):
    """loss.py:17-27 with log_softmax functional.py:81-86: host one-hot,
    log_softmax over axis 1, (-logp * onehot).sum() / N.  Returns (loss, cache)."""
    N, V = logits2d.shape
    onehot = np.zeros((N, V), dtype=F32)
    onehot[np.arange(N), labels.astype(np.int64)] = 1.0
    shifted = logits2d - logits2d.max(axis=1, keepdims=True)
    lse = np.log(np.exp(shifted).sum(axis=1, keepdims=True))
    logp = shifted - lse
    neg = logp * c32(-1)
    loss = (neg * onehot).sum() / c32(N)
    return loss, (logp, onehot, N)


def cross_entropy_bwd(cache):
    """Gradient of the CE loss w.r.t. the 2-D logits (the closures of div, sum,
    mul, neg-mul and log_softmax, functional.py:88-92)."""
    logp, onehot, N = cache
    g_sum = np.ones((), dtype=logp.dtype) / c32(N)
    g_prod = np.broadcast_to(g_sum, logp.shape)
    g_neg = onehot * g_prod
    g_logp = Holder(logp.shape, logp.dtype).add(c32(-1) * g_neg).g
    s = np.exp(logp)
    return g_logp - s * g_logp.sum(axis=1, keepdims=True)


def gpt_loss_and_grads(P, x, y, cfg: GPTConfig):
    """One forward + backward: returns (loss as Python float, logits, grads)
    with grads an OrderedDict of float32 arrays in parameter order."""
    logits, (idx, tdt, caches, cfn, clm, xdt) = gpt_forward(P, x, cfg, keep=True)
    B, T, V = logits.shape
    loss, cce = cross_entropy(logits.reshape(B * T, V), np.asarray(y).reshape(-1))
    G = OrderedDict((name, Holder(P[name].shape, F32)) for name, _, _ in param_spec(cfg))
    g_logits = Holder((B * T, V), logits.dtype).add(cross_entropy_bwd(cce)).g.reshape(B, T, V)
    C = cfg.n_embd
    h_xf = Holder((B, T, C), xdt)
    linear_bwd(g_logits, clm, h_xf, G["lm_head.weight"], G["lm_head.bias"])
    h_x = Holder((B, T, C), xdt)
    ln_bwd(h_xf.g, cfn, h_x, G["ln_f.gamma"], G["ln_f.beta"])
    g = h_x.g
    for i in reversed(range(cfg.n_layer)):
        pre = f"blocks.{i}."
        x_dt, x_shape, c1, cm, mid_dt, c2, cf1, cg, cf2, out_dt = caches[i]
        # x_out = x_mid + f2
        h_mid = Holder(x_shape, mid_dt).add(sum_to_shape(g, x_shape))
        g_f2 = Holder(x_shape, out_dt).add(sum_to_shape(g, x_shape)).g
        h_gl = Holder(cg[0].shape, cg[0].dtype)
        linear_bwd(g_f2, cf2, h_gl, G[pre + "mlp.layers.2.weight"], G[pre + "mlp.layers.2.bias"])
        h_f1 = Holder(cg[0].shape, cg[0].dtype)
        gelu_bwd(h_gl.g, cg, h_f1)
        h_h2 = Holder(x_shape, mid_dt)
        linear_bwd(h_f1.g, cf1, h_h2, G[pre + "mlp.layers.0.weight"], G[pre + "mlp.layers.0.bias"])
        ln_bwd(h_h2.g, c2, h_mid, G[pre + "ln2.gamma"], G[pre + "ln2.beta"])
        # x_mid = x + a
        g_mid = h_mid.g
        h_xin = Holder(x_shape, x_dt).add(sum_to_shape(g_mid, x_shape))
        g_a = Holder(x_shape, mid_dt).add(sum_to_shape(g_mid, x_shape)).g
        h_h = Holder(x_shape, c1[0].dtype)
        mha_bwd(g_a, cm, h_h, G, pre + "attn.", cfg)
        ln_bwd(h_h.g, c1, h_xin, G[pre + "ln1.gamma"], G[pre + "ln1.beta"])
        g = h_xin.g
    # x0 = tok + pos; tok = W_tok[idx] (np.add.at scatter, tensor.py:380-382)
    T_ = idx.shape[1]
    g_tok = Holder((B, T_, C), tdt).add(sum_to_shape(g, (B, T_, C))).g
    g_pos = Holder((T_, C), tdt).add(sum_to_shape(g, (T_, C))).g
    gw = np.zeros_like(P["tok_emb.weight"])
    np.add.at(gw, idx, g_tok)
    G["tok_emb.weight"].add(gw)
    gp = np.zeros_like(P["pos_emb.weight"])
    np.add.at(gp, np.arange(T_), g_pos)
    G["pos_emb.weight"].add(gp)
    grads = OrderedDict((k, h.g if h.g is not None else np.zeros(h.shape, F32)) for k, h in G.items())
    return float(loss), logits, grads


class Adam:
    """optim.py:37-59 (bias-corrected Adam, weight decay 0)."""

    def __init__(self, params, lr=3e-4, betas=(0.9, 0.999), eps=1e-8):
        self.lr, (self.b1, self.b2), self.eps = lr, betas, eps
        self.t = 0
        self.m = OrderedDict((k, np.zeros_like(v)) for k, v in params.items())
        self.v = OrderedDict((k, np.zeros_like(v)) for k, v in params.items())

    def step(self, params, grads):
        self.t += 1
        for k, p in params.items():
            g = grads[k].copy()
            self.m[k] = self.b1 * self.m[k] + (1 - self.b1) * g
            self.v[k] = self.b2 * self.v[k] + (1 - self.b2) * (g * g)
            m_hat = self.m[k] / (1 - self.b1 ** self.t)
            v_hat = self.v[k] / (1 - self.b2 ** self.t)
            p -= self.lr * m_hat / (np.sqrt(v_hat) + self.eps)


def train(cfg: GPTConfig, seed: int, B: int, steps: int, lr=3e-4, record_grads_at=(0,)):
    """The harness training loop (char_transformer.py:70-77 order: forward ->
    CE -> zero_grad -> backward -> Adam step) on seeded synthetic batches:
    rng = default_rng(seed); weights from init_params(cfg, rng); then each step
    draws its batch with draw_batch(rng, ...).  Returns (losses, grads_at,
    params) with grads_at {step: grads}."""
    rng = np.random.default_rng(seed)
    P = init_params(cfg, rng)
    opt = Adam(P, lr=lr)
    losses, grads_at = [], {}
    for it in range(steps):
        x, y = draw_batch(rng, cfg.vocab, B, cfg.block)
        loss, _, G = gpt_loss_and_grads(P, x, y, cfg)
        losses.append(loss)
        if it in record_grads_at:
            grads_at[it] = G
        opt.step(P, G)
    return losses, grads_at, P


def greedy_generate(P, cfg: GPTConfig, prompts, n_new):
    """Greedy variant of GPT.generate (transformer.py:93-104): crop to the block
    size, full forward, argmax (first maximum, np.argmax) of the last
    position's logits.  Returns (ids (B, T0 + n_new), top-2 margins (B, n_new))."""
    idx = np.asarray(prompts)
    margins = []
    for _ in range(n_new):
        cond = idx[:, -cfg.block:]
        logits = gpt_forward(P, cond, cfg)[:, -1, :]
        nxt = np.argmax(logits, axis=-1)
        top2 = np.sort(logits, axis=-1)[:, -2:]
        margins.append(top2[:, 1] - top2[:, 0])
        idx = np.concatenate([idx, nxt[:, None]], axis=1)
    return idx, np.stack(margins, axis=1)


def greedy_generate_cached(P, cfg: GPTConfig, prompts, n_new):
    """greedy_generate computed incrementally: a prefill forward over the
    prompt that keeps each layer's k/v, then one-token steps attending to the
    cached k/v.  The same per-row arithmetic as the full recompute (attention
    of one query over its prefix, same dtype flow), so the argmax sequence is
    the reference's up to last-bit summation-order differences; pinned against
    greedy_generate (itself pinned by the reference's tokens)."""
    idx = np.asarray(prompts)
    B, T0 = idx.shape
    H, D = cfg.n_head, cfg.head_dim
    cache = [[None, None] for _ in range(cfg.n_layer)]
    margins = []

    def run(tokens, t0):
        T = tokens.shape[1]
        x = P["tok_emb.weight"][tokens] + P["pos_emb.weight"][np.arange(t0, t0 + T)]
        for i in range(cfg.n_layer):
            pre = f"blocks.{i}."
            h, _ = ln_fwd(x, P[pre + "ln1.gamma"], P[pre + "ln1.beta"])
            a = pre + "attn."
            q, _ = linear_fwd(h, P[a + "q_proj.weight"], P[a + "q_proj.bias"])
            k, _ = linear_fwd(h, P[a + "k_proj.weight"], P[a + "k_proj.bias"])
            v, _ = linear_fwd(h, P[a + "v_proj.weight"], P[a + "v_proj.bias"])
            split = lambda t: t.reshape(B, T, H, D).transpose(0, 2, 1, 3)
            kc = split(k) if cache[i][0] is None else np.concatenate([cache[i][0], split(k)], axis=2)
            vc = split(v) if cache[i][1] is None else np.concatenate([cache[i][1], split(v)], axis=2)
            cache[i] = [kc, vc]
            qh = split(q)
            sc = np.asarray(np.float64(1.0 / np.sqrt(D)))
            s = (qh @ kc.swapaxes(-1, -2)) * sc
            Tk = kc.shape[2]
            mask = (np.triu(np.ones((T, Tk), dtype=F32), k=1 + (Tk - T)) * -1e9).astype(F32)
            s = s + mask
            e = np.exp(s - s.max(axis=-1, keepdims=True))
            p = e / e.sum(axis=-1, keepdims=True)
            o = (p @ vc).transpose(0, 2, 1, 3).reshape(B, T, cfg.n_embd)
            y, _ = linear_fwd(o, P[a + "out_proj.weight"], P[a + "out_proj.bias"])
            x = x + y
            h2, _ = ln_fwd(x, P[pre + "ln2.gamma"], P[pre + "ln2.beta"])
            f1, _ = linear_fwd(h2, P[pre + "mlp.layers.0.weight"], P[pre + "mlp.layers.0.bias"])
            gl, _ = gelu_fwd(f1)
            f2, _ = linear_fwd(gl, P[pre + "mlp.layers.2.weight"], P[pre + "mlp.layers.2.bias"])
            x = x + f2
        xf, _ = ln_fwd(x, P["ln_f.gamma"], P["ln_f.beta"])
        logits, _ = linear_fwd(xf[:, -1:, :], P["lm_head.weight"], P["lm_head.bias"])
        return logits[:, 0, :]

    t0, cur = 0, idx
    for _ in range(n_new):
        logits = run(cur, t0)
        nxt = np.argmax(logits, axis=-1)
        top2 = np.sort(logits, axis=-1)[:, -2:]
        margins.append(top2[:, 1] - top2[:, 0])
        t0 += cur.shape[1]
        idx = np.concatenate([idx, nxt[:, None]], axis=1)
        cur = nxt[:, None]
    return idx, np.stack(margins, axis=1)
