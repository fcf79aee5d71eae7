"""GPT on the device (the reference's transformer.py:14-104).

``MultiHeadAttention`` keeps the reference's constructor, attributes,
state_dict names and forward contract; its score/mask/softmax/value block
(transformer.py:36-44) is the fused ``F.causal_attention`` kernel, fed with
the strided (B, H, T, D) views that ``_split_heads`` makes.
"""
from __future__ import annotations

import math

import numpy as np

from . import device as dev
from . import functional as F
from .device import DeviceArray
from .layers import Dropout, Embedding, GELU, LayerNorm, Linear
from .module import Module, Sequential
from .tensor import Tensor, no_grad


# decode steps leave each block's second residual add to the next launch that
# reads the rows (TransformerBlock.forward_step_deferred) where the size
# limits allow; False keeps one reduce launch per block (forward_step)
_DEFERRED_STEP = True
# greedy decode steps run as one persistent launch each (mtx_decode_step_f32)
# where the model fits its limits; False keeps the multi-launch step above
_PERSISTENT_STEP = True


def _linear_into(x, lin, out):
    """out += x @ W + b, in place (inference only: no graph node)."""
    from .linalg import bmm

    bmm(x.data.t, lin.weight.data.t, out.data.t, beta=1.0, bias=lin.bias.data.t)
    return out


def _linear_ln_into(x, lin, out, ln):
    """out += x @ W + b in place, then (out, ln(out)); for one-token rows the
    normalisation is done by the launch that finishes the product
    (mtx_gemm_ln_f32).  Inference only: no graph nodes."""
    from . import kernels as K

    B, T, Cin = x.shape
    C = lin.weight.shape[1]
    if T == 1 and K.gemm_ln_fits(B, Cin, C):
        y = dev.empty((B, 1, C))
        K.gemm_ln(x.data.t.reshape(B, Cin), lin.weight.data.t, out.data.t.view(B, C), ln.gamma.data.t,
                  ln.beta.data.t, float(np.float32(ln.eps)), y.t.view(B, C), bias=lin.bias.data.t)
        return out, Tensor(y)
    _linear_into(x, lin, out)
    return out, ln(out)


class MultiHeadAttention(Module):
    def __init__(self, n_embd, n_head, dropout=0.0):
        super().__init__()
        assert n_embd % n_head == 0, "n_embd must be divisible by n_head"
        self.n_head = n_head
        self.head_dim = n_embd // n_head
        self.q_proj = Linear(n_embd, n_embd)
        self.k_proj = Linear(n_embd, n_embd)
        self.v_proj = Linear(n_embd, n_embd)
        self.out_proj = Linear(n_embd, n_embd)
        self.attn_drop = Dropout(dropout)
        self._qkv = None  # fused q/k/v projection for decode steps (fuse_qkv)

    def _split_heads(self, x, B, T):
        # (B, T, C) -> (B, n_head, T, head_dim), a strided view
        return x.reshape(B, T, self.n_head, self.head_dim).transpose(1, 2)

    def forward(self, x, residual=None):
        """Causal self-attention of x (transformer.py:36-44).  With `residual`
        (shaped like x) the result is residual + attention(x), the add done in
        the output projection's GEMM epilogue."""
        B, T, C = x.shape
        drop = {}
        if self.attn_drop.p > 0.0 and self.attn_drop._training:
            # attn_drop (transformer.py:43) inside the fused kernel: the mask
            # is drawn where the reference draws it (no other draw happens
            # between the projections and the softmax)
            keep, ks = F.attention_keep_mask((B, self.n_head, T, T), self.attn_drop.p)
            drop = {"keep": keep, "keep_scale": ks}
        scale = 1.0 / math.sqrt(self.head_dim)
        projs = (self.q_proj, self.k_proj, self.v_proj)
        if all(p.bias is not None for p in projs):
            # the three projections as one packed GEMM; attention reads the
            # heads from the packed tensor and writes its gradient there
            qkv = F.linear_qkv(x, *projs)
            out = F.causal_attention_packed(qkv, self.n_head, scale=scale, **drop)
        else:
            q, k, v = (self._split_heads(p(x), B, T) for p in projs)
            out = F.causal_attention(q, k, v, scale=scale, **drop)
        out = out.transpose(1, 2).reshape(B, T, C)
        if residual is not None:
            return F.linear(out, self.out_proj.weight, self.out_proj.bias, residual=residual)
        return self.out_proj(out)


    def forward_cached(self, x, cache, t0, residual=None, fused=False):
        """Inference-only step over positions [t0, t0 + T) of x (B, T, C):
        keys/values of these positions are written into cache = (k, v), each a
        (B, Tmax, C) DeviceArray, and attention runs against cache[:, :t0 + T]
        (bottom-right causal: query i sees keys <= t0 + i).  fused: the three
        projections as one GEMM over the fused q/k/v weight, which the caller
        has just refreshed (fuse_qkv).  With `residual` (shaped like x) the result is residual +
        attention(x), the add in the output projection's epilogue (same
        values as the separate add)."""
        from . import kernels as K

        B, T, C = x.shape
        H, D = self.n_head, self.head_dim
        rows = B * T
        if fused:
            W, b = self._qkv
            qkv = dev.empty((B, T, 3 * C))
            K.gemm(x.data.t.reshape(rows, C), W.data.t, qkv.t.view(rows, 3 * C), bias=b.data.t)
            q_t, k_t, v_t = qkv.t[:, :, :C], qkv.t[:, :, C:2 * C], qkv.t[:, :, 2 * C:]
        else:
            q_t, k_t, v_t = (p(x).data.t for p in (self.q_proj, self.k_proj, self.v_proj))
        kc, vc = cache
        K.ewise("COPY", kc.t[:, t0:t0 + T, :], k_t)
        K.ewise("COPY", vc.t[:, t0:t0 + T, :], v_t)
        Tk = t0 + T
        heads = lambda t: t.view(t.shape[0], t.shape[1], H, D).transpose(1, 2)
        qh = heads(q_t)
        kh = heads(kc.t[:, :Tk, :])
        vh = heads(vc.t[:, :Tk, :])
        out = dev.empty((B, T, H, D))
        if T == 1:  # one new token: the decode kernel (reads the cache once)
            K.attn_decode(qh, kh, vh, 1.0 / math.sqrt(D), out=out.t.transpose(1, 2))
        else:
            K.attn_fwd(qh, kh, vh, 1.0 / math.sqrt(D), True, out=out.t.transpose(1, 2))
        o = Tensor(out.reshape(B, T, C))
        if residual is None:
            return self.out_proj(o)
        y = dev.empty((B, T, C))
        K.gemm(o.data.t.reshape(rows, C), self.out_proj.weight.data.t, y.t.view(rows, C),
               bias=self.out_proj.bias.data.t if self.out_proj.bias is not None else None,
               act=K.GEMM_ACT_ADD, aux=residual.data.t.reshape(rows, C))
        return Tensor(y)


    def forward_step(self, x, cache, lengths, residual=None, ln=None):
        """One-token decode step whose positions live in device memory, so a
        recorded step replays unchanged: x (B, 1, C); this token's key/value
        go to cache row lengths[b] - 1 and attention runs over each
        sequence's first lengths[b] cached keys: one launch for both
        (mtx_decode_qkv_attn_f32) within its size limits, else the q/k/v
        GEMM writing the caches itself (mtx_gemm_step_f32, or
        mtx_kv_append_f32 past its limits) and mtx_attn_decode.
        With `residual` (B, 1, C) the output projection is accumulated into it
        in place (the block's residual add folded into the GEMM) and it is
        returned; with `ln` as well (the LayerNorm that reads the residual
        next), (residual, ln(residual)) is returned, the normalisation done
        with the projection (mtx_gemm_ln_f32)."""
        from . import kernels as K

        B, T, C = x.shape
        assert T == 1, "forward_step takes one token per sequence"
        H, D = self.n_head, self.head_dim
        if self._qkv is None:
            self.fuse_qkv()
        kc, vc = cache
        if K.qkv_attn_fits(H, D, kc.shape[1]):
            # one launch: the projection of this head's q, k, v (k and v into
            # the caches) and its attention (mtx_decode_qkv_attn_f32)
            out = dev.empty((B, 1, C))
            W, b = self._qkv
            K.qkv_attn_step(x.data.t.reshape(B, C), W.data.t, b.data.t, kc.t, vc.t, lengths, H,
                            1.0 / math.sqrt(D), out.t.view(B, C))
            return self._project_out(out, B, C, residual, ln)
        if K.step_fits(B, C):
            # one launch: q to its buffer, k and v straight into the caches
            q = dev.empty((B, 1, C)).t
            W, b = self._qkv
            K.gemm_step(x.data.t.reshape(B, C), W.data.t, bias=b.data.t, c=q.view(B, C),
                        kv=(kc.t, vc.t, lengths))
        else:
            qkv = F.linear(x, *self._qkv).data.t  # (B, 1, 3C): [q | k | v]
            q, k, v = qkv[..., :C], qkv[..., C:2 * C], qkv[..., 2 * C:]
            K.kv_append(k, kc.t, lengths)
            K.kv_append(v, vc.t, lengths)
        heads = lambda t: t.unflatten(2, (H, D)).transpose(1, 2)
        out = dev.empty((B, 1, H, D))
        K.attn_decode(heads(q), heads(kc.t), heads(vc.t), 1.0 / math.sqrt(D),
                      out=out.t.transpose(1, 2), lengths=lengths)
        return self._project_out(out.reshape(B, 1, C), B, C, residual, ln)

    def _project_out(self, out, B, C, residual, ln):
        """The output projection of a decode step's attention rows out (B, 1, C)."""
        if residual is not None:
            if ln is not None:
                return _linear_ln_into(Tensor(out), self.out_proj, residual, ln)
            return _linear_into(Tensor(out), self.out_proj, residual)
        return self.out_proj(Tensor(out))

    def fuse_qkv(self):
        """Concatenate the q/k/v projections into one (C, 3C) weight and (3C,)
        bias for decode steps (one GEMM instead of three).  A snapshot: call
        again after the weights change (generate_greedy does, per call).  The
        buffers are kept and refilled, so their addresses stay the same."""
        from . import kernels as K

        lins = (self.q_proj, self.k_proj, self.v_proj)
        Cin, C = self.q_proj.weight.shape
        if self._qkv is not None and tuple(self._qkv[0].shape) == (Cin, 3 * C):
            W, b = self._qkv[0].data, self._qkv[1].data
        else:
            W = dev.empty((Cin, 3 * C))
            b = dev.empty((3 * C,))
        K.pack3([p.weight.data.t.contiguous() for p in lins], W.t)
        K.pack3([p.bias.data.t.contiguous().view(1, C) for p in lins], b.t.view(1, 3 * C))
        self._qkv = (Tensor(W), Tensor(b))


class TransformerBlock(Module):
    """Pre-norm block: x + attn(ln1(x)), then x + mlp(ln2(x))."""

    def __init__(self, n_embd, n_head, dropout=0.0):
        super().__init__()
        self.ln1 = LayerNorm(n_embd)
        self.attn = MultiHeadAttention(n_embd, n_head, dropout)
        self.ln2 = LayerNorm(n_embd)
        self.mlp = Sequential(
            Linear(n_embd, 4 * n_embd),
            GELU(),
            Linear(4 * n_embd, n_embd),
            Dropout(dropout),
        )

    def forward(self, x):
        # the residual adds (transformer.py:64-65) happen in the epilogues of
        # the output projection and of fc2 (when the MLP's dropout is off)
        x = self.attn(self.ln1(x), residual=x)
        fc1, act, fc2, drop = self.mlp.layers
        if (isinstance(fc1, Linear) and isinstance(act, GELU) and isinstance(fc2, Linear)
                and fc1.bias is not None and fc2.bias is not None):
            # Linear -> GELU -> Linear as one node (GELU in the GEMM epilogues)
            if isinstance(drop, Dropout) and (not drop._training or drop.p == 0.0):
                x = F.mlp_gelu(self.ln2(x), fc1, fc2, residual=x)
            else:
                x = x + drop(F.mlp_gelu(self.ln2(x), fc1, fc2))
        else:
            x = x + self.mlp(self.ln2(x))
        return x

    def forward_cached(self, x, cache, t0, fused=False):
        """Inference-only forward over positions [t0, t0 + T) with the
        attention's keys and values cached: the residual adds in the GEMM
        epilogues of the output projection and fc2, fc1's GELU in its own
        epilogue (no pre-activation kept), the values of the layer-by-layer
        composition.  fused: the attention's q/k/v projections as one GEMM
        over its fused weight, refreshed by the caller (attn.fuse_qkv)."""
        from . import kernels as K

        fc1, act, fc2, drop = self.mlp.layers
        if not (isinstance(fc1, Linear) and isinstance(act, GELU) and isinstance(fc2, Linear)
                and fc1.bias is not None and fc2.bias is not None
                and (not drop._training or drop.p == 0.0)):
            x = x + self.attn.forward_cached(self.ln1(x), cache, t0, fused=fused)
            return x + self.mlp(self.ln2(x))
        x = self.attn.forward_cached(self.ln1(x), cache, t0, residual=x, fused=fused)
        B, T, C = x.shape
        rows, Hd = B * T, fc1.weight.shape[1]
        h = dev.empty((rows, Hd))
        K.gemm(self.ln2(x).data.t.reshape(rows, C), fc1.weight.data.t, h.t, bias=fc1.bias.data.t,
               act=K.GEMM_ACT_GELU)
        y = dev.empty((B, T, C))
        K.gemm(h.t, fc2.weight.data.t, y.t.view(rows, C), bias=fc2.bias.data.t, act=K.GEMM_ACT_ADD,
               aux=x.data.t.reshape(rows, C))
        return Tensor(y)

    def forward_step(self, x, cache, lengths, ln_in=None, next_ln=None):
        """Decode step (no autograd): x is updated in place, both residual
        adds folded into the out_proj / second MLP GEMMs (beta = 1), and
        ln2 done by the launch that finishes the output projection.
        ln_in: this block's ln1(x) when the caller already has it.  With
        next_ln (the LayerNorm that reads x next: the following block's ln1
        or ln_f) the step returns (x, next_ln(x)), the normalisation again
        done with the second MLP product; otherwise it returns x."""
        fc1, act, fc2, drop = self.mlp.layers
        if drop._training and drop.p > 0.0:
            raise NotImplementedError("decode steps run without dropout (use model.eval() or p = 0)")
        from . import kernels as K

        _, h_in = self.attn.forward_step(self.ln1(x) if ln_in is None else ln_in, cache, lengths, residual=x,
                                         ln=self.ln2)
        B, _, C = x.shape
        if K.step_fits(B, C) and isinstance(act, GELU):
            # fc1 with its GELU in one launch
            h = Tensor(dev.empty((B, 1, fc1.weight.shape[1])))
            K.gemm_step(h_in.data.t.reshape(B, C), fc1.weight.data.t, bias=fc1.bias.data.t,
                        c=h.data.t.view(B, -1), act=K.ACT_GELU)
        else:
            h = act(fc1(h_in))
        if next_ln is None:
            return _linear_into(h, fc2, x)
        return _linear_ln_into(h, fc2, x, next_ln)


    def deferred_step_fits(self, B, Tmax):
        """Whether forward_step_deferred takes B sequences with caches of Tmax
        rows (the size limits of its four launches)."""
        from . import kernels as K

        fc1, act, fc2, drop = self.mlp.layers
        C = self.ln1.gamma.shape[0]
        H = self.attn.n_head
        hid = fc1.weight.shape[1]
        return (isinstance(act, GELU) and not (drop._training and drop.p > 0.0)
                and K.qkv_attn_fits(H, C // H, Tmax) and C <= 1024
                and K.gemm_ln_fits(B, C, C) and K.step_fits(B, C) and K.gemm_ln_fits(B, hid, C))

    def forward_step_deferred(self, X, xi, pending, cache, lengths):
        """Decode step with the block's second residual add left pending: X is
        a pair of (B, 1, C) residual buffers, X[xi] the current one.  With
        pending = (partial products, count, bias) of the previous block's
        second MLP product, the q/k/v + attention launch adds them to X[xi]
        into X[1 - xi] (mtx_decode_qkv_attn_f32, which also applies ln1);
        out_proj adds its result into that buffer and applies ln2
        (mtx_gemm_ln_f32); fc1 with GELU (mtx_gemm_step_f32); fc2 only
        writes its partial products (mtx_gemm_partials_f32).  Returns the
        index of the buffer that now holds x and this block's pending update
        (the next block's launch, or the head's, adds it)."""
        from . import kernels as K

        fc1, act, fc2, drop = self.mlp.layers
        attn = self.attn
        if attn._qkv is None:
            attn.fuse_qkv()
        B, _, C = X[xi].shape
        H = attn.n_head
        kc, vc = cache
        cur = xi if pending is None else 1 - xi
        out = dev.empty((B, 1, C))
        W, b = attn._qkv
        K.qkv_attn_step(X[xi].t.view(B, C), W.data.t, b.data.t, kc.t, vc.t, lengths, H,
                        1.0 / math.sqrt(C // H), out.t.view(B, C), pending=pending,
                        x_out=X[cur].t.view(B, C) if pending is not None else None,
                        ln=(self.ln1.gamma.data.t, self.ln1.beta.data.t, float(np.float32(self.ln1.eps))))
        _, h_in = _linear_ln_into(Tensor(out), attn.out_proj, Tensor(X[cur]), self.ln2)
        h = dev.empty((B, 1, fc1.weight.shape[1]))
        K.gemm_step(h_in.data.t.reshape(B, C), fc1.weight.data.t, bias=fc1.bias.data.t, c=h.t.view(B, -1),
                    act=K.ACT_GELU)
        ws, ks = K.gemm_partials(h.t.view(B, -1), fc2.weight.data.t)
        return cur, (ws, ks, fc2.bias.data.t)


class GPT(Module):
    def __init__(self, vocab_size, block_size, n_embd=64, n_head=4, n_layer=2, dropout=0.0):
        super().__init__()
        self.block_size = block_size
        self.tok_emb = Embedding(vocab_size, n_embd)
        self.pos_emb = Embedding(block_size, n_embd)
        self.drop = Dropout(dropout)
        self.blocks = [TransformerBlock(n_embd, n_head, dropout) for _ in range(n_layer)]
        self.ln_f = LayerNorm(n_embd)
        self.lm_head = Linear(n_embd, vocab_size)

    def init_weights(self, rng, std=0.02):
        """Harness initialisation used by the benchmark configurations: in
        state_dict order, every Linear weight and Embedding table ~ N(0, std)
        (float64 standard normals * std, cast to float32), biases 0, LayerNorm
        gamma 1 / beta 0.  `rng` is a numpy Generator."""
        state = {}
        for name, arr in self.state_dict().items():
            if name.endswith(".gamma"):
                state[name] = np.ones(arr.shape, np.float32)
            elif name.endswith(".beta") or name.endswith(".bias"):
                state[name] = np.zeros(arr.shape, np.float32)
            else:
                state[name] = (rng.standard_normal(arr.shape) * std).astype(np.float32)
        self.load_state_dict(state)
        return self

    def _positions(self, T):
        cache = self.__dict__.setdefault("_pos_ids", {})
        if T not in cache:
            cache[T] = dev.index_array(np.arange(T))
        return cache[T]

    def forward(self, idx):
        """idx: (B, T) token ids, host ints or a device int64 DeviceArray."""
        if not isinstance(idx, DeviceArray):
            idx = np.asarray(idx)
        B, T = idx.shape
        assert T <= self.block_size, f"sequence length {T} exceeds block_size {self.block_size}"
        tok = self.tok_emb(idx)
        pos = self.pos_emb(self._positions(T))
        x = self.drop(tok + pos)
        for block in self.blocks:
            x = block(x)
        x = self.ln_f(x)
        return self.lm_head(x)

    def generate_greedy(self, idx, max_new_tokens, return_margins=False, graph=True):
        """Greedy decoding: argmax (first maximum, as np.argmax) of the last
        position's logits -- the C4 harness over transformer.py:93-104 -- with
        a KV cache: one prefill over the prompt, then one-token steps whose
        attention is the decode kernel against the cached keys and values.
        The loop stays on the device: each step's pick (mtx_greedy_pick_f32)
        lands in the id buffer the next step's embedding reads, and the same
        launch advances the step's positions (cache row, key count, position
        id), device counters.  Where the model fits its limits each step is
        one persistent launch (mtx_decode_step_f32, GPT._decode_step);
        otherwise a step is a chain of launches that replays unchanged: with
        graph=True the first one-token step runs eagerly, the second is
        recorded as a HIP graph and replayed for the rest.  With the
        persistent step the device state (caches, records, the step's inputs
        and workspace) is kept for the most recent prompt shape and, with
        graph=True, the prefill is recorded as a HIP graph on the second call
        for that shape and replayed after that, while the parameters keep
        their device buffers.  The host synchronises once, at the end.  Needs
        T0 + max_new_tokens <=
        block_size (beyond it the reference crops the context and recomputes
        positions, which a cache cannot reuse; use generate() then).
        Returns ids (B, T0 + n) and, if asked, the top-2 logit margins (B, n)."""
        from . import kernels as K

        idx = np.asarray(idx)
        B, T0 = idx.shape
        n = int(max_new_tokens)
        Tmax = T0 + n
        if Tmax > self.block_size:
            raise ValueError(f"prompt + new tokens = {Tmax} exceeds block_size {self.block_size}")
        if n < 1:
            return (idx.copy(), np.empty((B, 0))) if return_margins else idx.copy()
        C = self.tok_emb.weight.shape[1]
        if _PERSISTENT_STEP:
            out = self._generate_greedy_persistent(idx, n, return_margins, graph)
            if out is not None:
                return out
        caches = [(dev.empty((B, Tmax, C)), dev.empty((B, Tmax, C))) for _ in self.blocks]
        ids = dev.empty((Tmax, B), dtype="int64")  # time-major: a step's ids are contiguous
        margins = dev.empty((n, B))
        pos = self._positions(Tmax)

        with no_grad():
            # the fused q/k/v weights (a snapshot of the current weights) serve
            # the prefill and the decode steps
            for block in self.blocks:
                block.attn.fuse_qkv()
            # prefill over the prompt
            prompt = dev.index_array(idx)
            x = self.tok_emb(prompt) + self.pos_emb(DeviceArray(pos.t[:T0]))
            for block, cache in zip(self.blocks, caches):
                x = block.forward_cached(x, cache, 0, fused=True)
            x = self.ln_f(Tensor(x.data.t[:, T0 - 1:T0, :]))
            K.argmax_rows(self.lm_head(x).data.t.view(B, -1), idx=ids.t[T0], margin=margins.t[0])
            if n > 1:
                cur = ids.t[T0].clone()              # ids fed to the next step, then overwritten
                lengths = dev.full((B,), T0 + 1, "int32").t
                posd = dev.full((1,), T0, "int64").t
                x = dev.empty((B, 1, C))

                ln0 = self.blocks[0].ln1
                xn = dev.empty((B, 1, C))
                X = (x, dev.empty((B, 1, C)))
                V = self.lm_head.weight.shape[1]
                deferred = (_DEFERRED_STEP and C <= 1024 and V <= 256
                            and all(blk.deferred_step_fits(B, Tmax) for blk in self.blocks))

                def step_deferred():
                    # the token + position embeddings; each block's q/k/v +
                    # attention launch applies the previous block's pending
                    # second residual add and its own ln1, and the head launch
                    # the last block's and ln_f (mtx_head_pick_f32)
                    K.embedding2_fwd(self.tok_emb.weight.data.t, cur, self.pos_emb.weight.data.t, posd,
                                     x.t.view(B, C), ib_stride=0)
                    xi, pending = 0, None
                    for block, cache in zip(self.blocks, caches):
                        xi, pending = block.forward_step_deferred(X, xi, pending, cache, lengths)
                    lnf = self.ln_f
                    K.head_pick(X[xi].t.view(B, C), self.lm_head.weight.data.t, self.lm_head.bias.data.t, cur,
                                ids.t, lengths, posd, margins.t, t_base=T0, pending=pending,
                                ln=(lnf.gamma.data.t, lnf.beta.data.t, float(np.float32(lnf.eps))))

                def step():
                    if deferred:
                        return step_deferred()
                    # embeddings of this token and position and the first
                    # block's ln1 in one launch (mtx_embedding2_ln_fwd_f32)
                    K.embedding2_ln_fwd(self.tok_emb.weight.data.t, cur, self.pos_emb.weight.data.t, posd,
                                        x.t.view(B, C), ln0.gamma.data.t, ln0.beta.data.t,
                                        float(np.float32(ln0.eps)), xn.t.view(B, C), ib_stride=0)
                    h, hn = Tensor(x), Tensor(xn)
                    # each block's last launch also normalises its output for
                    # the next block's ln1 (ln_f after the last block)
                    for i, (block, cache) in enumerate(zip(self.blocks, caches)):
                        nxt = self.blocks[i + 1].ln1 if i + 1 < len(self.blocks) else self.ln_f
                        h, hn = block.forward_step(h, cache, lengths, ln_in=hn, next_ln=nxt)
                    # lm_head and the pick in one launch: the pick writes the
                    # next input, the id and margin records, and advances the
                    # positions (mtx_head_pick_f32)
                    K.head_pick(hn.data.t.view(B, C), self.lm_head.weight.data.t, self.lm_head.bias.data.t, cur,
                                ids.t, lengths, posd, margins.t, t_base=T0)

                ds = self._decode_step(caches, B, Tmax)
                if ds is not None:
                    # every remaining token step in one persistent launch;
                    # the status word is read once
                    ds(cur, ids.t, lengths, posd, margins=margins.t, t_base=T0, steps=n - 1)
                    ds.check()
                elif graph and n > 2:
                    from .graphs import Graph

                    step()  # eager first: the recorded step then finds every buffer allocated
                    g = Graph()
                    with g.capture():
                        step()
                    for s in range(2, n):
                        g.replay()
                else:
                    for s in range(1, n):
                        step()
        out = ids.t.numpy().T.copy()
        out[:, :T0] = idx
        if return_margins:
            return out, margins.t.numpy().T.astype(np.float64)
        return out

    def _param_ptrs(self):
        """Device addresses of every parameter and fused q/k/v buffer, and
        every dropout's mode: a cached decode state built on them is valid
        while they are unchanged (values may change in place)."""
        ptrs = [p.data.t.data_ptr() for p in self.parameters()]
        for blk in self.blocks:
            if blk.attn._qkv is not None:
                ptrs += [blk.attn._qkv[0].data.t.data_ptr(), blk.attn._qkv[1].data.t.data_ptr()]
        drops = [(m._training, m.p) for kind, _, m, _ in self._walk() if kind == "module" and isinstance(m, Dropout)]
        return tuple(ptrs), tuple(drops)

    def _greedy_state(self, B, T0):
        """Device state of greedy decoding with the persistent step for (B, T0)
        prompts, kept between calls (the most recent shape only): caches of
        block_size rows, the id and margin records, the step's inputs, the
        DecodeStep and, from the second call on, the prefill recorded as a HIP
        graph.  None where the persistent step does not apply."""
        st = self.__dict__.get("_greedy_st")
        if st is not None and st["key"] == (B, T0) and st["ptrs"] == self._param_ptrs():
            return st
        self.__dict__["_greedy_st"] = None  # the previous state (its graph, its buffers) goes first
        st = None
        Tm = self.block_size
        C = self.tok_emb.weight.shape[1]
        for block in self.blocks:
            block.attn.fuse_qkv()
        caches = [(dev.empty((B, Tm, C)), dev.empty((B, Tm, C))) for _ in self.blocks]
        ds = self._decode_step(caches, B, Tm)
        if ds is None:
            return None
        st = dict(key=(B, T0), ptrs=self._param_ptrs(), caches=caches, ds=ds, graph=None, calls=0,
                  ids=dev.empty((Tm, B), dtype="int64"), margins=dev.empty((Tm, B)),
                  prompt=dev.empty((B, T0), dtype="int64"), cur=dev.empty((B,), dtype="int64"),
                  lengths=dev.empty((B,), dtype="int32"), posd=dev.empty((1,), dtype="int64"),
                  lengths0=dev.full((B,), T0 + 1, "int32"), posd0=dev.full((1,), T0, "int64"))
        self.__dict__["_greedy_st"] = st
        return st

    def _generate_greedy_persistent(self, idx, n, return_margins, graph):
        """generate_greedy with the persistent decode step and the state of
        _greedy_state: the prompt is copied into the state's buffer, the
        prefill (fused q/k/v refreshed, the prompt's forward writing the
        caches, the first pick, the step inputs reset) runs eagerly on the
        first call for a shape and replays a recorded HIP graph after that
        (graph=True), then one launch runs the remaining token steps.  None
        where the persistent step does not apply."""
        from . import kernels as K

        B, T0 = idx.shape
        st = self._greedy_state(B, T0)
        if st is None:
            return None
        pos = self._positions(self.block_size)
        ids, margins = st["ids"], st["margins"]

        def prefill():
            for block in self.blocks:
                block.attn.fuse_qkv()
            x = self.tok_emb(st["prompt"]) + self.pos_emb(DeviceArray(pos.t[:T0]))
            for block, cache in zip(self.blocks, st["caches"]):
                x = block.forward_cached(x, cache, 0, fused=True)
            x = self.ln_f(Tensor(x.data.t[:, T0 - 1:T0, :]))
            K.argmax_rows(self.lm_head(x).data.t.view(B, -1), idx=ids.t[T0], margin=margins.t[0])
            st["cur"].t.copy_(ids.t[T0])
            st["lengths"].t.copy_(st["lengths0"].t)
            st["posd"].t.copy_(st["posd0"].t)

        st["prompt"].t.copy_(np.ascontiguousarray(idx, dtype=np.int64))
        with no_grad():
            if graph and st["calls"] > 0:
                if st["graph"] is None:
                    from .graphs import Graph

                    g = Graph()
                    with g.capture():
                        prefill()
                    st["graph"] = g
                st["graph"].replay()
            else:
                prefill()
            st["calls"] += 1
            if n > 1:
                try:
                    st["ds"](st["cur"].t, ids.t, st["lengths"].t, st["posd"].t, margins=margins.t, t_base=T0,
                             steps=n - 1)
                    st["ds"].check()
                except Exception:
                    self.__dict__["_greedy_st"] = None  # a failed step leaves its workspace unusable
                    raise
        out = ids.t[:T0 + n].numpy().T.copy()
        out[:, :T0] = idx
        if return_margins:
            return out, margins.t[:n].numpy().T.astype(np.float64)
        return out

    def _decode_step(self, caches, B, Tmax):
        """The persistent one-launch decode step (kernels.DecodeStep) for
        this model, or None where it does not apply: a block with an MLP
        other than Linear-GELU-Linear, active dropout, a Linear without bias,
        a head size other than 64 or a model beyond the kernel's limits."""
        from . import kernels as K

        C = self.tok_emb.weight.shape[1]
        V = self.lm_head.weight.shape[1]
        blocks = self.blocks
        if not (_PERSISTENT_STEP and blocks):
            return None
        hid = blocks[0].mlp.layers[0].weight.shape[1]
        if not K.decode_step_fits(len(blocks), C, C // 64, hid, V, Tmax) or self.lm_head.bias is None:
            return None
        layers = []
        for blk, (kc, vc) in zip(blocks, caches):
            fc1, act, fc2, drop = blk.mlp.layers
            attn = blk.attn
            if (attn.n_head * 64 != C or not isinstance(act, GELU) or (drop._training and drop.p > 0.0)
                    or (attn.attn_drop._training and attn.attn_drop.p > 0.0) or fc1.weight.shape[1] != hid
                    or any(lin.bias is None for lin in (fc1, fc2, attn.out_proj, attn.q_proj, attn.k_proj,
                                                        attn.v_proj))):
                return None
            if attn._qkv is None:
                attn.fuse_qkv()
            W, b = attn._qkv
            layers.append(dict(
                ln1_gamma=blk.ln1.gamma.data.t, ln1_beta=blk.ln1.beta.data.t,
                ln1_eps=float(np.float32(blk.ln1.eps)), w_qkv=W.data.t, b_qkv=b.data.t,
                w_out=attn.out_proj.weight.data.t, b_out=attn.out_proj.bias.data.t,
                ln2_gamma=blk.ln2.gamma.data.t, ln2_beta=blk.ln2.beta.data.t,
                ln2_eps=float(np.float32(blk.ln2.eps)), w_fc1=fc1.weight.data.t, b_fc1=fc1.bias.data.t,
                w_fc2=fc2.weight.data.t, b_fc2=fc2.bias.data.t, k_cache=kc.t, v_cache=vc.t))
        lnf = (self.ln_f.gamma.data.t, self.ln_f.beta.data.t, float(np.float32(self.ln_f.eps)))
        return K.DecodeStep(layers, self.tok_emb.weight.data.t, self.pos_emb.weight.data.t, lnf,
                            self.lm_head.weight.data.t, self.lm_head.bias.data.t, B, Tmax)

    def generate(self, idx, max_new_tokens, temperature=1.0):
        """Sample tokens as the reference does (transformer.py:93-104): each
        step takes the last position's logits / temperature, a softmax, and
        one np.random.choice per row from NumPy's global RNG, rows in order.
        The logits come from one-token KV-cache steps while the context fits
        block_size; once the reference would crop it (positions shift) they
        come from a full forward over the cropped context.  The softmax runs
        on the device; the host draws.  With active dropout (training mode,
        p > 0) every step is a full forward, as in the reference."""
        from . import kernels as K

        idx = np.asarray(idx)
        B, T0 = idx.shape
        n = int(max_new_tokens)
        blk = self.block_size
        out = np.empty((B, T0 + n), dtype=np.int64)
        out[:, :T0] = idx
        if n < 1:
            return out
        V = self.lm_head.weight.shape[1]
        C = self.tok_emb.weight.shape[1]
        temp = dev.const(float(temperature))
        mods = [self] + [m for kind, _, m, _ in self._walk() if kind == "module"]
        dropout_on = any(isinstance(m, Dropout) and m._training and m.p > 0.0 for m in mods)

        def sample(logits2d):
            scaled = dev.empty((B, V))
            K.ewise("DIV", scaled.t, logits2d, temp.t)
            probs = dev.empty((B, V))
            K.softmax_fwd(scaled.t, probs.t)
            p = probs.numpy().astype(np.float64)
            p /= p.sum(axis=-1, keepdims=True)
            return np.array([np.random.choice(V, p=pr) for pr in p])

        def last_logits(x):
            x = self.ln_f(Tensor(x.data.t[:, -1:, :]))
            return self.lm_head(x).data.t.view(B, V)

        with no_grad():
            ctx = T0
            caches = None
            if T0 <= blk and not dropout_on:
                caches = [(dev.empty((B, blk, C)), dev.empty((B, blk, C))) for _ in self.blocks]
                pos = self._positions(blk)
                x = self.tok_emb(dev.index_array(idx)) + self.pos_emb(DeviceArray(pos.t[:T0]))
                for block, cache in zip(self.blocks, caches):
                    x = block.forward_cached(x, cache, 0)
                logits = last_logits(x)
            else:
                logits = self.forward(out[:, max(0, ctx - blk):ctx]).data.t[:, -1, :]
            for i in range(n):
                out[:, ctx] = sample(logits)
                ctx += 1
                if i == n - 1:
                    break
                if caches is not None and ctx <= blk:
                    # the new token sits at position ctx - 1 of an uncropped context
                    t = ctx - 1
                    x = self.tok_emb(dev.index_array(out[:, t:t + 1])) + self.pos_emb(DeviceArray(pos.t[t:t + 1]))
                    for block, cache in zip(self.blocks, caches):
                        x = block.forward_cached(x, cache, t)
                    logits = last_logits(x)
                else:
                    caches = None
                    logits = self.forward(out[:, max(0, ctx - blk):ctx]).data.t[:, -1, :]
        return out
