"""NumPy restatement of the reference's causal attention sub-graph (oracle).

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg; never by the product.

The reference computes attention inside ``MultiHeadAttention.forward``
(transformer.py:36-44) from generic autograd ops:

    scores = (q @ k.transpose(-2, -1)) * (1.0 / np.sqrt(head_dim))
    scores = scores + Tensor(np.triu(np.ones((T, T), float32), k=1) * -1e9)
    attn   = F.softmax(scores, axis=-1)
    out    = attn @ v

Under NumPy 2 (the reference's pinned version) ``1.0/np.sqrt(D)`` is an
``np.float64`` scalar, ``Tensor.__init__`` keeps it as a 0-d float64 array
(tensor.py:53-54), and ``float32 array * float64 0-d array`` promotes to float64.
So q@k^T is an fp32 sgemm, and everything from the scale on is float64.
Gradient holders follow the dtype of the tensor they belong to
(``_accum_grad`` zero-inits with ``zeros_like(data)`` then adds in place,
tensor.py:29-33), so the grad of the fp32 ``q@k^T`` node is rounded to fp32
before the matmul backward produces dq and dk in fp32.

``reference_attention`` restates exactly that flow.  ``attention_f64`` is the
same mathematics carried out entirely in float64, and ``flash_forward`` /
``flash_backward`` the log-sum-exp formulation the GPU kernels implement.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
F64 = np.float64


def causal_mask(Tq: int, Tk: int) -> np.ndarray:
    """Boolean (Tq, Tk) mask of *hidden* entries.

    For Tq == Tk this is ``np.triu(ones, k=1) != 0`` (transformer.py:39).  For
    Tq < Tk the queries are the last Tq positions (bottom-right alignment), the
    rule the GPU library uses: key j is visible to query i iff j <= i + Tk - Tq.
    """
    i = np.arange(Tq)[:, None]
    j = np.arange(Tk)[None, :]
    return j > i + (Tk - Tq)


def _softmax_lastdim(x: np.ndarray) -> np.ndarray:
    """F.softmax forward, functional.py:62-66 (max-shift, exp, divide by sum)."""
    shifted = x - x.max(axis=-1, keepdims=True)
    exps = np.exp(shifted)
    return exps / exps.sum(axis=-1, keepdims=True)


def _softmax_backward(p: np.ndarray, gout: np.ndarray) -> np.ndarray:
    """F.softmax backward closure, functional.py:69-73."""
    g = gout * p
    return g - p * g.sum(axis=-1, keepdims=True)


def reference_attention(q, k, v, dout=None, scale=None, causal=True, keep=None, p=0.0):
    """The reference's attention sub-graph with its exact dtype flow.

    q, k, v: (..., T, D) float32 (the _split_heads views, transformer.py:26-28).
    dout: upstream gradient of ``out`` or None (forward only).
    keep: optional dropout keep mask (..., Tq, Tk) (nonzero = kept) with drop
    probability p: attn_drop (Dropout.forward, layers.py:115-122) between the
    softmax and attn @ v, ``attn * mask.astype(float32) * (1.0 / (1.0 - p))``,
    and its closure ``grad * mask * scale`` (layers.py:124-126).
    Returns (out, dq, dk, dv); grads are None when dout is None.

    Forward: transformer.py:36-44, with matmul tensor.py:207-208, the scalar
    multiply tensor.py:148-150 (fp32 * fp64 0-d -> fp64), mask add
    tensor.py:111-113, softmax functional.py:62-66.
    Backward: the closures in reverse topological order -- matmul
    tensor.py:210-218 (attn @ v), softmax functional.py:69-73, add
    tensor.py:115-119 (identity for scores), mul tensor.py:152-156
    (other.data * out.grad, accumulated into the fp32 q@k^T node's grad),
    matmul tensor.py:210-218 (q @ k^T), transpose tensor.py:338-340.
    """
    q = np.asarray(q, dtype=F32)
    k = np.asarray(k, dtype=F32)
    v = np.asarray(v, dtype=F32)
    Tq, D = q.shape[-2], q.shape[-1]
    Tk = k.shape[-2]
    if scale is None:
        scale = 1.0 / np.sqrt(D)  # np.float64, as in transformer.py:36
    scale64 = np.asarray(np.float64(scale))
    kt = np.swapaxes(k, -1, -2)
    qk = q @ kt  # fp32 (sgemm)
    scores = qk * scale64  # -> float64
    if causal:
        mask = (causal_mask(Tq, Tk).astype(F32) * F32(-1e9)).astype(F32)
        scores = scores + mask
    attn = _softmax_lastdim(scores)  # float64
    if keep is not None:
        dmask = (np.asarray(keep) != 0).astype(F32)
        dscale = 1.0 / (1.0 - p)
        attn_d = attn * dmask * dscale  # float64
    else:
        attn_d = attn
    out = attn_d @ v  # float64 @ float32 -> float64
    if dout is None:
        return out, None, None, None
    gout = np.asarray(dout, dtype=F64)
    # attn @ v backward (tensor.py:213-218); v's grad holder is fp32
    d_attn = gout @ np.swapaxes(v, -1, -2)
    dv = (np.swapaxes(attn_d, -1, -2) @ gout).astype(F32)
    if keep is not None:
        d_attn = d_attn * dmask * dscale  # dropout closure
    # softmax backward -> grad of scores (float64 node)
    d_scores = _softmax_backward(attn, d_attn)
    # mask add: identity; mul by scale: grad flows into the fp32 q@k^T node
    d_qk = (scale64 * d_scores).astype(F32)
    # q @ kt backward in fp32
    dq = (d_qk @ k).astype(F32)
    d_kt = np.swapaxes(q, -1, -2) @ d_qk
    dk = np.swapaxes(d_kt, -1, -2).astype(F32)
    return out, dq, dk, dv


def attention_f64(q, k, v, dout=None, scale=None, causal=True, keep=None, p_drop=0.0):
    """Same mathematics as reference_attention, entirely in float64 (with the
    same optional dropout keep mask / probability).

    Returns (out, p, dq, dk, dv, ds) where p is the probability matrix and ds
    the score gradient (grad w.r.t. scale * q k^T + mask), for invariant checks.
    """
    q = np.asarray(q, dtype=F64)
    k = np.asarray(k, dtype=F64)
    v = np.asarray(v, dtype=F64)
    Tq, D = q.shape[-2], q.shape[-1]
    Tk = k.shape[-2]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    if causal:
        s = np.where(causal_mask(Tq, Tk), -np.inf, s)
    p = _softmax_lastdim(s)
    z = 1.0 if keep is None else (np.asarray(keep) != 0) / (1.0 - p_drop)
    out = (p * z) @ v
    if dout is None:
        return out, p, None, None, None, None
    g = np.asarray(dout, dtype=F64)
    dv = np.swapaxes(p * z, -1, -2) @ g
    dp = (g @ np.swapaxes(v, -1, -2)) * z
    ds = _softmax_backward(p, dp)
    dq = scale * (ds @ k)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    return out, p, dq, dk, dv, ds


def flash_forward(q, k, v, scale, causal=True):
    """Log-sum-exp form: returns (out, lse) with lse_i = log sum_j exp(s_ij),
    s = scale * q k^T over visible keys.  Float64."""
    q = np.asarray(q, dtype=F64)
    k = np.asarray(k, dtype=F64)
    v = np.asarray(v, dtype=F64)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    if causal:
        s = np.where(causal_mask(q.shape[-2], k.shape[-2]), -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    out = (e @ v) / l
    lse = (m + np.log(l))[..., 0]
    return out, lse


def flash_backward(q, k, v, out, dout, lse, scale, causal=True):
    """Backward from saved (out, lse): P = exp(s - lse), delta = rowsum(dO*O),
    dS = P * (dO V^T - delta).  Float64.  Returns (dq, dk, dv)."""
    q = np.asarray(q, dtype=F64)
    k = np.asarray(k, dtype=F64)
    v = np.asarray(v, dtype=F64)
    out = np.asarray(out, dtype=F64)
    g = np.asarray(dout, dtype=F64)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    p = np.exp(s - np.asarray(lse, dtype=F64)[..., None])
    if causal:
        p = np.where(causal_mask(q.shape[-2], k.shape[-2]), 0.0, p)
    delta = (g * out).sum(axis=-1, keepdims=True)
    dp = g @ np.swapaxes(v, -1, -2)
    ds = p * (dp - delta)
    dq = scale * (ds @ k)
    dk = scale * (np.swapaxes(ds, -1, -2) @ q)
    dv = np.swapaxes(p, -1, -2) @ g
    return dq, dk, dv


def reference_attention_chunked(q, k, v, dout=None, scale=None, causal=True, chunk=1):
    """reference_attention over the leading (B, H) axes in chunks of `chunk`
    (b, h) slices, to bound memory at long T (one fp64 (T, T) matrix per
    slice).  Results are identical to the unchunked call: every slice is
    independent."""
    B, H = q.shape[0], q.shape[1]
    outs = []
    for b in range(B):
        row = []
        for h0 in range(0, H, chunk):
            sl = (slice(b, b + 1), slice(h0, h0 + chunk))
            row.append(reference_attention(q[sl], k[sl], v[sl],
                                           None if dout is None else dout[sl],
                                           scale, causal))
        outs.append([np.concatenate([r[i] for r in row], axis=1) if row[0][i] is not None else None
                     for i in range(4)])
    return tuple(np.concatenate([o[i] for o in outs], axis=0) if outs[0][i] is not None else None
                 for i in range(4))


def numerical_gradient(f, inputs, eps=1e-5):
    """Central differences in float64, one element at a time -- the method of
    the reference's grad_check.numerical_gradient (grad_check.py:5-38)."""
    grads = []
    for idx_in, x in enumerate(inputs):
        g = np.zeros_like(x, dtype=F64)
        it = np.nditer(x, flags=["multi_index"])
        while not it.finished:
            i = it.multi_index
            old = x[i]
            x[i] = old + eps
            fp = f()
            x[i] = old - eps
            fm = f()
            x[i] = old
            g[i] = (fp - fm) / (2 * eps)
            it.iternext()
        grads.append(g)
    return grads


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even) and return them
    as float32.  NaN/inf are not expected in the inputs."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(F32)


LOG2E = 1.4426950408889634


def _lazy_reference(s2, tile, tau):
    """The forward kernel's running reference per row: key tiles of `tile`
    keys in ascending order; the reference is set by the first tile with a
    visible key and moved to a later tile's max only when that max exceeds it
    by more than `tau` (log2 units).  Returns m_t (..., Tq, ntile): the
    reference in effect while tile t's probabilities are formed."""
    Tk = s2.shape[-1]
    nt = (Tk + tile - 1) // tile
    m = np.full(s2.shape[:-1], -np.inf)
    out = np.empty(s2.shape[:-1] + (nt,))
    for t in range(nt):
        tm = s2[..., t * tile:(t + 1) * tile].max(axis=-1)
        fresh = ~np.isfinite(m)
        move = np.where(fresh, np.isfinite(tm), tm - np.where(fresh, 0.0, m) > tau)
        m = np.where(move, tm, m)
        out[..., t] = m
    return out


def attention_bf16_emulated(q, k, v, dout, scale, causal=True, rounding=True, tile=64, tau=8.0,
                            onepass=False):
    """The bf16 kernels' arithmetic (mtx_attn_fwd / mtx_attn_bwd with bf16
    inputs) restated in float64 with bf16 round-to-nearest-even at exactly
    the points where the kernels round, for elementwise checks of the GPU
    results (the reference, transformer.py:36-44, has no bf16 path; its
    mathematics is attention_f64's).

    q, k, v, dout: bf16-valued float32 arrays (..., T, D).  The kernels round
      * the register operand pre-multiplied by c = scale*log2(e): Q*c in the
        forward and dQ passes, K*c in the dK/dV pass (scores come out in log2
        units);
      * the forward probabilities exp2(s - m_t) before P V and the row sum,
        with the running reference m_t of _lazy_reference (earlier tiles are
        rescaled by exp2(m_t - m_final) in fp32);
      * the output O (stored as bf16; delta = rowsum(dO * O) uses it);
      * P before dV = P^T dO, and dS = P (dP - delta) before dK = scale dS^T Q
        and dQ = scale dS K (P and dS themselves are formed in fp32 from the
        unrounded scores).
    onepass=True: dQ as the one-pass backward forms it, from the dK/dV pass's
      dS (scores from K*c) instead of a dQ pass's (scores from Q*c).
    rounding=False skips every rounding (then the result is attention_f64's
    up to float64 rounding).  Returns (out, lse, dq, dk, dv) in float64."""
    R = bf16_round if rounding else (lambda x: np.asarray(x, dtype=F64))
    q32, k32, v32, g32 = (np.asarray(a, dtype=F32) for a in (q, k, v, dout))
    q64, k64, v64, g64 = (a.astype(F64) for a in (q32, k32, v32, g32))
    c = F32(F32(scale) * F32(LOG2E)) if rounding else scale * LOG2E
    qs = R(q32 * c).astype(F64) if rounding else q64 * c
    ks = R(k32 * c).astype(F64) if rounding else k64 * c
    Tq, Tk = q32.shape[-2], k32.shape[-2]
    hidden = causal_mask(Tq, Tk) if causal else np.zeros((Tq, Tk), bool)

    # forward: S^T = K (Q c)^T, lazy reference, bf16 P for P V and the row sum
    s2 = np.where(hidden, -np.inf, qs @ np.swapaxes(k64, -1, -2))
    mt = _lazy_reference(s2, tile, tau)
    m_fin = mt[..., -1:]
    pt = np.empty_like(s2)
    w = np.empty_like(s2)
    for t in range(mt.shape[-1]):
        sl = slice(t * tile, (t + 1) * tile)
        mref = mt[..., t:t + 1]
        e = np.where(np.isfinite(s2[..., sl]), np.exp2(s2[..., sl] - np.where(np.isfinite(mref), mref, 0.0)), 0.0)
        pt[..., sl] = R(e).astype(F64)
        w[..., sl] = np.exp2(np.where(np.isfinite(mref), mref - m_fin, 0.0))
    pw = pt * w
    l = pw.sum(axis=-1, keepdims=True)
    out = (pw @ v64) / l
    lse = (m_fin[..., 0] + np.log2(l[..., 0])) * np.log(2.0)
    ob = R(out).astype(F64)

    # backward
    delta = (g64 * ob).sum(axis=-1, keepdims=True)
    nl = lse[..., None] * LOG2E
    dp = g64 @ np.swapaxes(v64, -1, -2)
    # dK/dV pass: S = Q (K c)^T
    pk = np.where(hidden, 0.0, np.exp2(np.where(hidden, 0.0, q64 @ np.swapaxes(ks, -1, -2)) - nl))
    dsk = pk * (dp - delta)
    dv = np.swapaxes(R(pk).astype(F64), -1, -2) @ g64
    dk = scale * (np.swapaxes(R(dsk).astype(F64), -1, -2) @ q64)
    if onepass:
        # the key-outer pass's dS, rounded for its dK product, times K
        dq = scale * (R(dsk).astype(F64) @ k64)
    else:
        # dQ pass: S^T = K (Q c)^T
        pq = np.where(hidden, 0.0, np.exp2(np.where(hidden, 0.0, qs @ np.swapaxes(k64, -1, -2)) - nl))
        dsq = pq * (dp - delta)
        dq = scale * (R(dsq).astype(F64) @ k64)
    return ob if rounding else out, lse, dq, dk, dv
