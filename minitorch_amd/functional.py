"""Stateless differentiable functions (the reference's functional.py, plus the
fused ops the GPU path adds).

Reference functions on the transformer's path, same names and semantics:
tanh, gelu, softmax, log_softmax (functional.py:39-97; relu and sigmoid, off
that path, are not provided).  Added fused ops, each one autograd
node with a hand-written backward (the precedent is the reference's Conv2d,
conv.py:66-95):
  linear(x, W, b)              x @ W + b with the bias in the GEMM epilogue
  linear_qkv(x, lq, lk, lv)    the three q/k/v projections as one packed GEMM
  mlp_gelu(x, fc1, fc2)        Linear -> GELU -> Linear, GELU in the GEMM epilogues
  causal_attention(q, k, v)    transformer.py:36-44 as one flash kernel
  causal_attention_packed      the same over a packed [q | k | v] tensor
"""
from __future__ import annotations

import math

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray
from .tensor import Tensor, _accum_grad, _grad_target, _own_grad, _parents, grad_enabled


def _track(*ts):
    return grad_enabled() and any(t.requires_grad for t in ts)


def _node(data, prev, op, backward, track):
    out = Tensor(data, requires_grad=track)
    if track:
        out._backward = backward
        out._prev = _parents(prev)
        out._op = op
    return out


def tanh(x):
    """Hyperbolic tangent (functional.py:39-51)."""
    data = dev.empty(x.shape)
    K.ewise("TANH", data.t, x.data.t)
    out = None

    def _backward():
        if x.requires_grad:
            g = dev.empty(x.shape)
            K.ewise("TANH_GRAD", g.t, out.data.t, out.grad.t)
            _accum_grad(x, g, owned=True)

    out = _node(data, (x,), "tanh", _backward, _track(x))
    return out


def gelu(x):
    """GELU, tanh approximation (functional.py:54-59), as one fused node: the
    same formula and float32 constants as the reference's 8-node composite."""
    xc = x.data.contiguous()
    data = dev.empty(x.shape)
    K.gelu_fwd(xc.t, data.t)
    out = None

    def _backward():
        if x.requires_grad:
            target, acc = _grad_target(x)
            K.gelu_bwd(xc.t, out.grad.contiguous().t, target.t, accumulate=acc)

    out = _node(data, (x,), "gelu", _backward, _track(x))
    return out


def _last_axis(x, axis):
    axis = axis % x.ndim
    if axis != x.ndim - 1:
        raise NotImplementedError("softmax over a non-last axis: transpose first")


def softmax(x, axis=-1, causal=False):
    """Softmax over the last axis (functional.py:62-78).  causal=True applies
    the causal mask of transformer.py:39-40 to a (..., Tq, L) score tensor:
    hidden entries come out exactly 0, as the reference's -1e9 add gives."""
    _last_axis(x, axis)
    xc = x.data.contiguous()
    data = dev.empty(x.shape)
    K.softmax_fwd(xc.t, data.t, causal_tq=x.shape[-2] if causal else 0)
    out = None

    def _backward():
        if x.requires_grad:
            target, acc = _grad_target(x)
            K.softmax_bwd(out.data.t, out.grad.contiguous().t, target.t, accumulate=acc)

    out = _node(data, (x,), "softmax", _backward, _track(x))
    return out


def log_softmax(x, axis=-1):
    """log(softmax(x)) over the last axis (functional.py:81-97)."""
    _last_axis(x, axis)
    xc = x.data.contiguous()
    data = dev.empty(x.shape)
    K.softmax_fwd(xc.t, data.t, log=True)
    out = None

    def _backward():
        if x.requires_grad:
            target, acc = _grad_target(x)
            K.softmax_bwd(out.data.t, out.grad.contiguous().t, target.t, log=True, accumulate=acc)

    out = _node(data, (x,), "log_softmax", _backward, _track(x))
    return out


def linear(x, weight, bias=None, residual=None):
    """x @ W + b (layers.py:31-37) as one node: bias fused into the GEMM
    epilogue; backward dX = dY W^T, dW = X^T dY (batch folded into the
    contraction), db = column sums of dY.  With `residual` (a tensor of the
    output's shape) the node is residual + (x @ W + b) -- the block's
    x + attn(...) (transformer.py:64) -- with the add in the same GEMM
    epilogue; the residual's gradient is dY."""
    from .linalg import bmm, matmul_data, matmul_grad_b

    if x.shape[-1] != weight.shape[0]:
        raise AssertionError(f"Linear expects last dim {weight.shape[0]}, got {x.shape[-1]}")
    N = weight.shape[1]
    out_shape = tuple(x.shape[:-1]) + (N,)
    data = dev.empty(out_shape)
    if residual is not None:
        if tuple(residual.shape) != out_shape or x.ndim < 2:
            raise AssertionError(f"linear: residual {tuple(residual.shape)} does not match output {out_shape}")
        rows = int(np.prod(out_shape[:-1]))
        x2 = x.data.t.reshape(rows, x.shape[-1])
        K.gemm(x2, weight.data.t, data.t.view(rows, N), bias=bias.data.t if bias is not None else None,
               act=K.GEMM_ACT_ADD, aux=residual.data.t.reshape(rows, N))
    else:
        xt = x.data.t if x.ndim >= 2 else x.data.t.unsqueeze(0)
        ot = data.t if x.ndim >= 2 else data.t.unsqueeze(0)
        bmm(xt, weight.data.t, ot, bias=bias.data.t if bias is not None else None)
    prev = (x, weight) + ((bias,) if bias is not None else ()) + ((residual,) if residual is not None else ())
    out = None

    def _backward():
        g = out.grad
        if residual is not None and residual.requires_grad:
            _accum_grad(residual, g)
        if x.requires_grad:
            target, acc = _grad_target(x)
            gt = g.t if x.ndim >= 2 else g.t.unsqueeze(0)
            tt = target.t if x.ndim >= 2 else target.t.unsqueeze(0)
            bmm(gt, weight.data.t.transpose(0, 1), tt, beta=1.0 if acc else 0.0)
        db_done = False
        if weight.requires_grad:
            db_done = matmul_grad_b(x.data, g, weight,
                                    bias=bias if bias is not None and bias.requires_grad else None)
        if bias is not None and bias.requires_grad and not db_done:
            target, acc = _grad_target(bias)
            K.reduce(g.t, list(range(g.ndim - 1)), target.t, accumulate=acc)

    out = _node(data, prev, "linear", _backward, _track(*prev))
    return out


def linear_qkv(x, lq, lk, lv):
    """q_proj(x), k_proj(x), v_proj(x) (transformer.py:32-34) as one node whose
    output is the packed (..., 3C) tensor [q | k | v]: one GEMM over the
    concatenated (C_in, 3C) weight with the concatenated bias in its epilogue.
    Backward: dX = dQKV W^T as one GEMM with K = 3C, dW = X^T dQKV as one
    (C_in, 3C) GEMM and db as one column reduction, each split back into the
    three Linears' gradients (mtx_unpack3_f32, accumulating like _accum_grad).
    The three layers keep their own parameters and state_dict keys."""
    from .linalg import bmm

    Ws = (lq.weight, lk.weight, lv.weight)
    bs = (lq.bias, lk.bias, lv.bias)
    Cin, C = Ws[0].shape
    if x.shape[-1] != Cin:
        raise AssertionError(f"Linear expects last dim {Cin}, got {x.shape[-1]}")
    wcat = dev.empty((Cin, 3 * C))
    K.pack3([w.data.t for w in Ws], wcat.t)
    bcat = dev.empty((1, 3 * C))
    K.pack3([b.data.t.view(1, C) for b in bs], bcat.t)
    data = dev.empty(tuple(x.shape[:-1]) + (3 * C,))
    xt = x.data.t if x.ndim >= 2 else x.data.t.unsqueeze(0)
    ot = data.t if x.ndim >= 2 else data.t.unsqueeze(0)
    bmm(xt, wcat.t, ot, bias=bcat.t.view(-1))
    prev = (x,) + Ws + bs
    out = None

    def _backward():
        g = out.grad
        g2 = g.t.reshape(-1, 3 * C)
        if x.requires_grad:
            target, acc = _grad_target(x)
            gt = g.t if x.ndim >= 2 else g.t.unsqueeze(0)
            tt = target.t if x.ndim >= 2 else target.t.unsqueeze(0)
            bmm(gt, wcat.t.transpose(0, 1), tt, beta=1.0 if acc else 0.0)
        need_db = any(b.requires_grad for b in bs)
        db = dev.empty((1, 3 * C)) if need_db else None
        if any(w.requires_grad for w in Ws):
            # dW and db (the column sums of dQKV) in one GEMM
            x2 = x.data.t.reshape(-1, Cin)
            dw = dev.empty((Cin, 3 * C))
            K.gemm(x2.transpose(0, 1), g2, dw.t, 1.0, 0.0, None, M=Cin, N=3 * C, K=x2.shape[0],
                   colsum=db.t.view(-1) if need_db else None)
            _unpack_grads(dw.t, Ws)
        elif need_db:
            K.reduce(g2, [0], db.t.view(-1))
        if need_db:
            _unpack_grads(db.t, bs, rows_view=(1, C))

    out = _node(data, prev, "linear_qkv", _backward, _track(*prev))
    return out


def mlp_gelu(x, fc1, fc2, residual=None):
    """fc2(gelu(fc1(x))) -- the MLP of TransformerBlock (transformer.py:56-59:
    Linear, GELU, Linear; Linear layers.py:31-37, F.gelu functional.py:54-59)
    -- as one node.  Forward: the fc1 GEMM applies GELU in its epilogue and
    also stores the pre-activation h the backward needs; then the fc2 GEMM.
    Backward: dW2, db2 from dY; dh = (dY W2^T) * gelu'(h) as one GEMM whose
    epilogue applies the GELU derivative; then dW1, db1 and dX from dh.  The
    two Linears keep their own parameters and state_dict keys.  With
    `residual` (shaped like the output) the node is residual + mlp(x) -- the
    block's x + mlp(...) (transformer.py:65) -- with the add in the fc2 GEMM's
    epilogue; the residual's gradient is dY."""
    W1, b1, W2, b2 = fc1.weight, fc1.bias, fc2.weight, fc2.bias
    Cin, Hd = W1.shape
    Cout = W2.shape[1]
    if x.shape[-1] != Cin or W2.shape[0] != Hd:
        raise AssertionError(f"MLP shapes do not chain: x {tuple(x.shape)}, fc1 {tuple(W1.shape)}, "
                             f"fc2 {tuple(W2.shape)}")
    lead = tuple(x.shape[:-1])
    rows = int(np.prod(lead)) if lead else 1
    x2 = x.data.t.reshape(rows, Cin)
    h = _empty((rows, Hd), x2.dtype)
    a = _empty((rows, Hd), x2.dtype)
    K.gemm(x2, W1.data.t, a, bias=b1.data.t, act=K.GEMM_ACT_GELU, aux=h)
    data = dev.empty(lead + (Cout,))
    if residual is not None:
        if tuple(residual.shape) != lead + (Cout,):
            raise AssertionError(f"mlp_gelu: residual {tuple(residual.shape)} does not match output")
        K.gemm(a, W2.data.t, data.t.view(rows, Cout), bias=b2.data.t, act=K.GEMM_ACT_ADD,
               aux=residual.data.t.reshape(rows, Cout))
    else:
        K.gemm(a, W2.data.t, data.t.view(rows, Cout), bias=b2.data.t)
    prev = (x, W1, b1, W2, b2) + ((residual,) if residual is not None else ())
    out = None

    def _backward():
        if residual is not None and residual.requires_grad:
            _accum_grad(residual, out.grad)
        g2 = out.grad.t.reshape(rows, Cout)
        _wgrad(a.transpose(0, 1), g2, W2, b2, Hd, Cout, rows)
        need_h = x.requires_grad or W1.requires_grad or b1.requires_grad
        if not need_h:
            return
        dh = _empty((rows, Hd), g2.dtype)
        K.gemm(g2, W2.data.t.transpose(0, 1), dh, act=K.GEMM_ACT_GELU_BWD, aux=h)
        _wgrad(x2.transpose(0, 1), dh, W1, b1, Cin, Hd, rows)
        if x.requires_grad:
            t, acc = _grad_target(x)
            K.gemm(dh, W1.data.t.transpose(0, 1), t.t.view(rows, Cin), 1.0, 1.0 if acc else 0.0, None)

    out = _node(data, prev, "mlp_gelu", _backward, _track(*prev))
    return out


def _wgrad(at, g, W, b, M, N, rows):
    """W.grad (+)= at @ g (at: (M, rows), g: (rows, N)) and b.grad (+)= the
    column sums of g, in one GEMM when both are wanted."""
    tw = tb = None
    if W.requires_grad:
        tw, accw = _grad_target(W)
    if b.requires_grad:
        tb, accb = _grad_target(b)
    if tw is not None:
        K.gemm(at, g, tw.t, 1.0, 1.0 if accw else 0.0, None, M=M, N=N, K=rows,
               colsum=tb.t if tb is not None else None, colsum_accumulate=tb is not None and accb)
    elif tb is not None:
        K.reduce(g, [0], tb.t, accumulate=accb)


def _unpack_grads(src, params, rows_view=None):
    """Split a packed (rows, 3C) gradient into the three parameters' gradients
    (fresh buffers, or added to existing ones)."""
    targets, acc = [], []
    for p in params:
        if p.requires_grad:
            t, a = _grad_target(p)
        else:
            t, a = dev.empty(p.shape), False  # computed and discarded
        targets.append(t.t if rows_view is None else t.t.view(*rows_view))
        acc.append(a)
    K.unpack3(src, targets, acc)


def causal_attention_packed(qkv, n_head, scale=None, keep=None, keep_scale=1.0):
    """causal_attention (transformer.py:36-44) over the q, k, v column blocks
    of one packed (B, T, 3C) tensor (linear_qkv's output).  The heads are
    strided views of it (strides (T*3C, D, 3C, 1), no copies), and the
    backward writes dq, dk, dv straight into the column blocks of qkv's
    gradient, so the packed projection's backward reads a single buffer.
    Returns the (B, H, T, D) output as causal_attention does."""
    t = qkv.data.t
    B, T, C3 = t.shape
    C = C3 // 3
    D = C // n_head
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    heads = lambda a: [a.view(B, T, 3, n_head, D)[:, :, i].transpose(1, 2) for i in range(3)]
    qt, kt, vt = heads(t)
    o = _empty((B, T, n_head, D), t.dtype).transpose(1, 2)
    drop = {} if keep is None else {"keep": keep, "keep_scale": float(keep_scale)}
    o, lse = K.attn_fwd(qt, kt, vt, scale, True, out=o, **drop)
    out = None

    def _backward():
        if not qkv.requires_grad:
            return
        g = out.grad.t
        do = g if _kernel_layout(g) else out.grad.contiguous().t
        target, acc = _grad_target(qkv)
        dq, dk, dv = heads(target.t)
        K.attn_bwd(qt, kt, vt, o, do, lse, scale, True, dq=dq, dk=dk, dv=dv, accumulate=acc, **drop)

    out = _node(DeviceArray(o), (qkv,), "causal_attention", _backward, _track(qkv))
    return out


def causal_attention(q, k, v, scale=None, keep=None, keep_scale=1.0):
    """softmax(q k^T * scale + causal mask) @ v for (B, H, T, D) tensors --
    exactly transformer.py:36-44 -- as one fused flash kernel (libmtx_hip
    mtx_attn_fwd / mtx_attn_bwd).  q, k, v may be the strided views that
    _split_heads makes (no copies); gradients come back in the same layout.
    keep: optional dropout keep-mask (a uint8 (B, H, T, ld) device tensor,
    see attention_keep_mask) applied to the softmax output with keep_scale =
    1/(1-p), the reference's attn_drop (transformer.py:43, layers.py:115-126);
    forward and backward use the same mask (mtx_attn_*_dropout)."""
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qt, kt, vt = q.data.t, k.data.t, v.data.t
    B, H, Tq, _ = qt.shape
    # the output is stored as (B, T, H, D), so merging the heads back to
    # (B, T, C) (transformer.py:45) is a view, not a copy
    o = _empty((B, Tq, H, D), qt.dtype).transpose(1, 2)
    drop = {} if keep is None else {"keep": keep, "keep_scale": float(keep_scale)}
    o, lse = K.attn_fwd(qt, kt, vt, scale, True, out=o, **drop)
    out = None

    def _backward():
        g = out.grad.t
        do = g if _kernel_layout(g) else out.grad.contiguous().t
        need = [t.requires_grad for t in (q, k, v)]
        if not any(need):
            return
        tgt = []
        for t in (q, k, v):
            if t.requires_grad and t.grad is not None:
                _own_grad(t)
                tgt.append((t.grad.t, True))
            else:
                buf = dev.DeviceArray(_empty_like(t.data.t))
                tgt.append((buf.t, False))
        acc_all = all(a for _, a in tgt)
        none_acc = not any(a for _, a in tgt)
        if acc_all or none_acc:
            K.attn_bwd(qt, kt, vt, o, do, lse, scale, True, dq=tgt[0][0], dk=tgt[1][0], dv=tgt[2][0],
                       accumulate=acc_all, **drop)
            for t, (buf, acc) in zip((q, k, v), tgt):
                if t.requires_grad and not acc:
                    t.grad = DeviceArray(buf)
        else:
            dq, dk, dv = K.attn_bwd(qt, kt, vt, o, do, lse, scale, True, **drop)
            for t, gbuf in zip((q, k, v), (dq, dk, dv)):
                if t.requires_grad:
                    _accum_grad(t, DeviceArray(gbuf), owned=True)

    out = _node(DeviceArray(o), (q, k, v), "causal_attention", _backward, _track(q, k, v))
    return out


# Source of attention dropout masks.  "host": np.random.rand(B, H, Tq, Tk) > p
# from NumPy's global RNG, the reference's draw (layers.py:120) at the same
# point of the forward, so a seeded run reproduces the reference's masks;
# "device": the Philox4x32-10 generator on the GPU (mtx_dropout_keep_philox),
# with a counter offset that advances per mask.
_DROPOUT_RNG = {"mode": "host", "seed": 0, "offset": 0}


def set_attention_dropout_rng(mode: str = "host", seed: int = 0) -> None:
    """Choose where attention dropout masks come from ("host" or "device");
    "device" restarts the Philox stream at (seed, offset 0)."""
    if mode not in ("host", "device"):
        raise ValueError(f"unknown dropout RNG mode {mode!r}")
    _DROPOUT_RNG.update(mode=mode, seed=int(seed), offset=0)


def attention_keep_mask(shape, p: float):
    """Keep-mask of a (B, H, Tq, Tk) attention matrix for drop probability p,
    as the fused kernels take it (uint8 (B, H, Tq, ld), ld = Tk rounded up to
    a multiple of 4).  Returns (mask, keep_scale)."""
    from . import _lib

    if _lib.capturing():
        # a recorded step would replay this draw (host mask or Philox
        # offset) unchanged on every call
        raise RuntimeError("attention dropout masks cannot be drawn inside a recorded (captured) step")
    B, H, Tq, Tk = (int(x) for x in shape)
    keep_scale = float(np.float32(1.0 / (1.0 - p)))
    if _DROPOUT_RNG["mode"] == "device":
        mask, _DROPOUT_RNG["offset"] = K.dropout_keep_philox(
            (B, H, Tq, Tk), p, _DROPOUT_RNG["seed"], _DROPOUT_RNG["offset"])
        return mask, keep_scale
    ld = K.keep_ld(Tk)
    host = np.zeros((B, H, Tq, ld), dtype=np.uint8)
    host[..., :Tk] = np.random.rand(B, H, Tq, Tk) > p
    return dev.from_host(host, dtype=np.uint8).t, keep_scale


def _empty(shape, dtype):
    return dev.empty_buf(shape, dtype)


def _kernel_layout(t):
    """A (B, H, T, D) view the attention kernels take as it is: unit d stride,
    16-byte aligned base and other strides."""
    vec = 16 // t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(s % vec == 0 for s in t.stride()[:-1]))


def _empty_like(t):
    """An uninitialised float32 buffer with t's shape in t's memory order."""
    return dev.empty_like_layout(t, "float32")


def cross_entropy(logits, labels):
    """Mean softmax cross-entropy of (N, V) logits against integer labels
    (loss.py:17-27: log_softmax + one-hot NLL, divided by N), fused."""
    N, V = logits.shape
    if isinstance(labels, DeviceArray):
        # device-resident labels: range is the caller's responsibility (the
        # kernel clamps; it never reads out of bounds)
        labels_d = dev.index_array(labels)
        if labels_d.size != N:
            raise ValueError("one label per row expected")
        labels_d = labels_d.reshape(N)
    else:
        lab = np.asarray(labels).reshape(-1)
        if lab.size != N:
            raise ValueError("one label per row expected")
        if lab.size and (lab.min() < 0 or lab.max() >= V):
            raise IndexError("label out of range")
        labels_d = dev.index_array(lab.astype(np.int64))
    xc = logits.data.contiguous()
    row_loss = dev.empty((N,))
    lse = dev.empty((N,))
    K.xent_fwd(xc.t, labels_d.t, row_loss.t, lse.t)
    data = dev.empty(())
    K.reduce(row_loss.t, [0], data.t.view(1), alpha=1.0 / N)
    out = None

    def _backward():
        if logits.requires_grad:
            target, acc = _grad_target(logits)
            K.xent_bwd(xc.t, labels_d.t, lse.t, out.grad.t.view(1), 1.0 / N, target.t, accumulate=acc)

    out = _node(data, (logits,), "cross_entropy", _backward, _track(logits))
    return out
