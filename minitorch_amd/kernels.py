"""Thin Python wrappers over the libmtx_hip entry points.

Each function takes device arrays (``device.DevBuf``: pointer, shape,
element strides, dtype), validates shapes on the host, calls the C ABI on the
current HIP stream and returns the outputs, allocating those not given with
the library's caching allocator.  Errors raise ``ValueError`` (bad
arguments, found before any HIP call) or ``MtxError`` (HIP failure).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L
from . import device as dev
from .device import dtype_name as _dt


def _need_cuda(*ts):
    for t in ts:
        if not getattr(t, "is_cuda", False) or not hasattr(t, "data_ptr"):
            raise ValueError("minitorch_amd kernels take device arrays")


def _bhtd(name, t):
    if t.dim() != 4:
        raise ValueError(f"{name}: expected a (B, H, T, D) tensor, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: the last (d) dimension must be contiguous")


def pack3(srcs, dst):
    """dst (rows, 3*cols) = [s0 | s1 | s2] for three contiguous fp32 (rows,
    cols) tensors (mtx_pack3_f32)."""
    s0, s1, s2 = srcs
    rows, cols = s0.shape
    _need_cuda(s0, s1, s2, dst)
    for t in (s0, s1, s2):
        if tuple(t.shape) != (rows, cols) or not t.is_contiguous() or _dt(t) != "float32":
            raise ValueError("pack3: sources must be contiguous fp32 tensors of one shape")
    if tuple(dst.shape) != (rows, 3 * cols) or not dst.is_contiguous() or _dt(dst) != "float32":
        raise ValueError(f"pack3: dst must be contiguous fp32 ({rows}, {3 * cols})")
    L.call("mtx_pack3_f32", L.ptr(s0), L.ptr(s1), L.ptr(s2), rows, cols, L.ptr(dst),
           L.stream_handle())
    return dst


def unpack3(src, dsts, accumulate=(False, False, False)):
    """d_b (rows, cols) (+)= src[:, b*cols:(b+1)*cols] (mtx_unpack3_f32)."""
    d0, d1, d2 = dsts
    rows, cols = d0.shape
    _need_cuda(src, d0, d1, d2)
    for t in (d0, d1, d2):
        if tuple(t.shape) != (rows, cols) or not t.is_contiguous() or _dt(t) != "float32":
            raise ValueError("unpack3: targets must be contiguous fp32 tensors of one shape")
    if tuple(src.shape) != (rows, 3 * cols) or not src.is_contiguous() or _dt(src) != "float32":
        raise ValueError(f"unpack3: src must be contiguous fp32 ({rows}, {3 * cols})")
    mask = sum(1 << i for i, a in enumerate(accumulate) if a)
    L.call("mtx_unpack3_f32", L.ptr(src), rows, cols, L.ptr(d0), L.ptr(d1), L.ptr(d2), mask,
           L.stream_handle())


def _check_keep(keep, B, H, Tq, Tk):
    """A dropout keep-mask as the kernels take it: contiguous uint8
    (B, H, Tq, ld) with ld >= Tk, ld % 4 == 0 (nonzero = kept)."""
    if _dt(keep) != "uint8" or not keep.is_contiguous() or keep.dim() != 4:
        raise ValueError("keep must be a contiguous uint8 (B,H,Tq,ld) tensor")
    if tuple(keep.shape[:3]) != (B, H, Tq) or keep.shape[3] < Tk or keep.shape[3] % 4:
        raise ValueError(f"keep shape {tuple(keep.shape)} does not fit (B,H,Tq)={(B, H, Tq)}, Tk={Tk}")
    if not getattr(keep, "is_cuda", False):
        raise ValueError("keep must be a device array")
    return keep.shape[3]


def keep_ld(Tk: int) -> int:
    """Row stride (bytes) of a keep-mask for Tk keys."""
    return (Tk + 3) // 4 * 4


def dropout_keep_philox(shape, p: float, seed: int, offset: int, out=None):
    """Keep-mask (B, H, Tq, keep_ld(Tk)) uint8 for dropout probability p, from
    the device Philox4x32-10 generator (mtx_dropout_keep_philox): element
    e of the logical (B*H*Tq, Tk) array uses output word e % 4 of counter
    offset + e // 4.  Returns (mask, next offset)."""
    B, H, Tq, Tk = (int(x) for x in shape)
    ld = keep_ld(Tk)
    if out is None:
        out = dev.empty_buf((B, H, Tq, ld), "uint8").fill_(0)
    rows = B * H * Tq
    L.call("mtx_dropout_keep_philox", L.ptr(out), rows, Tk, ld, float(p), int(seed) & (2**64 - 1),
           int(offset) & (2**64 - 1), L.stream_handle())
    return out, offset + (rows * Tk + 3) // 4


def attn_fwd(q, k, v, scale: float, causal: bool = True, out=None, lse=None, keep=None,
             keep_scale: float = 1.0):
    """Fused attention forward.  q: (B,H,Tq,D), k/v: (B,H,Tk,D), fp32 or bf16,
    any strides with a contiguous last dim.  Returns (out, lse) with out like q
    and lse fp32 (B,H,Tq).  keep: optional dropout keep-mask (see
    _check_keep); then out = (P * keep * keep_scale) @ v."""
    _need_cuda(q, k, v)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _bhtd(name, t)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if k.shape != (B, H, Tk, D) or v.shape != (B, H, Tk, D):
        raise ValueError(f"shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if not (_dt(q) == _dt(k) == _dt(v)):
        raise ValueError("q, k, v must share a dtype")
    if out is None:
        out = dev.empty_buf((B, H, Tq, D), _dt(q))
    if lse is None:
        lse = dev.empty_buf((B, H, Tq), "float32")
    _bhtd("out", out)
    if not lse.is_contiguous() or tuple(lse.shape) != (B, H, Tq) or _dt(lse) != "float32":
        raise ValueError("lse must be a contiguous fp32 (B,H,Tq) tensor")
    if keep is not None:
        ld = _check_keep(keep, B, H, Tq, Tk)
        L.call("mtx_attn_fwd_dropout", L.dtype_code(q), B, H, Tq, Tk, D,
               L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
               L.ptr(out), L.strides(out), L.ptr(lse), float(scale), int(bool(causal)),
               L.ptr(keep), ld, float(keep_scale), L.stream_handle())
        return out, lse
    L.call("mtx_attn_fwd", L.dtype_code(q), B, H, Tq, Tk, D,
           L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
           L.ptr(out), L.strides(out), L.ptr(lse), float(scale), int(bool(causal)),
           L.stream_handle())
    return out, lse


def attn_decode(q, k, v, scale: float, out=None, lse=None, lengths=None):
    """Decode-step attention: q (B,H,1,D) against k/v (B,H,L,D) (any strides
    with a contiguous last dim, e.g. head views of (B,T,C) caches).  lengths:
    optional int32 device tensor (B,): sequence b uses its first lengths[b]
    keys.  Returns (out (B,H,1,D) like q, lse fp32 (B,H) or None)."""
    _need_cuda(q, k, v)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _bhtd(name, t)
    B, H, Tq, D = q.shape
    Lk = k.shape[2]
    if Tq != 1 or k.shape != (B, H, Lk, D) or v.shape != (B, H, Lk, D):
        raise ValueError(f"shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if not (_dt(q) == _dt(k) == _dt(v)):
        raise ValueError("q, k, v must share a dtype")
    if out is None:
        out = dev.empty_buf((B, H, 1, D), _dt(q))
    _bhtd("out", out)
    if lse is not None and (not lse.is_contiguous() or tuple(lse.shape) != (B, H) or _dt(lse) != "float32"):
        raise ValueError("lse must be a contiguous fp32 (B,H) tensor")
    if lengths is not None and (_dt(lengths) != "int32" or tuple(lengths.shape) != (B,)
                                or not lengths.is_contiguous() or not lengths.is_cuda):
        raise ValueError("lengths must be a contiguous int32 device tensor of shape (B,)")
    L.call("mtx_attn_decode", L.dtype_code(q), B, H, Lk, D,
           L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
           L.ptr(out), L.strides(out), L.ptr(lse) if lse is not None else None,
           L.ptr(lengths) if lengths is not None else None, float(scale),
           L.stream_handle())
    return out, lse


DECODE_STEP_WIDTHS = (128, 256, 384, 512)
_DECODE_LAYER_KEYS = ("ln1_gamma", "ln1_beta", "w_qkv", "b_qkv", "w_out", "b_out", "ln2_gamma", "ln2_beta",
                      "w_fc1", "b_fc1", "w_fc2", "b_fc2", "k_cache", "v_cache")


def decode_step_fits(n_layer, C, n_head, F, V, Tmax):
    """Whether mtx_decode_step_f32 runs the model: head size 64 with C in
    {128, 256, 384, 512}, MLP width F = 4C, V <= 256, up to 16 blocks and
    1024 cache rows."""
    return (C in DECODE_STEP_WIDTHS and C == 64 * n_head and F == 4 * C
            and 1 <= V <= 256 and 1 <= n_layer <= 16 and 1 <= Tmax <= 1024)


class DecodeStep:
    """A GPT's greedy decode step as one persistent, cooperative launch
    (mtx_decode_step_f32): embeddings, every block, ln_f, lm_head and the
    pick, with grid-wide barriers between stages.

    layers: one dict per block of fp32 device arrays, contiguous, weights
    (in, out): ln1_gamma, ln1_beta, w_qkv (C, 3C) [q | k | v], b_qkv, w_out
    (C, C), b_out, ln2_gamma, ln2_beta, w_fc1 (C, F), b_fc1, w_fc2 (F, C),
    b_fc2, k_cache and v_cache (B, Tmax, C), plus ln1_eps and ln2_eps
    floats.  tok_emb (n_tok, C), pos_emb (n_pos, C), lnf = (gamma, beta,
    eps), w_head (C, V), b_head (V,).  The workspace (barrier words, residual
    rows, partial products) is allocated and zeroed here; the steps of one
    DecodeStep run in order on one stream."""

    def __init__(self, layers, tok_emb, pos_emb, lnf, w_head, b_head, B, Tmax):
        C = tok_emb.shape[1]
        F = layers[0]["w_fc1"].shape[1]
        V = w_head.shape[1]
        H = C // 64
        if not decode_step_fits(len(layers), C, H, F, V, Tmax):
            raise ValueError("decode_step: model outside the persistent step's limits")
        arrays = [tok_emb, pos_emb, lnf[0], lnf[1], w_head, b_head]
        for y in layers:
            arrays += [y[k] for k in _DECODE_LAYER_KEYS]
        for t in arrays:
            _need_cuda(t)
            if _dt(t) != "float32" or not t.is_contiguous():
                raise ValueError("decode_step: model arrays must be contiguous fp32 device arrays")
        shapes = {"w_qkv": (C, 3 * C), "b_qkv": (3 * C,), "w_out": (C, C), "b_out": (C,), "w_fc1": (C, F),
                  "b_fc1": (F,), "w_fc2": (F, C), "b_fc2": (C,), "ln1_gamma": (C,), "ln1_beta": (C,),
                  "ln2_gamma": (C,), "ln2_beta": (C,), "k_cache": (B, Tmax, C), "v_cache": (B, Tmax, C)}
        for i, y in enumerate(layers):
            for k, s in shapes.items():
                if tuple(y[k].shape) != s:
                    raise ValueError(f"decode_step: layer {i} {k} has shape {tuple(y[k].shape)}, expected {s}")
        if tuple(w_head.shape) != (C, V) or tuple(b_head.shape) != (V,) or pos_emb.shape[1] != C:
            raise ValueError("decode_step: head or embedding shapes do not match")
        self.B, self.C, self.Tmax, self.V = B, C, Tmax, V
        self._arrays = arrays  # kept alive: the structs below hold their addresses
        self._layers = (L.DecodeLayer * len(layers))()
        for i, y in enumerate(layers):
            for k in _DECODE_LAYER_KEYS:
                setattr(self._layers[i], k, y[k].data_ptr())
            self._layers[i].ln1_eps = float(y["ln1_eps"])
            self._layers[i].ln2_eps = float(y["ln2_eps"])
        m = L.DecodeModel()
        m.n_layer, m.B, m.C, m.n_head, m.F, m.V, m.Tmax = len(layers), B, C, H, F, V, Tmax
        m.tok_emb, m.n_tok = tok_emb.data_ptr(), tok_emb.shape[0]
        m.pos_emb, m.n_pos = pos_emb.data_ptr(), pos_emb.shape[0]
        m.layers = self._layers
        m.lnf_gamma, m.lnf_beta, m.lnf_eps = lnf[0].data_ptr(), lnf[1].data_ptr(), float(lnf[2])
        m.w_head, m.b_head = w_head.data_ptr(), b_head.data_ptr()
        self._model = m
        nbytes = L.lib().mtx_decode_step_workspace_bytes(B, C, H, F)
        self.workspace = dev.zeros(((nbytes + 3) // 4,), "int32").t
        self._ws_bytes = self.workspace.numel() * 4

    def __call__(self, cur, ids, lengths, pos, margins=None, t_base=0, wait_limit_us=0, steps=1):
        """`steps` token steps in one launch.  A step reads cur (B,) int64
        and pos (1,) int64, appends to the caches at row lengths[b] - 1,
        writes the pick to cur and ids (Tmax, B) at row lengths[b], the top-2
        margin to margins (n, B) at row lengths[b] - t_base, then lengths +=
        1 and pos += 1.  wait_limit_us bounds each grid-wide wait (0: the
        library's 2 s; negative: every wait fails, for tests of the failure
        path)."""
        B = self.B
        _need_cuda(cur, ids, lengths, pos)
        if _dt(cur) != "int64" or cur.numel() != B or not cur.is_contiguous():
            raise ValueError("decode_step: cur must be contiguous int64 (B,)")
        if _dt(ids) != "int64" or ids.dim() != 2 or ids.shape[1] != B or not ids.is_contiguous():
            raise ValueError("decode_step: ids must be contiguous int64 (Tmax, B)")
        if _dt(lengths) != "int32" or lengths.numel() != B or not lengths.is_contiguous():
            raise ValueError("decode_step: lengths must be contiguous int32 (B,)")
        if _dt(pos) != "int64" or pos.numel() < 1:
            raise ValueError("decode_step: pos must be int64")
        if margins is not None and (_dt(margins) != "float32" or margins.dim() != 2 or margins.shape[1] != B
                                    or not margins.is_contiguous()):
            raise ValueError("decode_step: margins must be contiguous fp32 (n, B)")
        L.call("mtx_decode_step_f32", ctypes.addressof(self._model), int(steps), L.ptr(cur), L.ptr(ids),
               L.ptr(margins) if margins is not None else None, int(t_base),
               margins.shape[0] if margins is not None else 0, L.ptr(lengths), L.ptr(pos),
               L.ptr(self.workspace), self._ws_bytes, int(wait_limit_us), L.stream_handle())

    def check(self):
        """Synchronise and raise MtxError if a step's grid-wide wait ran out
        (that step's results are incomplete; later steps did nothing)."""
        L.call("mtx_decode_step_status", L.ptr(self.workspace), L.stream_handle())

    def reset(self):
        """Clear the barrier words and the error word."""
        L.call("mtx_decode_step_reset", L.ptr(self.workspace), L.stream_handle())


QKV_ATTN_MAX_C, QKV_ATTN_MAX_T = 1024, 2048


def qkv_attn_fits(H, D, Tmax):
    """True when mtx_decode_qkv_attn_f32 takes heads of size D, H*D columns
    and caches of Tmax rows."""
    return D in (64, 128) and H * D <= QKV_ATTN_MAX_C and 1 <= Tmax <= QKV_ATTN_MAX_T


def _pending_args(pending, ln, rows, C):
    """ctypes arguments (pws, pks, pbias) and (gamma, beta, eps) of the
    pending-update input mode of mtx_decode_qkv_attn_f32 / mtx_head_pick_f32."""
    if ln is None:
        if pending is not None:
            raise ValueError("pending partial products need the LayerNorm (ln)")
        return (None, 0, None), (None, None, 0.0)
    gamma, beta, eps = ln
    if gamma.numel() != C or beta.numel() != C or not (gamma.is_contiguous() and beta.is_contiguous()):
        raise ValueError(f"ln: gamma and beta must be contiguous with {C} elements")
    if C > 1024:
        raise ValueError("the LayerNorm input mode needs rows of at most 1024 values")
    lnargs = (L.ptr(gamma), L.ptr(beta), float(eps))
    if pending is None:
        return (None, 0, None), lnargs
    ws, ks, pbias = pending
    if not 1 <= int(ks) <= 8 or ws.numel() * ws.element_size() < int(ks) * rows * C * 4:
        raise ValueError("pending: 1 to 8 partial products of (rows, C) fp32")
    if pbias is not None and (pbias.numel() != C or not pbias.is_contiguous()):
        raise ValueError(f"pending: bias must be contiguous with {C} elements")
    return (L.ptr(ws), int(ks), L.ptr(pbias) if pbias is not None else None), lnargs


def gemm_partials(a, b, ws=None):
    """mtx_gemm_partials_f32: the K ranges' partial products of a (M, K) @
    b (K, N) into ws ([ks][M][N] fp32; allocated when None).  Returns
    (ws, ks).  Summed in range order they are mtx_gemm_ln_f32's product."""
    import ctypes

    M, Kd = a.shape[-2], a.shape[-1]
    N = b.shape[-1]
    if _dt(a) != "float32" or _dt(b) != "float32" or b.shape[-2] != Kd:
        raise ValueError("gemm_partials: fp32 a (M, K) and b (K, N)")
    nbytes = L.lib().mtx_gemm_ln_workspace_bytes(M, N, Kd)
    if ws is None:
        ws = dev.empty_buf((nbytes // 4,), "float32")
    ks = ctypes.c_int(0)
    L.call("mtx_gemm_partials_f32", int(M), int(N), int(Kd), L.ptr(a), int(a.stride(-2)), int(a.stride(-1)),
           L.ptr(b), int(b.stride(-2)), int(b.stride(-1)), L.ptr(ws), ws.numel() * ws.element_size(),
           ctypes.byref(ks), L.stream_handle())
    return ws, ks.value


def qkv_attn_step(x, w, bias, kc, vc, lengths, n_head, scale, out, pending=None, x_out=None, ln=None):
    """mtx_decode_qkv_attn_f32: one decode step's q/k/v projection and
    attention in one launch.  x (B, C) the input rows, w (C, 3C) and bias
    (3C,) the packed [q | k | v] projection; this step's k and v go to row
    lengths[b] - 1 of the caches kc / vc (B, Tmax, C), and out (B, C)
    receives softmax(scale q k^T) v over each sequence's first lengths[b]
    cached rows, head h in columns h*D .. h*D + D - 1.  Without ln the rows
    of x are the normalised input; with ln = (gamma, beta, eps) they are raw
    residual rows r (plus, with pending = (ws, ks, bias), the previous
    block's pending update r = (sum of the ks partial products + bias) + x,
    written to x_out) and the projection reads LayerNorm(r)."""
    _need_cuda(x, w, kc, vc, lengths, out)
    B, C = x.shape
    H = int(n_head)
    D = C // H
    Bc, Tmax, Ck = kc.shape
    if H * D != C or tuple(w.shape) != (C, 3 * C) or Ck != C or Bc < B or tuple(out.shape) != (B, C):
        raise ValueError("qkv_attn_step: x (B, C), w (C, 3C), caches (>= B, T, C), out (B, C)")
    if tuple(vc.shape) != tuple(kc.shape) or tuple(vc.stride()) != tuple(kc.stride()) or kc.stride(2) != 1:
        raise ValueError("qkv_attn_step: k/v caches must share shape and strides, unit column stride")
    if x.stride(1) != 1 or w.stride(1) != 1 or out.stride(1) != 1:
        raise ValueError("qkv_attn_step: x, w and out need unit column strides")
    if bias is not None and (bias.numel() != 3 * C or not bias.is_contiguous()):
        raise ValueError("qkv_attn_step: bias must be contiguous (3C,)")
    if _dt(lengths) != "int32" or lengths.numel() < B or not lengths.is_contiguous():
        raise ValueError("qkv_attn_step: lengths must be contiguous int32 with >= B entries")
    pargs, lnargs = _pending_args(pending, ln, B, C)
    if x_out is not None and (ln is None or tuple(x_out.shape) != (B, C) or x_out.stride(1) != 1):
        raise ValueError("qkv_attn_step: x_out (B, C) with a unit column stride, with ln")
    L.call("mtx_decode_qkv_attn_f32", B, H, D, L.ptr(x), x.stride(0), *pargs,
           L.ptr(x_out) if x_out is not None else None, x_out.stride(0) if x_out is not None else 0, *lnargs,
           L.ptr(w), w.stride(0), L.ptr(bias) if bias is not None else None, L.ptr(kc), L.ptr(vc),
           kc.stride(0), kc.stride(1), Tmax, L.ptr(lengths), float(scale), L.ptr(out), out.stride(0),
           L.stream_handle())
    return out


def argmax_rows(x, idx=None, margin=None):
    """First-maximum index of each row of a fp32 (rows, cols) device tensor
    (np.argmax) and, if `margin` is given, largest - second largest.  idx:
    int64 (rows,) or a strided column view; returns (idx, margin)."""
    _need_cuda(x)
    if _dt(x) != "float32" or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a fp32 (rows, cols) tensor with contiguous rows")
    rows, cols = x.shape
    if idx is None:
        idx = dev.empty_buf((rows,), "int64")
    if _dt(idx) != "int64" or idx.numel() != rows:
        raise ValueError("idx must be int64 with one entry per row")
    if margin is not None and (_dt(margin) != "float32" or margin.numel() != rows):
        raise ValueError("margin must be fp32 with one entry per row")
    L.call("mtx_argmax_f32", rows, cols, L.ptr(x), x.stride(0), L.ptr(idx), idx.stride(0) if idx.dim() else 1,
           L.ptr(margin) if margin is not None else None, margin.stride(0) if margin is not None else 0,
           L.stream_handle())
    return idx, margin


def kv_append(x, cache, lengths):
    """cache[b, lengths[b] - 1, :] = x[b, 0, :]: x (B, 1, C) fp32, cache
    (B, T, C) fp32 with contiguous rows, lengths int32 device (B,)."""
    _need_cuda(x, cache, lengths)
    B, T, C = cache.shape
    if _dt(x) != "float32" or _dt(cache) != "float32" or tuple(x.shape) != (B, 1, C):
        raise ValueError(f"kv_append: x{tuple(x.shape)} / cache{tuple(cache.shape)} mismatch (fp32 needed)")
    if x.stride(2) != 1 or cache.stride(2) != 1 or _dt(lengths) != "int32" or tuple(lengths.shape) != (B,):
        raise ValueError("kv_append: contiguous rows and int32 lengths (B,) needed")
    L.call("mtx_kv_append_f32", B, C, T, L.ptr(x), x.stride(0), L.ptr(cache), cache.stride(0), cache.stride(1),
           L.ptr(lengths), L.stream_handle())


def decode_advance(lengths, pos=None):
    """lengths += 1 (int32 device (B,)) and pos += 1 (int64 device (1,))."""
    _need_cuda(lengths)
    if _dt(lengths) != "int32" or lengths.dim() != 1 or not lengths.is_contiguous():
        raise ValueError("lengths must be a contiguous int32 device vector")
    if pos is not None and (_dt(pos) != "int64" or not pos.is_cuda):
        raise ValueError("pos must be an int64 device tensor")
    L.call("mtx_decode_advance", lengths.numel(), L.ptr(lengths), L.ptr(pos) if pos is not None else None,
           L.stream_handle())


def attn_bwd(q, k, v, out, dout, lse, scale: float, causal: bool = True,
             dq=None, dk=None, dv=None, accumulate: bool = False, workspace=None,
             phases: int = L.ATTN_BWD_ALL, keep=None, keep_scale: float = 1.0):
    """Fused attention backward.  Returns fp32 (dq, dk, dv).  With
    accumulate=True the given dq/dk/dv are added to instead of overwritten.
    keep/keep_scale: the forward's dropout mask (all phases only)."""
    _need_cuda(q, k, v, out, dout, lse)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out), ("dout", dout)):
        _bhtd(name, t)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if tuple(out.shape) != tuple(q.shape) or tuple(dout.shape) != tuple(q.shape):
        raise ValueError("out and dout must have q's shape")
    if not (_dt(q) == _dt(k) == _dt(v) == _dt(out) == _dt(dout)):
        raise ValueError("q, k, v, out, dout must share a dtype")
    if dq is None:
        dq = dev.empty_buf((B, H, Tq, D), "float32")
    if dk is None:
        dk = dev.empty_buf((B, H, Tk, D), "float32")
    if dv is None:
        dv = dev.empty_buf((B, H, Tk, D), "float32")
    for name, t, shp in (("dq", dq, (B, H, Tq, D)), ("dk", dk, (B, H, Tk, D)), ("dv", dv, (B, H, Tk, D))):
        if tuple(t.shape) != shp or _dt(t) != "float32":
            raise ValueError(f"{name} must be fp32 with shape {shp}")
        _bhtd(name, t)
    nbytes = L.lib().mtx_attn_bwd_workspace_bytes(B, H, Tq)
    if workspace is None:
        workspace = dev.empty_buf((nbytes,), "uint8")
    if keep is not None:
        if int(phases) != L.ATTN_BWD_ALL:
            raise ValueError("the dropout backward runs all phases")
        ld = _check_keep(keep, B, H, Tq, Tk)
        L.call("mtx_attn_bwd_dropout", L.dtype_code(q), B, H, Tq, Tk, D,
               L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
               L.ptr(out), L.strides(out), L.ptr(dout), L.strides(dout), L.ptr(lse),
               L.ptr(dq), L.strides(dq), L.ptr(dk), L.strides(dk), L.ptr(dv), L.strides(dv),
               L.ptr(workspace), workspace.numel() * workspace.element_size(),
               float(scale), int(bool(causal)), int(bool(accumulate)), L.ptr(keep), ld,
               float(keep_scale), L.stream_handle())
        return dq, dk, dv
    L.call("mtx_attn_bwd_phase", int(phases), L.dtype_code(q), B, H, Tq, Tk, D,
           L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
           L.ptr(out), L.strides(out), L.ptr(dout), L.strides(dout), L.ptr(lse),
           L.ptr(dq), L.strides(dq), L.ptr(dk), L.strides(dk), L.ptr(dv), L.strides(dv),
           L.ptr(workspace), workspace.numel() * workspace.element_size(),
           float(scale), int(bool(causal)), int(bool(accumulate)), L.stream_handle())
    return dq, dk, dv


def attn_bwd_noalloc(q, k, v, out, dout, lse, scale: float, causal: bool, dq, dk, dv,
                     accumulate: bool = False):
    """mtx_attn_bwd_noalloc: attn_bwd into caller-given dq/dk/dv with the
    library's fixed device scratch for delta (no allocation of any kind; at
    most ATTN_SCRATCH_BYTES / 4 rows B*H*Tq)."""
    _need_cuda(q, k, v, out, dout, lse, dq, dk, dv)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out), ("dout", dout), ("dq", dq), ("dk", dk),
                    ("dv", dv)):
        _bhtd(name, t)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    L.call("mtx_attn_bwd_noalloc", L.dtype_code(q), B, H, Tq, Tk, D,
           L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
           L.ptr(out), L.strides(out), L.ptr(dout), L.strides(dout), L.ptr(lse),
           L.ptr(dq), L.strides(dq), L.ptr(dk), L.strides(dk), L.ptr(dv), L.strides(dv),
           float(scale), int(bool(causal)), int(bool(accumulate)), L.stream_handle())
    return dq, dk, dv


# ---------------------------------------------------------------------------
# generic elementwise / reductions
# ---------------------------------------------------------------------------

def _i64(seq):
    seq = tuple(int(x) for x in seq)
    return (L.C.c_int64 * max(1, len(seq)))(*seq)


def _bstrides(t, shape):
    """Element strides of `t` broadcast to `shape` (0 on broadcast axes)."""
    nd = len(shape)
    ts, tst = tuple(t.shape), tuple(t.stride())
    pad = nd - len(ts)
    if pad < 0:
        raise ValueError(f"cannot broadcast shape {ts} to {tuple(shape)}")
    out = []
    for d in range(nd):
        if d < pad:
            out.append(0)
            continue
        sz = ts[d - pad]
        if sz == shape[d]:
            out.append(tst[d - pad] if sz != 1 else 0)
        elif sz == 1:
            out.append(0)
        else:
            raise ValueError(f"cannot broadcast shape {ts} to {tuple(shape)}")
    return out


def ewise(op: str, out, a=None, b=None, alpha: float = 1.0, beta: float = 0.0, accumulate=False):
    """out (+)= op(a, b), broadcasting a and b to out's shape."""
    shape = tuple(out.shape)
    nd = len(shape)
    if nd > 8:
        raise ValueError("at most 8 dimensions")
    sa = _i64(_bstrides(a, shape)) if a is not None else None
    sb = _i64(_bstrides(b, shape)) if b is not None else None
    L.call("mtx_ewise_f32", L.EW[op], nd, _i64(shape),
           L.ptr(a) if a is not None else None, sa,
           L.ptr(b) if b is not None else None, sb,
           L.ptr(out), _i64(out.stride()), float(alpha), float(beta), int(bool(accumulate)),
           L.stream_handle())
    return out


def fill(out, value: float):
    shape = tuple(out.shape)
    L.call("mtx_ewise_f32", L.EW["FILL"], len(shape), _i64(shape), None, None, None, None,
           L.ptr(out), _i64(out.stride()), float(value), 0.0, 0, L.stream_handle())
    return out


def reduce(a, axes, out, op=L.RED_SUM, alpha: float = 1.0, accumulate=False):
    """out (+)= alpha * reduce(a over `axes`); out is contiguous with the kept
    axes of a in order (any shape with that many elements)."""
    shape = tuple(a.shape)
    nd = len(shape)
    axes = {ax % nd for ax in axes} if nd else set()
    mask = (L.C.c_int * max(1, nd))(*[1 if d in axes else 0 for d in range(nd)])
    shp = _i64(shape)
    ws_bytes = L.lib().mtx_reduce_workspace_bytes(nd, shp, mask)
    ws = dev.empty_buf((ws_bytes,), "uint8") if ws_bytes else None
    if not out.is_contiguous():
        raise ValueError("reduce output must be contiguous")
    L.call("mtx_reduce_f32", int(op), nd, shp, L.ptr(a), _i64(a.stride()), mask, L.ptr(out),
           float(alpha), int(bool(accumulate)), L.ptr(ws) if ws is not None else None, ws_bytes,
           L.stream_handle())
    return out


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

GEMM_ACT_NONE, GEMM_ACT_GELU, GEMM_ACT_GELU_BWD, GEMM_ACT_ADD = 0, 1, 2, 4


def gemm_ln_fits(M, K, N):
    """Whether mtx_gemm_ln_f32 takes an (M, K) @ (K, N) product."""
    return 1 <= M <= 64 and 1 <= K <= 4096 and 1 <= N <= 2048


def gemm_ln(a, b, c, gamma, beta_ln, eps, y, bias=None, alpha=1.0, beta=1.0):
    """c = alpha * a @ b + bias + beta * c, then y = LayerNorm(rows of c)
    with gamma, beta_ln, eps (mtx_gemm_ln_f32: a decode step's residual
    projection and the LayerNorm after it; a (M, K) with M <= 64, b (K, N),
    c and y (M, N) with unit column strides)."""
    M, K = a.shape[-2], a.shape[-1]
    N = b.shape[-1]
    for name, t in (("a", a), ("b", b), ("c", c), ("y", y), ("gamma", gamma), ("beta", beta_ln)):
        if _dt(t) != "float32":
            raise ValueError(f"gemm_ln: {name} must be fp32")
    if tuple(c.shape[-2:]) != (M, N) or tuple(y.shape[-2:]) != (M, N) or c.stride(-1) != 1 or y.stride(-1) != 1:
        raise ValueError(f"gemm_ln: c and y must be ({M}, {N}) with unit column strides")
    if gamma.numel() != N or beta_ln.numel() != N or not (gamma.is_contiguous() and beta_ln.is_contiguous()):
        raise ValueError(f"gemm_ln: gamma and beta must be contiguous with N={N} elements")
    ws_bytes = L.lib().mtx_gemm_ln_workspace_bytes(M, N, K)
    ws = dev.empty_buf((ws_bytes,), "uint8") if ws_bytes else None
    L.call("mtx_gemm_ln_f32", int(M), int(N), int(K), float(alpha), L.ptr(a), int(a.stride(-2)),
           int(a.stride(-1)), L.ptr(b), int(b.stride(-2)), int(b.stride(-1)), float(beta), L.ptr(c),
           int(c.stride(-2)), L.ptr(bias) if bias is not None else None, L.ptr(gamma), L.ptr(beta_ln),
           float(eps), L.ptr(y), int(y.stride(-2)), L.ptr(ws) if ws is not None else None, ws_bytes,
           L.stream_handle())
    return y


GEMM_FP32, GEMM_BF16X3 = L.MTX_GEMM_FP32, L.MTX_GEMM_BF16X3


def set_gemm_mode(mode: int) -> int:
    """Select how products of at least 128 x 128 are computed
    (mtx_gemm_set_mode): GEMM_BF16X3 (the default: fp32 values split into
    three bf16 pieces on the bf16 matrix cores, fp32-accurate) or GEMM_FP32
    (fp32 MFMA).  Returns the previous mode."""
    prev = int(L.lib().mtx_gemm_get_mode())
    L.call("mtx_gemm_set_mode", int(mode))
    return prev


def get_gemm_mode() -> int:
    return int(L.lib().mtx_gemm_get_mode())


def set_attn_mode(mode: int) -> int:
    """Select how fp32 attention with 64-wide heads computes its
    products (mtx_attn_set_mode): GEMM_BF16X3 (the default: three bf16
    pieces per fp32 value on the bf16 matrix cores) or GEMM_FP32 (fp32
    MFMA).  Returns the previous mode."""
    prev = int(L.lib().mtx_attn_get_mode())
    L.call("mtx_attn_set_mode", int(mode))
    return prev


def get_attn_mode() -> int:
    return int(L.lib().mtx_attn_get_mode())


ATTN_BWD_TWOPASS, ATTN_BWD_ONEPASS = L.ATTN_BWD_TWOPASS, L.ATTN_BWD_ONEPASS


def set_attn_bwd_mode(mode: int) -> int:
    """Select how the backward of bf16 attention with D <= 64 runs
    (mtx_attn_set_bwd_mode): ATTN_BWD_TWOPASS (the default: deterministic
    dQ and dK/dV passes) or ATTN_BWD_ONEPASS (one key-outer kernel writes
    dK/dV and adds dQ with fp32 atomics, after a delta kernel that zeroes
    dq).  Returns the previous mode."""
    prev = int(L.lib().mtx_attn_get_bwd_mode())
    L.call("mtx_attn_set_bwd_mode", int(mode))
    return prev


def get_attn_bwd_mode() -> int:
    return int(L.lib().mtx_attn_get_bwd_mode())


def attn_bwd_onepass_used(dtype: str, D: int) -> bool:
    """Whether attn_bwd (all phases, no dropout) takes the one-pass kernels
    for this input dtype and head size."""
    return dtype == "bfloat16" and D <= 64 and get_attn_bwd_mode() == ATTN_BWD_ONEPASS


def gemm(a, b, c, alpha=1.0, beta=0.0, bias=None, M=None, N=None, K=None, batch=1,
         sa=None, sb=None, sc=None, act=GEMM_ACT_NONE, aux=None, colsum=None, colsum_accumulate=False):
    """C = alpha*A@B + beta*C (+bias) with explicit (row, col, batch) strides
    for each operand; defaults take them from 2-D/3-D tensors.  act/aux: the
    GELU epilogues of mtx_gemm_act_f32 (aux shaped like C: the pre-activation
    written by act 1, read by act 2), or GEMM_ACT_ADD: C = ... + aux (a
    residual stream, not C itself).  colsum: a contiguous (N,) tensor that
    receives (or, with colsum_accumulate, adds) the column sums of B -- a
    Linear layer's bias gradient next to its weight gradient
    (mtx_gemm_wgrad_f32: batch 1, alpha 1, no bias or activation)."""
    if sa is None:
        sa = (a.stride(-2), a.stride(-1), a.stride(0) if a.dim() == 3 else 0)
    if sb is None:
        sb = (b.stride(-2), b.stride(-1), b.stride(0) if b.dim() == 3 else 0)
    if sc is None:
        sc = (c.stride(-2), c.stride(-1), c.stride(0) if c.dim() == 3 else 0)
    M = a.shape[-2] if M is None else M
    K = a.shape[-1] if K is None else K
    N = b.shape[-1] if N is None else N
    for name, t in (("A", a), ("B", b), ("C", c), ("bias", bias), ("aux", aux)):
        if t is not None and _dt(t) != "float32":
            raise ValueError(f"gemm: {name} must be fp32 (got {t.dtype})")
    # one operand stride must be unit; otherwise the caller passes a copy
    ws_bytes = L.lib().mtx_gemm_workspace_bytes(M, N, K, batch)
    ws = dev.empty_buf((ws_bytes,), "uint8") if ws_bytes else None
    if colsum is not None:
        if batch != 1 or alpha != 1.0 or bias is not None or act != GEMM_ACT_NONE:
            raise ValueError("gemm: colsum needs batch 1, alpha 1 and no bias or activation")
        if _dt(colsum) != "float32" or colsum.numel() != N or not colsum.is_contiguous():
            raise ValueError(f"gemm: colsum must be a contiguous fp32 tensor of N={N} elements")
        L.call("mtx_gemm_wgrad_f32", int(M), int(N), int(K), L.ptr(a), int(sa[0]), int(sa[1]),
               L.ptr(b), int(sb[0]), int(sb[1]), float(beta), L.ptr(c), int(sc[0]), int(sc[1]),
               L.ptr(colsum), int(bool(colsum_accumulate)),
               L.ptr(ws) if ws is not None else None, ws_bytes, L.stream_handle())
        return c
    if act != GEMM_ACT_NONE:
        if aux is not None:
            if tuple(aux.shape[-2:]) != (M, N) or _dt(aux) != "float32":
                raise ValueError(f"gemm: aux must be fp32 with C's shape ({M}, {N})")
            sx = (aux.stride(-2), aux.stride(-1), aux.stride(0) if aux.dim() == 3 else 0)
        elif act in (GEMM_ACT_GELU_BWD, GEMM_ACT_ADD):
            raise ValueError("gemm: this epilogue needs aux")
        else:
            sx = (0, 0, 0)
        L.call("mtx_gemm_act_f32", int(M), int(N), int(K), int(batch),
               float(alpha), L.ptr(a), int(sa[0]), int(sa[1]), int(sa[2]),
               L.ptr(b), int(sb[0]), int(sb[1]), int(sb[2]),
               float(beta), L.ptr(c), int(sc[0]), int(sc[1]), int(sc[2]),
               L.ptr(bias) if bias is not None else None, int(act),
               L.ptr(aux) if aux is not None else None, int(sx[0]), int(sx[1]), int(sx[2]),
               L.ptr(ws) if ws is not None else None, ws_bytes, L.stream_handle())
        return c
    L.call("mtx_gemm_f32", int(M), int(N), int(K), int(batch),
           float(alpha), L.ptr(a), int(sa[0]), int(sa[1]), int(sa[2]),
           L.ptr(b), int(sb[0]), int(sb[1]), int(sb[2]),
           float(beta), L.ptr(c), int(sc[0]), int(sc[1]), int(sc[2]),
           L.ptr(bias) if bias is not None else None,
           L.ptr(ws) if ws is not None else None, ws_bytes, L.stream_handle())
    return c


# size limits of mtx_gemm_step_f32 (one-launch decode-step projections)
STEP_MAX_M, STEP_MAX_K = 64, 512
ACT_NONE, ACT_GELU = 0, 1


def step_fits(M, K):
    """True when mtx_gemm_step_f32 takes an (M, K) activation."""
    return 1 <= M <= STEP_MAX_M and 1 <= K <= STEP_MAX_K


def gemm_step(a, b, bias=None, c=None, beta=0.0, act=ACT_NONE, kv=None):
    """One decode-step projection: P = a @ b + bias, a (M, K) with unit k
    stride, b (K, N) with unit n stride.  Columns of P go to c (M, Nc) as
    act(P + beta*c); with kv = (kcache, vcache, lengths) the last 2*Ck columns
    go to the caches (B, T, Ck) at row lengths[m] - 1 instead (Nc = N - 2*Ck)."""
    M, Kd = a.shape
    N = b.shape[1]
    if a.stride(1) != 1 or b.stride(1) != 1 or b.shape[0] != Kd:
        raise ValueError("gemm_step: a (M, K) and b (K, N) need unit inner strides")
    if kv is not None:
        kc, vc, lengths = kv
        _need_cuda(kc, vc, lengths)
        Bc, T, Ck = kc.shape
        if tuple(vc.shape) != tuple(kc.shape) or tuple(vc.stride()) != tuple(kc.stride()) or kc.stride(2) != 1 \
                or Bc < M:
            raise ValueError("gemm_step: k/v caches must be (B >= M, T, C) with equal strides")
        if _dt(lengths) != "int32" or lengths.numel() < M:
            raise ValueError("gemm_step: lengths must be int32 with >= M entries")
        nc = N - 2 * Ck
        cache_args = (L.ptr(kc), L.ptr(vc), kc.stride(0), kc.stride(1), T, L.ptr(lengths))
    else:
        nc = N
        cache_args = (None, None, 0, 0, 0, None)
    if nc < 0:
        raise ValueError("gemm_step: N too small for the cache columns")
    if nc > 0:
        if c is None or tuple(c.shape) != (M, nc) or c.stride(1) != 1:
            raise ValueError(f"gemm_step: c must be ({M}, {nc}) with unit column stride")
    L.call("mtx_gemm_step_f32", int(M), int(N), int(Kd), L.ptr(a), a.stride(0), L.ptr(b), b.stride(0),
           float(beta), L.ptr(c) if nc > 0 else None, c.stride(0) if nc > 0 else 0,
           L.ptr(bias) if bias is not None else None, int(act), int(nc), *cache_args, L.stream_handle())
    return c


def greedy_pick(x, cur, ids, lengths, pos=None, margins=None, t_base=0):
    """mtx_greedy_pick_f32: per row of x (rows, cols) the first-maximum index
    to cur (int64 (rows,)) and to ids[lengths[row], row] (int64 (Tmax, rows)),
    the top-2 margin to margins[lengths[row] - t_base, row] (float32
    (n, rows)); then lengths += 1 (int32 (rows,)) and pos += 1."""
    _need_cuda(x, cur, ids, lengths)
    rows, cols = x.shape
    if _dt(x) != "float32" or x.stride(1) != 1:
        raise ValueError("greedy_pick: x must be fp32 with contiguous rows")
    if _dt(cur) != "int64" or cur.numel() != rows or not cur.is_contiguous():
        raise ValueError("greedy_pick: cur must be contiguous int64 (rows,)")
    if _dt(ids) != "int64" or ids.dim() != 2 or ids.shape[1] != rows or not ids.is_contiguous():
        raise ValueError("greedy_pick: ids must be contiguous int64 (Tmax, rows)")
    if _dt(lengths) != "int32" or lengths.numel() != rows or not lengths.is_contiguous():
        raise ValueError("greedy_pick: lengths must be contiguous int32 (rows,)")
    if pos is not None and _dt(pos) != "int64":
        raise ValueError("greedy_pick: pos must be int64")
    if margins is not None and (_dt(margins) != "float32" or margins.dim() != 2 or margins.shape[1] != rows
                                or not margins.is_contiguous()):
        raise ValueError("greedy_pick: margins must be contiguous fp32 (n, rows)")
    L.call("mtx_greedy_pick_f32", rows, cols, L.ptr(x), x.stride(0), L.ptr(cur), L.ptr(ids), ids.shape[0],
           L.ptr(margins) if margins is not None else None, int(t_base),
           margins.shape[0] if margins is not None else 0, L.ptr(lengths),
           L.ptr(pos) if pos is not None else None, L.stream_handle())


def embedding2_fwd(wa, ia, wb, ib, out, ib_stride=1):
    """out (n, C) = wa[ia] + wb[ib] (mtx_embedding2_fwd_f32); ib_stride 0
    broadcasts ib[0]."""
    Va, C = wa.shape
    Vb = wb.shape[0]
    n = ia.numel()
    if _dt(ia) != "int64" or _dt(ib) != "int64" or wb.shape[1] != C or out.shape[-1] != C:
        raise ValueError("embedding2: int64 ids and tables / output of one width")
    if wa.stride(1) != 1 or wb.stride(1) != 1 or out.stride(-1) != 1 or not ia.is_contiguous():
        raise ValueError("embedding2: rows must be contiguous")
    if ib_stride and ib.numel() < n:
        raise ValueError("embedding2: ib has fewer ids than ia")
    L.call("mtx_embedding2_fwd_f32", L.ptr(wa), wa.stride(0), Va, L.ptr(ia), L.ptr(wb), wb.stride(0), Vb,
           L.ptr(ib), int(ib_stride), L.ptr(out), out.stride(-2) if out.dim() >= 2 else C, n, C, L.stream_handle())
    return out


def embedding2_ln_fwd(wa, ia, wb, ib, out, gamma, beta, eps, y, ib_stride=1):
    """out (n, C) = wa[ia] + wb[ib] and y = LayerNorm(out) with gamma, beta,
    eps in one launch (mtx_embedding2_ln_fwd_f32)."""
    Va, C = wa.shape
    Vb = wb.shape[0]
    n = ia.numel()
    if _dt(ia) != "int64" or _dt(ib) != "int64" or wb.shape[1] != C or out.shape[-1] != C or y.shape[-1] != C:
        raise ValueError("embedding2_ln: int64 ids and tables / outputs of one width")
    if (wa.stride(1) != 1 or wb.stride(1) != 1 or out.stride(-1) != 1 or y.stride(-1) != 1
            or not ia.is_contiguous()):
        raise ValueError("embedding2_ln: rows must be contiguous")
    if gamma.numel() != C or beta.numel() != C or not (gamma.is_contiguous() and beta.is_contiguous()):
        raise ValueError("embedding2_ln: gamma and beta must be contiguous with C elements")
    if ib_stride and ib.numel() < n:
        raise ValueError("embedding2_ln: ib has fewer ids than ia")
    L.call("mtx_embedding2_ln_fwd_f32", L.ptr(wa), wa.stride(0), Va, L.ptr(ia), L.ptr(wb), wb.stride(0), Vb,
           L.ptr(ib), int(ib_stride), L.ptr(out), out.stride(-2) if out.dim() >= 2 else C, n, C,
           L.ptr(gamma), L.ptr(beta), float(eps), L.ptr(y), y.stride(-2) if y.dim() >= 2 else C,
           L.stream_handle())
    return y


def head_pick(x, w, bias, cur, ids, lengths, pos=None, margins=None, t_base=0, pending=None, ln=None):
    """mtx_head_pick_f32: logits = x @ w + bias per row of x (rows, K), w
    (K, V), then the pick of greedy_pick on them (cur, ids, margins,
    lengths, pos) in one launch.  With ln = (gamma, beta, eps) the rows are
    raw (plus pending = (ws, ks, bias) as in qkv_attn_step) and the product
    reads their LayerNorm."""
    _need_cuda(x, w, cur, ids, lengths)
    rows, Kd = x.shape
    V = w.shape[1]
    if _dt(x) != "float32" or _dt(w) != "float32" or x.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("head_pick: x and w must be fp32 with contiguous rows")
    if w.shape[0] != Kd or (bias is not None and (bias.numel() != V or not bias.is_contiguous())):
        raise ValueError("head_pick: w must be (K, V) and bias (V,)")
    if _dt(cur) != "int64" or cur.numel() != rows or not cur.is_contiguous():
        raise ValueError("head_pick: cur must be contiguous int64 (rows,)")
    if _dt(ids) != "int64" or ids.dim() != 2 or ids.shape[1] != rows or not ids.is_contiguous():
        raise ValueError("head_pick: ids must be contiguous int64 (Tmax, rows)")
    if _dt(lengths) != "int32" or lengths.numel() != rows or not lengths.is_contiguous():
        raise ValueError("head_pick: lengths must be contiguous int32 (rows,)")
    if pos is not None and _dt(pos) != "int64":
        raise ValueError("head_pick: pos must be int64")
    if margins is not None and (_dt(margins) != "float32" or margins.dim() != 2 or margins.shape[1] != rows
                                or not margins.is_contiguous()):
        raise ValueError("head_pick: margins must be contiguous fp32 (n, rows)")
    pargs, lnargs = _pending_args(pending, ln, rows, Kd)
    L.call("mtx_head_pick_f32", rows, Kd, V, L.ptr(x), x.stride(0), *pargs, *lnargs, L.ptr(w), w.stride(0),
           L.ptr(bias) if bias is not None else None, L.ptr(cur), L.ptr(ids), ids.shape[0],
           L.ptr(margins) if margins is not None else None, int(t_base),
           margins.shape[0] if margins is not None else 0, L.ptr(lengths),
           L.ptr(pos) if pos is not None else None, L.stream_handle())


# ---------------------------------------------------------------------------
# row kernels
# ---------------------------------------------------------------------------

def _rows(t):
    """(rows, L, leading stride) of a tensor whose last axis is contiguous and
    whose leading axes collapse to one row index."""
    if t.stride(-1) != 1:
        raise ValueError("last axis must be contiguous")
    Lx = t.shape[-1]
    rows = t.numel() // Lx if Lx else 0
    if t.dim() == 1:
        return 1, Lx, Lx
    # leading axes must collapse with a single stride
    ld = t.stride(-2)
    expect = ld * t.shape[-2]
    for d in range(t.dim() - 3, -1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            raise ValueError("leading axes do not collapse")
        expect *= t.shape[d]
    return rows, Lx, ld


def softmax_fwd(x, y, causal_tq=0, log=False):
    rx, Lx, ldx = _rows(x)
    _, _, ldy = _rows(y)
    L.call("mtx_softmax_fwd_f32", L.ptr(x), ldx, L.ptr(y), ldy, rx, Lx, int(causal_tq), int(log),
           L.stream_handle())
    return y


def softmax_bwd(y, dy, dx, log=False, accumulate=False):
    r, Lx, ldy = _rows(y)
    _, _, lddy = _rows(dy)
    _, _, lddx = _rows(dx)
    L.call("mtx_softmax_bwd_f32", L.ptr(y), ldy, L.ptr(dy), lddy, L.ptr(dx), lddx, r, Lx, int(log),
           int(bool(accumulate)), L.stream_handle())
    return dx


def layernorm_fwd(x, gamma, beta, y, mean, std, eps):
    r, C, ldx = _rows(x)
    _, _, ldy = _rows(y)
    L.call("mtx_layernorm_fwd_f32", L.ptr(x), ldx, L.ptr(gamma), L.ptr(beta), L.ptr(y), ldy,
           L.ptr(mean), L.ptr(std), r, C, float(eps), L.stream_handle())
    return y


def layernorm_bwd(x, gamma, mean, std, dy, dx=None, dgamma=None, dbeta=None, accumulate=False,
                  accumulate_params=None, addend=None):
    """dx and/or dgamma, dbeta in one pass over x and dy.  `accumulate` adds
    into dx; `accumulate_params` (default: same as `accumulate`) adds into
    dgamma and dbeta; `addend` (rows, C) is added to dx instead (dx = the
    LayerNorm gradient + addend; not with `accumulate`)."""
    if accumulate_params is None:
        accumulate_params = accumulate
    flags = (1 if accumulate else 0) | (2 if accumulate_params else 0)
    r, C, ldx = _rows(x)
    _, _, lddy = _rows(dy)
    lddx = _rows(dx)[2] if dx is not None else C
    ldadd = _rows(addend)[2] if addend is not None else 0
    ws = None
    ws_bytes = 0
    if dgamma is not None:
        ws_bytes = L.lib().mtx_layernorm_bwd_workspace_bytes(r, C)
        ws = dev.empty_buf((ws_bytes,), "uint8")
    L.call("mtx_layernorm_bwd_f32", L.ptr(x), ldx, L.ptr(gamma), L.ptr(mean), L.ptr(std),
           L.ptr(dy), lddy, L.ptr(dx) if dx is not None else None, lddx,
           L.ptr(addend) if addend is not None else None, ldadd,
           L.ptr(dgamma) if dgamma is not None else None, L.ptr(dbeta) if dbeta is not None else None,
           r, C, flags, L.ptr(ws) if ws is not None else None, ws_bytes,
           L.stream_handle())


def gelu_fwd(x, y):
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("gelu: contiguous tensors only")
    L.call("mtx_gelu_fwd_f32", L.ptr(x), L.ptr(y), x.numel(), L.stream_handle())
    return y


def gelu_bwd(x, dy, dx, accumulate=False):
    if not (x.is_contiguous() and dy.is_contiguous() and dx.is_contiguous()):
        raise ValueError("gelu_bwd: contiguous tensors only")
    L.call("mtx_gelu_bwd_f32", L.ptr(x), L.ptr(dy), L.ptr(dx), x.numel(), int(bool(accumulate)),
           L.stream_handle())
    return dx


def xent_fwd(logits, labels, row_loss, lse):
    r, V, ld = _rows(logits)
    L.call("mtx_xent_fwd_f32", L.ptr(logits), ld, L.ptr(labels), L.ptr(row_loss), L.ptr(lse), r, V,
           L.stream_handle())


def xent_bwd(logits, labels, lse, gscalar, scale, dlogits, accumulate=False):
    r, V, ld = _rows(logits)
    _, _, ldd = _rows(dlogits)
    L.call("mtx_xent_bwd_f32", L.ptr(logits), ld, L.ptr(labels), L.ptr(lse), L.ptr(gscalar),
           float(scale), L.ptr(dlogits), ldd, r, V, int(bool(accumulate)), L.stream_handle())


def embedding_fwd(weight, idx, out):
    V, C = weight.shape
    L.call("mtx_embedding_fwd_f32", L.ptr(weight), weight.stride(0), V, L.ptr(idx), idx.numel(),
           L.ptr(out), C, C, L.stream_handle())
    return out


def embedding_bwd(idx, grad, dweight, accumulate=False):
    """dweight (+)= scatter-add of grad rows by idx.  Small tables use a
    one-hot GEMM on MFMA (onehot^T @ grad); large ones the row-owner kernel.
    Both are deterministic."""
    V, C = dweight.shape
    n = idx.numel()
    if V <= 4096 and n * V <= (1 << 27):
        onehot = dev.empty_buf((n, V), "float32")
        L.call("mtx_onehot_f32", L.ptr(idx), n, V, L.ptr(onehot), L.stream_handle())
        gemm(onehot.t(), grad, dweight, beta=1.0 if accumulate else 0.0, M=V, N=C, K=n, batch=1,
             sa=(1, V, 0), sb=(grad.stride(0), grad.stride(1), 0), sc=(dweight.stride(0), dweight.stride(1), 0))
        return dweight
    L.call("mtx_embedding_bwd_f32", L.ptr(idx), idx.numel(), L.ptr(grad), C, L.ptr(dweight),
           dweight.stride(0), V, C, int(bool(accumulate)), L.stream_handle())
    return dweight


class AdamTable:
    """Device table for the one-launch multi-tensor Adam (layout of the C
    struct AdamEntry: p, g, m, v, n, block0 -- six 64-bit words)."""

    def __init__(self, params, grads, ms, vs):
        n = len(params)
        sizes = (L.C.c_int64 * n)(*[p.numel() for p in params])
        b0 = (L.C.c_int64 * n)()
        total = L.C.c_int64()
        L.call("mtx_adam_blocks", sizes, n, b0, L.C.byref(total))
        rows = []
        for i in range(n):
            rows.append([params[i].data_ptr(), grads[i].data_ptr(), ms[i].data_ptr(), vs[i].data_ptr(),
                         params[i].numel(), b0[i]])
        host = np.array(rows, dtype=np.int64).reshape(n, 6)
        self.table = dev.from_host(host, np.int64).t
        self.n = n
        self.total_blocks = int(total.value)


def adam_bias_table(beta1, beta2, first_step, length):
    """Host float32 table of the bias corrections (1 - beta1^t, 1 - beta2^t)
    for steps first_step .. first_step + length - 1, entry (t - 1) % length."""
    out = np.empty(2 * length, dtype=np.float32)
    L.call("mtx_adam_bias_table", float(beta1), float(beta2), int(first_step), int(length),
           out.ctypes.data_as(L.C.c_void_p))
    return out


def adam_step_dev(table: AdamTable, lr, beta1, beta2, eps, weight_decay, step_dev, bias_dev):
    """Adam with the step count in device memory (step_dev int32 (1,),
    incremented by the launch) and bias corrections from bias_dev (2*len
    float32, adam_bias_table): a launch that replays unchanged in a graph."""
    L.call("mtx_adam_dev_f32", L.ptr(table.table), table.n, table.total_blocks, float(lr), float(beta1),
           float(beta2), float(eps), float(weight_decay), L.ptr(step_dev), L.ptr(bias_dev),
           bias_dev.numel() // 2, L.stream_handle())


def zero_grads(table: AdamTable):
    """Zero every gradient the table points at, in one launch."""
    L.call("mtx_zero_grads_f32", L.ptr(table.table), table.n, table.total_blocks, L.stream_handle())


def adam_step(table: AdamTable, lr, beta1, beta2, eps, weight_decay, step):
    L.call("mtx_adam_f32", L.ptr(table.table), table.n, table.total_blocks, float(lr), float(beta1),
           float(beta2), float(eps), float(weight_decay), int(step), L.stream_handle())
