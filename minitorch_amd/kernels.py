"""Thin Python wrappers over the libmtx_hip entry points.

Each function takes torch device tensors (device memory only -- no torch
compute is used), validates shapes on the host, calls the C ABI on the current
HIP stream and returns the output tensors.  Errors raise ``ValueError`` (bad
arguments, found before any HIP call) or ``MtxError`` (HIP failure).
"""
from __future__ import annotations

import torch

from . import _lib as L


def _need_cuda(*ts):
    for t in ts:
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError("minitorch_amd kernels take device tensors (torch.cuda)")


def _bhtd(name, t):
    if t.dim() != 4:
        raise ValueError(f"{name}: expected a (B, H, T, D) tensor, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: the last (d) dimension must be contiguous")


def attn_fwd(q, k, v, scale: float, causal: bool = True, out=None, lse=None):
    """Fused attention forward.  q: (B,H,Tq,D), k/v: (B,H,Tk,D), fp32 or bf16,
    any strides with a contiguous last dim.  Returns (out, lse) with out like q
    and lse fp32 (B,H,Tq)."""
    _need_cuda(q, k, v)
    for name, t in (("q", q), ("k", k), ("v", v)):
        _bhtd(name, t)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if k.shape != (B, H, Tk, D) or v.shape != (B, H, Tk, D):
        raise ValueError(f"shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    if out is None:
        out = torch.empty((B, H, Tq, D), dtype=q.dtype, device=q.device)
    if lse is None:
        lse = torch.empty((B, H, Tq), dtype=torch.float32, device=q.device)
    _bhtd("out", out)
    if not lse.is_contiguous() or lse.shape != (B, H, Tq) or lse.dtype != torch.float32:
        raise ValueError("lse must be a contiguous fp32 (B,H,Tq) tensor")
    L.call("mtx_attn_fwd", L.dtype_code(q), B, H, Tq, Tk, D,
           L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
           L.ptr(out), L.strides(out), L.ptr(lse), float(scale), int(bool(causal)),
           L.stream_handle(q.device))
    return out, lse


def attn_bwd(q, k, v, out, dout, lse, scale: float, causal: bool = True,
             dq=None, dk=None, dv=None, accumulate: bool = False, workspace=None,
             phases: int = L.ATTN_BWD_ALL):
    """Fused attention backward.  Returns fp32 (dq, dk, dv).  With
    accumulate=True the given dq/dk/dv are added to instead of overwritten."""
    _need_cuda(q, k, v, out, dout, lse)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out), ("dout", dout)):
        _bhtd(name, t)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if out.shape != q.shape or dout.shape != q.shape:
        raise ValueError("out and dout must have q's shape")
    if not (q.dtype == k.dtype == v.dtype == out.dtype == dout.dtype):
        raise ValueError("q, k, v, out, dout must share a dtype")
    f32 = torch.float32
    if dq is None:
        dq = torch.empty((B, H, Tq, D), dtype=f32, device=q.device)
    if dk is None:
        dk = torch.empty((B, H, Tk, D), dtype=f32, device=q.device)
    if dv is None:
        dv = torch.empty((B, H, Tk, D), dtype=f32, device=q.device)
    for name, t, shp in (("dq", dq, (B, H, Tq, D)), ("dk", dk, (B, H, Tk, D)), ("dv", dv, (B, H, Tk, D))):
        if tuple(t.shape) != shp or t.dtype != f32:
            raise ValueError(f"{name} must be fp32 with shape {shp}")
        _bhtd(name, t)
    nbytes = L.lib().mtx_attn_bwd_workspace_bytes(B, H, Tq)
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    L.call("mtx_attn_bwd_phase", int(phases), L.dtype_code(q), B, H, Tq, Tk, D,
           L.ptr(q), L.strides(q), L.ptr(k), L.strides(k), L.ptr(v), L.strides(v),
           L.ptr(out), L.strides(out), L.ptr(dout), L.strides(dout), L.ptr(lse),
           L.ptr(dq), L.strides(dq), L.ptr(dk), L.strides(dk), L.ptr(dv), L.strides(dv),
           L.ptr(workspace), workspace.numel() * workspace.element_size(),
           float(scale), int(bool(causal)), int(bool(accumulate)), L.stream_handle(q.device))
    return dq, dk, dv
