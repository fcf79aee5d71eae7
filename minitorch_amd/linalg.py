"""Batched matrix products on the device (Tensor.__matmul__, tensor.py:207-223).

``matmul_data`` follows NumPy's ``@``: broadcasting batch axes, 1-D operands
promoted and squeezed.  Transposed operands are passed to the GEMM kernel as
stride swaps.  Two launch shapes avoid per-matrix loops:
  * when B does not vary over the batch (a weight), the batch axes of A and C
    are folded into the row dimension: one large GEMM;
  * otherwise the batch axes are collapsed into one strided batch index when
    their strides allow, and looped over only when they do not.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray


def _unit_ok(t):
    return t.stride(-1) == 1 or t.stride(-2) == 1 or t.shape[-1] == 1 or t.shape[-2] == 1


def _fix(t):
    return t if _unit_ok(t) else t.contiguous()


def _collapse(ts, nb):
    """If the first nb axes of every tensor in ts collapse into one index with
    a single stride, return those strides, else None."""
    out = []
    for t in ts:
        if nb == 0:
            out.append(0)
            continue
        shp, st = t.shape[:nb], t.stride()[:nb]
        s = None
        expect = None
        ok = True
        for d in range(nb - 1, -1, -1):
            if shp[d] == 1:
                continue
            if s is None:
                s = st[d]
                expect = st[d] * shp[d]
            else:
                if st[d] != expect:
                    ok = False
                    break
                expect = st[d] * shp[d]
        if not ok:
            return None
        out.append(0 if s is None else s)
    return out


def _rows_fold(t, nb):
    """Stride of the row index if t's batch axes and its row axis collapse
    into one row index, else None."""
    st = _collapse([t.as_strided(t.shape[:nb + 1], t.stride()[:nb + 1])], nb + 1)
    return None if st is None else st[0]


def bmm(at, bt, ct, alpha=1.0, beta=0.0, bias=None):
    """ct[...] = alpha * at @ bt + beta * ct (+ bias), device arrays with
    broadcastable batch axes; ct has the full batch shape."""
    at, bt = _fix(at), _fix(bt)
    batch = tuple(ct.shape[:-2])
    nb = len(batch)
    M, Kd = at.shape[-2], at.shape[-1]
    N = bt.shape[-1]
    ae = at.expand(batch + (M, Kd))
    be = bt.expand(batch + (Kd, N))
    if nb and all(s == 0 for s in be.stride()[:nb]):
        ra, rc = _rows_fold(ae, nb), _rows_fold(ct, nb)
        if ra is not None and rc is not None:
            rows = int(np.prod(batch)) * M
            K.gemm(ae, be, ct, alpha, beta, bias, M=rows, N=N, K=Kd, batch=1,
                   sa=(ra if rows > 1 else ae.stride(-2), ae.stride(-1), 0),
                   sb=(be.stride(-2), be.stride(-1), 0),
                   sc=(rc if rows > 1 else ct.stride(-2), ct.stride(-1), 0))
            return ct
    st = _collapse([ae, be, ct], nb)
    if st is not None:
        nbat = int(np.prod(batch)) if nb else 1
        K.gemm(ae, be, ct, alpha, beta, bias, M=M, N=N, K=Kd, batch=nbat,
               sa=(ae.stride(-2), ae.stride(-1), st[0]),
               sb=(be.stride(-2), be.stride(-1), st[1]),
               sc=(ct.stride(-2), ct.stride(-1), st[2]))
        return ct
    for i in range(batch[0]):
        bmm(ae[i], be[i], ct[i], alpha, beta, bias)
    return ct


def matmul_data(a: DeviceArray, b: DeviceArray) -> DeviceArray:
    at, bt = a.t, b.t
    a1, b1 = at.dim() == 1, bt.dim() == 1
    if a1:
        at = at.unsqueeze(0)
    if b1:
        bt = bt.unsqueeze(-1)
    if at.shape[-1] != bt.shape[-2]:
        raise ValueError(f"matmul: shapes {tuple(a.shape)} and {tuple(b.shape)} not aligned")
    batch = tuple(np.broadcast_shapes(tuple(at.shape[:-2]), tuple(bt.shape[:-2])))
    out = dev.empty_buf(batch + (at.shape[-2], bt.shape[-1]), "float32")
    bmm(at, bt, out)
    if a1:
        out = out.squeeze(-2)
    if b1:
        out = out.squeeze(-1)
    return DeviceArray(out)


def matmul_grad_b(a: DeviceArray, g: DeviceArray, other, bias=None):
    """Accumulate dB = A^T @ G, summed to B's shape, into other.grad
    (tensor.py:216-218).  With `bias` (a Linear's bias, x @ W + b), its
    gradient -- the column sums of G -- comes out of the same GEMM where the
    2-D weight path applies; returns True when it did."""
    from .tensor import _accum_grad, _grad_target, _sum_to_shape

    at, gt = a.t, g.t
    if at.dim() == 1:
        at = at.unsqueeze(0)
        gt = gt.unsqueeze(-2)
    if other.ndim == 1:
        gt = gt.unsqueeze(-1)
    batch = tuple(gt.shape[:-2])
    nb = len(batch)
    if other.ndim <= 2 and nb:
        ae = _fix(at.expand(batch + tuple(at.shape[-2:])))
        ra, rg = _rows_fold(ae, nb), _rows_fold(gt, nb)
        if ra is not None and rg is not None:
            rows = int(np.prod(batch)) * ae.shape[-2]
            target, acc = _grad_target(other)
            tt = target.t if other.ndim == 2 else target.t.view(-1, 1)
            tb, accb = (None, False)
            if bias is not None and other.ndim == 2 and bias.ndim == 1 and bias.shape[0] == gt.shape[-1]:
                tb, accb = _grad_target(bias)
            K.gemm(ae, gt, tt, 1.0, 1.0 if acc else 0.0, None,
                   M=ae.shape[-1], N=gt.shape[-1], K=rows, batch=1,
                   sa=(ae.stride(-1), ra, 0), sb=(rg, gt.stride(-1), 0), sc=(tt.stride(0), tt.stride(1), 0),
                   colsum=tb.t if tb is not None else None, colsum_accumulate=accb)
            return tb is not None
    res = dev.empty(batch + (at.shape[-1], gt.shape[-1]))
    bmm(at.transpose(-1, -2), gt, res.t)
    if other.ndim == 1:
        res = res.reshape(*res.shape[:-1])
    _accum_grad(other, _sum_to_shape(res, other.shape), owned=True)
    return False
