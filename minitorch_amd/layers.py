"""Layers (the reference's layers.py:7-131) on the device.

Initialisation draws come from NumPy's global RNG exactly as in the reference
(np.random.randn for Linear and Embedding, layers.py:19-25, 96-98), so seeding
np.random gives the same initial weights as the reference.  Linear runs as one
fused GEMM node (bias in the epilogue), LayerNorm as one fused row kernel,
GELU as one fused elementwise kernel.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from . import functional as F
from . import kernels as K
from .device import DeviceArray
from .module import Module
from .tensor import Tensor, _grad_target, _grad_target_addend, grad_enabled, _parents


class Linear(Module):
    """y = x @ W + b with W stored (in, out) (layers.py:7-37)."""

    def __init__(self, in_features, out_features, bias=True, init="kaiming"):
        super().__init__()
        assert in_features > 0 and out_features > 0, "features must be positive"
        if init == "xavier":
            scale = np.sqrt(2.0 / (in_features + out_features))
        else:
            scale = np.sqrt(2.0 / in_features)
        self.weight = Tensor((np.random.randn(in_features, out_features) * scale).astype(np.float32),
                             requires_grad=True)
        self.bias = Tensor(np.zeros(out_features, dtype=np.float32), requires_grad=True) if bias else None

    def forward(self, x):
        assert x.shape[-1] == self.weight.shape[0], \
            f"Linear expects last dim {self.weight.shape[0]}, got {x.shape[-1]}"
        return F.linear(x, self.weight, self.bias)


class GELU(Module):
    def forward(self, x):
        return F.gelu(x)


class LayerNorm(Module):
    """Normalise over the last axis (layers.py:73-89): biased variance, eps
    inside the square root; one fused kernel each way."""

    def __init__(self, num_features, eps=1e-5):
        super().__init__()
        assert num_features > 0, "num_features must be positive"
        self.gamma = Tensor(np.ones(num_features, dtype=np.float32), requires_grad=True)
        self.beta = Tensor(np.zeros(num_features, dtype=np.float32), requires_grad=True)
        self.eps = eps

    def forward(self, x):
        C = self.gamma.shape[0]
        assert x.shape[-1] == C, f"LayerNorm expects last dim {C}, got {x.shape[-1]}"
        xc = x.data.contiguous()
        rows = xc.size // C
        y = dev.empty(x.shape)
        mean = dev.empty((rows,))
        std = dev.empty((rows,))
        K.layernorm_fwd(xc.t.view(rows, C), self.gamma.data.t, self.beta.data.t, y.t.view(rows, C),
                        mean.t, std.t, float(np.float32(self.eps)))
        gamma, beta = self.gamma, self.beta
        track = grad_enabled() and any(t.requires_grad for t in (x, gamma, beta))
        out = Tensor(y, requires_grad=track)
        if track:
            def _backward():
                g = out.grad.contiguous().t.view(rows, C)
                dx = dgam = dbet = add = None
                acc_x = acc_p = False
                if x.requires_grad:
                    # x's other contribution (the residual add's) is read as
                    # an addend when it is still held by reference
                    tx, acc_x, ad = _grad_target_addend(x)
                    dx = tx.t.view(rows, C)
                    add = ad.t.view(rows, C) if ad is not None else None
                if gamma.requires_grad or beta.requires_grad:
                    tg, ag = _grad_target(gamma)
                    tb, ab = _grad_target(beta)
                    if ag != ab:  # one of them already held a gradient: keep it simple
                        raise RuntimeError("LayerNorm parameters with mismatched grad state")
                    dgam, dbet, acc_p = tg.t, tb.t, ag
                if dx is not None or dgam is not None:
                    K.layernorm_bwd(xc.t.view(rows, C), gamma.data.t, mean.t, std.t, g, dx=dx,
                                    dgamma=dgam, dbeta=dbet, accumulate=acc_x, accumulate_params=acc_p,
                                    addend=add)

            out._backward = _backward
            out._prev = _parents((x, gamma, beta))
            out._op = "layernorm"
        return out


class Embedding(Module):
    """Lookup table (layers.py:92-104): weight[idx] gathers rows; the backward
    scatters with repeated ids adding up (np.add.at)."""

    def __init__(self, num_embeddings, embed_dim):
        super().__init__()
        assert num_embeddings > 0 and embed_dim > 0, "sizes must be positive"
        self.weight = Tensor((np.random.randn(num_embeddings, embed_dim) * 0.02).astype(np.float32),
                             requires_grad=True)

    def forward(self, idx):
        if isinstance(idx, DeviceArray):
            return self.weight[idx]
        return self.weight[np.asarray(idx)]


class Dropout(Module):
    """Inverted dropout (layers.py:107-131).  Identity in eval mode or with
    p == 0 (the same Tensor is returned).  The keep-mask is drawn on the host
    from NumPy's global RNG, as the reference draws it."""

    def __init__(self, p=0.5):
        super().__init__()
        assert 0.0 <= p < 1.0, "dropout probability must be in [0, 1)"
        self.p = p

    def forward(self, x):
        if not self._training or self.p == 0.0:
            return x
        mask = (np.random.rand(*x.shape) > self.p).astype(np.float32) * np.float32(1.0 / (1.0 - self.p))
        return x * Tensor(mask)
