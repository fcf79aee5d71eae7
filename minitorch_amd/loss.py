"""Losses (the reference's loss.py:6-27)."""
from __future__ import annotations

import numpy as np

from . import functional as F
from .device import DeviceArray
from .tensor import Tensor


def cross_entropy_loss(input, target):
    """Softmax cross-entropy of (N, V) logits (loss.py:17-27).  `target` holds
    class indices (a Tensor, array or list; one per row) or one-hot rows."""
    t = target.data if isinstance(target, Tensor) else target
    if isinstance(t, DeviceArray) and t.t.dtype == "int64":
        return F.cross_entropy(input, t)  # device-resident class indices
    if isinstance(t, DeviceArray):
        t = t.numpy()
    t = np.asarray(t)
    if t.ndim == 1 or (t.ndim == 2 and t.shape[1] == 1):
        return F.cross_entropy(input, t.reshape(-1).astype(np.int64))
    onehot = target if isinstance(target, Tensor) else Tensor(t)
    log_probs = F.log_softmax(input, axis=1)
    return (-log_probs * onehot).sum() / input.shape[0]
