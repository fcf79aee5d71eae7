"""Optimisers (the reference's optim.py:5-59).

Adam updates every parameter tensor in a single kernel launch (a device table
of (param, grad, m, v) pointers), with the reference's float32 arithmetic.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from . import kernels as K


class Optimizer:
    def __init__(self, params, lr=1e-3, weight_decay=0.0):
        self.params = list(params)
        self.lr = lr
        self.weight_decay = weight_decay
        self._capturable = False
        self._table = None
        self._key = None

    def zero_grad(self):
        """Drop the gradients (optim.py:11-13); in capturable mode the
        persistent buffers are refilled with zeros instead, so their addresses
        stay the ones a recorded step uses."""
        if self._capturable and self._table is not None and self._table_current():
            # the persistent buffers are the ones the pointer table lists:
            # one launch zeroes them all
            K.zero_grads(self._table)
            return
        for p in self.params:
            if self._capturable and p.grad is not None:
                K.fill(p.grad.t, 0.0)
            else:
                p.grad = None

    def _table_current(self):
        live = [i for i, p in enumerate(self.params) if p.requires_grad and p.grad is not None]
        key = tuple((self.params[i].data.t.data_ptr(), self.params[i].grad.t.data_ptr()) for i in live)
        return key == self._key and all(self.params[i].grad.t.is_contiguous() for i in live)

    def step(self):
        raise NotImplementedError


class Adam(Optimizer):
    """Bias-corrected Adam (optim.py:37-59)."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        super().__init__(params, lr, weight_decay)
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.t = 0
        self.m = [dev.zeros(p.shape) for p in self.params]
        self.v = [dev.zeros(p.shape) for p in self.params]
        self._table = None
        self._key = None

    def capturable(self, window: int = 4096):
        """Make step() replayable as part of a recorded HIP graph: every
        trainable parameter keeps a persistent gradient buffer (zero-filled by
        zero_grad; accumulating into zeros gives the same bits as a first
        write), and the step count lives in device memory, the bias
        corrections coming from a host-filled table that covers `window`
        steps at a time (refilled between steps by prepare()).  Returns self.

        Difference from the reference in this mode: the reference's Adam
        skips a parameter whose grad is None (optim.py:47-48), but here every
        trainable parameter always holds a (possibly all-zero) gradient, so a
        parameter that receives no gradient in some step after earlier steps
        gave it one is still updated (its m and v decay and it moves by
        lr * m_hat / (sqrt(v_hat) + eps)).  GPT training uses every parameter
        in every step, where the two agree; use the eager mode for models that
        leave parameters out of some steps."""
        for p in self.params:
            if p.requires_grad and p.grad is None:
                p.grad = dev.zeros(p.shape)
        self._step_dev = dev.full((1,), self.t, "int32").t
        self._bias_dev = dev.empty((2 * window,)).t
        self._bias_first = None
        self._capturable = True
        self.prepare()
        live = [i for i, p in enumerate(self.params) if p.requires_grad and p.grad is not None]
        if live:
            self._adam_table(live)  # built now: a recording cannot upload it
        return self

    def prepare(self):
        """Host work before the next step (eager, recorded or replayed): make
        the bias table cover step t + 1.  A no-op unless capturable."""
        if not self._capturable:
            return
        t_next = self.t + 1
        n = self._bias_dev.numel() // 2
        f = self._bias_first
        if f is None or not (f <= t_next < f + n):
            host = K.adam_bias_table(self.beta1, self.beta2, t_next, n)
            self._bias_dev.copy_(host)
            self._bias_first = t_next

    def step(self):
        if self._capturable:
            self.prepare()
            self.t += 1
            live = [i for i, p in enumerate(self.params) if p.requires_grad and p.grad is not None]
            if live:
                self._adam_table(live)
                K.adam_step_dev(self._table, self.lr, self.beta1, self.beta2, self.eps, self.weight_decay,
                                self._step_dev, self._bias_dev)
            return
        self.t += 1
        live = [i for i, p in enumerate(self.params) if p.requires_grad and p.grad is not None]
        if not live:
            return
        self._adam_table(live)
        K.adam_step(self._table, self.lr, self.beta1, self.beta2, self.eps, self.weight_decay, self.t)

    def _adam_table(self, live):
        """The device table of (param, grad, m, v) pointers, rebuilt only when
        a pointer changed."""
        for i in live:
            p = self.params[i]
            if not p.grad.t.is_contiguous():
                p.grad = p.grad.copy()
        key = tuple((self.params[i].data.t.data_ptr(), self.params[i].grad.t.data_ptr()) for i in live)
        if key != self._key:
            self._table = K.AdamTable([self.params[i].data.t for i in live],
                                      [self.params[i].grad.t for i in live],
                                      [self.m[i].t for i in live], [self.v[i].t for i in live])
            self._key = key

    def state_dict(self):
        """Host copy of the optimizer state for checkpoint / resume: the step
        count `t` and the moment estimates `m.<i>`, `v.<i>` in parameter order.
        (The reference keeps this state in memory only, optim.py:43-45.)"""
        state = {"t": np.asarray(self.t, dtype=np.int64)}
        for i in range(len(self.params)):
            state[f"m.{i}"] = self.m[i].numpy().copy()
            state[f"v.{i}"] = self.v[i].numpy().copy()
        return state

    def load_state_dict(self, state):
        """Restore a state_dict() (same parameter list, same shapes); the
        moment buffers are overwritten in place."""
        for i, p in enumerate(self.params):
            for name, buf in (("m", self.m[i]), ("v", self.v[i])):
                arr = np.asarray(state[f"{name}.{i}"], dtype=np.float32)
                if arr.shape != tuple(p.shape):
                    raise ValueError(f"{name}.{i}: shape {arr.shape} does not match parameter {tuple(p.shape)}")
                buf.t.copy_(dev.from_host(arr).t)
        self.t = int(state["t"])
        if self._capturable:
            self._step_dev.fill_(self.t)
            self._bias_first = None
            self.prepare()

    def save(self, path):
        np.savez(path, **self.state_dict())

    def load(self, path):
        with np.load(path) as data:
            self.load_state_dict({k: data[k] for k in data.files})
        return self
