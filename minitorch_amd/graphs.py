"""A step recorded once as a HIP graph and replayed.

Launch-bound loops (a small model's training step: a few hundred short
kernels and their Python dispatch) are recorded once with
torch.cuda.CUDAGraph on the library's stream and replayed; every kernel,
buffer address and argument of the recorded step is reused, so the step must
read no host state that changes between calls:

* inputs are device tensors; each call copies its arguments into static
  buffers the recorded step reads (device-to-device, outside the graph);
* the optimizer runs in capturable mode (optim.Adam.capturable: persistent
  gradient buffers, step count in device memory), and its host-side
  bookkeeping (the step count, the bias-correction table) is advanced around
  each replay;
* the first `warmup` calls run eagerly (they create cached constants, the
  optimizer's pointer table and the gradient buffers), the next one is
  recorded and then replayed, so every call performs one real step.

The reference has no counterpart (it runs every op eagerly on the CPU,
char_transformer.py:70-77).
"""
from __future__ import annotations

import torch

from .device import DeviceArray


class CapturedStep:
    """fn(*inputs) -> output, replayed from a HIP graph after `warmup` eager
    calls.  `inputs` are DeviceArrays or torch device tensors of a fixed
    shape and dtype; the returned object is the output of the recorded call,
    whose buffers every replay overwrites."""

    def __init__(self, fn, optimizer=None, warmup: int = 2):
        self.fn = fn
        self.opt = optimizer
        self.warmup = warmup
        self.calls = 0
        self.graph = None
        self.out = None
        self._static = None
        if optimizer is not None and not optimizer._capturable:
            raise ValueError("the optimizer must be in capturable mode (optimizer.capturable())")
        if warmup < 1:
            # first calls create cached device constants (host -> device
            # copies), which a recording cannot contain
            raise ValueError("a captured step needs at least one eager warm-up call")

    def _stage(self, inputs):
        tens = [x.t if isinstance(x, DeviceArray) else x for x in inputs]
        if self._static is None:
            self._static = [torch.empty_like(t) for t in tens]
            self._wrap = [isinstance(x, DeviceArray) for x in inputs]
        if len(tens) != len(self._static):
            raise ValueError("a captured step takes the same number of inputs on every call")
        for s, t in zip(self._static, tens):
            if t.shape != s.shape or t.dtype != s.dtype:
                raise ValueError(f"input {tuple(t.shape)} {t.dtype} does not match the recorded "
                                 f"{tuple(s.shape)} {s.dtype}")
            s.copy_(t)
        return [DeviceArray(s) if w else s for s, w in zip(self._static, self._wrap)]

    def __call__(self, *inputs):
        args = self._stage(inputs)
        if self.calls < self.warmup:
            self.calls += 1
            return self.fn(*args)
        if self.graph is None:
            t0 = self.opt.t if self.opt is not None else None
            if self.opt is not None:
                self.opt.prepare()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self.out = self.fn(*args)
            # recording ran no kernel: the step is still to be taken
            if self.opt is not None:
                self.opt.t = t0
            self.graph = graph
        if self.opt is not None:
            self.opt.prepare()
        self.graph.replay()
        if self.opt is not None:
            self.opt.t += 1
        self.calls += 1
        return self.out
