"""Steps recorded once as a HIP graph and replayed (mtx_graph_* entry points).

Launch-bound loops (a small model's training step: a few hundred short
kernels and their Python dispatch; a decode step) are recorded once on the
library's capture stream and replayed on the null stream, where the eager
work runs; every kernel, buffer address and argument of the recorded step is
reused, so the step must read no host state that changes between calls:

* inputs are device arrays; each call copies its arguments into static
  buffers the recorded step reads (device-to-device, outside the graph);
* the optimizer runs in capturable mode (optim.Adam.capturable: persistent
  gradient buffers, step count in device memory), and its host-side
  bookkeeping (the step count, the bias-correction table) is advanced around
  each replay;
* the first `warmup` calls run eagerly (they create cached constants, the
  optimizer's pointer table and the gradient buffers), the next one is
  recorded and then replayed, so every call performs one real step.

Memory the recorded launches use comes from the graph's private pool of the
library's allocator (see mtx_malloc), so eager work never reuses it while the
graph exists.  The reference has no counterpart (it runs every op eagerly on
the CPU, char_transformer.py:70-77).
"""
from __future__ import annotations

import ctypes as C
from contextlib import contextmanager

from . import _lib as L
from . import device as dev
from .device import DeviceArray

_CAPTURE_STREAM = [None]


def _capture_stream():
    if _CAPTURE_STREAM[0] is None:
        dev.device()
        s = C.c_void_p()
        L.call("mtx_stream_create", C.byref(s))
        _CAPTURE_STREAM[0] = s
    return _CAPTURE_STREAM[0]


class Graph:
    """One recorded HIP graph.  ``with g.capture(): ...`` records every launch
    the block issues (none of them runs); ``g.replay()`` runs them all."""

    def __init__(self):
        self._h = None

    @contextmanager
    def capture(self):
        if self._h is not None:
            raise RuntimeError("this graph is already recorded")
        if L.capturing():
            raise RuntimeError("a capture is already in progress")
        dev.synchronize()
        s = _capture_stream()
        L.call("mtx_graph_begin", s)
        L._STREAM[0] = s
        ok = False
        try:
            yield self
            ok = True
        finally:
            L._STREAM[0] = None
            h = C.c_void_p()
            rc = L.lib().mtx_graph_end(s, C.byref(h))
            if ok:
                L.check("mtx_graph_end", rc)
                self._h = h
            elif rc == 0:
                L.lib().mtx_graph_destroy(h)
            # else: the block raised and the capture failed too; the library
            # has already released the capture's memory pool, and the
            # block's own exception is the one that propagates

    def replay(self):
        if self._h is None:
            raise RuntimeError("nothing recorded")
        L.call("mtx_graph_launch", self._h, None)

    def __del__(self):
        try:
            if self._h is not None:
                L.lib().mtx_graph_destroy(self._h)
                self._h = None
        except Exception:
            pass


def _buf(x):
    return x.t if isinstance(x, DeviceArray) else x


class CapturedStep:
    """fn(*inputs) -> output, replayed from a HIP graph after `warmup` eager
    calls.  `inputs` are DeviceArrays (or DevBufs) of a fixed shape and
    dtype; the returned object is the output of the recorded call, whose
    buffers every replay overwrites."""

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
        bufs = [_buf(x) for x in inputs]
        if self._static is None:
            self._static = [dev.empty_buf(b.shape, b.dtype) for b in bufs]
            self._wrap = [isinstance(x, DeviceArray) for x in inputs]
        if len(bufs) != len(self._static):
            raise ValueError("a captured step takes the same number of inputs on every call")
        for s, b in zip(self._static, bufs):
            if tuple(b.shape) != tuple(s.shape) or dev.dtype_name(b) != s.dtype:
                raise ValueError(f"input {tuple(b.shape)} {dev.dtype_name(b)} does not match the recorded "
                                 f"{tuple(s.shape)} {s.dtype}")
            s.copy_(b)
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
            graph = Graph()
            with graph.capture():
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
