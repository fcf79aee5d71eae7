"""Module system (the reference's module.py:5-134): parameter discovery by
attribute walk, train/eval flags, dotted state_dict names and .npz save/load.

state_dict() returns host NumPy arrays (a device-to-host copy) under exactly
the reference's key names, and load_state_dict() accepts NumPy arrays, so
weights move between this package and the reference unchanged.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from .device import DeviceArray
from .tensor import Tensor


def _dedup(params):
    seen, out = set(), []
    for p in params:
        if id(p) not in seen:
            seen.add(id(p))
            out.append(p)
    return out


class Module:
    """Base class for layers and models (module.py:17-118)."""

    def __init__(self):
        self._training = True

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def _children(self):
        for name, val in self.__dict__.items():
            if isinstance(val, (list, tuple)):
                for i, item in enumerate(val):
                    yield f"{name}.{i}", item
            else:
                yield name, val

    def parameters(self):
        params = []
        for _, val in self._children():
            if isinstance(val, Tensor) and val.requires_grad:
                params.append(val)
            elif isinstance(val, Module):
                params.extend(val.parameters())
        return _dedup(params)

    def train(self):
        self._training = True
        for _, val in self._children():
            if isinstance(val, Module):
                val.train()
        return self

    def eval(self):
        self._training = False
        for _, val in self._children():
            if isinstance(val, Module):
                val.eval()
        return self

    def save(self, path):
        np.savez(path, **self.state_dict())

    def load(self, path):
        with np.load(path) as data:
            self.load_state_dict({k: data[k] for k in data.files})
        return self

    def state_dict(self):
        state = {}
        for name, val in self.__dict__.items():
            if isinstance(val, Tensor) and val.requires_grad:
                state[name] = val.data.numpy().copy()
            elif isinstance(val, Module):
                for k, v in val.state_dict().items():
                    state[f"{name}.{k}"] = v
            elif isinstance(val, (list, tuple)):
                for i, item in enumerate(val):
                    if isinstance(item, Module):
                        for k, v in item.state_dict().items():
                            state[f"{name}.{i}.{k}"] = v
        return state

    def load_state_dict(self, state):
        for name, val in self.__dict__.items():
            if isinstance(val, Tensor) and val.requires_grad:
                if name in state:
                    v = state[name]
                    val.data = v.copy() if isinstance(v, DeviceArray) else dev.from_host(v)
            elif isinstance(val, Module):
                prefix = f"{name}."
                child = {k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)}
                if child:
                    val.load_state_dict(child)
            elif isinstance(val, (list, tuple)):
                for i, item in enumerate(val):
                    if isinstance(item, Module):
                        prefix = f"{name}.{i}."
                        child = {k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)}
                        if child:
                            item.load_state_dict(child)


class Sequential(Module):
    """Chain of modules (module.py:121-134)."""

    def __init__(self, *layers):
        super().__init__()
        self.layers = list(layers)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x
