"""Module system (the reference's module.py:5-134): parameter discovery by
attribute walk, train/eval flags, dotted state_dict names and .npz save/load.

Everything here is one walk over the module tree, ``Module._walk``, which
visits a module's attributes in insertion order and yields every trainable
tensor with its dotted key and every sub-module.  What is shared with the
reference is the contract, not the code:

* the key of a trainable tensor is its attribute path, list items by index
  (``blocks.0.attn.q_proj.weight``, ``mlp.layers.2.bias``), in attribute
  insertion order -- the keys and order of the reference's state_dict
  (module.py:81-94), so weights move between the two unchanged;
* parameters() also includes trainable tensors held directly in a list
  attribute (the reference's parameters() does, its state_dict() does not),
  each tensor once, first occurrence first (module.py:5-15, 33-46).

state_dict() returns host NumPy arrays (a device-to-host copy) and
load_state_dict() accepts NumPy arrays or device arrays.
"""
from __future__ import annotations

import numpy as np

from . import device as dev
from .device import DeviceArray
from .tensor import Tensor


def _trainable(x) -> bool:
    return isinstance(x, Tensor) and x.requires_grad


class Module:
    """Base class for layers and models (module.py:17-118)."""

    def __init__(self):
        self._training = True

    def forward(self, *args, **kwargs):
        raise NotImplementedError

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    # -- the tree walk ------------------------------------------------------
    def _children(self):
        """(name, value, listed) for each attribute value, list and tuple
        items flattened as name.i (listed=True)."""
        for name, val in self.__dict__.items():
            if isinstance(val, (list, tuple)):
                for i, item in enumerate(val):
                    yield f"{name}.{i}", item, True
            else:
                yield name, val, False

    def _walk(self, prefix=""):
        """Depth-first, attribute order: ("tensor", key, tensor, listed) for a
        trainable tensor, ("module", key, module, listed) for a sub-module
        (its own entries follow it)."""
        for name, val, listed in self._children():
            key = prefix + name
            if _trainable(val):
                yield "tensor", key, val, listed
            elif isinstance(val, Module):
                yield "module", key, val, listed
                yield from val._walk(key + ".")

    def _named_state(self):
        """(key, tensor) pairs of the state dict: trainable tensors that are
        attributes of some module (not list items)."""
        for kind, key, val, listed in self._walk():
            if kind == "tensor" and not listed:
                yield key, val

    # -- the reference's interface ------------------------------------------
    def parameters(self):
        by_id = {}
        for kind, _, val, _ in self._walk():
            if kind == "tensor":
                by_id.setdefault(id(val), val)
        return list(by_id.values())

    def _set_mode(self, training: bool):
        self._training = training
        for kind, _, val, _ in self._walk():
            if kind == "module":
                val._training = training
        return self

    def train(self):
        return self._set_mode(True)

    def eval(self):
        return self._set_mode(False)

    def state_dict(self):
        return {key: t.data.numpy().copy() for key, t in self._named_state()}

    def load_state_dict(self, state):
        for key, t in self._named_state():
            if key in state:
                v = state[key]
                t.data = v.copy() if isinstance(v, DeviceArray) else dev.from_host(v)

    def save(self, path):
        np.savez(path, **self.state_dict())

    def load(self, path):
        with np.load(path, allow_pickle=False) as z:
            self.load_state_dict(dict(z.items()))
        return self


class Sequential(Module):
    """Chain of modules (module.py:121-134)."""

    def __init__(self, *layers):
        super().__init__()
        self.layers = list(layers)

    def forward(self, x):
        for layer in self.layers:
            x = layer(x)
        return x
