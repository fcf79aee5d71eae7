"""GPU autograd Tensor with the reference's interface (tensor.py).

Same public surface and the same op-node protocol as the reference
(tensor.py:36-537): every op returns a new ``Tensor`` whose ``_backward``
closure accumulates gradients into its inputs, ``_prev`` holds the inputs and
``_op`` names the op; ``backward()`` seeds ones and runs the closures in
reverse topological order (iterative post-order DFS, tensor.py:453-477).

Differences, all on purpose:
  * ``data`` and ``grad`` are ``DeviceArray``s in GPU memory and every
    operation runs in libmtx_hip.so.  Values are float32 throughout; the
    reference's NumPy-2 promotion to float64 after the attention scale is not
    reproduced (the parity tests state their tolerances).
  * A gradient that is written for the first time goes straight into a new
    buffer (the reference zero-fills, then adds: same values).
  * Python scalars in arithmetic become cached device constants.
  * ``_prev`` is a tuple of the distinct inputs in argument order, not a set:
    the backward walk, and so the order in which a tensor's consumers add
    into its gradient, is the same on every run (the reference's order
    follows set iteration, i.e. object addresses), which makes training
    bit-reproducible.
"""
from __future__ import annotations

import numbers

import numpy as np

from . import device as dev
from . import kernels as K
from .device import DeviceArray


def _parents(inputs):
    """Distinct inputs in first-occurrence order (an op's ``_prev``)."""
    return tuple(dict.fromkeys(inputs))

_grad_enabled = True


class no_grad:
    """Context manager that disables graph construction (tensor.py:7-17)."""

    def __enter__(self):
        global _grad_enabled
        self._prev = _grad_enabled
        _grad_enabled = False
        return self

    def __exit__(self, *args):
        global _grad_enabled
        _grad_enabled = self._prev


def grad_enabled() -> bool:
    return _grad_enabled


def _bshape(a, b):
    return tuple(np.broadcast_shapes(tuple(a), tuple(b)))


def _sum_to_shape(g: DeviceArray, shape) -> DeviceArray:
    """tensor.py:20-26: sum away leading axes, then the axes that are 1 in
    `shape`.  Returns `g` itself when nothing needs reducing."""
    shape = tuple(shape)
    if g.shape == shape:
        return g
    extra = g.ndim - len(shape)
    axes = list(range(extra))
    axes += [extra + i for i, s in enumerate(shape) if s == 1 and g.shape[extra + i] != 1]
    out = dev.empty(shape)
    K.reduce(g.t, axes, out.t)
    return out


# ids of the non-leaf tensors that have exactly one consumer in the graph the
# running backward() walks (set by Tensor.backward)
_single_consumer: set = set()
# a non-leaf tensor with several consumers takes its first gradient by
# reference too (False: as a copy)
_ALIAS_FIRST_GRAD = True


def _accum_grad(tensor: "Tensor", grad: DeviceArray, owned: bool = False):
    """tensor.py:29-33.  `owned` marks a freshly computed buffer with
    tensor's shape that nobody else references: it becomes the gradient
    without a copy.  A non-leaf tensor with a single consumer receives exactly
    one gradient per backward pass, which is final (its producer ran first),
    so it takes that buffer (or view, e.g. through reshape / transpose) as its
    gradient without a copy; such an alias is copied into a buffer of its own
    before anything accumulates into it."""
    if tensor.grad is None:
        if owned and grad.shape == tensor.shape and grad.t.is_contiguous():
            tensor.grad = grad
            tensor._grad_alias = False
            return
        if (id(tensor) in _single_consumer or (_ALIAS_FIRST_GRAD and tensor._prev)) and grad.shape == tensor.shape:
            # a non-leaf's first gradient is taken by reference: nothing
            # writes that buffer again in this backward pass, and every later
            # in-place write to tensor.grad copies it first (_own_grad) or
            # reads it as an addend (_grad_target_addend)
            tensor.grad = grad
            tensor._grad_alias = True
            return
        tensor.grad = dev.empty(tensor.shape)
        tensor._grad_alias = False
        K.ewise("COPY", tensor.grad.t, grad.t)
    else:
        _own_grad(tensor)
        K.ewise("COPY", tensor.grad.t, grad.t, accumulate=True)


def _own_grad(tensor: "Tensor"):
    """Give tensor a gradient buffer of its own (copy an alias) before it is
    written in place."""
    if tensor.grad is not None and getattr(tensor, "_grad_alias", False):
        own = dev.empty(tensor.shape)
        K.ewise("COPY", own.t, tensor.grad.t)
        tensor.grad = own
        tensor._grad_alias = False


def _grad_target(tensor: "Tensor"):
    """(buffer, accumulate) for a kernel that writes tensor's gradient
    directly: a new buffer the first time, else the existing one in
    accumulate mode."""
    if tensor.grad is None:
        tensor.grad = dev.empty(tensor.shape)
        tensor._grad_alias = False
        return tensor.grad, False
    _own_grad(tensor)
    return tensor.grad, True


def _grad_target_addend(tensor: "Tensor"):
    """(buffer, accumulate, addend) for a kernel that writes tensor's
    gradient directly and can add a second input: when tensor.grad is a
    reference to another buffer (its first contribution, see _accum_grad), a
    new buffer plus that reference as the addend, so the kernel writes
    new = own + addend with no copy; otherwise _grad_target's answer and no
    addend."""
    if tensor.grad is not None and getattr(tensor, "_grad_alias", False) and tensor.grad.t.is_contiguous():
        addend = tensor.grad
        tensor.grad = dev.empty(tensor.shape)
        tensor._grad_alias = False
        return tensor.grad, False, addend
    t, acc = _grad_target(tensor)
    return t, acc, None


def _as_tensor(x) -> "Tensor":
    if isinstance(x, Tensor):
        return x
    if isinstance(x, numbers.Number):
        return Tensor(dev.const(float(x)))
    return Tensor(x)


class Tensor:
    """An n-dimensional float32 array in GPU memory that records operations
    for reverse-mode autodiff (tensor.py:36-49)."""

    def __init__(self, data, *, requires_grad=False):
        if isinstance(data, DeviceArray):
            self.data = data
        elif isinstance(data, dev.DevBuf):
            self.data = DeviceArray(data)
        else:
            self.data = dev.from_host(data)
        self.requires_grad = requires_grad and _grad_enabled
        self.grad = None
        self._backward = lambda: None
        self._prev = ()
        self._op = ""

    # ---------------------------------------------------------------- props
    @property
    def shape(self):
        return self.data.shape

    @property
    def ndim(self):
        return self.data.ndim

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def T(self):
        return self.transpose()

    def size(self, dim=None):
        return self.data.size if dim is None else self.data.shape[dim]

    def numpy(self):
        return self.data.numpy()

    # ---------------------------------------------------------- constructors
    @staticmethod
    def zeros(*shape, requires_grad=False):
        return Tensor(dev.zeros(shape), requires_grad=requires_grad)

    @staticmethod
    def ones(*shape, requires_grad=False):
        return Tensor(dev.full(shape, 1.0), requires_grad=requires_grad)

    @staticmethod
    def randn(*shape, requires_grad=False):
        return Tensor(np.random.randn(*shape).astype(np.float32), requires_grad=requires_grad)

    def _should_track(self, *others):
        return _grad_enabled and any(t.requires_grad for t in (self, *others))

    def _node(self, data, prev, op, backward, track):
        out = Tensor(data, requires_grad=track)
        if track:
            out._backward = backward
            out._prev = _parents(prev)
            out._op = op
        return out

    # ------------------------------------------------------------ arithmetic
    def _ew2(self, other, op):
        out = dev.empty(_bshape(self.shape, other.shape))
        K.ewise(op, out.t, self.data.t, other.data.t)
        return out

    def __add__(self, other):
        other = _as_tensor(other)
        track = self._should_track(other)
        out = None

        def _backward():
            for t in (self, other):
                if t.requires_grad:
                    _accum_grad(t, _sum_to_shape(out.grad, t.shape))

        out = self._node(self._ew2(other, "ADD"), (self, other), "add", _backward, track)
        return out

    def __radd__(self, other):
        return self.__add__(other)

    def __sub__(self, other):
        other = _as_tensor(other)
        track = self._should_track(other)
        out = None

        def _backward():
            if self.requires_grad:
                _accum_grad(self, _sum_to_shape(out.grad, self.shape))
            if other.requires_grad:
                neg = dev.empty(out.shape)
                K.ewise("NEG", neg.t, out.grad.t)
                _accum_grad(other, _sum_to_shape(neg, other.shape), owned=True)

        out = self._node(self._ew2(other, "SUB"), (self, other), "sub", _backward, track)
        return out

    def __rsub__(self, other):
        return _as_tensor(other).__sub__(self)

    def __mul__(self, other):
        other = _as_tensor(other)
        track = self._should_track(other)
        out = None

        def _backward():
            for t, o in ((self, other), (other, self)):
                if t.requires_grad:
                    g = dev.empty(out.shape)
                    K.ewise("MUL", g.t, o.data.t, out.grad.t)
                    _accum_grad(t, _sum_to_shape(g, t.shape), owned=True)

        out = self._node(self._ew2(other, "MUL"), (self, other), "mul", _backward, track)
        return out

    def __rmul__(self, other):
        return self.__mul__(other)

    def __truediv__(self, other):
        other = _as_tensor(other)
        track = self._should_track(other)
        out = None

        def _backward():
            if self.requires_grad:
                g = dev.empty(out.shape)
                K.ewise("DIV", g.t, out.grad.t, other.data.t)
                _accum_grad(self, _sum_to_shape(g, self.shape), owned=True)
            if other.requires_grad:
                # -a / b**2 * g
                b2 = dev.empty(other.shape)
                K.ewise("SQUARE", b2.t, other.data.t)
                g = dev.empty(out.shape)
                K.ewise("DIV", g.t, self.data.t, b2.t)
                K.ewise("MUL", g.t, g.t, out.grad.t)
                K.ewise("NEG", g.t, g.t)
                _accum_grad(other, _sum_to_shape(g, other.shape), owned=True)

        out = self._node(self._ew2(other, "DIV"), (self, other), "div", _backward, track)
        return out

    def __rtruediv__(self, other):
        return _as_tensor(other).__truediv__(self)

    def __pow__(self, other):
        other = _as_tensor(other)
        track = self._should_track(other)
        out = None

        def _backward():
            if self.requires_grad:
                # b * a**(b-1) * g
                bm1 = dev.empty(other.shape)
                K.ewise("SCALE_SHIFT", bm1.t, other.data.t, alpha=1.0, beta=-1.0)
                g = dev.empty(out.shape)
                K.ewise("POW", g.t, self.data.t, bm1.t)
                K.ewise("MUL", g.t, g.t, other.data.t)
                K.ewise("MUL", g.t, g.t, out.grad.t)
                _accum_grad(self, _sum_to_shape(g, self.shape), owned=True)
            if other.requires_grad:
                # a**b * log(|a| + 1e-12) * g
                la = dev.empty(self.shape)
                K.ewise("ABS", la.t, self.data.t)
                K.ewise("SCALE_SHIFT", la.t, la.t, alpha=1.0, beta=1e-12)
                K.ewise("LOG", la.t, la.t)
                g = dev.empty(out.shape)
                K.ewise("MUL", g.t, out.data.t, la.t)
                K.ewise("MUL", g.t, g.t, out.grad.t)
                _accum_grad(other, _sum_to_shape(g, other.shape), owned=True)

        out = self._node(self._ew2(other, "POW"), (self, other), "pow", _backward, track)
        return out

    def __neg__(self):
        return self * -1

    # ---------------------------------------------------------------- matmul
    def __matmul__(self, other):
        track = self._should_track(other)
        out = None

        def _backward():
            from .linalg import matmul_data

            g = out.grad
            if self.requires_grad:
                ga = matmul_data(g, other.data.swapaxes(-1, -2))
                _accum_grad(self, _sum_to_shape(ga, self.shape), owned=True)
            if other.requires_grad:
                from .linalg import matmul_grad_b

                matmul_grad_b(self.data, g, other)

        from .linalg import matmul_data

        out = self._node(matmul_data(self.data, other.data), (self, other), "matmul", _backward, track)
        return out

    # ------------------------------------------------------------- reductions
    def _norm_axes(self, axis):
        if axis is None:
            return tuple(range(self.ndim))
        if isinstance(axis, int):
            return (axis % self.ndim,)
        return tuple(a % self.ndim for a in axis)

    def _reduce(self, axis, keepdims, alpha, op=0):
        axes = self._norm_axes(axis)
        kept = [s for i, s in enumerate(self.shape) if i not in axes]
        out = dev.empty(kept)
        K.reduce(self.data.t, axes, out.t, op=op, alpha=alpha)
        if keepdims:
            out = out.reshape(*[1 if i in axes else s for i, s in enumerate(self.shape)])
        return out, axes

    def sum(self, axis=None, keepdims=False):
        """Sum over `axis` (or all elements).  tensor.py:227-242."""
        data, axes = self._reduce(axis, keepdims, 1.0)
        track = self.requires_grad and _grad_enabled
        out = None

        def _backward():
            if self.requires_grad:
                g = out.grad
                g = g.reshape(*[1 if i in axes else s for i, s in enumerate(self.shape)])
                _accum_grad(self, g.broadcast_to(self.shape))

        out = self._node(data, (self,), "sum", _backward, track)
        return out

    def mean(self, axis=None, keepdims=False):
        """Mean over `axis` (or all elements).  tensor.py:244-267."""
        axes = self._norm_axes(axis)
        count = int(np.prod([self.shape[a] for a in axes])) if axes else 1
        data, _ = self._reduce(axis, keepdims, 1.0 / count)
        track = self.requires_grad and _grad_enabled
        out = None

        def _backward():
            if self.requires_grad:
                g = out.grad.reshape(*[1 if i in axes else s for i, s in enumerate(self.shape)])
                tmp = dev.empty(self.shape)
                K.ewise("SCALE_SHIFT", tmp.t, g.broadcast_to(self.shape).t, alpha=1.0 / count, beta=0.0)
                _accum_grad(self, tmp, owned=True)

        out = self._node(data, (self,), "mean", _backward, track)
        return out

    # ---------------------------------------------------------------- shapes
    def reshape(self, *shape):
        """A view with a new shape when the layout allows, else a copy
        (tensor.py:317-329)."""
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        data = self.data.reshape(*shape)
        track = self.requires_grad and _grad_enabled
        out = None

        def _backward():
            if self.requires_grad:
                _accum_grad(self, out.grad.reshape(*self.shape))

        out = self._node(data, (self,), "reshape", _backward, track)
        return out

    def transpose(self, dim0=-2, dim1=-1):
        """Swap two axes (a strided view, no copy).  tensor.py:331-345."""
        axes = list(range(self.ndim))
        axes[dim0], axes[dim1] = axes[dim1], axes[dim0]
        data = self.data.transpose(axes)
        track = self.requires_grad and _grad_enabled
        out = None

        def _backward():
            if self.requires_grad:
                _accum_grad(self, out.grad.transpose(axes))

        out = self._node(data, (self,), "transpose", _backward, track)
        return out

    def __getitem__(self, key):
        """Basic indexing (a strided view) or an integer index array on the
        first axis (a gather, as Embedding uses: tensor.py:374-387)."""
        track = self.requires_grad and _grad_enabled
        out = None
        if isinstance(key, (np.ndarray, list, DeviceArray)) and not (
                isinstance(key, np.ndarray) and key.dtype == bool):
            if self.ndim != 2:
                raise NotImplementedError("index arrays are supported on 2-D tensors (embedding tables)")
            if not isinstance(key, DeviceArray):
                # host ids are range-checked here; device-resident ids are the
                # caller's responsibility (the kernel clamps, it never reads out of bounds)
                ids = np.asarray(key)
                if ids.size and (ids.min() < 0 or ids.max() >= self.shape[0]):
                    raise IndexError(f"index out of range for axis 0 of size {self.shape[0]}")
            idx = dev.index_array(key)
            C = self.shape[1]
            data = dev.empty(tuple(idx.shape) + (C,))
            K.embedding_fwd(self.data.t, idx.t.reshape(-1), data.t.view(-1, C))

            def _backward():
                if self.requires_grad:
                    target, acc = _grad_target(self)
                    K.embedding_bwd(idx.t.reshape(-1), out.grad.contiguous().t.reshape(-1, C), target.t,
                                    accumulate=acc)

            out = self._node(data, (self,), "getitem", _backward, track)
            return out
        keys = key if isinstance(key, tuple) else (key,)
        if not all(k is None or k is Ellipsis or isinstance(k, (int, slice, np.integer)) for k in keys):
            raise NotImplementedError("only basic indexing (ints, slices, None, ...) or an integer "
                                      "index array on axis 0 is supported")
        data = DeviceArray(self.data.t[key])

        def _backward():
            if self.requires_grad:
                target, acc = _grad_target(self)
                if not acc:
                    K.fill(target.t, 0.0)
                K.ewise("COPY", target.t[key], out.grad.t, accumulate=True)

        out = self._node(data, (self,), "getitem", _backward, track)
        return out

    # ------------------------------------------------------------ elementwise
    def _unary(self, op, name, grad_fn):
        data = dev.empty(self.shape)
        K.ewise(op, data.t, self.data.t)
        track = self.requires_grad and _grad_enabled
        out = None

        def _backward():
            if self.requires_grad:
                _accum_grad(self, grad_fn(out), owned=True)

        out = self._node(data, (self,), name, _backward, track)
        return out

    def exp(self):
        """Elementwise e**x (tensor.py:391-402)."""
        def gf(out):
            g = dev.empty(self.shape)
            K.ewise("MUL", g.t, out.data.t, out.grad.t)
            return g
        return self._unary("EXP", "exp", gf)

    def log(self):
        """log(max(x, 1e-12)) (tensor.py:404-415)."""
        def gf(out):
            g = dev.empty(self.shape)
            K.ewise("RECIP_CLAMP", g.t, self.data.t)
            K.ewise("MUL", g.t, g.t, out.grad.t)
            return g
        return self._unary("LOG", "log", gf)

    # --------------------------------------------------------------- autograd
    def backward(self):
        """Reverse-mode autodiff from this scalar (tensor.py:453-477)."""
        assert self.data.size == 1, "backward() only works on scalar tensors - call .sum() or .mean() first"
        if self.grad is None:
            self.grad = dev.full(self.shape, 1.0)
        topo = []
        visited = set()
        stack = [(self, False)]
        while stack:
            node, processed = stack.pop()
            if processed:
                topo.append(node)
                continue
            if node in visited:
                continue
            visited.add(node)
            stack.append((node, True))
            for child in node._prev:
                if child not in visited:
                    stack.append((child, False))
        # consumers per tensor; gradients aliased in an earlier pass get
        # buffers of their own first (their sources may be accumulated into)
        counts: dict = {}
        for node in topo:
            _own_grad(node)
            for child in node._prev:
                counts[id(child)] = counts.get(id(child), 0) + 1
        global _single_consumer
        _single_consumer = {id(n) for n in topo if n._prev and counts.get(id(n), 0) == 1}
        try:
            for node in reversed(topo):
                node._backward()
        finally:
            _single_consumer = set()

    def zero_grad(self):
        self.grad = None

    def detach(self):
        return Tensor(self.data, requires_grad=False)

    def clone(self):
        return Tensor(self.data.copy(), requires_grad=self.requires_grad)

    def __repr__(self):
        return f"Tensor(data={self.data.numpy()}, grad={None if self.grad is None else self.grad.numpy()})"

    def __len__(self):
        return self.data.shape[0]

    def __float__(self):
        return float(self.data.numpy())
