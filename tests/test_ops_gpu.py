"""GPU parity of the GEMM, elementwise, reduction, row, embedding and Adam
kernels (through minitorch_amd.kernels and the Tensor API) against NumPy.

fp32 bar: |gpu - ref| <= 1e-5 + 1e-4 * |ref| elementwise, except where a test
states a looser, justified bound (long float32 dot products).
"""
import sys

import numpy as np
import pytest
from devarrays import H, T as _T, empty

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def T(x):
    return _T(np.ascontiguousarray(x, dtype=np.float32))


def close(got, ref, rtol=1e-4, atol=1e-5, name=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    lim = atol + rtol * np.abs(ref)
    assert np.all(err <= lim), f"{name}: max err {err.max():.3e} (max |ref| {np.abs(ref).max():.3e})"


@pytest.fixture(params=["bf16x3", "fp32"])
def gemm_mode(request, dev):
    """Each GEMM test runs under both product kernels for shapes of at least
    128 x 128: the bf16 three-piece split (the default) and fp32 MFMA."""
    from minitorch_amd import kernels as Kn

    prev = Kn.set_gemm_mode(Kn.GEMM_BF16X3 if request.param == "bf16x3" else Kn.GEMM_FP32)
    yield request.param
    Kn.set_gemm_mode(prev)


def dot_tol(K):
    """Elementwise tolerance for a float32 dot product of length K with N(0,1)
    entries: rounding error grows like sqrt(K) * 2^-24 * |terms|."""
    return 2e-6 * np.sqrt(K) * 4


@pytest.mark.parametrize("M,N,K,ta,tb,batch,bias", [
    (1, 1, 1, False, False, 1, False),
    (7, 5, 3, False, False, 1, True),
    (64, 64, 64, False, False, 1, False),
    (130, 70, 33, True, False, 1, True),
    (129, 257, 100, False, True, 3, False),
    (256, 65, 384, False, False, 1, True),
    (384, 1536, 4096, True, False, 1, False),   # weight-gradient shape: split-K path
    (33, 17, 2000, True, True, 2, False),
    # M <= 64 rows (decode steps): the one-launch skinny kernel
    (64, 1152, 384, False, False, 1, True),
    (64, 384, 512, False, False, 1, True),
    (64, 65, 384, False, False, 1, True),
    (50, 100, 500, True, True, 2, False),
    (64, 384, 1536, False, False, 1, True),     # skinny, K split over 3 workgroups
    (17, 40, 1000, True, False, 2, True),       # skinny split, scalar A loads, batched
    (64, 64, 4100, False, False, 1, False),     # K past the skinny range: tiled split-K
    # >= 128 x 128 and >= 2^27 multiply-adds, with K >= 1024 or >= 256 tiles of
    # 128 x 128: the bf16-split kernel in its default mode
    (256, 384, 1400, False, True, 1, True),     # ragged last k-tile, B contiguous along k
    (300, 260, 1111, True, True, 2, True),      # edge tiles on both sides, both operands transposed
    (4100, 1000, 33, False, False, 1, True),    # row strides of 33: no aligned vector loads
    (1000, 130, 5000, True, False, 1, False),   # split K with edge tiles
    (1024, 1024, 16, False, False, 8, True),    # one k-tile, batched
])
def test_gemm(dev, gemm_mode, M, N, K, ta, tb, batch, bias):
    from minitorch_amd import kernels as Kn

    _say(f"[gemm] {gemm_mode} M={M} N={N} K={K} ta={ta} tb={tb} batch={batch} bias={bias}")
    rng = np.random.default_rng(M * 7 + N + K)
    a = rng.standard_normal((batch, K, M) if ta else (batch, M, K), dtype=np.float32)
    b = rng.standard_normal((batch, N, K) if tb else (batch, K, N), dtype=np.float32)
    c0 = rng.standard_normal((batch, M, N), dtype=np.float32)
    bs = rng.standard_normal(N, dtype=np.float32)
    ta_, tb_, tc = T(a), T(b), T(c0)
    av = ta_.transpose(1, 2) if ta else ta_
    bv = tb_.transpose(1, 2) if tb else tb_
    Kn.gemm(av, bv, tc, alpha=0.5, beta=2.0, bias=T(bs) if bias else None, batch=batch)
    A = np.swapaxes(a, 1, 2) if ta else a
    B = np.swapaxes(b, 1, 2) if tb else b
    ref = 0.5 * (A.astype(np.float64) @ B) + 2.0 * c0 + (bs if bias else 0)
    close(H(tc), ref, rtol=1e-4, atol=dot_tol(K), name="gemm")


def test_ewise_broadcast_and_accumulate(dev):
    from minitorch_amd import kernels as Kn

    _say("[ewise]")
    rng = np.random.default_rng(1)
    a = rng.standard_normal((4, 1, 6), dtype=np.float32)
    b = rng.standard_normal((3, 1), dtype=np.float32) + 3.0
    out = empty((4, 3, 6))
    for op, f in (("ADD", np.add), ("SUB", np.subtract), ("MUL", np.multiply), ("DIV", np.divide)):
        Kn.ewise(op, out, T(a), T(b))
        close(H(out), f(a.astype(np.float64), b), name=op)
    Kn.ewise("POW", out, T(np.abs(a) + 0.5), T(b))
    close(H(out), (np.abs(a) + 0.5).astype(np.float64) ** b, rtol=2e-6 * 10, name="pow")
    for op, f in (("EXP", np.exp), ("TANH", np.tanh), ("NEG", np.negative),
                  ("LOG", lambda x: np.log(np.maximum(x, 1e-12)))):
        o = empty((4, 1, 6))
        Kn.ewise(op, o, T(a))
        close(H(o), f(a.astype(np.float64)), rtol=1e-5, name=op)
    # accumulate into a strided (transposed) output
    base = rng.standard_normal((6, 5), dtype=np.float32)
    ob = T(base)
    src = rng.standard_normal((5, 6), dtype=np.float32)
    Kn.ewise("COPY", ob.t(), T(src), accumulate=True)
    close(H(ob), base + src.T, name="accumulate-strided")


@pytest.mark.parametrize("shape,axes", [((5, 7), [0]), ((5, 7), [1]), ((3, 4, 5), [0, 1]),
                                        ((16384, 384), [0]), ((2, 3, 4, 5), [1, 3]), ((7,), [0]),
                                        ((64, 256, 384), [0, 1]), ((1, 5, 1, 7), [0, 2]),
                                        ((3, 1, 4, 5), [0, 1, 2]), ((4, 6, 8), [0, 2])])
def test_reduce_sum(dev, shape, axes):
    from minitorch_amd import kernels as Kn

    _say(f"[reduce] {shape} {axes}")
    rng = np.random.default_rng(2)
    a = rng.standard_normal(shape, dtype=np.float32)
    kept = [s for i, s in enumerate(shape) if i not in axes]
    out = empty(kept if kept else (1,))
    Kn.reduce(T(a), axes, out, alpha=0.5)
    ref = 0.5 * a.astype(np.float64).sum(axis=tuple(axes))
    R = int(np.prod([shape[i] for i in axes]))
    close(H(out).reshape(np.shape(ref)), ref, atol=dot_tol(R), name="reduce")


def test_reduce_merged_dims_bit_identical(dev):
    """Reducing (B, T, C) over (B, T) merges the two reduced dims into one of
    B*T rows; the result must be bit-identical to reducing the (B*T, C) view,
    and a transposed (non-mergeable) input must still match float64."""
    from minitorch_amd import kernels as Kn

    rng = np.random.default_rng(9)
    a = rng.standard_normal((64, 256, 384), dtype=np.float32)
    ta = T(a)
    o3 = empty((384,))
    o2 = empty((384,))
    Kn.reduce(ta, [0, 1], o3)
    Kn.reduce(ta.reshape(64 * 256, 384), [0], o2)
    assert np.array_equal(H(o3), H(o2))
    tt = ta.transpose(0, 2)  # (384, 256, 64), strides (1, 384, 98304)
    ot = empty((256,))
    Kn.reduce(tt, [0, 2], ot)
    close(H(ot), a.astype(np.float64).sum(axis=(0, 2)), atol=dot_tol(64 * 384), name="reduce-strided")


@pytest.mark.parametrize("rows,L,causal", [(3, 5, 0), (64, 65, 0), (40, 256, 256), (8, 1000, 0)])
def test_softmax_and_log_softmax(dev, rows, L, causal):
    from minitorch_amd import kernels as Kn
    from oracle.attention import causal_mask

    _say(f"[softmax] rows={rows} L={L} causal={causal}")
    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, L), dtype=np.float32) * 3
    dy = rng.standard_normal((rows, L), dtype=np.float32)
    xs = x.astype(np.float64)
    if causal:
        m = np.tile(causal_mask(causal, L), (rows // causal + 1, 1))[:rows]
        xs = np.where(m, -np.inf, xs)
    p = np.exp(xs - xs.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    y = empty((rows, L))
    Kn.softmax_fwd(T(x), y, causal_tq=causal)
    close(H(y), p, name="softmax")
    dx = empty((rows, L))
    Kn.softmax_bwd(y, T(dy), dx)
    g = dy * p
    close(H(dx), g - p * g.sum(-1, keepdims=True), name="softmax_bwd")
    if not causal:
        ly = empty((rows, L))
        Kn.softmax_fwd(T(x), ly, log=True)
        lp = np.log(p)
        close(H(ly), lp, atol=1e-5, name="log_softmax")
        Kn.softmax_bwd(ly, T(dy), dx, log=True)
        close(H(dx), dy - p * dy.sum(-1, keepdims=True), name="log_softmax_bwd")


@pytest.mark.parametrize("rows,C", [(5, 64), (300, 384), (17, 1536), (3, 33), (4099, 384), (1000, 2048),
                                    (301, 128), (301, 256), (301, 512), (301, 768), (301, 1024)])
def test_layernorm(dev, rows, C):
    from minitorch_amd import kernels as Kn
    from oracle.gpt import Holder, ln_bwd, ln_fwd

    _say(f"[layernorm] rows={rows} C={C}")
    rng = np.random.default_rng(4)
    x = rng.standard_normal((rows, C), dtype=np.float32) * 2 + 1
    gam = rng.standard_normal(C, dtype=np.float32)
    bet = rng.standard_normal(C, dtype=np.float32)
    dy = rng.standard_normal((rows, C), dtype=np.float32)
    y = empty((rows, C))
    mean = empty((rows,))
    std = empty((rows,))
    tx = T(x)
    Kn.layernorm_fwd(tx, T(gam), T(bet), y, mean, std, float(np.float32(1e-5)))
    ry, cache = ln_fwd(x.astype(np.float64), gam, bet)
    close(H(y), ry, name="ln_fwd")
    dx = empty((rows, C))
    dg = empty((C,))
    db = empty((C,))
    Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dx=dx)
    Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dgamma=dg, dbeta=db)
    hx, hg, hb = Holder(x.shape, np.float64), Holder((C,), np.float64), Holder((C,), np.float64)
    ln_bwd(dy.astype(np.float64), cache, hx, hg, hb)
    close(H(dx), hx.g, atol=1e-4 * np.sqrt(C) / 10, name="ln_dx")
    close(H(dg), hg.g, atol=dot_tol(rows), name="ln_dgamma")
    close(H(db), hb.g, atol=dot_tol(rows), name="ln_dbeta")
    # one fused call: dx added into a held gradient, dgamma / dbeta overwritten
    base = rng.standard_normal((rows, C), dtype=np.float32)
    dx2 = T(base)
    dg2 = T(np.full(C, 7.0, np.float32))
    db2 = T(np.full(C, -3.0, np.float32))
    Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dx=dx2, dgamma=dg2, dbeta=db2, accumulate=True,
                     accumulate_params=False)
    close(H(dx2), hx.g + base, atol=1e-4 * np.sqrt(C) / 10, name="ln_dx_fused_acc")
    assert np.array_equal(H(dg2), H(dg)) and np.array_equal(H(db2), H(db))
    # and the other way round: parameters accumulate, dx overwritten
    Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dx=dx2, dgamma=dg2, dbeta=db2, accumulate=False,
                     accumulate_params=True)
    close(H(dx2), hx.g, atol=1e-4 * np.sqrt(C) / 10, name="ln_dx_fused")
    close(H(dg2), 2 * hg.g, atol=2 * dot_tol(rows), name="ln_dgamma_acc")
    close(H(db2), 2 * hb.g, atol=2 * dot_tol(rows), name="ln_dbeta_acc")
    # an addend instead of accumulation: the same bits as accumulating into a
    # copy of it, with and without the parameter gradients; the addend unchanged
    for with_params in (False, True):
        acc_buf = T(base)
        kw = dict(dgamma=empty((C,)), dbeta=empty((C,))) if with_params else {}
        Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dx=acc_buf, accumulate=True, accumulate_params=False, **kw)
        add_src, out = T(base), empty((rows, C))
        kw = dict(dgamma=empty((C,)), dbeta=empty((C,))) if with_params else {}
        Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dx=out, addend=add_src, **kw)
        assert np.array_equal(H(out), H(acc_buf)), f"addend vs accumulate (params={with_params})"
        assert np.array_equal(H(add_src), base)
    with pytest.raises(ValueError):
        Kn.layernorm_bwd(tx, T(gam), mean, std, T(dy), dx=dx2, accumulate=True, addend=T(base))


def test_gelu(dev):
    from minitorch_amd import kernels as Kn
    from oracle.gpt import Holder, gelu_bwd, gelu_fwd

    _say("[gelu]")
    rng = np.random.default_rng(5)
    x = rng.standard_normal(10001, dtype=np.float32) * 3
    dy = rng.standard_normal(10001, dtype=np.float32)
    y = empty((10001,))
    Kn.gelu_fwd(T(x), y)
    ry, cache = gelu_fwd(x.astype(np.float64))
    close(H(y), ry, name="gelu")
    dx = empty((10001,))
    Kn.gelu_bwd(T(x), T(dy), dx)
    h = Holder(x.shape, np.float64)
    gelu_bwd(dy.astype(np.float64), cache, h)
    close(H(dx), h.g, name="gelu_bwd")


def test_cross_entropy_and_embedding(dev):
    import minitorch_amd as mt
    from oracle.gpt import cross_entropy, cross_entropy_bwd

    _say("[xent+embedding]")
    rng = np.random.default_rng(6)
    N, V, C = 300, 65, 48
    logits = rng.standard_normal((N, V), dtype=np.float32)
    labels = rng.integers(0, V, N)
    t = mt.Tensor(logits, requires_grad=True)
    loss = mt.cross_entropy_loss(t, mt.Tensor(labels.astype(np.float32)))
    loss.backward()
    rl, cache = cross_entropy(logits.astype(np.float64), labels)
    assert abs(float(loss) - float(rl)) < 1e-5 * abs(float(rl))
    close(t.grad.numpy(), cross_entropy_bwd(cache), atol=1e-7, name="xent_grad")
    W = rng.standard_normal((V, C), dtype=np.float32)
    ids = rng.integers(0, V, (4, 75))
    g = rng.standard_normal((4, 75, C), dtype=np.float32)
    tw = mt.Tensor(W, requires_grad=True)
    e = tw[ids]
    close(e.numpy(), W[ids], rtol=0, atol=0, name="gather")
    (e * mt.Tensor(g)).sum().backward()
    ref = np.zeros_like(W, dtype=np.float64)
    np.add.at(ref, ids, g)
    close(tw.grad.numpy(), ref, atol=dot_tol(300), name="scatter_add")


def test_adam_matches_oracle(dev):
    import minitorch_amd as mt
    from minitorch_amd.device import DeviceArray
    from oracle.gpt import Adam as OAdam

    _say("[adam]")
    rng = np.random.default_rng(7)
    shapes = [(5,), (33, 7), (300,), (2, 3, 4)]
    ps = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    tp = [mt.Tensor(p.copy(), requires_grad=True) for p in ps]
    opt = mt.Adam(tp, lr=3e-4)
    op = {str(i): p.copy() for i, p in enumerate(ps)}
    oopt = OAdam(op, lr=3e-4)
    for step in range(3):
        gs = [rng.standard_normal(s).astype(np.float32) for s in shapes]
        for t, g in zip(tp, gs):
            t.grad = mt.Tensor(g).data
        # one gradient a view at a 4-byte offset: that tensor takes the
        # kernel's scalar (unaligned) path
        wide = mt.Tensor(np.concatenate([[0.0], gs[2]]).astype(np.float32)).data
        tp[2].grad = DeviceArray(wide.t[1:])
        opt.step()
        oopt.step(op, {str(i): g for i, g in enumerate(gs)})
    # every operation is a separately rounded float32 one, as in NumPy
    for i, t in enumerate(tp):
        assert np.array_equal(t.numpy(), op[str(i)]), f"adam p{i} differs from the float32 oracle"


def test_adam_capturable_zero_grad_and_step(dev):
    """Capturable Adam: zero_grad zeroes every persistent gradient buffer in
    one launch (the pointer table's g fields; sizes straddle the 256-element
    blocks), the buffers keep their addresses, and steps with the device step
    count match the oracle's Adam."""
    import minitorch_amd as mt
    from minitorch_amd import device as mdev
    from oracle.gpt import Adam as OAdam

    _say("[adam capturable zero_grad]")
    rng = np.random.default_rng(17)
    shapes = [(5,), (33, 8), (256,), (257,), (2, 3, 4)]
    ps = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    tp = [mt.Tensor(p.copy(), requires_grad=True) for p in ps]
    opt = mt.Adam(tp, lr=3e-4).capturable(window=2)
    addrs = [t.grad.t.data_ptr() for t in tp]
    op = {str(i): p.copy() for i, p in enumerate(ps)}
    oopt = OAdam(op, lr=3e-4)
    for step in range(3):
        gs = [rng.standard_normal(s).astype(np.float32) for s in shapes]
        for t, g in zip(tp, gs):
            t.grad.t.copy_(mdev.from_host(g).t)
        opt.step()
        oopt.step(op, {str(i): g for i, g in enumerate(gs)})
        opt.zero_grad()
        mdev.synchronize()
        for i, t in enumerate(tp):
            assert t.grad.t.data_ptr() == addrs[i]
            assert not np.any(t.grad.numpy()), f"grad {i} not zeroed after step {step}"
    for i, t in enumerate(tp):
        assert np.array_equal(t.numpy(), op[str(i)]), f"adam p{i} differs from the float32 oracle"


def test_tensor_autograd_like_reference_checks(dev):
    """Analytic GPU gradients of the reference's test_grads.py cases
    (add/mul broadcast 76-85, matmul-batched 96-99, matmul-broadcast-batch
    102-105, mean-axis 116-119, reshape 150-153, transpose 156-159, tanh
    176-179, softmax 188-191, log_softmax 194-197) against float64 NumPy."""
    import minitorch_amd as mt
    from minitorch_amd import functional as F

    _say("[tensor autograd]")
    rng = np.random.default_rng(8)

    def run(f_gpu, f_np, *arrs):
        ts = [mt.Tensor(a, requires_grad=True) for a in arrs]
        out = f_gpu(*ts)
        (out * mt.Tensor(np.ones(out.shape, np.float32))).sum().backward()
        # numerical reference: float64 central differences of the NumPy form
        from oracle.attention import numerical_gradient

        xs = [a.astype(np.float64).copy() for a in arrs]
        num = numerical_gradient(lambda: float(np.sum(f_np(*xs))), xs, eps=1e-6)
        for t, n in zip(ts, num):
            close(t.grad.numpy(), n, rtol=1e-3, atol=1e-4, name=f_gpu.__name__ if hasattr(f_gpu, "__name__") else "")

    r = lambda *s: rng.standard_normal(s).astype(np.float32)
    run(lambda a, b: a + b, lambda a, b: a + b, r(3, 4), r(4))
    run(lambda a, b: a * b, lambda a, b: a * b, r(3, 4), r(3, 1))
    run(lambda a, b: a / b, lambda a, b: a / b, r(3, 4), np.abs(r(3, 4)) + 0.5)
    run(lambda a, b: a @ b, lambda a, b: a @ b, r(2, 3, 4), r(2, 4, 5))
    run(lambda a, b: a @ b, lambda a, b: a @ b, r(2, 3, 4), r(4, 5))
    run(lambda a: a.mean(axis=1), lambda a: a.mean(axis=1), r(3, 4))
    run(lambda a: a.reshape(4, 3).transpose(), lambda a: a.reshape(4, 3).T, r(3, 4))
    run(lambda a: F.tanh(a), np.tanh, r(3, 4))
    run(lambda a: F.softmax(a) * mt.Tensor(np.arange(4, dtype=np.float32)),
        lambda a: (np.exp(a) / np.exp(a).sum(-1, keepdims=True)) * np.arange(4), r(3, 4))
    run(lambda a: F.log_softmax(a) * mt.Tensor(np.arange(4, dtype=np.float32)),
        lambda a: (a - np.log(np.exp(a).sum(-1, keepdims=True))) * np.arange(4), r(3, 4))
    run(lambda a: (a ** 3), lambda a: a ** 3, r(3, 4))
    run(lambda a: a.exp(), np.exp, r(3, 4))


def test_embedding_backward_both_paths(dev):
    """Small tables take the one-hot GEMM path, large ones (V > 4096) the
    row-owner scatter kernel; both must equal np.add.at with repeated ids."""
    from minitorch_amd import kernels as Kn

    for V, n, C in ((65, 5000, 96), (5000, 700, 40)):
        _say(f"[embedding bwd] V={V} n={n} C={C}")
        rng = np.random.default_rng(V)
        ids = rng.integers(0, min(V, 50), n)  # heavy repetition
        g = rng.standard_normal((n, C), dtype=np.float32)
        base = rng.standard_normal((V, C), dtype=np.float32)
        dw = T(base)
        Kn.embedding_bwd(_T(ids, "int64"), T(g), dw, accumulate=True)
        ref = base.astype(np.float64).copy()
        np.add.at(ref, ids, g)
        close(H(dw), ref, atol=dot_tol(n), name=f"embedding_bwd V={V}")


def test_view_gradients_alias_and_accumulate_like_reference(dev):
    """Gradients through reshape / transpose views reach a single-consumer
    tensor without a copy; the values, a second backward pass without
    zero_grad (which accumulates, as the reference's _accum_grad does), a
    tensor used twice by one node and the attention output's strided
    gradient all match NumPy."""
    import minitorch_amd as mt
    import minitorch_amd.functional as F

    _say("[autograd] view aliasing")
    rng = np.random.default_rng(12)
    xa = rng.standard_normal((2, 6, 8), dtype=np.float32)
    wa = rng.standard_normal((2, 2, 6, 4), dtype=np.float32)
    x = mt.Tensor(xa, requires_grad=True)
    w = mt.Tensor(wa)
    h = x * 2.0                                   # non-leaf, one consumer (the reshape)
    v = h.reshape(2, 6, 2, 4).transpose(1, 2)     # (2, 2, 6, 4) view of h
    loss = (v * w).sum()
    loss.backward()
    gx = 2.0 * wa.transpose(0, 2, 1, 3).reshape(2, 6, 8)
    close(x.grad.numpy(), gx, name="x.grad")
    close(h.grad.numpy(), wa.transpose(0, 2, 1, 3).reshape(2, 6, 8), name="h.grad")
    # second pass without zero_grad: every gradient (intermediate ones
    # included) accumulates once more, as in the reference
    loss.backward()
    # the reference's semantics: loss.grad stays 1, and every intermediate
    # gradient accumulates its upstream's already accumulated one, so after
    # two passes (v*w).grad = 2, v.grad = w + 2w = 3w, the reshape's input
    # w' + 3w' = 4w', h.grad = w' + 4w' = 5w' and x.grad = 2w' + 2*5w' = 12w'
    Wt = wa.transpose(0, 2, 1, 3).reshape(2, 6, 8)
    close(v.grad.numpy(), 3 * wa, name="v.grad after two passes")
    close(h.grad.numpy(), 5 * Wt, name="h.grad after two passes")
    close(x.grad.numpy(), 12 * Wt, name="x.grad after two passes")
    # a tensor used twice by one node (x * x through a view)
    y = mt.Tensor(xa, requires_grad=True)
    r = y.reshape(2, 48)
    (r * r).sum().backward()
    close(y.grad.numpy(), 2 * xa, name="x*x")
    # attention output: gradient arriving through transpose / reshape (strided)
    B, H, T, D = 2, 3, 17, 16
    q, k, vv = (mt.Tensor(rng.standard_normal((B, T, H * D), dtype=np.float32), requires_grad=True)
                for _ in range(3))
    heads = lambda t: t.reshape(B, T, H, D).transpose(1, 2)
    o = F.causal_attention(heads(q), heads(k), heads(vv))
    m = o.transpose(1, 2).reshape(B, T, H * D)
    dy = rng.standard_normal((B, T, H * D), dtype=np.float32)
    (m * mt.Tensor(dy)).sum().backward()
    from oracle.attention import reference_attention
    sp = lambda a: a.reshape(B, T, H, D).transpose(0, 2, 1, 3)
    ro, rdq, rdk, rdv = reference_attention(sp(q.data.numpy()), sp(k.data.numpy()), sp(vv.data.numpy()),
                                            sp(dy), 1.0 / np.sqrt(D), True)
    mg = lambda a: a.transpose(0, 2, 1, 3).reshape(B, T, H * D)
    close(m.numpy(), mg(ro), name="attn out")
    for t, r_ in ((q, rdq), (k, rdk), (vv, rdv)):
        close(t.grad.numpy(), mg(r_), name="attn grad")


@pytest.mark.parametrize("rows,cols", [(1, 5), (7, 384), (384, 384), (3, 6)])
def test_pack3_unpack3(dev, rows, cols):
    """mtx_pack3_f32 / mtx_unpack3_f32 against NumPy concatenation and
    slicing, with every accumulate-mask bit (vector and scalar paths)."""

    from minitorch_amd import kernels as K

    rng = np.random.default_rng(rows * 1000 + cols)
    src = [rng.standard_normal((rows, cols), dtype=np.float32) for _ in range(3)]
    ts = [_T(a) for a in src]
    packed = empty((rows, 3 * cols))
    K.pack3(ts, packed)
    np.testing.assert_array_equal(packed.numpy(), np.concatenate(src, axis=1))
    base = [rng.standard_normal((rows, cols), dtype=np.float32) for _ in range(3)]
    for mask in range(8):
        acc = [bool(mask >> i & 1) for i in range(3)]
        outs = [_T(b.copy()) for b in base]
        K.unpack3(packed, outs, acc)
        for i in range(3):
            expect = src[i] + base[i] if acc[i] else src[i]
            np.testing.assert_array_equal(outs[i].numpy(), expect)


@pytest.mark.parametrize("M,N,K", [(37, 50, 23), (512, 1536, 384), (2048, 2048, 384), (96, 80, 8192),
                                   (300, 260, 5000)])
def test_gemm_gelu_epilogues(dev, gemm_mode, M, N, K):
    """mtx_gemm_act_f32: act 1 = gelu(A@B + bias) with the pre-activation in
    aux, act 2 = (A@B) * gelu'(aux), against NumPy float64 (the K = 8192 case
    takes the split-K path, whose reduce applies the epilogue; 2048 x 2048
    the split-bf16 kernel's own epilogue in its default mode, 512 x 1536 --
    48 tiles of 128 x 128 with K < 1024 -- the fp32 kernel in both)."""

    from minitorch_amd import kernels as K_

    rng = np.random.default_rng(M + N + K)
    a = (rng.standard_normal((M, K), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.standard_normal((K, N), dtype=np.float32)
    bias = rng.standard_normal(N, dtype=np.float32)
    ta, tb, tbias = (_T(x) for x in (a, b, bias))
    c = empty((M, N))
    h = empty((M, N))
    K_.gemm(ta, tb, c, bias=tbias, act=K_.GEMM_ACT_GELU, aux=h)
    v = a.astype(np.float64) @ b.astype(np.float64) + bias
    c0, c1 = 0.7978845834732056, 0.044714998453855515
    t = np.tanh(c0 * (v + c1 * v ** 3))
    gelu = 0.5 * v * (1 + t)
    dgelu = 0.5 * (1 + t) + 0.5 * v * (1 - t * t) * c0 * (1 + 3 * c1 * v * v)
    tol = lambda r: 1e-5 + 1e-4 * np.abs(r)
    assert np.all(np.abs(h.numpy() - v) <= tol(v))
    assert np.all(np.abs(c.numpy() - gelu) <= tol(gelu))
    d = empty((M, N))
    K_.gemm(ta, tb, d, act=K_.GEMM_ACT_GELU_BWD, aux=h)
    ref = (a.astype(np.float64) @ b.astype(np.float64)) * dgelu
    assert np.all(np.abs(d.numpy() - ref) <= tol(ref) + 1e-5 * np.abs(ref).max())


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,acc", [(384, 1152, 16384, False), (384, 65, 4096, True), (200, 130, 777, False),
                                       (64, 48, 300, True), (7, 5, 3, False), (384, 384, 0, True),
                                       (130, 300, 4001, True), (1536, 384, 16384, False)])
def test_gemm_wgrad_colsum(dev, gemm_mode, M, N, K, acc):
    """mtx_gemm_wgrad_f32: dW = A @ B (+ beta C) and the column sums of B (a
    Linear's bias gradient) from one launch, against NumPy float64.  The
    first case takes the split-K path (the sums go through the reduce), the
    odd shapes the edge-tile loaders, K = 0 gives C = beta C and sums of 0."""

    from minitorch_amd import kernels as K_

    _say(f"[gemm_wgrad] M={M} N={N} K={K} acc={acc}")
    rng = np.random.default_rng(M * 7 + N + K)
    # A as the transposed view of a (K, M) activation, as the weight gradient uses it
    x = rng.standard_normal((K, M), dtype=np.float32)
    g = rng.standard_normal((K, N), dtype=np.float32)
    c0 = rng.standard_normal((M, N), dtype=np.float32)
    s0 = rng.standard_normal(N, dtype=np.float32)
    tx, tg = T(x), T(g)
    c = T(c0)
    s = T(s0)
    beta = 1.0 if acc else 0.0
    K_.gemm(tx.transpose(0, 1), tg, c, 1.0, beta, None, M=M, N=N, K=K, colsum=s, colsum_accumulate=acc)
    ref_c = x.astype(np.float64).T @ g.astype(np.float64) + (c0 if acc else 0)
    ref_s = g.astype(np.float64).sum(0) + (s0 if acc else 0)
    close(H(c), ref_c, atol=dot_tol(max(K, 1)) * 2, name="wgrad_c")
    close(H(s), ref_s, atol=dot_tol(max(K, 1)) * 2, name="wgrad_colsum")
    # the same tiled product without the column sums gives the same C (M <= 64
    # products without them take the skinny kernel instead)
    c2 = T(c0)
    K_.gemm(tx.transpose(0, 1), tg, c2, 1.0, beta, None, M=M, N=N, K=K)
    if M > 64:
        assert np.array_equal(H(c2), H(c))
    else:
        close(H(c2), H(c), atol=dot_tol(max(K, 1)) * 2, name="wgrad_vs_plain")


@pytest.mark.parametrize("M,N,K", [(37, 50, 23), (16384, 384, 384), (96, 80, 8192), (64, 384, 2048),
                                   (200, 300, 3000)])
def test_gemm_residual_epilogue(dev, gemm_mode, M, N, K):
    """mtx_gemm_act_f32 act 4: C = A@B + bias + aux (a residual stream),
    against NumPy float64; the K = 8192 case takes the split-K path, whose
    reduce applies the add."""

    from minitorch_amd import kernels as K_

    _say(f"[gemm_residual] M={M} N={N} K={K}")
    rng = np.random.default_rng(M + 3 * N + K)
    a = (rng.standard_normal((M, K), dtype=np.float32) / np.float32(np.sqrt(K))).astype(np.float32)
    b = rng.standard_normal((K, N), dtype=np.float32)
    bias = rng.standard_normal(N, dtype=np.float32)
    res = rng.standard_normal((M, N), dtype=np.float32)
    c = empty((M, N))
    K_.gemm(T(a), T(b), c, bias=T(bias), act=K_.GEMM_ACT_ADD, aux=T(res))
    ref = a.astype(np.float64) @ b.astype(np.float64) + bias + res
    close(H(c), ref, atol=dot_tol(K), name="gemm_residual")
    with pytest.raises(ValueError):
        K_.gemm(T(a), T(b), c, act=K_.GEMM_ACT_ADD, aux=c)  # the residual cannot be C itself


@pytest.mark.parametrize("M,N,K", [(64, 384, 1536), (64, 384, 384), (64, 64, 256), (7, 130, 700), (33, 384, 384),
                                   (1, 2048, 4096), (64, 1000, 3000), (16, 64, 16), (5, 100, 7)])
def test_gemm_ln_matches_gemm_then_layernorm(dev, M, N, K):
    """mtx_gemm_ln_f32 (x += h @ W + b, then LayerNorm of x's rows: a decode
    step's residual projection and the LayerNorm after it) against float64
    NumPy and against mtx_gemm_f32 followed by mtx_layernorm_fwd_f32 on the
    same inputs (the two differ only in how K's partial sums are grouped);
    split counts 1 to 8, rows of 1 to 32 values per lane; a second call on
    the same inputs gives the same bits (the split and its order are
    fixed)."""
    from minitorch_amd import kernels as Kn
    from oracle.gpt import ln_fwd

    _say(f"[gemm_ln] M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    h = rng.standard_normal((M, K), dtype=np.float32)
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    b = rng.standard_normal(N, dtype=np.float32)
    x0 = rng.standard_normal((M, N), dtype=np.float32)
    gam = rng.standard_normal(N, dtype=np.float32)
    bet = rng.standard_normal(N, dtype=np.float32)
    eps = float(np.float32(1e-5))
    xf, yf = T(x0), empty((M, N))
    Kn.gemm_ln(T(h), T(w), xf, T(gam), T(bet), eps, yf, bias=T(b))
    xs, ys = T(x0), empty((M, N))
    Kn.gemm(T(h), T(w), xs, beta=1.0, bias=T(b))
    Kn.layernorm_fwd(xs, T(gam), T(bet), ys, empty((M,)), empty((M,)), eps)
    xf2, yf2 = T(x0), empty((M, N))
    Kn.gemm_ln(T(h), T(w), xf2, T(gam), T(bet), eps, yf2, bias=T(b))
    assert np.array_equal(H(xf), H(xf2)) and np.array_equal(H(yf), H(yf2))
    close(H(xf), H(xs), atol=dot_tol(K), name="gemm_ln x vs gemm")
    close(H(yf), H(ys), rtol=1e-4, atol=1e-4, name="gemm_ln y vs layernorm")
    xr = x0.astype(np.float64) + h.astype(np.float64) @ w + b
    close(H(xf), xr, atol=dot_tol(K), name="gemm_ln x")
    close(H(xs), xr, atol=dot_tol(K), name="gemm x")
    yr = ln_fwd(H(xf).astype(np.float64), gam.astype(np.float64), bet.astype(np.float64), 1e-5)[0]
    close(H(yf), yr, rtol=1e-4, atol=1e-4, name="gemm_ln y")


def test_gemm_nonfinite_and_near_overflow(dev, gemm_mode):
    """Inputs at the edge of the fp32 range, under both product kernels (a
    512 x 512 x 1024 product runs on the bf16-split kernel in its default
    mode, K split four ways).  Row 0
    of A holds 3.4e38 (finite, but above bf16's largest finite value
    3.39e38), row 1 holds +Inf; B's first row is 0.5.  fp32 MFMA: row 0 is
    the finite fp32 result, row 1 is +Inf.  Split mode: both rows are NaN
    (the high bf16 piece of 3.4e38 rounds to Inf, and Inf - Inf follows), as
    documented for mtx_gemm_set_mode.  Every other row is unaffected."""
    from minitorch_amd import kernels as Kn

    _say(f"[gemm edge values] {gemm_mode}")
    M = N = 512
    K = 1024
    rng = np.random.default_rng(99)
    a = 0.1 * rng.standard_normal((M, K), dtype=np.float32)
    b = 0.1 * rng.standard_normal((K, N), dtype=np.float32)
    a[0, 0] = np.float32(3.4e38)
    a[1, 0] = np.inf
    b[0, :] = 0.5
    tc = T(np.zeros((M, N), np.float32))
    Kn.gemm(T(a), T(b), tc)
    c = H(tc)
    ref = a[2:].astype(np.float64) @ b
    close(c[2:], ref, rtol=1e-4, atol=dot_tol(K), name="rows 2..")
    if gemm_mode == "fp32":
        ref0 = a[0].astype(np.float64) @ b
        assert np.all(np.isfinite(c[0]))
        np.testing.assert_allclose(c[0], ref0, rtol=1e-5)
        assert np.all(c[1] == np.inf)
    else:
        assert np.all(np.isnan(c[0])) and np.all(np.isnan(c[1]))


def test_failed_capture_releases_its_pool(dev):
    """A capture that fails at mtx_graph_end (invalidated by synchronising
    the capturing stream) releases its memory pool: a block freed into that
    pool during the capture is reused by the next allocation of its size."""
    import ctypes as C

    from minitorch_amd import _lib as L

    _say("[graph capture failure]")
    lib = L.lib()
    L.call("mtx_device_sync")
    L.call("mtx_empty_cache")  # no cached general-pool block of this size
    s = C.c_void_p()
    L.call("mtx_stream_create", C.byref(s))
    nbytes = 37 << 20
    p = C.c_void_p()
    L.call("mtx_malloc", C.byref(p), nbytes)
    try:
        L.call("mtx_graph_begin", s)
        h = C.c_void_p()
        try:
            L.call("mtx_free", p)  # goes to the capture's pool
            rc_sync = lib.mtx_stream_sync(s)
        finally:
            rc_end = lib.mtx_graph_end(s, C.byref(h))
        if rc_end == 0:
            lib.mtx_graph_destroy(h)
            pytest.skip(f"the runtime did not invalidate the capture (sync rc {rc_sync})")
        assert rc_sync != 0
        q = C.c_void_p()
        L.call("mtx_malloc", C.byref(q), nbytes)
        assert q.value == p.value, "the failed capture's pool kept the block"
        L.call("mtx_free", q)
        # the failure is not reported again by the next launch
        t = T(np.ones(1000, np.float32))
        from minitorch_amd import kernels as Kn

        Kn.ewise("COPY", t, t)
        L.call("mtx_device_sync")
    finally:
        L.call("mtx_device_sync")
        L.call("mtx_stream_destroy", s)
