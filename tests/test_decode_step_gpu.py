"""The persistent decode step (mtx_decode_step_f32: one cooperative launch per
greedy token step, grid-wide barriers between stages) on the GPU.

  * Tokens identical to the oracle's cached greedy decoding (oracle/gpt.py,
    pinned by the reference's own greedy tokens) and top-2 margins within
    1e-4 of the oracle's, for every kernel instance the models below reach:
    row widths C = 128, 256, 384, 512, logits per lane for V <= 128 and
    V <= 256 (V = 256: every lane's four logits in use), odd batch sizes (a
    stage-A item with one sequence, a stage-B item with fewer than 8 rows;
    a batch of one), one to six blocks, and batches with more
    stage-A and stage-B items than resident workgroups (C = 128, B = 300;
    C = 384, B = 96; C = 512, B = 72, where fc1's weight slab shares stage
    A's LDS), so that workgroups run several items of a stage and request
    later items' weight slabs inside the stage.
  * The multi-launch step (the chain of mtx_decode_qkv_attn_f32 ...
    mtx_head_pick_f32) gives the same tokens, margins within 2e-5.
  * Deterministic: two runs give bit-identical tokens and margins.
  * The bounded grid-wide wait: a step whose waits are told to fail at once
    (wait_limit_us < 0) ends every workgroup, leaves lengths unchanged,
    reports the failure through mtx_decode_step_status, and the following
    steps on the same workspace do nothing until mtx_decode_step_reset;
    after the reset a step gives the chain's token.
  * Steps per launch: five launches of one step and one launch of five
    steps agree bit for bit.
  * One workspace shared in turn by launches of different grid sizes gives
    the results of workspaces of their own (each launch counts its barriers
    from the base the launch before it left).
  * generate_greedy's kept state (prefill replayed from a HIP graph from the
    second call of a shape) gives the oracle's tokens call after call, sees
    weights changed in place, and is rebuilt for new parameter buffers or a
    new prompt shape.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _model(cfg, seed):
    import minitorch_amd as mt
    from oracle.gpt import init_params

    P = init_params(cfg, np.random.default_rng(seed))
    model = mt.GPT(cfg.vocab, cfg.block, cfg.n_embd, cfg.n_head, cfg.n_layer, dropout=0.0)
    model.load_state_dict(P)
    model.eval()
    return model, P


CASES = [
    # (vocab, block, n_embd, n_head, n_layer), B, T0, n_new
    ((65, 64, 128, 2, 3), 5, 7, 40),
    ((200, 48, 256, 4, 2), 9, 3, 30),
    ((65, 40, 512, 8, 1), 3, 5, 20),
    ((65, 256, 384, 6, 6), 64, 32, 16),
    ((65, 24, 128, 2, 2), 300, 3, 6),
    ((65, 16, 384, 6, 1), 96, 3, 6),
    ((65, 16, 512, 8, 1), 72, 3, 6),
    ((256, 40, 256, 4, 2), 1, 4, 20),
]


@pytest.mark.parametrize("shape,B,T0,n", CASES)
def test_persistent_matches_oracle_and_chain(dev, monkeypatch, shape, B, T0, n):
    import minitorch_amd.transformer as tr
    from oracle.gpt import GPTConfig, greedy_generate_cached

    cfg = GPTConfig(*shape)
    _say(f"[decode_step] C={cfg.n_embd} H={cfg.n_head} L={cfg.n_layer} V={cfg.vocab} B={B} T0={T0} n={n}")
    model, P = _model(cfg, 40 + cfg.n_embd)
    prompts = np.random.default_rng(41).integers(0, cfg.vocab, (B, T0))
    import minitorch_amd.device as dv

    assert tr._PERSISTENT_STEP
    probe = [(dv.empty((B, T0 + n, cfg.n_embd)), dv.empty((B, T0 + n, cfg.n_embd))) for _ in range(cfg.n_layer)]
    assert model._decode_step(probe, B, T0 + n) is not None, "the persistent step must be the path under test"
    del probe
    toks, margins = model.generate_greedy(prompts, n, return_margins=True)
    ref, rmarg = greedy_generate_cached(P, cfg, prompts, n)
    np.testing.assert_array_equal(toks, ref)
    np.testing.assert_allclose(margins, rmarg, rtol=0, atol=1e-4)
    monkeypatch.setattr(tr, "_PERSISTENT_STEP", False)
    t_chain, m_chain = model.generate_greedy(prompts, n, return_margins=True)
    np.testing.assert_array_equal(toks, t_chain)
    np.testing.assert_allclose(margins, m_chain, rtol=0, atol=2e-5)


def test_persistent_is_deterministic(dev):
    from oracle.gpt import GPTConfig

    _say("[decode_step] two runs, bit-identical")
    cfg = GPTConfig(65, 64, 256, 4, 3)
    model, _ = _model(cfg, 43)
    prompts = np.random.default_rng(44).integers(0, cfg.vocab, (17, 9))
    t1, m1 = model.generate_greedy(prompts, 30, return_margins=True)
    t2, m2 = model.generate_greedy(prompts, 30, return_margins=True)
    np.testing.assert_array_equal(t1, t2)
    np.testing.assert_array_equal(m1, m2)


def test_wait_failure_is_reported_and_cleared(dev, monkeypatch):
    import minitorch_amd.transformer as tr
    from minitorch_amd import _lib as L
    from minitorch_amd import device as dv
    from minitorch_amd.tensor import no_grad
    from oracle.gpt import GPTConfig

    _say("[decode_step] bounded wait: forced failure, status, reset")
    cfg = GPTConfig(65, 32, 128, 2, 2)
    B, T0 = 6, 5
    model, _ = _model(cfg, 45)
    prompts = np.random.default_rng(46).integers(0, cfg.vocab, (B, T0))
    monkeypatch.setattr(tr, "_PERSISTENT_STEP", False)
    want = model.generate_greedy(prompts, 2)[:, T0 + 1]  # the chain's first decode-step token
    monkeypatch.setattr(tr, "_PERSISTENT_STEP", True)

    # the state generate_greedy builds before its first decode step
    from minitorch_amd import kernels as K

    Tmax = T0 + 2
    C = cfg.n_embd
    caches = [(dv.empty((B, Tmax, C)), dv.empty((B, Tmax, C))) for _ in model.blocks]
    ids = dv.empty((Tmax, B), dtype="int64")
    margins = dv.empty((2, B))
    pos = model._positions(Tmax)
    with no_grad():
        x = model.tok_emb(dv.index_array(prompts)) + model.pos_emb(dv.DeviceArray(pos.t[:T0]))
        for block, cache in zip(model.blocks, caches):
            x = block.forward_cached(x, cache, 0)
        from minitorch_amd.tensor import Tensor

        h = model.ln_f(Tensor(x.data.t[:, T0 - 1:T0, :]))
        K.argmax_rows(model.lm_head(h).data.t.view(B, -1), idx=ids.t[T0], margin=margins.t[0])
    cur = ids.t[T0].clone()
    lengths = dv.full((B,), T0 + 1, "int32").t
    posd = dv.full((1,), T0, "int64").t
    ds = model._decode_step(caches, B, Tmax)
    assert ds is not None
    assert B // 2 * cfg.n_head >= 2  # at least two workgroups, so some workgroup waits

    ds(cur, ids.t, lengths, posd, margins=margins.t, t_base=T0, wait_limit_us=-1)
    with pytest.raises(L.MtxError, match="wait ran out"):
        ds.check()
    np.testing.assert_array_equal(lengths.numpy(), np.full(B, T0 + 1))
    assert int(posd.numpy()[0]) == T0
    # a later step on the failed workspace does nothing, whatever its limit
    ds(cur, ids.t, lengths, posd, margins=margins.t, t_base=T0)
    with pytest.raises(L.MtxError, match="wait ran out"):
        ds.check()
    np.testing.assert_array_equal(lengths.numpy(), np.full(B, T0 + 1))
    # cleared, the step runs: the chain's token, lengths and position advanced
    ds.reset()
    ds(cur, ids.t, lengths, posd, margins=margins.t, t_base=T0)
    ds.check()
    np.testing.assert_array_equal(lengths.numpy(), np.full(B, T0 + 2))
    assert int(posd.numpy()[0]) == T0 + 1
    np.testing.assert_array_equal(ids.numpy()[T0 + 1], want)
    np.testing.assert_array_equal(cur.numpy(), want)


def _prefilled(model, prompts, Tmax, n_margins):
    """The state generate_greedy builds before its first decode step: the
    prompt's caches, the first pick in ids[T0] and cur, lengths T0 + 1,
    position T0."""
    from minitorch_amd import device as dv
    from minitorch_amd import kernels as K
    from minitorch_amd.tensor import Tensor, no_grad

    B, T0 = prompts.shape
    C = model.tok_emb.weight.shape[1]
    caches = [(dv.empty((B, Tmax, C)), dv.empty((B, Tmax, C))) for _ in model.blocks]
    ids = dv.empty((Tmax, B), dtype="int64")
    margins = dv.empty((n_margins, B))
    pos = model._positions(Tmax)
    with no_grad():
        x = model.tok_emb(dv.index_array(prompts)) + model.pos_emb(dv.DeviceArray(pos.t[:T0]))
        for block, cache in zip(model.blocks, caches):
            x = block.forward_cached(x, cache, 0)
        h = model.ln_f(Tensor(x.data.t[:, T0 - 1:T0, :]))
        K.argmax_rows(model.lm_head(h).data.t.view(B, -1), idx=ids.t[T0], margin=margins.t[0])
    cur = ids.t[T0].clone()
    lengths = dv.full((B,), T0 + 1, "int32").t
    posd = dv.full((1,), T0, "int64").t
    return caches, ids, margins, cur, lengths, posd


def test_steps_per_launch_agree(dev):
    """Five token steps as five launches and as one launch (the picks,
    lengths and position passed between steps inside the kernel) give the
    same ids and margins, bit for bit."""
    from oracle.gpt import GPTConfig

    _say("[decode_step] 5 launches of one step vs one launch of 5 steps")
    cfg = GPTConfig(65, 32, 256, 4, 2)
    B, T0, n = 7, 6, 5
    model, _ = _model(cfg, 47)
    prompts = np.random.default_rng(48).integers(0, cfg.vocab, (B, T0))
    Tmax = T0 + 1 + n
    outs = []
    for per_launch in (1, n):
        caches, ids, margins, cur, lengths, posd = _prefilled(model, prompts, Tmax, n + 1)
        ds = model._decode_step(caches, B, Tmax)
        for _ in range(n // per_launch):
            ds(cur, ids.t, lengths, posd, margins=margins.t, t_base=T0, steps=per_launch)
        ds.check()
        outs.append((ids.numpy()[T0:T0 + n + 1].copy(), margins.numpy().copy(), lengths.numpy().copy()))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    np.testing.assert_array_equal(outs[0][2], np.full(B, T0 + 1 + n))
    np.testing.assert_array_equal(outs[1][2], np.full(B, T0 + 1 + n))


def test_workspace_shared_across_grid_sizes(dev):
    """One workspace used in turn by steps of two batch sizes whose grids
    differ (8 and 24 workgroups at C = 128, neither launch's barrier count a
    multiple of the other grid): every step gives the ids and margins, bit
    for bit, of the same steps on workspaces of their own."""
    from oracle.gpt import GPTConfig

    _say("[decode_step] one workspace, grids of 8 and 24 workgroups in turn")
    cfg = GPTConfig(65, 32, 128, 2, 2)
    T0, n = 4, 4
    Tmax = T0 + 1 + n
    model, _ = _model(cfg, 49)
    prompts = {B: np.random.default_rng(50 + B).integers(0, cfg.vocab, (B, T0)) for B in (5, 17)}

    def run(shared):
        states, steps = {}, {}
        for B in (5, 17):
            states[B] = _prefilled(model, prompts[B], Tmax, n + 1)
            steps[B] = model._decode_step(states[B][0], B, Tmax)
        if shared:
            steps[5].workspace, steps[5]._ws_bytes = steps[17].workspace, steps[17]._ws_bytes
        for _ in range(n):
            for B in (5, 17):
                _, ids, margins, cur, lengths, posd = states[B]
                steps[B](cur, ids.t, lengths, posd, margins=margins.t, t_base=T0)
        for B in (5, 17):
            steps[B].check()
        return {B: (states[B][1].numpy()[T0:T0 + n + 1].copy(), states[B][2].numpy().copy()) for B in (5, 17)}

    own, shared = run(False), run(True)
    for B in (5, 17):
        np.testing.assert_array_equal(shared[B][0], own[B][0])
        np.testing.assert_array_equal(shared[B][1], own[B][1])


def test_greedy_state_kept_across_calls(dev):
    """generate_greedy keeps the persistent step's device state for the most
    recent prompt shape: repeated calls (the prefill eager on the first call,
    recorded as a HIP graph on the second, replayed after that) give the
    oracle's tokens for each call's prompts; a weight changed in place is
    read by the replayed prefill and the step; parameters given new buffers
    (load_state_dict) or another prompt shape rebuild the state."""
    from oracle.gpt import GPTConfig, greedy_generate_cached, init_params

    _say("[decode_step] state kept across generate_greedy calls")
    cfg = GPTConfig(65, 48, 128, 2, 2)
    B, T0, n = 6, 5, 12
    model, P = _model(cfg, 51)
    rng = np.random.default_rng(52)

    def check(P_, B_=B, T0_=T0, n_=n, graph=True):
        prompts = rng.integers(0, cfg.vocab, (B_, T0_))
        toks, marg = model.generate_greedy(prompts, n_, return_margins=True, graph=graph)
        ref, rmarg = greedy_generate_cached(P_, cfg, prompts, n_)
        np.testing.assert_array_equal(toks, ref)
        np.testing.assert_allclose(marg, rmarg, rtol=0, atol=1e-4)

    for _ in range(3):
        check(P)
    st = model.__dict__["_greedy_st"]
    assert st is not None and st["graph"] is not None and st["calls"] == 3
    newb = (rng.standard_normal(cfg.vocab) * 0.5).astype(np.float32)
    model.lm_head.bias.data.t.copy_(newb)
    P["lm_head.bias"] = newb
    check(P)
    assert model.__dict__["_greedy_st"] is st
    P2 = init_params(cfg, np.random.default_rng(53))
    model.load_state_dict(P2)
    check(P2)
    st2 = model.__dict__["_greedy_st"]
    assert st2 is not st and st2["calls"] == 1
    check(P2, B_=4, T0_=7)
    assert model.__dict__["_greedy_st"]["key"] == (4, 7)
    # one new token (the prefill's pick only, no decode launch), then the
    # prefill run eagerly on a kept state
    check(P2, B_=4, T0_=7, n_=1)
    check(P2, B_=4, T0_=7, graph=False)
