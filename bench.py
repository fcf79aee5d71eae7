#!/usr/bin/env python3
"""Benchmark of the causal-MHA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

A *step* is one fused causal-attention forward + backward over the whole batch
of config C3 (B=8, H=16, T=2048, D=64, bf16 Q/K/V,
fp32 accumulation, LSE and gradients), the configuration the throughput
target (>= 50% of the dense bf16 MFMA peak) is quoted on.  Inputs are synthetic (seeded N(0,1)*0.5,
rounded to bf16) and resident in HBM before timing starts.

value = algorithmic causal FLOPs (7*B*H*T^2*D per fwd+bwd) / step time, in
TFLOP/s.  The same JSON line carries:
  roofline      -- the dominant kernel: its algorithmic FLOPs per launch over
                   its average launch time (HIP events on the launch stream)
                   against the 2516.6 TFLOP/s dense-bf16 MFMA peak;
  cpu_baseline  -- the NumPy restatement of the reference (oracle/, the
                   reference's own NumPy semantics) timed on this host on a
                   bounded sample of (b,h) slices of the same workload;
  also          -- config C1 (fp32, B=32,H=8,T=256,D=64) on the same kernels,
                   and per-phase timings.
Every timed loop runs after ~30 ms of its own launches, untimed (SETTLE_MS:
the GPU's clock transient after idle gaps), and W warm-up calls; the C3 leg
also reports its cold-start step time.  Only one GPU is used: --gpus > 1 exits
with a message.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

PEAK_BF16 = 2516.6  # TFLOP/s, dense bf16 MFMA, MI355X
PEAK_FP32 = 157.3   # TFLOP/s, fp32 MFMA
PEAK_HBM = 8000.0   # GB/s


def attn_flops(B, H, T, D):
    """Algorithmic causal FLOPs: fwd 2*B*H*T^2*D, bwd 5*B*H*T^2*D."""
    u = B * H * T * T * D
    return 2 * u, 5 * u


class _Event:
    """A HIP event of the library runtime (mtx_event_*), recorded on the
    stream the package launches on."""

    def __init__(self):
        import ctypes as C

        from minitorch_amd import _lib as L

        self._C, self._L = C, L
        self.h = C.c_void_p()
        L.call("mtx_event_create", C.byref(self.h))

    def record(self):
        self._L.call("mtx_event_record", self.h, self._L.stream_handle())

    def elapsed_time(self, end) -> float:
        ms = self._C.c_float(0.0)
        self._L.call("mtx_event_elapsed_ms", self.h, end.h, self._C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            self._L.lib().mtx_event_destroy(self.h)
        except Exception:
            pass


def _events():
    return _Event(), _Event()


def _sync():
    from minitorch_amd import device as D

    D.synchronize()


# Every timed loop first runs its own launches, untimed, for SETTLE_MS of GPU
# time, then its warm-up calls, then the timed calls.  After an idle gap of
# more than a few milliseconds (host work between legs: input generation,
# model construction) the GPU runs the first ~2 ms of a heavy MFMA load at
# full speed and the next ~20 ms about 20% slower before it settles; on the C3
# step, 5 warm-up + 20 timed steps measured 0.39 ms per step after 10 ms to 1 s
# of idle and 0.33 ms right after the same load (profiles/attn_c3_power_transient.md).
# A 20-step window would otherwise time that transient instead of the rate a
# continuously running job sees.  The C3 leg also reports its cold-start time
# (no settling, right after the inputs are uploaded) beside the settled one.
SETTLE_MS = 30.0
SETTLE_MAX_CALLS = 1000


def settle(fn, ms=SETTLE_MS):
    """Run fn() untimed for about `ms` of GPU time (its duration estimated
    from one call, at most SETTLE_MAX_CALLS calls), ending without a
    synchronisation so the GPU does not idle before what follows."""
    if ms <= 0:
        return
    e0, e1 = _events()
    e0.record()
    fn()
    e1.record()
    _sync()
    t = max(e0.elapsed_time(e1), 1e-3)
    for _ in range(min(SETTLE_MAX_CALLS, int(math.ceil(ms / t)))):
        fn()


def time_loop(fn, steps, warmup, settle_ms=SETTLE_MS):
    """Average ms per call of fn() over `steps` calls after `warmup` calls
    (preceded by `settle_ms` of untimed calls), bracketed by device
    synchronisation and HIP events on the launch stream."""
    settle(fn, settle_ms)
    for _ in range(warmup):
        fn()
    _sync()
    e0, e1 = _events()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    _sync()
    return e0.elapsed_time(e1) / steps


def make_inputs(B, H, T, D, dtype, seed, scale_qkv):
    """Seeded inputs, drawn q, k, v, dO in that order; bf16 rounding (RNE) on
    the host copy to the device.  Returns (host fp32 copies of the device
    values, device arrays)."""
    from minitorch_amd import device as Dv
    from oracle.attention import bf16_round

    rng = np.random.default_rng(seed)
    shp = (B, H, T, D)
    arrs = [scale_qkv * rng.standard_normal(shp, dtype=np.float32) for _ in range(3)]
    arrs.append(rng.standard_normal(shp, dtype=np.float32))
    dev = [Dv.from_host(a, dtype).t for a in arrs]
    host = [bf16_round(a) if dtype == "bfloat16" else a for a in arrs]
    return host, dev


def bench_attention(B, H, T, D, dtype, seed, scale_qkv, steps, warmup, cold=False):
    from minitorch_amd import _lib as L
    from minitorch_amd import device as Dv
    from minitorch_amd import kernels as K

    arrs, (q, k, v, do) = make_inputs(B, H, T, D, dtype, seed, scale_qkv)
    scale = 1.0 / math.sqrt(D)
    o, lse = K.attn_fwd(q, k, v, scale, True)
    dq, dk, dv = K.attn_bwd(q, k, v, o, do, lse, scale, True)
    ws = Dv.empty_buf((L.lib().mtx_attn_bwd_workspace_bytes(B, H, T),), "uint8")

    def step():
        K.attn_fwd(q, k, v, scale, True, out=o, lse=lse)
        K.attn_bwd(q, k, v, o, do, lse, scale, True, dq=dq, dk=dk, dv=dv, workspace=ws)

    cold_ms = time_loop(step, steps, warmup, settle_ms=0) if cold else None
    ms_step = time_loop(step, steps, warmup)
    # per-kernel averages (each phase is one kernel launch).  Two-pass: the dQ
    # pass also computes delta = rowsum(dO*O), which the dK/dV pass reads.
    # One-pass: "prep" computes delta and zeroes dq, "dkdvq" is the key-outer
    # kernel that writes dK/dV and adds dQ.
    ms_fwd = time_loop(lambda: K.attn_fwd(q, k, v, scale, True, out=o, lse=lse), steps, 2)
    ph = {}
    if K.attn_bwd_onepass_used(dtype, D):
        phases = (("prep", L.ATTN_BWD_ONEPASS | L.ATTN_BWD_DELTA),
                  ("dkdvq", L.ATTN_BWD_ONEPASS | L.ATTN_BWD_DQ | L.ATTN_BWD_DKDV))
    else:
        phases = (("dq", L.ATTN_BWD_DELTA | L.ATTN_BWD_DQ), ("dkdv", L.ATTN_BWD_DKDV))
    for name, mask in phases:
        ph[name] = time_loop(lambda m=mask: K.attn_bwd(q, k, v, o, do, lse, scale, True, dq=dq, dk=dk,
                                                       dv=dv, workspace=ws, phases=m), steps, 2)
    _sync()
    r = dict(ms_step=ms_step, ms_fwd=ms_fwd, **{f"ms_{k}": v for k, v in ph.items()})
    if cold:
        r["ms_step_cold"] = cold_ms
    return r, arrs


def c3_series(nwin=30, per=5):
    """The C3 step's time over consecutive windows of `per` steps (HIP events
    between the windows, no synchronisation inside a run of windows): once
    right after the same load, and after idle gaps of 10 ms to 1 s.  Prints
    one line per run, ms per step for each window."""
    from minitorch_amd import _lib as L
    from minitorch_amd import device as Dv
    from minitorch_amd import kernels as K

    B, H, T, D = 8, 16, 2048, 64
    _, (q, k, v, do) = make_inputs(B, H, T, D, "bfloat16", 3, 0.5)
    scale = 1.0 / math.sqrt(D)
    o, lse = K.attn_fwd(q, k, v, scale, True)
    dq, dk, dv = K.attn_bwd(q, k, v, o, do, lse, scale, True)
    ws = Dv.empty_buf((L.lib().mtx_attn_bwd_workspace_bytes(B, H, T),), "uint8")

    def step():
        K.attn_fwd(q, k, v, scale, True, out=o, lse=lse)
        K.attn_bwd(q, k, v, o, do, lse, scale, True, dq=dq, dk=dk, dv=dv, workspace=ws)

    def run(tag):
        evs = [_Event() for _ in range(nwin + 1)]
        evs[0].record()
        for w in range(nwin):
            for _ in range(per):
                step()
            evs[w + 1].record()
        _sync()
        ms = [evs[i].elapsed_time(evs[i + 1]) / per for i in range(nwin)]
        print(f"[series] {tag}: " + " ".join(f"{x:.3f}" for x in ms), file=sys.stderr, flush=True)

    step()
    _sync()
    run("after setup (~1 s idle)")
    run("right after the same load")
    for idle in (0.01, 0.05, 0.2, 1.0):
        time.sleep(idle)
        run(f"after {idle * 1e3:.0f} ms idle")
    run("right after the same load")


def attn_bytes(B, H, T, D, esize):
    """Algorithmic HBM bytes (read, write) per launch of each attention pass:
    every input read once, every output written once.  q/k/v/o/dO have
    `esize`-byte elements, lse/delta and the gradients are fp32."""
    t, r = B * H * T * D * esize, B * H * T * 4
    g = B * H * T * D * 4
    return {"fwd": (3 * t, t + r),                      # q, k, v -> o, lse
            "dq": (5 * t + r, g + r),                   # q, k, v, o, dO, lse -> dQ, delta
            "dkdv": (4 * t + 2 * r, 2 * g)}             # q, k, v, dO, lse, delta -> dK, dV


def short_t_report(name, B, H, T, D, r):
    """Per-pass time and algorithmic HBM rate of a short-T attention config."""
    out = {}
    for ph, (rd, wr) in attn_bytes(B, H, T, D, 4).items():
        ms = r[f"ms_{ph}"]
        out[ph] = {"us": round(ms * 1e3, 2), "bytes": rd + wr,
                   "GBps": round((rd + wr) / (ms * 1e-3) / 1e9, 1),
                   "frac_of_hbm": round((rd + wr) / (ms * 1e-3) / 1e9 / PEAK_HBM, 4)}
    print(f"[bench] {name} B={B} H={H} T={T} D={D} fp32: step {r['ms_step'] * 1e3:.2f} us; {out}",
          file=sys.stderr)


def cpu_baseline_attention(arrs, T, D, budget_s=15.0):
    """Time the NumPy restatement of the reference sub-graph (fwd + autograd
    bwd, transformer.py:36-44 with its float64 promotion) over successive
    (b,h) slices of the same inputs until `budget_s` seconds are spent."""
    from oracle.attention import reference_attention

    q, k, v, do = arrs
    B, H = q.shape[:2]
    slices = [(b, h) for b in range(B) for h in range(H)]
    done = 0
    t0 = time.perf_counter()
    for b, h in slices:
        sl = (slice(b, b + 1), slice(h, h + 1))
        reference_attention(q[sl], k[sl], v[sl], do[sl], 1.0 / math.sqrt(D), True)
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    f, bwd = attn_flops(1, done, T, D)
    return (f + bwd) / dt / 1e12, done, dt


C0_CFG = dict(vocab=65, block=32, n_embd=64, n_head=4, n_layer=2, B=16)
C2_CFG = dict(vocab=65, block=256, n_embd=384, n_head=6, n_layer=6, B=64)
# sequences per step of the C2 CPU baseline (a full B=64 step of the NumPy
# restatement took over 10 minutes on an 8-core host, too long for the default
# run; 8 sequences take about 18 s there)
C2_CPU_B = 8


def gpt_flops_per_step(c):
    """Model FLOPs of one training step: 6 * (matmul params) * tokens plus the
    causal attention products 3 * L * (2 * B * T^2 * C) (fwd 1x, bwd 2x of the
    causal-halved 4*B*T^2*C)."""
    C, V, L, B, T = c["n_embd"], c["vocab"], c["n_layer"], c["B"], c["block"]
    n_mm = L * (4 * C * C + 8 * C * C) + C * V
    return 6 * n_mm * B * T + 3 * L * (2 * B * T * T * C)


def bench_c4(n_new=224):
    """Config C4: greedy decoding with the C2 model (weights N(0, 0.02) from
    default_rng(2), biases 0, eval mode) of 64 prompts of 32 ids drawn from
    default_rng(4), + n_new tokens each: prefill, then one-token steps with the
    KV cache (GPT.generate_greedy: decode kernel, device-side pick, one step
    recorded as a HIP graph and replayed).  The timed region is the whole
    generate call, ids on the host at the end.  Also times the decode
    attention kernel alone at the longest step (L = 256, fp32 cache) with HIP
    events and reports its read bandwidth (K and V once)."""
    import minitorch_amd as mt

    c = C2_CFG
    model = mt.GPT(c["vocab"], c["block"], c["n_embd"], c["n_head"], c["n_layer"], dropout=0.0)
    model.init_weights(np.random.default_rng(2))
    model.eval()
    prompts = np.random.default_rng(4).integers(0, c["vocab"], (64, 32))
    import minitorch_amd.transformer as tr

    def timed():
        model.generate_greedy(prompts, 8)  # warm-up (library load, allocator)
        _sync()
        best, toks = None, None
        for _ in range(2):
            t0 = time.perf_counter()
            toks = model.generate_greedy(prompts, n_new)
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
        return best, toks

    def name(persistent):
        return ("persistent: the 223 token steps after the prefill's pick in one cooperative launch "
                "(mtx_decode_step_f32)" if persistent
                else "chain: 32 launches per token step, recorded once as a HIP graph and replayed")

    mode = tr._PERSISTENT_STEP
    best, toks = timed()
    assert toks.shape == (64, 32 + n_new)
    tr._PERSISTENT_STEP = not mode
    try:
        other, toks2 = timed()
    finally:
        tr._PERSISTENT_STEP = mode
    assert np.array_equal(toks, toks2), "the two decode-step structures disagree"
    dk = bench_decode_kernel(c)
    return {"tokens_per_s": round(64 * n_new / best, 1), "ms_total": round(best * 1e3, 2),
            "ms_per_token_step": round(best * 1e3 / n_new, 4),
            "decode_step": name(mode),
            "other_decode_step": {"structure": name(not mode), "ms_per_token_step": round(other * 1e3 / n_new, 4),
                                  "tokens_per_s": round(64 * n_new / other, 1), "same_tokens": True},
            "decode_kernel": dk,
            "config": "C2 model (6x384, 6 heads), 64 prompts x 32 ids, +224 greedy tokens, fp32, KV cache"}


def bench_decode_kernel(c, graph=True, sets=8):
    """The decode attention kernel alone at the longest C4 step (B = 64, the
    C2 model's heads, L = 256, fp32 cache): microseconds per launch from HIP
    events and the read bandwidth (K and V once), twice: on one cache (its
    50 MB stay in the 256 MB MALL between launches) and cycling over `sets`
    caches (8 x 50 MB: each launch reads a cache the previous 7 launches have
    pushed out, i.e. from HBM -- the situation of the decode step, whose 6
    layers hold 6 such caches).  graph=False launches it 25 times eagerly on
    one cache and times nothing (a short workload for counter passes)."""
    from minitorch_amd import device as Dv
    from minitorch_amd import kernels as K
    from minitorch_amd.graphs import Graph

    B, H, L, D = 64, c["n_head"], 256, c["n_embd"] // c["n_head"]
    g = np.random.default_rng(4)
    q = Dv.from_host(g.standard_normal((B, H, 1, D), dtype=np.float32)).t
    caches = []
    for _ in range(sets if graph else 1):
        caches.append((Dv.from_host(g.standard_normal((B, L, H * D), dtype=np.float32)).t,
                       Dv.from_host(g.standard_normal((B, L, H * D), dtype=np.float32)).t))
    heads = lambda t: t.view(B, L, H, D).transpose(1, 2)
    out = Dv.empty_buf(q.shape)

    def launch(i=0):
        kc, vc = caches[i]
        K.attn_decode(q, heads(kc), heads(vc), D ** -0.5, out=out)

    if not graph:
        for _ in range(25):
            launch()
        _sync()
        return None
    for i in range(sets):
        launch(i)
    _sync()
    nbytes = 2 * B * H * L * D * 4
    res = {"L": L, "bytes_per_launch": nbytes}
    # launches recorded in a HIP graph and replayed: launched one by one from
    # Python the loop is bound by the host's per-call path (~17 us), not by
    # the kernel
    for name, order in (("one_cache", [0] * 24), ("rotating", [i % sets for i in range(3 * sets)])):
        graph = Graph()
        with graph.capture():
            for i in order:
                launch(i)
        ms = time_loop(graph.replay, 20, 3) / len(order)
        res[name] = {"us_per_launch": round(ms * 1e3, 3), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "frac_of_hbm": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM, 4)}
    res["note"] = (f"one_cache: the same 50 MB K+V every launch (MALL-resident); rotating: {sets} caches "
                   f"({sets * nbytes / 1e6:.0f} MB) in turn, each read after the other {sets - 1} evicted it")
    return res


def bench_gpt(c, seed, steps, warmup, graph=False):
    """Training steps (forward, cross-entropy, zero_grad, backward, Adam
    lr 3e-4) on seeded synthetic token batches already resident on the GPU.
    With graph=True the step runs through minitorch_amd.CapturedStep (Adam in
    capturable mode): two eager calls, the third recorded as a HIP graph and
    replayed from then on (each call copies its batch into the recorded
    step's input buffers), so the host's per-kernel dispatch leaves the
    timed loop.  Returns ms per step and the losses of the timed steps."""
    import minitorch_amd as mt
    from minitorch_amd import device as D

    rng = np.random.default_rng(seed)
    model = mt.GPT(c["vocab"], c["block"], c["n_embd"], c["n_head"], c["n_layer"], dropout=0.0)
    model.init_weights(rng)
    opt = mt.Adam(model.parameters(), lr=3e-4)
    model.train()
    B, T, V = c["B"], c["block"], c["vocab"]
    if graph:
        warmup = max(warmup, 3)  # two eager calls, then the recorded one
    batches = []
    for _ in range(warmup + steps):
        ids = rng.integers(0, V, (B, T + 1))
        batches.append((D.index_array(ids[:, :-1]), D.index_array(ids[:, 1:].reshape(-1))))
    losses = []

    def train_step(x, y):
        logits = model(x)
        loss = mt.cross_entropy_loss(logits.reshape(B * T, V), mt.Tensor(y))
        opt.zero_grad()
        loss.backward()
        opt.step()
        return loss

    if graph:
        opt.capturable()
        captured = mt.CapturedStep(train_step, opt, warmup=2)

    def step(i):
        return captured(*batches[i]) if graph else train_step(*batches[i])

    for i in range(warmup):
        step(i)
    _sync()
    e0, e1 = _events()
    e0.record()
    last = []
    for i in range(warmup, warmup + steps):
        loss = step(i)
        # a replayed step overwrites the recorded loss buffer: keep a copy
        last.append(loss.data.t.clone() if graph else loss)
    e1.record()
    _sync()
    losses = [float(l_.numpy()) if isinstance(l_, D.DevBuf) else float(l_) for l_ in last]
    return e0.elapsed_time(e1) / steps, losses


def cpu_baseline_gpt(c, budget_s, B_sample):
    """The NumPy restatement of the reference training step (oracle/gpt.py:
    forward, cross-entropy, hand-derived backward with the reference's dtype
    flow, Adam) on a batch of B_sample sequences, repeated until budget_s."""
    from oracle.gpt import Adam, GPTConfig, draw_batch, gpt_loss_and_grads, init_params

    cfg = GPTConfig(c["vocab"], c["block"], c["n_embd"], c["n_head"], c["n_layer"])
    rng = np.random.default_rng(0)
    P = init_params(cfg, rng)
    opt = Adam(P, lr=3e-4)
    n = 0
    t0 = time.perf_counter()
    while True:
        x, y = draw_batch(rng, cfg.vocab, B_sample, cfg.block)
        _, _, G = gpt_loss_and_grads(P, x, y, cfg)
        opt.step(P, G)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return n * B_sample * cfg.block / dt, n, dt


def cpu_baseline_c4():
    """The reference's generation loop restated in NumPy (oracle/gpt.py
    greedy_generate: a full forward over the context per token, as
    transformer.py:93-104 does) for the C4 model and its 64 sequences: one
    step timed at the middle context of the run (143 ids; the 224 steps span
    32 .. 255).  A step's cost is linear in the context plus a small
    quadratic attention term, so this is the run's mean step time to about 1%.
    Returns (tokens/s, step s)."""
    from oracle.gpt import GPTConfig, greedy_generate, init_params

    c = C2_CFG
    cfg = GPTConfig(c["vocab"], c["block"], c["n_embd"], c["n_head"], c["n_layer"])
    P = init_params(cfg, np.random.default_rng(2))
    ctx = np.random.default_rng(4).integers(0, c["vocab"], (64, 143))
    t0 = time.perf_counter()
    greedy_generate(P, cfg, ctx, 1)
    dt = time.perf_counter() - t0
    return 64 / dt, dt


def pmc_traffic(kernel):
    """HBM bytes per launch of `kernel` at C3 from the committed rocprofv3 PMC
    summary (profiles/pmc_traffic.json), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)["bytes_per_launch"][kernel]
        return int(rec["read"] + rec["write"])
    except Exception:
        return None


def host_info():
    """CPU model, visible cores and NumPy's BLAS, for the CPU-baseline record."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas = None
    try:
        cfg = np.show_config(mode="dicts")
        b = cfg.get("Build Dependencies", {}).get("blas", {})
        blas = f"{b.get('name', '?')} {b.get('version', '')}".strip()
    except Exception:
        pass
    try:
        ncpu = len(os.sched_getaffinity(0))
    except Exception:
        ncpu = os.cpu_count()
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": ncpu,
            "numpy": np.__version__, "blas": blas, "blas_threads": blas_threads()}


def blas_threads():
    for var in ("OPENBLAS_NUM_THREADS", "OMP_NUM_THREADS", "MKL_NUM_THREADS"):
        if os.environ.get(var):
            return int(os.environ[var])
    try:
        return len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--gemm-mode", choices=("bf16x3", "fp32"), default="bf16x3",
                    help="--only gpt2/gpt0: the product kernel for shapes of >= 128 x 128")
    ap.add_argument("--attn-mode", choices=("bf16x3", "fp32"), default="bf16x3",
                    help="--only c1/gpt2/gpt0: the product kernel of fp32 attention (64-wide heads)")
    ap.add_argument("--decode", choices=("default", "persistent", "chain"), default="default",
                    help="the greedy decode step of the C4 leg: one persistent launch or the chain of launches")
    ap.add_argument("--bwd-mode", choices=("default", "onepass", "twopass"), default="default",
                    help="the attention backward structure for the C3/C1 legs (mtx_attn_set_bwd_mode)")
    ap.add_argument("--only", choices=("all", "c3", "c3series", "c1", "c0attn", "c4", "c4eager", "c4step", "c4kernel",
                                       "gpt2", "gpt0"),
                    default="all",
                    help="profiling aid: run only one attention config and print no JSON line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="profiling aid: run 5 device copies of MIB MiB (a kernel of known HBM "
                         "traffic, for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(attention shards by (b,h) with no exchange). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    from minitorch_amd import device as Dv

    try:
        Dv.device()
    except RuntimeError as e:
        print(f"no GPU visible: {e}", file=sys.stderr)
        sys.exit(1)

    if args.decode != "default":
        import minitorch_amd.transformer as _tr

        _tr._PERSISTENT_STEP = args.decode == "persistent"
    if args.bwd_mode != "default":
        from minitorch_amd import kernels as _K

        _K.set_attn_bwd_mode(_K.ATTN_BWD_ONEPASS if args.bwd_mode == "onepass" else _K.ATTN_BWD_TWOPASS)
    if args.calibrate_copy:
        from minitorch_amd import kernels as K

        n = args.calibrate_copy * (1 << 20) // 4
        src = Dv.full((n,), 1.0).t
        dst = Dv.empty_buf((n,))
        for _ in range(5):
            K.ewise("COPY", dst, src)
        _sync()
        print(f"[bench] copied {args.calibrate_copy} MiB x5", file=sys.stderr)
        return
    if args.only in ("gpt2", "gpt0"):
        from minitorch_amd import kernels as _K

        c = C2_CFG if args.only == "gpt2" else C0_CFG
        if args.gemm_mode == "fp32":
            _K.set_gemm_mode(_K.GEMM_FP32)
        if args.attn_mode == "fp32":
            _K.set_attn_mode(_K.GEMM_FP32)
        # the modes as the library reports them, not as requested
        gm = "bf16x3" if _K.get_gemm_mode() == _K.GEMM_BF16X3 else "fp32"
        am = "bf16x3" if _K.get_attn_mode() == _K.GEMM_BF16X3 else "fp32"
        for graph in (True, False):
            ms, losses = bench_gpt(c, 2, args.steps, args.warmup, graph=graph)
            print(f"[bench] {args.only} ({'graph' if graph else 'eager'}, gemm {gm}, "
                  f"attention {am}): {ms:.3f} ms/step, "
                  f"{c['B'] * c['block'] / (ms * 1e-3):.0f} tokens/s, losses {losses}", file=sys.stderr)
        return
    if args.only == "c3series":
        c3_series()
        return
    if args.only == "c4eager":
        # the C4 run with the chain of launches, every decode step launched
        # eagerly (no HIP graph): the same kernels, for a kernel-by-kernel trace
        import minitorch_amd as mt
        import minitorch_amd.transformer as _tr

        _tr._PERSISTENT_STEP = False

        c = C2_CFG
        model = mt.GPT(c["vocab"], c["block"], c["n_embd"], c["n_head"], c["n_layer"], dropout=0.0)
        model.init_weights(np.random.default_rng(2))
        model.eval()
        prompts = np.random.default_rng(4).integers(0, c["vocab"], (64, 32))
        model.generate_greedy(prompts, 8, graph=False)
        _sync()
        t0 = time.perf_counter()
        model.generate_greedy(prompts, 224, graph=False)
        dt = time.perf_counter() - t0
        print(f"[bench] C4 eager steps: {dt * 1e3 / 224:.3f} ms per token step", file=sys.stderr)
        return
    if args.only == "c4step":
        # the C4 run with the persistent decode step only (one launch per
        # token step, no graph): a short workload for kernel traces
        import minitorch_amd as mt
        import minitorch_amd.transformer as _tr

        _tr._PERSISTENT_STEP = True
        c = C2_CFG
        model = mt.GPT(c["vocab"], c["block"], c["n_embd"], c["n_head"], c["n_layer"], dropout=0.0)
        model.init_weights(np.random.default_rng(2))
        model.eval()
        prompts = np.random.default_rng(4).integers(0, c["vocab"], (64, 32))
        model.generate_greedy(prompts, 8)
        _sync()
        t0 = time.perf_counter()
        model.generate_greedy(prompts, 224)
        dt = time.perf_counter() - t0
        print(f"[bench] C4 persistent steps: {dt * 1e3 / 224:.4f} ms per token step", file=sys.stderr)
        return
    if args.only == "c4kernel":
        bench_decode_kernel(C2_CFG, graph=False)
        print("[bench] decode kernel x25 (B=64, H=6, L=256, D=64, fp32)", file=sys.stderr)
        return
    if args.only == "c4":
        print(f"[bench] C4 {bench_c4()}", file=sys.stderr)
        return
    if args.attn_mode == "fp32":
        from minitorch_amd import kernels as _K

        _K.set_attn_mode(_K.GEMM_FP32)
    if args.only == "c1":
        r1, _ = bench_attention(32, 8, 256, 64, "float32", 1, 1.0, args.steps, args.warmup)
        print(f"[bench] C1 {r1}", file=sys.stderr)
        short_t_report("C1", 32, 8, 256, 64, r1)
        return
    if args.only == "c0attn":
        # the attention of the C0 model (4 heads of 16, T = 32, batch 16)
        r0, _ = bench_attention(16, 4, 32, 16, "float32", 1, 1.0, args.steps, args.warmup)
        short_t_report("C0 attention", 16, 4, 32, 16, r0)
        return

    # ---- C3: headline ----
    B, H, T, D = 8, 16, 2048, 64
    print(f"[bench] C3 bf16 B={B} H={H} T={T} D={D}: {args.warmup} warmup + {args.steps} steps",
          file=sys.stderr, flush=True)
    r3, arrs3 = bench_attention(B, H, T, D, "bfloat16", 3, 0.5, args.steps, args.warmup, cold=True)
    ms_cold = r3.pop("ms_step_cold")
    f3, b3 = attn_flops(B, H, T, D)
    tflops = (f3 + b3) / (r3["ms_step"] * 1e-3) / 1e12
    # dominant kernel and its algorithmic FLOPs: fwd kernel = 2u; one-pass
    # key-outer kernel = S, dP, dV, dK, dQ = 5u (its prep kernel is HBM-bound
    # O(T*D) work); two-pass: dK/dV pass = S, dP, dV, dK = 4u, dQ pass = the
    # dQ product only (its S/dP recompute is already counted in the dK/dV
    # pass, and its delta rowsum is O(T*D)) = 1u.
    u = B * H * T * T * D
    kern = {"attn_fwd": (r3["ms_fwd"], 2 * u)}
    if "ms_dkdvq" in r3:
        kern.update({"attn_dkdvq": (r3["ms_dkdvq"], 5 * u), "attn_prep": (r3["ms_prep"], 0)})
    else:
        kern.update({"attn_dkdv": (r3["ms_dkdv"], 4 * u), "attn_dq": (r3["ms_dq"], 1 * u)})
    dom = max(kern, key=lambda k_: kern[k_][0])
    ms_dom, fl_dom = kern[dom]
    achieved = fl_dom / (ms_dom * 1e-3) / 1e12
    print(f"[bench] C3 step {r3['ms_step']:.3f} ms = {tflops:.1f} TFLOP/s (cold start {ms_cold:.3f} ms = "
          f"{(f3 + b3) / (ms_cold * 1e-3) / 1e12:.1f}); phases {r3}", file=sys.stderr, flush=True)
    # the same step with the other backward structure, for comparison
    from minitorch_amd import kernels as _K

    cur_bwd = _K.get_attn_bwd_mode()
    other_bwd = _K.ATTN_BWD_TWOPASS if cur_bwd == _K.ATTN_BWD_ONEPASS else _K.ATTN_BWD_ONEPASS
    other_name = "two-pass" if other_bwd == _K.ATTN_BWD_TWOPASS else "one-pass"
    _K.set_attn_bwd_mode(other_bwd)
    try:
        r3b, _ = bench_attention(B, H, T, D, "bfloat16", 3, 0.5, args.steps, args.warmup)
    finally:
        _K.set_attn_bwd_mode(cur_bwd)
    print(f"[bench] C3 {other_name} step {r3b['ms_step']:.3f} ms = "
          f"{(f3 + b3) / (r3b['ms_step'] * 1e-3) / 1e12:.1f} TFLOP/s; phases {r3b}", file=sys.stderr, flush=True)
    if args.only == "c3":
        return

    # ---- C1: fp32 ----
    print("[bench] C1 fp32 B=32 H=8 T=256 D=64", file=sys.stderr, flush=True)
    r1, _ = bench_attention(32, 8, 256, 64, "float32", 1, 1.0, args.steps, args.warmup)
    f1, b1 = attn_flops(32, 8, 256, 64)
    tflops1 = (f1 + b1) / (r1["ms_step"] * 1e-3) / 1e12

    # ---- GPT training: C2 (GPT-small char model) and C0 (tiny) ----
    print("[bench] GPT C2 training (B=64, T=256, 6x384)", file=sys.stderr, flush=True)
    # the mean over 20 steps, the length of the compared loss curve
    ms_c2, losses_c2 = bench_gpt(C2_CFG, 2, 20, 3, graph=True)
    ms_c2_eager, _ = bench_gpt(C2_CFG, 2, 5, 2)
    # the same replayed step with the products of >= 128 x 128 on the fp32
    # MFMA kernel instead of the default three-piece bf16 split
    from minitorch_amd import kernels as _K

    prev_mode = _K.set_gemm_mode(_K.GEMM_FP32)
    try:
        ms_c2_f32, losses_c2_f32 = bench_gpt(C2_CFG, 2, 20, 3, graph=True)
    finally:
        _K.set_gemm_mode(prev_mode)
    tok_c2 = C2_CFG["B"] * C2_CFG["block"] / (ms_c2 * 1e-3)
    fl_c2 = gpt_flops_per_step(C2_CFG)
    print(f"[bench] C2 {ms_c2:.2f} ms/step = {tok_c2:.0f} tokens/s, losses {losses_c2}", file=sys.stderr,
          flush=True)
    print("[bench] GPT C0 training (B=16, T=32, 2x64)", file=sys.stderr, flush=True)
    ms_c0, _ = bench_gpt(C0_CFG, 0, args.steps, 3, graph=True)
    ms_c0_eager, _ = bench_gpt(C0_CFG, 0, args.steps, 3)
    tok_c0 = C0_CFG["B"] * C0_CFG["block"] / (ms_c0 * 1e-3)

    print("[bench] C4 greedy decoding (64 x (32 + 224) tokens)", file=sys.stderr, flush=True)
    c4 = bench_c4()
    print(f"[bench] C4 {c4['tokens_per_s']:.0f} tokens/s", file=sys.stderr, flush=True)

    cpu = None
    cpu_gpt = None
    if not args.no_cpu:
        print(f"[bench] CPU baseline (NumPy restatement, ~{args.cpu_budget:.0f}s)", file=sys.stderr, flush=True)
        cv, nsl, dt = cpu_baseline_attention(arrs3, T, D, args.cpu_budget)
        cpu = {"value": round(cv, 6), "unit": "TFLOP/s", "cores": blas_threads(), "kind": "port",
               "sample": f"{nsl} of {B * H} (b,h) slices of C3 (T=2048, D=64), fwd+bwd through the "
                         f"NumPy restatement of the reference sub-graph (fp32 q@k^T, fp64 from the "
                         f"scale on), {dt:.1f}s; TFLOP/s on the algorithmic causal count",
               "host": host_info()}
        print("[bench] CPU baseline, GPT C2 step on 8 sequences (NumPy restatement)", file=sys.stderr, flush=True)
        tps2, n2, dt2 = cpu_baseline_gpt(C2_CFG, args.cpu_budget / 2, C2_CPU_B)
        tps0, n0, dt0 = cpu_baseline_gpt(C0_CFG, 3.0, C0_CFG["B"])
        tps4, dt4 = cpu_baseline_c4()
        c4["cpu_baseline"] = {"value": round(tps4, 2), "unit": "tokens/s", "cores": blas_threads(), "kind": "port",
                              "sample": f"one greedy step for all 64 sequences at the run's middle context "
                                        f"(143 ids of 32..255; {dt4:.1f}s), the mean step of the 224 to about 1%; "
                                        f"full-recompute NumPy restatement of GPT.generate (oracle/gpt.py)"}
        cpu_gpt = {"C2_tokens_per_s": round(tps2, 2), "C0_tokens_per_s": round(tps0, 1),
                   "cores": blas_threads(), "kind": "port",
                   "sample": f"C2 model, {n2} training steps on {C2_CPU_B} sequences of 256 tokens ({dt2:.1f}s; "
                             f"a B=64 step of the restatement took over 10 minutes on an 8-core host); "
                             f"C0, {n0} full B=16 steps ({dt0:.1f}s); NumPy restatement of the "
                             f"reference step (oracle/gpt.py)"}

    line = {
        "metric": "causal-MHA fwd+bwd TFLOP/s (C3: B=8,H=16,T=2048,D=64 bf16)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r3["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 q/k/v, N(0,1) dO, rounded to bf16)",
        "config": {"workload": "C3 causal MHA fwd+bwd", "B": B, "H": H, "T": T, "D": D,
                   "causal": True, "parallelism": "none (1 GPU)"},
        "pct_of_peak": round(100 * tflops / PEAK_BF16, 2),
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_BF16, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16, 4),
                     "traffic": pmc_traffic(dom), "ms_per_launch": round(ms_dom, 4),
                     "flops_per_launch": fl_dom},
        "cpu_baseline": cpu,
        "settle_ms": SETTLE_MS,
        "also": {
            "C3_phase_ms": {k_: round(v_, 4) for k_, v_ in r3.items()},
            "C3_backward": ("one-pass (mtx_attn_set_bwd_mode MTX_ATTN_BWD_ONEPASS): a delta kernel "
                            "that zeroes dq, then one key-outer kernel writing dK/dV and adding dQ with "
                            "fp32 atomics" if "ms_dkdvq" in r3 else
                            "two passes (the default, MTX_ATTN_BWD_TWOPASS: dQ query-outer with delta, "
                            "then dK/dV key-outer; deterministic)"),
            "C3_other_backward": {
                "mode": other_name,
                "ms_per_step": round(r3b["ms_step"], 4),
                "tflops": round((f3 + b3) / (r3b["ms_step"] * 1e-3) / 1e12, 2),
                "phase_ms": {k_: round(v_, 4) for k_, v_ in r3b.items()},
                "note": "the same step with the other backward structure (mtx_attn_set_bwd_mode); "
                        "one-pass phases: prep = delta + dq zeroed, dkdvq = key-outer kernel with "
                        "dQ atomics"},
            "C3_cold_start": {"ms_per_step": round(ms_cold, 4),
                              "tflops": round((f3 + b3) / (ms_cold * 1e-3) / 1e12, 2),
                              "note": f"{args.warmup} warm-up + {args.steps} timed steps right after the "
                                      "inputs are uploaded (about 1 s of GPU idle), without the settling "
                                      "period: the GPU's clock transient after idle"},
            "C1_fp32": {"tflops": round(tflops1, 3), "pct_of_fp32_peak": round(100 * tflops1 / PEAK_FP32, 2),
                        "ms_per_step": round(r1["ms_step"], 4),
                        "phase_ms": {k_: round(v_, 4) for k_, v_ in r1.items()}},
            "gpt_train": {
                "C2": {"tokens_per_s": round(tok_c2, 1), "ms_per_step": round(ms_c2, 3),
                       "model_tflops": round(fl_c2 / (ms_c2 * 1e-3) / 1e12, 2),
                       "pct_of_fp32_peak": round(100 * fl_c2 / (ms_c2 * 1e-3) / 1e12 / PEAK_FP32, 2),
                       "config": "vocab 65, n_embd 384, 6 heads, 6 layers, T=256, B=64, fp32, Adam 3e-4",
                       "losses": [round(x, 5) for x in losses_c2],
                       "mode": "step replayed from a HIP graph (CapturedStep)",
                       "gemm": "fp32 products of >= 128 x 128 as three-piece bf16 splits on the bf16 "
                               "matrix cores (fp32-accurate; mtx_gemm_set_mode MTX_GEMM_BF16X3, the default)",
                       "ms_per_step_eager": round(ms_c2_eager, 3),
                       "fp32_mfma_gemm": {"ms_per_step": round(ms_c2_f32, 3),
                                          "tokens_per_s": round(C2_CFG["B"] * C2_CFG["block"] / (ms_c2_f32 * 1e-3), 1),
                                          "losses": [round(x, 5) for x in losses_c2_f32],
                                          "note": "the same replayed step with every product on the fp32 "
                                                  "MFMA kernel (MTX_GEMM_FP32)"}},
                "C0": {"tokens_per_s": round(tok_c0, 1), "ms_per_step": round(ms_c0, 3),
                       "config": "vocab 65, n_embd 64, 4 heads, 2 layers, T=32, B=16, fp32",
                       "mode": "step replayed from a HIP graph (CapturedStep)",
                       "ms_per_step_eager": round(ms_c0_eager, 3)},
                "cpu_baseline": cpu_gpt,
            },
            "C4_greedy_decode": c4,
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
