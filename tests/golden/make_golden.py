#!/usr/bin/env python3
"""Write the golden fixtures in tests/golden/ by running the REFERENCE itself.

Run in the build container only (the reference is mounted at
/root/reference; it never travels to the GPU box and nothing else imports it):

    python tests/golden/make_golden.py            # attention, MHA, C0 train (+ dropout), greedy
    python tests/golden/make_golden.py --c2       # also the C2 20-step loss curve (slow)
    python tests/golden/make_golden.py --only-c4  # the C4 greedy tokens (slow, ~30 min)

These are the functions no closed form, finite difference or library
cross-check pins (the composed training step as the reference executes it,
with NumPy 2's float64 promotion and float32 gradient holders; the greedy
sequence its forward produces).  Each fixture stores its inputs' seeds and the
reference's outputs.  Inputs are generated with the same helpers the oracle
uses (oracle.gpt.init_params / draw_batch), and the reference model's
state_dict keys are checked against oracle.gpt.param_spec first.
"""
from __future__ import annotations

import argparse
import gc
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
REFERENCE = Path("/root/reference")
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(REFERENCE))

import minitorch as mt  # noqa: E402  (the reference)
from minitorch import functional as RF  # noqa: E402

from oracle.gpt import C0, C2, GPTConfig, draw_batch, init_params, param_spec  # noqa: E402


def ref_model(cfg: GPTConfig, rng):
    model = mt.GPT(cfg.vocab, cfg.block, cfg.n_embd, cfg.n_head, cfg.n_layer, dropout=0.0)
    names = [n for n, _, _ in param_spec(cfg)]
    sd = model.state_dict()
    assert list(sd.keys()) == names, "state_dict key order differs from oracle.gpt.param_spec"
    for n, shp, _ in param_spec(cfg):
        assert sd[n].shape == shp, (n, sd[n].shape, shp)
    model.load_state_dict(init_params(cfg, rng))
    return model


def attention_subgraph(path):
    """transformer.py:36-44 through the reference's Tensor ops, B=2,H=3,T=17,D=16."""
    rng = np.random.default_rng(200)
    B, H, T, D = 2, 3, 17, 16
    q, k, v, do = (rng.standard_normal((B, H, T, D), dtype=np.float32) for _ in range(4))
    tq, tk, tv = (mt.Tensor(a.copy(), requires_grad=True) for a in (q, k, v))
    scores = (tq @ tk.transpose(-2, -1)) * (1.0 / np.sqrt(D))
    mask = np.triu(np.ones((T, T), dtype=np.float32), k=1) * -1e9
    scores = scores + mt.Tensor(mask)
    attn = RF.softmax(scores, axis=-1)
    out = attn @ tv
    (out * mt.Tensor(do)).sum().backward()
    np.savez(path, q=q, k=k, v=v, do=do, out=out.data, dq=tq.grad, dk=tk.grad, dv=tv.grad,
             out_dtype=str(out.data.dtype), dq_dtype=str(tq.grad.dtype))
    print(f"wrote {path.name}: out {out.data.dtype}, dq {tq.grad.dtype}")


def mha_module(path):
    """A whole MultiHeadAttention (transformer.py:14-46), n_embd=48, 3 heads,
    x (2,17,48); loss = sum(y * dy)."""
    rng = np.random.default_rng(201)
    C, H, B, T = 48, 3, 2, 17
    mha = mt.MultiHeadAttention(C, H, dropout=0.0)
    w = {}
    for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
        w[name + ".weight"] = (rng.standard_normal((C, C)) * 0.1).astype(np.float32)
        w[name + ".bias"] = (rng.standard_normal(C) * 0.1).astype(np.float32)
    mha.load_state_dict(w)
    x = rng.standard_normal((B, T, C), dtype=np.float32)
    dy = rng.standard_normal((B, T, C), dtype=np.float32)
    tx = mt.Tensor(x.copy(), requires_grad=True)
    y = mha(tx)
    (y * mt.Tensor(dy)).sum().backward()
    grads = {f"grad.{n}": getattr(getattr(mha, n.split(".")[0]), n.split(".")[1]).grad for n in w}
    np.savez(path, x=x, dy=dy, y=y.data, dx=tx.grad, **{f"param.{k}": v for k, v in w.items()}, **grads)
    print(f"wrote {path.name}: y {y.data.dtype}, dx {tx.grad.dtype}")


def sample_index(shape, n, seed):
    r = np.random.default_rng(seed)
    return np.stack([r.integers(0, s, n) for s in shape], axis=1)


def train_curve(cfg: GPTConfig, seed: int, B: int, steps: int, path, full_grads_max=4096):
    """The harness loop (char_transformer.py:70-77) on the reference: loss per
    step; at step 0 the logits of batch row 0, every parameter's gradient L2
    norm, full gradients of small parameters and 64 sampled entries of each
    large one."""
    rng = np.random.default_rng(seed)
    model = ref_model(cfg, rng)
    opt = mt.Adam(model.parameters(), lr=3e-4)
    model.train()
    names = [n for n, _, _ in param_spec(cfg)]
    losses, extra = [], {}
    t0 = time.time()
    for it in range(steps):
        x, y = draw_batch(rng, cfg.vocab, B, cfg.block)
        logits = model(x)
        Bb, T, V = logits.shape
        loss = mt.cross_entropy_loss(logits.reshape(Bb * T, V), mt.Tensor(y.reshape(-1)))
        opt.zero_grad()
        loss.backward()
        if it == 0:
            extra["logits0_row0"] = logits.data[0]
            extra["logits_dtype"] = str(logits.data.dtype)
            norms = []
            for n, p in zip(names, model.parameters()):
                g = p.grad.astype(np.float64)
                norms.append(np.sqrt((g * g).sum()))
                if p.grad.size <= full_grads_max:
                    extra[f"grad.{n}"] = p.grad.copy()
                else:
                    ix = sample_index(p.grad.shape, 64, 7)
                    extra[f"gidx.{n}"] = ix
                    extra[f"gval.{n}"] = p.grad[tuple(ix.T)]
            extra["grad_norms"] = np.array(norms)
        opt.step()
        losses.append(float(loss.data))
        # drop this step's graph before the next forward builds one (at C2 the
        # reference's float64 graph is ~30 GB)
        del logits, loss
        for p in model.parameters():
            p.grad = None
        gc.collect()
        print(f"  step {it:2d} loss {losses[-1]:.10f}  ({time.time() - t0:.1f}s)", flush=True)
        # saved after every step (write + rename) so a long run leaves a usable prefix
        tmp = path.with_name(path.stem + ".part.npz")
        np.savez(tmp, losses=np.array(losses), seed=seed, B=B, steps=len(losses), names=np.array(names),
                 **extra)
        tmp.replace(path)
    print(f"wrote {path.name}")


def train_curve_dropout(cfg: GPTConfig, seed: int, B: int, steps: int, p: float, dseed: int, path):
    """The harness loop with dropout p in every Dropout of the model (the
    embedding dropout, each block's attn_drop and MLP dropout, transformer.py:
    75-76, 24, 60), the reference's demo setting (char_transformer.py:62).
    Masks come from NumPy's global RNG seeded with np.random.seed(dseed) after
    the model is built, in the reference's draw order.  Loss per step."""
    rng = np.random.default_rng(seed)
    model = mt.GPT(cfg.vocab, cfg.block, cfg.n_embd, cfg.n_head, cfg.n_layer, dropout=p)
    model.load_state_dict(init_params(cfg, rng))
    opt = mt.Adam(model.parameters(), lr=3e-4)
    model.train()
    np.random.seed(dseed)
    losses = []
    for it in range(steps):
        x, y = draw_batch(rng, cfg.vocab, B, cfg.block)
        logits = model(x)
        Bb, T, V = logits.shape
        loss = mt.cross_entropy_loss(logits.reshape(Bb * T, V), mt.Tensor(y.reshape(-1)))
        opt.zero_grad()
        loss.backward()
        opt.step()
        losses.append(float(loss.data))
        print(f"  step {it:2d} loss {losses[-1]:.10f}", flush=True)
    np.savez(path, losses=np.array(losses), seed=seed, B=B, steps=steps, p=p, dseed=dseed)
    print(f"wrote {path.name}")


def greedy(path, seed=100, B=4, T0=8, n_new=24):
    """Greedy decoding harness over the reference forward: argmax of
    model(idx[:, -block:]).data[:, -1, :] (transformer.py:97-98), eval mode,
    no_grad; C0-size model."""
    rng = np.random.default_rng(seed)
    model = ref_model(C0, rng)
    model.eval()
    prompts = rng.integers(0, C0.vocab, (B, T0))
    idx = prompts.copy()
    margins = []
    with mt.no_grad():
        for _ in range(n_new):
            logits = model(idx[:, -C0.block:]).data[:, -1, :]
            nxt = np.argmax(logits, axis=-1)
            top2 = np.sort(logits, axis=-1)[:, -2:]
            margins.append(top2[:, 1] - top2[:, 0])
            idx = np.concatenate([idx, nxt[:, None]], axis=1)
    np.savez(path, prompts=prompts, tokens=idx, margins=np.stack(margins, 1), seed=seed)
    print(f"wrote {path.name}: min top-2 margin {np.min(margins):.3e}")


def greedy_c4(path, n_new=224):
    """Config C4 through the reference's own forward: the C2 model (weights
    from init_params(C2, default_rng(2))), eval mode, no_grad, prompts
    default_rng(4).integers(0, 65, (64, 32)), 224 greedy steps, each the
    argmax of model(idx[:, -block:]).data[:, -1, :] (transformer.py:93-98,
    full recompute as the reference generates).  Written after every step
    (write + rename), so a long run leaves a usable prefix; `steps` says how
    many tokens each row holds beyond the prompt.  A run resumes from such a
    prefix (each step depends only on the ids so far)."""
    model = ref_model(C2, np.random.default_rng(2))
    model.eval()
    prompts = np.random.default_rng(4).integers(0, C2.vocab, (64, 32))
    idx = prompts.copy()
    margins = []
    start = 0
    if path.exists():
        z = np.load(path, allow_pickle=False)
        assert np.array_equal(z["prompts"], prompts), "saved prefix is for other prompts"
        start = int(z["steps"])
        idx = z["tokens"].copy()
        margins = list(z["margins"].T)
        print(f"  resuming after {start} steps", flush=True)
    t0 = time.time()
    with mt.no_grad():
        for it in range(start, n_new):
            logits = model(idx[:, -C2.block:]).data[:, -1, :]
            nxt = np.argmax(logits, axis=-1)
            top2 = np.sort(logits, axis=-1)[:, -2:]
            margins.append(top2[:, 1] - top2[:, 0])
            idx = np.concatenate([idx, nxt[:, None]], axis=1)
            # the step's graph holds reference cycles (node <-> closure): free
            # it now, or ~0.5 GB per step accumulates until the cyclic collector runs
            del logits
            gc.collect()
            tmp = path.with_name(path.stem + ".part.npz")
            np.savez_compressed(tmp, prompts=prompts, tokens=idx, margins=np.stack(margins, 1),
                                steps=it + 1)
            tmp.replace(path)
            print(f"  C4 step {it:3d}  ({time.time() - t0:.1f}s)", flush=True)
    print(f"wrote {path.name}: min top-2 margin {np.min(margins):.3e}")


def sampling(path, seed=300, B=4, T0=8, temperature=0.8):
    """The reference's sampling GPT.generate (transformer.py:93-104) on a
    C0-size model, NumPy's global RNG seeded with np.random.seed: 16 new
    tokens (the context stays within block_size = 32) and, from the same
    state, 40 more from a fresh prompt (the context outgrows block_size, so
    the reference crops it)."""
    rng = np.random.default_rng(seed)
    model = ref_model(C0, rng)
    model.eval()
    prompts = rng.integers(0, C0.vocab, (B, T0))
    np.random.seed(seed)
    with mt.no_grad():
        short = model.generate(prompts, 16, temperature=temperature)
        long = model.generate(prompts[:, :4], 40, temperature=temperature)
    np.savez(path, prompts=prompts, short=short, long=long, seed=seed, temperature=temperature)
    print(f"wrote {path.name}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--c2", action="store_true", help="also run the C2 20-step curve (slow)")
    ap.add_argument("--only-c2", action="store_true")
    ap.add_argument("--only-sampling", action="store_true")
    ap.add_argument("--only-dropout", action="store_true")
    ap.add_argument("--only-c4", action="store_true",
                    help="only the C4 greedy run through the reference forward (slow)")
    ap.add_argument("--c2-out", default=str(HERE / "c2_train.npz"),
                    help="where the C2 curve goes (a long run can write beside the committed fixture)")
    args = ap.parse_args()
    if args.only_sampling:
        sampling(HERE / "sampling_c0.npz")
        return
    if args.only_dropout:
        train_curve_dropout(C0, 0, 16, 10, 0.1, 1234, HERE / "c0_train_dropout.npz")
        return
    if args.only_c4:
        greedy_c4(HERE / "c4_greedy_ref.npz")
        return
    if not args.only_c2:
        attention_subgraph(HERE / "attn_subgraph.npz")
        mha_module(HERE / "mha_module.npz")
        print("C0 training, 20 steps")
        train_curve(C0, 0, 16, 20, HERE / "c0_train.npz")
        greedy(HERE / "greedy_c0.npz")
        sampling(HERE / "sampling_c0.npz")
        train_curve_dropout(C0, 0, 16, 10, 0.1, 1234, HERE / "c0_train_dropout.npz")
    if args.c2 or args.only_c2:
        print("C2 training, 20 steps")
        train_curve(C2, 2, 64, 20, Path(args.c2_out))


if __name__ == "__main__":
    main()
