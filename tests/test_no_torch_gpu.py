"""The product path without PyTorch: a fresh Python process that never
imports torch runs (1) the integration guide's NumPy-only ctypes snippet
(the code block marked "numpy-only attention round trip"), verbatim, checked against the oracle at the fp32 bar; (2) C0 training
through minitorch_amd (eager, then a HIP-graph-captured step) against the
reference's own loss curve; (3) greedy decoding (KV cache, replayed decode
step) against the reference's tokens; (4) __graft_entry__.smoke().  The
process asserts at the end that 'torch' is not in sys.modules."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parents[1]

SCRIPT = r'''
import sys, re
from pathlib import Path
import numpy as np
ROOT = Path(sys.argv[1]); sys.path.insert(0, str(ROOT)); sys.path.insert(0, str(ROOT / "tests"))

# (1) the integration guide's snippet, exactly as written there
text = (ROOT / "INTEGRATION.md").read_text()
snippet = re.search(r"```python\n(# numpy-only attention round trip\n.*?)```", text, re.S).group(1)
ns = {}
cwd = Path.cwd()
import os; os.chdir(ROOT)
exec(compile(snippet, "INTEGRATION.md", "exec"), ns)
os.chdir(cwd)
from oracle.attention import reference_attention
ref = reference_attention(ns["q"], ns["k"], ns["v"], ns["dout"], ns["scale"], True)
for name, got, r in zip(("out", "dq", "dk", "dv"), (ns["out"], ns["dq"], ns["dk"], ns["dv"]), ref):
    err = np.abs(got - r)
    assert np.all(err <= 1e-5 + 1e-4 * np.abs(r)), (name, float(err.max()))
print("snippet ok", flush=True)

# (2) C0 training, eager and captured, against the reference's loss curve
import minitorch_amd as mt
from minitorch_amd import device as D
from oracle.gpt import C0, draw_batch, init_params
g = np.load(ROOT / "tests" / "golden" / "c0_train.npz", allow_pickle=False)
for captured in (False, True):
    rng = np.random.default_rng(int(g["seed"]))
    model = mt.GPT(C0.vocab, C0.block, C0.n_embd, C0.n_head, C0.n_layer, dropout=0.0)
    model.load_state_dict(init_params(C0, rng))
    opt = mt.Adam(model.parameters(), lr=3e-4)
    model.train()
    B, T, V = int(g["B"]), C0.block, C0.vocab

    def step(x, y):
        logits = model(x)
        loss = mt.cross_entropy_loss(logits.reshape(B * T, V), mt.Tensor(y))
        opt.zero_grad()
        loss.backward()
        opt.step()
        return loss

    if captured:
        opt.capturable()
        step = mt.CapturedStep(step, opt, warmup=2)
    losses = []
    for _ in range(8):
        x, y = draw_batch(rng, V, B, T)
        losses.append(float(step(D.index_array(x), D.index_array(y.reshape(-1)))))
    ref_l = g["losses"][:8]
    assert np.all(np.abs(np.array(losses) - ref_l) <= 1e-4 * ref_l), (captured, losses, ref_l)
    print("c0 ok", captured, losses[-1], flush=True)

# (3) greedy decoding with the KV cache and the replayed step
gg = np.load(ROOT / "tests" / "golden" / "greedy_c0.npz", allow_pickle=False)
rng = np.random.default_rng(int(gg["seed"]))
model = mt.GPT(C0.vocab, C0.block, C0.n_embd, C0.n_head, C0.n_layer, dropout=0.0)
model.load_state_dict(init_params(C0, rng))
model.eval()
toks = model.generate_greedy(gg["prompts"], gg["tokens"].shape[1] - gg["prompts"].shape[1])
assert np.array_equal(toks, gg["tokens"]), "greedy tokens differ"
print("greedy ok", flush=True)

# (4) the driver's smoke
import __graft_entry__
__graft_entry__.smoke()
assert "torch" not in sys.modules, "torch was imported"
print("NO_TORCH_OK", flush=True)
'''


def test_product_path_runs_without_torch(dev, tmp_path):
    env = dict(os.environ)
    proc = subprocess.run([sys.executable, "-u", "-c", SCRIPT, str(ROOT)], capture_output=True, text=True,
                          timeout=600, env=env, cwd=str(tmp_path))
    print(proc.stdout[-3000:], proc.stderr[-3000:])
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "NO_TORCH_OK" in proc.stdout
