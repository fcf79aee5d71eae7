#!/usr/bin/env python3
"""Write tests/golden/c4_greedy.npz: the oracle's greedy tokens for config C4.

C4: the C2 model (vocab 65, n_embd 384, 6 heads,
6 layers, block 256), weights from oracle.gpt.init_params(C2,
default_rng(2)), eval mode; prompts = default_rng(4).integers(0, 65, (64, 32));
224 greedy steps.  Computed by oracle.gpt.greedy_generate_cached, which is
pinned to the reference's own greedy tokens by tests/test_oracle.py (the full
oracle run takes minutes, too long for a test, hence a fixture).

    python tests/golden/make_c4_fixture.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.gpt import C2, greedy_generate_cached, init_params  # noqa: E402


def main():
    P = init_params(C2, np.random.default_rng(2))
    prompts = np.random.default_rng(4).integers(0, C2.vocab, (64, 32))
    toks, margins = greedy_generate_cached(P, C2, prompts, 224)
    np.savez_compressed(HERE / "c4_greedy.npz", prompts=prompts, tokens=toks,
                        margins=margins.astype(np.float32))
    print("min top-2 margin", margins.min())


if __name__ == "__main__":
    main()
