"""NumPy restatement of the Philox4x32-10 counter-based generator and of the
dropout keep-mask the device generator (mtx_dropout_keep_philox) writes.

TEST INFRASTRUCTURE ONLY -- imported by tests/; never by the product.

Philox4x32-10 is the generator of Salmon, Moraes, Dror and Shaw, "Parallel
random numbers: as easy as 1, 2, 3" (SC'11): a 128-bit counter (c0..c3) and a
64-bit key (k0, k1); ten rounds, each
    (hi0, lo0) = M0 * c0,   (hi1, lo1) = M1 * c2      (32x32 -> 64-bit products)
    c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0)
with the key advanced by the Weyl constants (W0, W1) before every round but
the first.  Pinned by the published known-answer vectors (tests/test_dropout.py).

The keep mask replaces the reference's host draw np.random.rand(*shape) > p
(layers.py:120) where the mask feeds a fused kernel: element e (row-major
over rows x cols) takes output word e % 4 of counter offset + e // 4 (upper
64 bits of the counter zero), u = (word >> 8) * 2^-24, keep = u > p.
"""
from __future__ import annotations

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """ctr: (N, 4) integers < 2^32, key: (k0, k1).  Returns (N, 4) uint32."""
    c = np.asarray(ctr, dtype=np.uint64).reshape(-1, 4)
    c0, c1, c2, c3 = (c[:, i].copy() for i in range(4))
    k0, k1 = np.uint64(int(key[0]) & MASK32), np.uint64(int(key[1]) & MASK32)
    m0, m1, m32 = np.uint64(M0), np.uint64(M1), np.uint64(MASK32)
    for r in range(10):
        if r:
            k0 = (k0 + np.uint64(W0)) & m32
            k1 = (k1 + np.uint64(W1)) & m32
        p0 = m0 * c0  # < 2^64: exact in uint64
        p1 = m1 * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & m32
        hi1, lo1 = p1 >> np.uint64(32), p1 & m32
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return np.stack([c0, c1, c2, c3], axis=1).astype(np.uint32)


def keep_mask(rows: int, cols: int, p: float, seed: int, offset: int = 0) -> np.ndarray:
    """(rows, cols) uint8 keep mask as mtx_dropout_keep_philox draws it."""
    n = rows * cols
    calls = (n + 3) // 4
    t = np.arange(calls, dtype=np.uint64) + np.uint64(offset)
    ctr = np.zeros((calls, 4), dtype=np.uint64)
    ctr[:, 0] = t & np.uint64(MASK32)
    ctr[:, 1] = t >> np.uint64(32)
    words = philox4x32_10(ctr, (seed & MASK32, (seed >> 32) & MASK32)).reshape(-1)[:n]
    u = (words >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)
    return (u > np.float32(p)).astype(np.uint8).reshape(rows, cols)
