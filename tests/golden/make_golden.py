"""Writes the small golden fixtures in this directory from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Each fixture golden_<dtype>.npz holds, for one weight dtype, seeded f32
weights and activations and what the oracle computes from them: the
canonical GGUF weight blocks, the canonical activation blocks (Q8_0 or Q8_K),
the per-block integer dot products and the f32 matmul output.  The oracle is
itself pinned (known-answer test, brute force, closed forms); these fixtures
freeze its outputs so that a later change to it, or to a device kernel, shows
up as a byte difference.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

# (name, dtype id, m, k, n): small enough to stay a few tens of KB each
CASES = [
    ("q8_0", oracle.Q8_0, 3, 256, 16),
    ("q4_0", oracle.Q4_0, 3, 256, 16),
    ("q4k", oracle.Q4K, 3, 512, 16),
    ("q6k", oracle.Q6K, 3, 512, 16),
    ("q4_1", oracle.Q4_1, 3, 256, 16),
    ("q5_0", oracle.Q5_0, 3, 256, 16),
    ("q5_1", oracle.Q5_1, 3, 256, 16),
    ("q2k", oracle.Q2K, 3, 512, 16),
    ("q3k", oracle.Q3K, 3, 512, 16),
    ("q5k", oracle.Q5K, 3, 512, 16),
]
SEED = 299792458


def make(name, dt, m, k, n):
    rng = np.random.default_rng(SEED + dt)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    # a few edge values: an all-zero activation row segment and a tie in |x|
    x[0, :32] = 0.0
    x[1, 5], x[1, 9] = 1.5, -1.5
    wb = oracle.from_float(dt, w)
    ab = oracle.quantize_lhs(dt, x)
    ints = oracle.block_ints(dt, wb, ab, m, n, k)
    y = oracle.matmul(dt, x, wb, n)
    np.savez(os.path.join(HERE, f"golden_{name}.npz"), dtype=np.int32(dt), m=np.int32(m),
             k=np.int32(k), n=np.int32(n), w=w, x=x, w_blocks=wb, act_blocks=ab,
             block_ints=ints, y=y)


if __name__ == "__main__":
    for c in CASES:
        make(*c)
        print("wrote", c[0])
