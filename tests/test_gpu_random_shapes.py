"""Seeded random shapes across every route of `matmul_t`.

The configured shapes and the hand-picked edge cases pin each kernel at the
sizes it was tuned for; these cases draw (dtype, m, n, k) at random around
the route boundaries instead: m from 1 to 700, so every route and both
sides of each crossover are hit (matvec, the wavefront-split and split-K
skinny kernels, the prefill kernel, the tiled kernel and its half-empty-tail
instance); n ragged against every tile width; k any whole number of blocks
(super-blocks for the K-quants); the six padded-block dtypes, which run on
the matvec kernels at every m, are drawn the same way.  Reference semantics: k_quants::matmul
(k_quants.rs:1996-2011) over each dtype's vec_dot; the oracle's matmul is
the check, to the f32 bar (1e-3 relative L2, 2e-3 max relative per row).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14
Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K = 3, 6, 7, 10, 11, 13
M_CHOICES = [1, 2, 3, 4, 5, 8, 9, 15, 16, 17, 31, 32, 33, 40, 63, 64, 65, 96, 127, 128, 129, 200, 256,
             257, 384, 511, 512, 513, 600, 700]


def cases(count: int = 120, seed: int = 20261202, dtypes=(Q4K, Q6K, Q4_0, Q8_0)):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        dt = dtypes[i % len(dtypes)]
        m = int(M_CHOICES[rng.integers(len(M_CHOICES))])
        n = int(rng.integers(1, 640))
        if dt in (Q4K, Q6K, Q2K, Q3K, Q5K):
            k = 256 * int(rng.integers(1, 13))
        else:
            k = 64 * int(rng.integers(1, 40))  # 2..78 blocks of 32
        out.append((dt, m, n, k))
    return out


@pytest.mark.parametrize("dt,m,n,k", cases() + cases(36, 19937, (Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K)))
def test_random_shape(orc, dev, dt, m, n, k):
    from tests.test_gpu_parity import assert_close, upload

    rng = np.random.default_rng(1000 * dt + 7 * m + 3 * n + k)
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} m={m} n={n} k={k}")
