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


def group_cases(count: int = 24, seed: int = 4242):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        dt = [Q4K, Q6K, Q4_0, Q8_0][i % 4]
        m = int(M_CHOICES[rng.integers(len(M_CHOICES))])
        ns = tuple(int(v) for v in rng.integers(1, 400, size=int(rng.integers(1, 4))))
        k = 256 * int(rng.integers(1, 9))
        out.append((dt, m, ns, k))
    return out


@pytest.mark.parametrize("dt,m,ns,k", group_cases())
def test_random_group(orc, dev, dt, m, ns, k):
    """One to three weights on one activation (llama.rs:156-158), at random
    rows and widths: the joined matvec or skinny launch, or one shared
    quantize then a matmul per weight."""
    from tests.test_gpu_parity import assert_close, upload
    from xn_amd.quantized import matmul_t_group

    rng = np.random.default_rng(5000 + dt + 11 * m + sum(ns) + k)
    blocks = [orc.from_float(dt, rng.normal(0, 0.02, (n, k))) for n in ns]
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qts = [upload(b, n, k, dt, dev) for b, n in zip(blocks, ns)]
    dsts = [torch.full((m, n), float("nan"), dtype=torch.float32, device=dev) for n in ns]
    matmul_t_group(qts, m, k, torch.from_numpy(x).to(dev), dsts)
    for i, (b, n) in enumerate(zip(blocks, ns)):
        assert_close(dsts[i].cpu().numpy(), orc.matmul(dt, x, b, n), f"group dt={dt} m={m} k={k} weight {i} n={n}")


def mlp_cases(count: int = 16, seed: int = 777):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        dt, down_dt = [(Q4K, Q6K), (Q4K, Q4K), (Q6K, Q6K), (Q4_0, Q4_0)][i % 4]
        m = int(M_CHOICES[rng.integers(len(M_CHOICES))])
        k = 256 * int(rng.integers(1, 9))
        f = 256 * int(rng.integers(1, 9))
        n = int(rng.integers(1, 400))
        out.append((dt, down_dt, m, k, f, n))
    return out


@pytest.mark.parametrize("dt,down_dt,m,k,f,n", mlp_cases())
def test_random_mlp(orc, dev, dt, down_dt, m, k, f, n):
    """The SwiGLU MLP entry (llama.rs:236-264) at random rows and widths: h
    against the oracle's silu(x . gate) * (x . up), y against the oracle's
    down projection of the device's h."""
    from tests.test_gpu_parity import _silu, assert_close, upload
    from xn_amd.quantized import mlp_t

    rng = np.random.default_rng(6000 + 7 * dt + down_dt + m + k + f + n)
    gb = orc.from_float(dt, rng.normal(0, 0.02, (f, k)))
    ub = orc.from_float(dt, rng.normal(0, 0.02, (f, k)))
    db = orc.from_float(down_dt, rng.normal(0, 0.02, (n, f)))
    g, u, d = upload(gb, f, k, dt, dev), upload(ub, f, k, dt, dev), upload(db, n, f, down_dt, dev)
    xh = rng.normal(0, 1, (m, k)).astype(np.float32)
    h = torch.empty((m, f), dtype=torch.float32, device=dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    mlp_t(g, u, d, m, torch.from_numpy(xh).to(dev), h, y)
    want_h = _silu(orc.matmul(dt, xh, gb, f).astype(np.float64)) * orc.matmul(dt, xh, ub, f)
    assert_close(h.cpu().numpy(), want_h, f"mlp h dt={dt} m={m} k={k} f={f}")
    assert_close(y.cpu().numpy(), orc.matmul(down_dt, h.cpu().numpy(), db, n), f"mlp y dt={dt} m={m} f={f} n={n}")
