"""GPU parity at every configured shape.

The HIP path runs through the C ABI on full-size weights; the checker is the
AVX2 restatement of xn's CPU path (`oracle.cpu_matmul`: quantize_lhs, then
vec_dot per 128-column task, k_quants.rs:52-90, 1996-2026, avx.rs), which
`tests/test_oracle.py::test_avx2_baseline_agrees` pins to the scalar oracle.
Weights are N(0, 0.02) quantized on the device (byte-identical to the CPU
quantizer, `test_gpu_parity.py::test_device_weight_quantizer_bit_exact`), and
the checker reads the very blocks the device holds back through `raw_data`.
The vocab-sized lm_head uses random GGUF blocks (every quant, scale and min
bit pattern; f16 scales drawn at the magnitude a quantized N(0, 0.02) weight
has), since it is the block decode, not the quantizer, being tested there.

Bars as in test_gpu_parity: relative L2 <= 1e-3 and per-row max relative
error <= 2e-3.
"""
import os

import numpy as np
import pytest
import torch

from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4K, Q6K = 2, 8, 12, 14
SEED = 299792458


@pytest.fixture(scope="module")
def checker(orc):
    orc.cpu_pool_init(min(16, os.cpu_count() or 1))
    return orc


class Weights:
    """Device-quantized weights of the configured shapes, with their GGUF bytes
    for the checker; at most a few held at once."""

    def __init__(self, dev):
        self.dev = dev
        self.cache = {}

    def get(self, dt, n, k, tag=0):
        from xn_amd import GgmlDType, QTensor

        key = (dt, n, k, tag)
        if key not in self.cache:
            if len(self.cache) >= 3:
                self.cache.pop(next(iter(self.cache)))
            g = torch.Generator(device=self.dev).manual_seed(SEED + 7 * dt + n + 3 * k + 11 * tag)
            w = torch.randn((n, k), generator=g, device=self.dev, dtype=torch.float32) * 0.02
            qt = QTensor.quantize_f32(w, (n, k), GgmlDType(dt))
            del w
            blocks = np.frombuffer(qt.data(), dtype=np.uint8)
            self.cache[key] = (qt, blocks)
        return self.cache[key]


@pytest.fixture(scope="module")
def weights(dev):
    w = Weights(dev)
    yield w
    w.cache.clear()
    torch.cuda.empty_cache()


def random_blocks(orc, dt, n, k, rng):
    """Random GGUF blocks of dtype Q4K / Q6K with sane f16 scales."""
    nb = n * (k // 256)
    b = rng.integers(0, 256, (nb, orc.TYPE_SIZE[dt]), dtype=np.uint8)
    if dt == Q4K:  # d, dmin at bytes 0..3
        d = rng.uniform(2e-4, 6e-4, nb).astype(np.float16)
        dmin = rng.uniform(1e-4, 4e-4, nb).astype(np.float16)
        b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        b[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    else:  # Q6K: ql[128] qh[64] scales[16] d
        d = rng.uniform(2e-5, 6e-5, nb).astype(np.float16)
        b[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def x_rows(m, k, seed):
    return np.random.default_rng(seed).normal(0, 1, (m, k)).astype(np.float32)


def run_matmul_t(qt, x, n, dev):
    m, k = x.shape
    dst = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    return dst.cpu().numpy()


# ------------------------------------------------------------ config 1
def test_config1_q8_0_matvec(checker, weights, dev):
    qt, blocks = weights.get(Q8_0, 4096, 4096)
    x = x_rows(1, 4096, SEED)
    assert_close(run_matmul_t(qt, x, 4096, dev), checker.cpu_matmul(Q8_0, x, blocks, 4096), "config 1")


# ------------------------------------------------------------ config 2
@pytest.mark.parametrize("fused", [True, False])
def test_config2_q4_0_ffn_block(checker, weights, dev, fused):
    """h = silu(x Wg^T) * (x Wu^T), y = h Wd^T (llama.rs:258-264) at 4096 -> 14336 -> 4096,
    with the SiLU-gated one-launch kernel or two matmul_t calls and a host SiLU."""
    from xn_amd.quantized import matmul_t_silu_gate

    k, f = 4096, 14336
    g, gb = weights.get(Q4_0, f, k, 0)
    u, ub = weights.get(Q4_0, f, k, 1)
    d, db = weights.get(Q4_0, k, f, 2)
    x = x_rows(1, k, SEED + 2)
    xd = torch.from_numpy(x).to(dev)
    h = torch.empty((1, f), device=dev)
    if fused:
        matmul_t_silu_gate(g, u, (1, k, f), xd, h)
    else:
        gg = torch.empty((1, f), device=dev)
        uu = torch.empty((1, f), device=dev)
        g.matmul_t((1, k, f), xd, gg)
        u.matmul_t((1, k, f), xd, uu)
        h = gg / (1.0 + torch.exp(0.0 - gg)) * uu
    y = torch.empty((1, k), device=dev)
    d.matmul_t((1, f, k), h, y)
    gw = checker.cpu_matmul(Q4_0, x, gb, f).astype(np.float64)
    hw = (gw / (1.0 + np.exp(0.0 - gw)) * checker.cpu_matmul(Q4_0, x, ub, f)).astype(np.float32)
    assert_close(h.cpu().numpy(), hw, "config 2 h")
    assert_close(y.cpu().numpy(), checker.cpu_matmul(Q4_0, hw, db, k), "config 2 y")


# ------------------------------------------------------------ config 3
@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 14336), (14336, 4096), (8192, 28672)])
def test_config3_q4k_sweep(checker, weights, dev, k, n):
    """Q4_K matvec sweep at M = 1, 2, 4, 8 (the matvec up to m = 4, the
    skinny kernel at m = 8: the wavefront-split form where it applies,
    split-K on 8192 -> 28672)."""
    qt, blocks = weights.get(Q4K, n, k)
    for m in (1, 2, 4, 8):
        x = x_rows(m, k, SEED + m + k)
        assert_close(run_matmul_t(qt, x, n, dev), checker.cpu_matmul(Q4K, x, blocks, n),
                     f"config 3 k={k} n={n} m={m}")


# ------------------------------------------------------------ config 4
@pytest.mark.parametrize("dt", [Q4K, Q6K])
def test_config4_prefill(checker, weights, dev, dt):
    """Prefill K = 4096 -> N = 14336 at M = 64, 256, 512, 2048 through matmul_t
    (M = 64: skinny route; above: the tiled int8-MFMA kernel), plus the tiled
    kernel forced at M = 64 and the pre-quantized entry the bench times at 512."""
    from xn_amd.quantized import matmul_preq, quantize_lhs, set_route

    k, n = 4096, 14336
    qt, blocks = weights.get(dt, n, k)
    for m in (64, 256, 512, 2048):
        x = x_rows(m, k, SEED + m)
        assert_close(run_matmul_t(qt, x, n, dev), checker.cpu_matmul(dt, x, blocks, n),
                     f"config 4 dt={dt} m={m}")
    x = x_rows(64, k, SEED + 64)
    set_route(2)
    try:
        got = run_matmul_t(qt, x, n, dev)
    finally:
        set_route(0)
    assert_close(got, checker.cpu_matmul(dt, x, blocks, n), f"config 4 dt={dt} m=64 forced tiled")
    m = 512
    x = x_rows(m, k, SEED + 9)
    ws = qt.workspace(m)
    y = torch.full((m, n), float("nan"), device=dev)
    quantize_lhs(qt.dtype(), torch.from_numpy(x).to(dev), ws, m, k)
    matmul_preq(qt, m, ws, y)
    assert_close(y.cpu().numpy(), checker.cpu_matmul(dt, x, blocks, n), f"config 4 dt={dt} preq m=512")


@pytest.mark.parametrize("m", [96, 384, 512, 513])
def test_config4_prefill_route_boundary(checker, weights, dev, m):
    """Config 4's Q4_K weight on either side of the row count where the
    prefill route switches kernels: 64-row tiles with the K range split
    across workgroups (m = 96), 128-row tiles (m = 384, 512) and, past it,
    the 256 x 128 tiled kernel (m = 513)."""
    k, n = 4096, 14336
    qt, blocks = weights.get(Q4K, n, k)
    x = x_rows(m, k, SEED + 31 * m)
    assert_close(run_matmul_t(qt, x, n, dev), checker.cpu_matmul(Q4K, x, blocks, n), f"config 4 boundary m={m}")


# ------------------------------------------------------------ config 5
@pytest.mark.parametrize("dt,k,n", [(Q4K, 4096, 4096), (Q4K, 4096, 1024), (Q4K, 4096, 14336),
                                    (Q6K, 14336, 4096)])
def test_config5_layer_shapes(checker, weights, dev, dt, k, n):
    """Every layer QMatMul shape of the decode step at batch 1 and 16 (q/o,
    k/v, gate/up, down)."""
    qt, blocks = weights.get(dt, n, k)
    for m in (1, 16):
        x = x_rows(m, k, SEED + 5 * m + n)
        assert_close(run_matmul_t(qt, x, n, dev), checker.cpu_matmul(dt, x, blocks, n),
                     f"config 5 dt={dt} k={k} n={n} m={m}")


def test_config5_lm_head(checker, dev):
    """lm_head: Q6_K 4096 -> 128256 at batch 1 and 16."""
    from xn_amd import GgmlDType, QTensor

    k, n = 4096, 128256
    blocks = random_blocks(checker, Q6K, n, k, np.random.default_rng(SEED + 6))
    qt = QTensor.from_gguf_bytes(blocks, (n, k), GgmlDType.Q6K, dev)
    try:
        for m in (1, 16):
            x = x_rows(m, k, SEED + 17 * m)
            assert_close(run_matmul_t(qt, x, n, dev), checker.cpu_matmul(Q6K, x, blocks, n), f"lm_head m={m}")
    finally:
        del qt
        torch.cuda.empty_cache()


def test_config5_random_q4k_blocks(checker, dev):
    """Q4_K 4096 -> 14336 on random blocks (every 6-bit scale/min pattern) at
    the matvec, skinny and tiled routes."""
    from xn_amd import GgmlDType, QTensor

    k, n = 4096, 14336
    blocks = random_blocks(checker, Q4K, n, k, np.random.default_rng(SEED + 4))
    qt = QTensor.from_gguf_bytes(blocks, (n, k), GgmlDType.Q4K, dev)
    for m in (1, 16, 512):
        x = x_rows(m, k, SEED + 31 * m)
        assert_close(run_matmul_t(qt, x, n, dev), checker.cpu_matmul(Q4K, x, blocks, n), f"random q4k m={m}")


@pytest.mark.parametrize("m", [1, 16])
def test_config5_qkv_group(checker, weights, dev, m):
    """q, k, v (4096 -> 4096, 1024, 1024) in one grouped call (llama.rs:156-158)."""
    from xn_amd.quantized import matmul_t_group

    k = 4096
    ns = (4096, 1024, 1024)
    ws = [weights.get(Q4K, n, k, 10 + i) for i, n in enumerate(ns)]
    x = x_rows(m, k, SEED + 40 + m)
    dsts = [torch.full((m, n), float("nan"), device=dev) for n in ns]
    matmul_t_group([w[0] for w in ws], m, k, torch.from_numpy(x).to(dev), dsts)
    for i, ((_, blocks), n) in enumerate(zip(ws, ns)):
        assert_close(dsts[i].cpu().numpy(), checker.cpu_matmul(Q4K, x, blocks, n), f"qkv m={m} weight {i}")


@pytest.mark.parametrize("m", [1, 16])
def test_config5_silu_gate(checker, weights, dev, m):
    """gate/up 4096 -> 14336 Q4_K with the SiLU gate (llama.rs:258-264)."""
    from xn_amd.quantized import matmul_t_silu_gate

    k, n = 4096, 14336
    (g, gb), (u, ub) = weights.get(Q4K, n, k, 20), weights.get(Q4K, n, k, 21)
    x = x_rows(m, k, SEED + 50 + m)
    dst = torch.full((m, n), float("nan"), device=dev)
    matmul_t_silu_gate(g, u, (m, k, n), torch.from_numpy(x).to(dev), dst)
    gw = checker.cpu_matmul(Q4K, x, gb, n).astype(np.float64)
    want = gw / (1.0 + np.exp(0.0 - gw)) * checker.cpu_matmul(Q4K, x, ub, n)
    assert_close(dst.cpu().numpy(), want, f"silu gate m={m}")
