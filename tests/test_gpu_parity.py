"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars (from the path's contract):
  * activation quantization (Q8_0, Q8_K), weight quantization, repack round
    trips, dequantization and per-block integer dots: bit-exact;
  * f32 matmul outputs: relative L2 <= 1e-3 and, per output row,
    max |got - want| / max |want| <= 2e-3.
"""
import numpy as np
import pytest
import torch

from tests import _formats as F

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, Q4K, Q6K, Q8K = 2, 8, 12, 14, 15
WEIGHT_DTYPES = [Q4_0, Q8_0, Q4K, Q6K]
REL_L2 = 1e-3
ROW_MAX_REL = 2e-3


def assert_close(got: np.ndarray, want: np.ndarray, what: str = "") -> None:
    got = got.reshape(want.shape).astype(np.float64)
    want = want.astype(np.float64)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert rel <= REL_L2, f"{what}: relative L2 {rel:.3e}"
    w2 = want.reshape(-1, want.shape[-1])
    g2 = got.reshape(-1, want.shape[-1])
    row = np.abs(g2 - w2).max(axis=1) / np.maximum(np.abs(w2).max(axis=1), 1e-30)
    assert row.max() <= ROW_MAX_REL, f"{what}: row max relative error {row.max():.3e} (row {row.argmax()})"


def upload(orc_blocks: np.ndarray, n: int, k: int, dt: int, dev):
    from xn_amd import GgmlDType, QTensor

    return QTensor.from_gguf_bytes(orc_blocks, (n, k), GgmlDType(dt), dev)


# ------------------------------------------------- activation quantizers
@pytest.mark.parametrize("act", [Q8_0, Q8K])
@pytest.mark.parametrize("m,k", [(1, 256), (3, 4096), (8, 14336), (33, 512)])
def test_act_quantizer_bit_exact(orc, dev, act, m, k):
    from xn_amd.quantized import quantize_act_blocks

    rng = np.random.default_rng(1000 + m + act)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    x[0, :256] = 0.0  # an all-zero block
    if k >= 512:
        x[-1, 256:512] = rng.normal(0, 1e-30, 256).astype(np.float32)  # tiny values, subnormal scales
        x[-1, 300], x[-1, 301] = -3.5, 3.5  # tie on |x|: first wins
    want = orc.from_float(act, x)
    got = quantize_act_blocks(act, torch.from_numpy(x).to(dev), m, k).cpu().numpy()
    assert np.array_equal(got, want)


def test_act_quantizer_edge_values(orc, dev):
    from xn_amd.quantized import quantize_act_blocks

    rng = np.random.default_rng(7)
    k = 256
    rows = [
        np.full(k, 1.0, np.float32),
        np.full(k, -2.5, np.float32),
        np.where(np.arange(k) % 2 == 0, 1e4, -1e4).astype(np.float32),
        (np.arange(k, dtype=np.float32) - 128) * np.float32(0.5),  # exact halves -> round away from 0
        rng.normal(0, 1e6, k).astype(np.float32),
        rng.normal(0, 1e-6, k).astype(np.float32),
    ]
    # a NaN (dropped from the block maximum; its quant is min(NaN, 127) = 127
    # for Q8_K, `NaN as i8` = 0 for Q8_0) and infinities (Rust `as i8`
    # saturation and NaN products)
    for pos, val in ((5, np.nan), (9, np.inf), (40, -np.inf)):
        r = rng.normal(0, 1, k).astype(np.float32)
        r[pos] = val
        rows.append(r)
    x = np.stack(rows)
    for act in (Q8_0, Q8K):
        want = orc.from_float(act, x)
        got = quantize_act_blocks(act, torch.from_numpy(x).to(dev), x.shape[0], k).cpu().numpy()
        assert np.array_equal(got, want), f"act dtype {act}"


# ------------------------------------------- weight storage round trips
@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
def test_upload_raw_data_round_trip(orc, dev, dt):
    rng = np.random.default_rng(2000 + dt)
    n, k = 37, 1024
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    qt = upload(blocks, n, k, dt, dev)
    assert qt.storage_size_in_bytes() == blocks.size
    assert qt.data() == blocks.tobytes()


@pytest.mark.parametrize("dt", [Q4K, Q6K])
def test_raw_data_round_trip_random_bytes(orc, dev, dt):
    """Any byte pattern survives repack -> unrepack (the repack is a bijection)."""
    rng = np.random.default_rng(2100 + dt)
    n, k = 5, 768
    blocks = rng.integers(0, 256, n * (k // 256) * orc.TYPE_SIZE[dt]).astype(np.uint8)
    qt = upload(blocks, n, k, dt, dev)
    assert qt.data() == blocks.tobytes()


@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
def test_dequantize_bit_exact(orc, dev, dt):
    rng = np.random.default_rng(3000 + dt)
    n, k = 19, 1536
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    qt = upload(blocks, n, k, dt, dev)
    got = qt.dequantize().cpu().numpy().reshape(-1)
    want = orc.to_float(dt, blocks)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
def test_device_weight_quantizer_bit_exact(orc, dev, dt):
    from xn_amd import GgmlDType, QTensor

    rng = np.random.default_rng(4000 + dt)
    n, k = 24, 2048
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w[1] = 0.0
    w[2] = 0.125
    w[3, :256] = np.linspace(-1, 1, 256, dtype=np.float32)
    qt = QTensor.quantize_f32(torch.from_numpy(w).to(dev), (n, k), GgmlDType(dt))
    assert qt.data() == orc.from_float(dt, w).tobytes()


# ----------------------------------------------------- integer block dots
@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
def test_block_ints_bit_exact(orc, dev, dt):
    from xn_amd.quantized import block_ints, lhs_workspace, quantize_lhs

    rng = np.random.default_rng(5000 + dt)
    m, n, k = 3, 21, 1024
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    ws = lhs_workspace(qt.dtype(), m, k, dev)
    quantize_lhs(qt.dtype(), torch.from_numpy(x).to(dev), ws, m, k)
    got = block_ints(qt, m, ws).cpu().numpy().astype(np.int64)
    want = F.block_ints_bruteforce(dt, blocks, orc.quantize_lhs(dt, x), m, n, k)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- matmul
@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 17])
@pytest.mark.parametrize("entry", ["matmul_t", "matmul_t_abi", "matmul_t_split"])
def test_matmul_small(orc, dev, dt, m, entry):
    rng = np.random.default_rng(6000 + 31 * dt + m)
    n, k = 300, 2048
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    getattr(qt, entry)((m, k, n), torch.from_numpy(x).to(dev), dst)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} m={m} {entry}")


@pytest.mark.parametrize("dt,k,n", [
    (Q8_0, 4096, 4096),   # config 1
    (Q4_0, 4096, 14336),  # config 2 gate/up
    (Q4_0, 14336, 4096),  # config 2 down
    (Q4K, 4096, 4096),    # config 3
    (Q4K, 4096, 14336),
    (Q4K, 14336, 4096),
    (Q6K, 14336, 4096),   # config 5 FFN down
    (Q4K, 4096, 1792),    # an 8-way column-parallel shard of gate/up
    (Q6K, 1792, 4096),    # an 8-way row-parallel shard of down
])
# m = 3 and 4: the matvec, or for Q4_K / Q6_K weights with K >= 4096 and
# 2048 < N <= K the skinny kernel; m = 5 and 8: the skinny kernel for
# Q4_K / Q6_K, the matvec for the other dtypes
@pytest.mark.parametrize("m", [1, 3, 4, 5, 8])
def test_matmul_config_shapes(orc, dev, dt, k, n, m):
    rng = np.random.default_rng(7000 + dt + k + n + m)
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    blocks = orc.from_float(dt, w)
    del w
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} k={k} n={n} m={m}")


@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("m,n,k", [(64, 512, 4096), (130, 512, 4096), (300, 200, 768), (9, 129, 256),
                                   (257, 384, 1280), (16, 512, 7168), (24, 1000, 4096), (128, 384, 512),
                                   (129, 384, 512), (640, 300, 512)])
def test_matmul_prefill_sizes(orc, dev, dt, m, n, k):
    """The int8-MFMA route (forced): ragged m and n against the tiles
    (Q4_K up to 512 rows: the prefill kernel's 64- or 128-row by 256-column
    tiles; Q6_K and Q4_K past 512 rows: the 256 x 128 tiled kernel, whose
    instance for a last row tile at most half full drops the MFMAs of the
    wavefronts past m: tails of 128 (that instance) and 129 (the other)),
    1-28 super-blocks, and grids small enough to be split along K (partial
    sums added in a second kernel)."""
    from xn_amd.quantized import set_route

    rng = np.random.default_rng(8000 + dt + m + n + k)
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    set_route(2)
    try:
        qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    finally:
        set_route(0)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} m={m} n={n} k={k}")


@pytest.mark.parametrize("dt,m", [(Q4K, 96), (Q4K, 512), (Q6K, 300), (Q6K, 64)])
def test_matmul_prefill_long_k(orc, dev, dt, m):
    """The prefill-sized routes at the down projection's K = 14336 (56
    super-blocks per row; 4096 -> 14336 is the only K of the config-4
    prefill shapes): Q4_K on the prefill kernel (at N = 256, 64-row tiles
    split 28 ways along K), Q6_K on the tiled kernel (300 rows: its
    half-empty-tail instance, split along K) and on the skinny kernel (64
    rows), at the auto route."""
    rng = np.random.default_rng(8200 + dt + m)
    k, n = 14336, 256
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} m={m} k={k}")


@pytest.mark.parametrize("m,n,k", [(4, 301, 2304), (5, 77, 768), (7, 130, 8448), (8, 257, 256), (12, 99, 2304),
                                   (16, 64, 4096)])
def test_matmul_q4k_multirow_matvec(orc, dev, m, n, k):
    """Q4_K on the matvec route (forced) from 4 rows, where the staged
    activation image is interleaved by row in groups of 64 chunks: K whose
    chunk count is not a multiple of 64, rows past the launch's 4 or 8, and
    m above 8 (a second launch)."""
    from xn_amd.quantized import set_route

    rng = np.random.default_rng(8300 + m + n + k)
    blocks = orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, Q4K, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    set_route(1)
    try:
        # quantize_lhs + matmul_preq: the workspace (non-fused) matvec kernels
        qt.matmul_t_split((m, k, n), torch.from_numpy(x).to(dev), dst)
    finally:
        set_route(0)
    assert_close(dst.cpu().numpy(), orc.matmul(Q4K, x, blocks, n), f"m={m} n={n} k={k}")


@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("m,n,k", [(1, 300, 2048), (2, 300, 2048), (5, 129, 768), (7, 40, 256), (8, 512, 4096),
                                   (8, 100, 8192), (16, 200, 1024), (31, 384, 2304), (33, 256, 1280),
                                   (64, 130, 512)])
def test_matmul_skinny(orc, dev, dt, m, n, k):
    """The skinny int8-MFMA route (forced) for 1 <= m <= 64: 16-row tiles (K
    split across a workgroup's wavefronts, with fewer super-blocks than
    wavefronts at K = 256 and eight wavefronts at K = 8192), one and two
    32-row tiles, ragged n against the column tiles, split-K."""
    from xn_amd.quantized import set_route

    rng = np.random.default_rng(8500 + dt + m + n + k)
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    set_route(3)
    try:
        qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    finally:
        set_route(0)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} m={m} n={n} k={k}")


def test_qlinear_vs_linear(dev):
    """tests/quantized_tests.rs:14-118: QLinear(Q8_0) vs f32 Linear, 64->32,
    batch 4 (and 2x3 3-D input), max error < 0.3, with and without bias."""
    from xn_amd import GgmlDType, QLinear

    g = torch.Generator().manual_seed(299792458)
    w = torch.randn(32, 64, generator=g)
    b = torch.randn(32, generator=g)
    for xs in (torch.randn(4, 64, generator=g), torch.randn(2, 3, 64, generator=g)):
        for bias in (None, b):
            ref = xs @ w.T + (0 if bias is None else bias)
            ql = QLinear.from_linear(w.to(dev), None if bias is None else bias.to(dev), GgmlDType.Q8_0)
            out = ql.forward(xs.to(dev)).cpu()
            assert out.shape == ref.shape
            assert (out - ref).abs().max().item() < 0.3


# ------------------------------------------------------------ error paths
def test_errors(orc, dev):
    from xn_amd import GgmlDType, QTensor, XnqError

    rng = np.random.default_rng(9)
    blocks = orc.from_float(Q4K, rng.normal(0, 0.02, (4, 256)))
    with pytest.raises(XnqError, match="divisible"):
        QTensor.from_gguf_bytes(blocks, (8, 128), GgmlDType.Q4K, dev)
    with pytest.raises(XnqError, match="not supported"):
        QTensor.from_gguf_bytes(np.zeros(512, np.uint8), (1, 256), GgmlDType.F16, dev)
    qt = QTensor.from_gguf_bytes(blocks, (4, 256), GgmlDType.Q4K, dev)
    lhs = torch.zeros(512, device=dev)
    dst = torch.zeros(8, device=dev)
    with pytest.raises(XnqError, match="does not match"):
        qt.matmul_t((1, 512, 4), lhs, dst)
    with pytest.raises(XnqError, match="unexpected lhs length"):
        qt.matmul_t((2, 256, 4), lhs[:100], dst)
    # m = 0 is a no-op
    qt.matmul_t((0, 256, 4), lhs[:0], dst[:0])


# ------------------------------------------------ decode-step groups
def _silu(v):
    return v / (1.0 + np.exp(0.0 - v))


@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
@pytest.mark.parametrize("m,k,n", [(1, 2048, 300), (1, 4096, 1000), (3, 2048, 300), (1, 12288, 96), (9, 1024, 64),
                                   (16, 4096, 512), (16, 2048, 300), (80, 1024, 256)])
def test_silu_gate(orc, dev, dt, m, k, n):
    """SwiGLU of llama.rs:258-264: silu(x . gate) * (x . up), one kernel at m = 1;
    above, one shared activation quantize then a matmul per weight (skinny
    split-K at m = 16, tiled MFMA at m = 80 for the K-quants)."""
    from xn_amd.quantized import matmul_t_silu_gate

    rng = np.random.default_rng(8100 + dt + m + k + n)
    gb = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    ub = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    g, u = upload(gb, n, k, dt, dev), upload(ub, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    matmul_t_silu_gate(g, u, (m, k, n), torch.from_numpy(x).to(dev), dst)
    want = _silu(orc.matmul(dt, x, gb, n).astype(np.float64)) * orc.matmul(dt, x, ub, n)
    assert_close(dst.cpu().numpy(), want, f"silu_gate dt={dt} m={m} k={k} n={n}")


@pytest.mark.parametrize("dt", WEIGHT_DTYPES)
@pytest.mark.parametrize("m,ns", [(1, (300,)), (1, (512, 128, 128)), (1, (40, 7)), (2, (200, 64, 64)),
                                  (5, (300, 96, 40)), (8, (512, 128, 128)),
                                  (16, (512, 128, 128)), (16, (200, 72, 40)), (40, (300, 96)), (80, (256, 64))])
def test_matmul_group(orc, dev, dt, m, ns):
    """q, k, v projections of one activation (llama.rs:156-158) in one launch."""
    from xn_amd.quantized import matmul_t_group

    k = 2048
    rng = np.random.default_rng(8200 + dt + m + sum(ns))
    blocks = [orc.from_float(dt, rng.normal(0, 0.02, (n, k))) for n in ns]
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qts = [upload(b, n, k, dt, dev) for b, n in zip(blocks, ns)]
    dsts = [torch.full((m, n), float("nan"), dtype=torch.float32, device=dev) for n in ns]
    matmul_t_group(qts, m, k, torch.from_numpy(x).to(dev), dsts)
    for i, (b, n) in enumerate(zip(blocks, ns)):
        assert_close(dsts[i].cpu().numpy(), orc.matmul(dt, x, b, n), f"group dt={dt} m={m} weight {i} n={n}")


@pytest.mark.parametrize("m", [2, 3, 5])
def test_group_decode_shapes(orc, dev, m):
    """q/k/v (4096 -> 4096, 1024, 1024) and the gate/up pair (4096 -> 14336)
    of config 5 at few rows: q/k/v as one joined skinny launch from m = 2,
    the gate/up pair from m = 3 (the matvec at m = 2)."""
    from xn_amd.quantized import matmul_t_group, matmul_t_silu_gate

    k = 4096
    rng = np.random.default_rng(8300 + m)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    ns = (4096, 1024, 1024)
    blocks = [orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)).astype(np.float32)) for n in ns]
    qts = [upload(b, n, k, Q4K, dev) for b, n in zip(blocks, ns)]
    dsts = [torch.full((m, n), float("nan"), dtype=torch.float32, device=dev) for n in ns]
    matmul_t_group(qts, m, k, xd, dsts)
    for i, (b, n) in enumerate(zip(blocks, ns)):
        assert_close(dsts[i].cpu().numpy(), orc.matmul(Q4K, x, b, n), f"qkv m={m} weight {i}")
    del qts, blocks
    n = 14336
    gb = orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    ub = orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)).astype(np.float32))
    g, u = upload(gb, n, k, Q4K, dev), upload(ub, n, k, Q4K, dev)
    dst = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    matmul_t_silu_gate(g, u, (m, k, n), xd, dst)
    want = _silu(orc.matmul(Q4K, x, gb, n).astype(np.float64)) * orc.matmul(Q4K, x, ub, n)
    assert_close(dst.cpu().numpy(), want, f"gate/up m={m}")


def test_matmul_group_mixed_dtypes(orc, dev):
    """Weights of different dtypes share no kernel: one matmul per weight."""
    from xn_amd.quantized import matmul_t_group

    k = 1024
    rng = np.random.default_rng(8300)
    specs = [(Q4K, 96), (Q6K, 64), (Q8_0, 32)]
    blocks = [orc.from_float(dt, rng.normal(0, 0.02, (n, k))) for dt, n in specs]
    x = rng.normal(0, 1, (1, k)).astype(np.float32)
    qts = [upload(b, n, k, dt, dev) for b, (dt, n) in zip(blocks, specs)]
    dsts = [torch.empty((1, n), dtype=torch.float32, device=dev) for _, n in specs]
    matmul_t_group(qts, 1, k, torch.from_numpy(x).to(dev), dsts)
    for d, b, (dt, n) in zip(dsts, blocks, specs):
        assert_close(d.cpu().numpy(), orc.matmul(dt, x, b, n), f"mixed group dt={dt}")


# ------------------------------------------------ stream capture
def test_capture_graph_replay(orc, dev):
    """Launches captured with xnq_capture_begin/end (Device::capture_begin /
    capture_end, cuda_backend/mod.rs:251-283) replay to the eager results,
    on every replay, with eager work and new inputs between replays."""
    from xn_amd.quantized import capture, matmul_t_silu_gate

    rng = np.random.default_rng(8400)
    k, n = 1024, 256
    b4 = orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)))
    bg = orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)))
    bu = orc.from_float(Q4K, rng.normal(0, 0.02, (n, k)))
    b6 = orc.from_float(Q6K, rng.normal(0, 0.02, (n, k)))
    q4, g, u, q6 = (upload(b, n, k, dt, dev) for b, dt in ((b4, Q4K), (bg, Q4K), (bu, Q4K), (b6, Q6K)))
    xs = {m: torch.zeros((m, k), dtype=torch.float32, device=dev) for m in (1, 16, 300)}
    ys = {name: torch.zeros((m, n), dtype=torch.float32, device=dev)
          for name, m in (("mv", 1), ("gate", 1), ("sk", 16), ("mf", 300), ("t6", 300))}
    ws16 = torch.empty(max(q6.matmul_t_workspace_size(16), 1), dtype=torch.uint8, device=dev)
    ws300 = torch.empty(max(q4.matmul_t_workspace_size(300), 1), dtype=torch.uint8, device=dev)
    ws6 = torch.empty(max(q6.matmul_t_workspace_size(300), 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream(dev)

    def run():
        q4.matmul_t((1, k, n), xs[1], ys["mv"])
        matmul_t_silu_gate(g, u, (1, k, n), xs[1], ys["gate"])
        q6.matmul_t_ws((16, k, n), xs[16], ws16, ys["sk"])
        q4.matmul_t_ws((300, k, n), xs[300], ws300, ys["mf"])
        q6.matmul_t_ws((300, k, n), xs[300], ws6, ys["t6"])  # tiled kernel, half-empty last tile, K split

    torch.cuda.synchronize()
    with capture(stream) as c:
        run()
    assert c.graph is not None
    for rep in range(3):
        host = {m: rng.normal(0, 1, (m, k)).astype(np.float32) for m in xs}
        with torch.cuda.stream(stream):
            for m in xs:
                xs[m].copy_(torch.from_numpy(host[m]))
            for y in ys.values():
                y.fill_(float("nan"))
        stream.synchronize()
        c.graph.launch(stream)
        stream.synchronize()
        got = {name: y.clone() for name, y in ys.items()}
        with torch.cuda.stream(stream):
            for y in ys.values():
                y.fill_(float("nan"))
            run()
        stream.synchronize()
        for name, y in ys.items():
            assert torch.equal(got[name], y), f"replay {rep}: {name} differs from the eager result"
        if rep == 0:
            assert_close(got["mv"].cpu().numpy(), orc.matmul(Q4K, host[1], b4, n), "captured matvec")
            assert_close(got["sk"].cpu().numpy(), orc.matmul(Q6K, host[16], b6, n), "captured skinny")
            assert_close(got["mf"].cpu().numpy(), orc.matmul(Q4K, host[300], b4, n), "captured prefill")
            assert_close(got["t6"].cpu().numpy(), orc.matmul(Q6K, host[300], b6, n), "captured tiled")


def test_matmul_t_refuses_to_allocate_in_capture(orc, dev):
    from xn_amd._lib import XnqError
    from xn_amd.quantized import capture

    rng = np.random.default_rng(8500)
    k, n = 1024, 64
    qt = upload(orc.from_float(Q4K, rng.normal(0, 0.02, (n, k))), n, k, Q4K, dev)
    x = torch.zeros((300, k), dtype=torch.float32, device=dev)
    y = torch.zeros((300, n), dtype=torch.float32, device=dev)
    from xn_amd import _lib

    stream = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    with pytest.raises(XnqError, match="inside a stream capture"):
        with capture(stream):
            st = _lib.load().xnq_qtensor_matmul_t(qt.storage.handle, 300, k, n, x.data_ptr(), y.data_ptr(),
                                                  stream.cuda_stream)
            _lib.check(st)


@pytest.mark.parametrize("nbytes", [16, 4096, 1 << 20, (3 << 20) + 48])
def test_stream_read_folds_every_word(dev, nbytes):
    """The bare-read measurement hook reads every 32-bit word: its XOR fold
    equals numpy's, including a ragged tail past the last full round."""
    from xn_amd.measure import stream_read

    host = np.random.default_rng(nbytes).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(host.view(np.uint8).copy()).to(dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream_read(buf, sink)
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(host)
    assert int(sink.cpu().numpy().view(np.uint32)[0]) == int(want)



@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("m", [9, 16, 40])
def test_skinny_split_k_back_to_back(orc, dev, dt, m):
    """Split-K skinny calls that share one workspace (activation image and
    partial sums), six queued back to back with different activations and no
    host synchronisation, plain and SiLU-gated, each checked against the
    oracle."""
    from xn_amd.quantized import matmul_t_silu_gate

    k, n = 4096, 1280
    rng = np.random.default_rng(8700 + dt + m)
    wb = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    ub = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    w, u = upload(wb, n, k, dt, dev), upload(ub, n, k, dt, dev)
    xs = [rng.normal(0, 1, (m, k)).astype(np.float32) for _ in range(6)]
    ws = torch.empty(max(w.matmul_t_workspace_size(m), 1), dtype=torch.uint8, device=dev)
    outs, gated = [], []
    for x in xs:
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        w.matmul_t_ws((m, k, n), torch.from_numpy(x).to(dev), ws, y)
        outs.append(y)
        h = torch.empty((m, n), dtype=torch.float32, device=dev)
        matmul_t_silu_gate(w, u, (m, k, n), torch.from_numpy(x).to(dev), h)
        gated.append(h)
    for i, x in enumerate(xs):
        want = orc.matmul(dt, x, wb, n)
        assert_close(outs[i].cpu().numpy(), want, f"call {i} dt={dt} m={m}")
        want_h = _silu(want.astype(np.float64)) * orc.matmul(dt, x, ub, n)
        assert_close(gated[i].cpu().numpy(), want_h, f"gated call {i} dt={dt} m={m}")


@pytest.mark.parametrize("dt,down_dt", [(Q4K, Q6K), (Q6K, Q4K), (Q4_0, Q4K)])
@pytest.mark.parametrize("m", [1, 4, 16, 40, 80])
def test_mlp_t(orc, dev, dt, down_dt, m):
    """The SwiGLU MLP entry (llama.rs:236-264): h and y are the bits that
    silu_gate followed by matmul_t produce (on the small-batch MFMA route the
    gate/up split-sum also quantizes h for the down projection), and match
    the oracle."""
    from xn_amd.quantized import matmul_t_silu_gate, mlp_t

    k, f, n = 2048, 1024, 384
    rng = np.random.default_rng(8800 + 7 * dt + down_dt + m)
    gb = orc.from_float(dt, rng.normal(0, 0.02, (f, k)))
    ub = orc.from_float(dt, rng.normal(0, 0.02, (f, k)))
    db = orc.from_float(down_dt, rng.normal(0, 0.02, (n, f)))
    g, u, d = upload(gb, f, k, dt, dev), upload(ub, f, k, dt, dev), upload(db, n, f, down_dt, dev)
    x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float32)).to(dev)
    h = torch.empty((m, f), dtype=torch.float32, device=dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    mlp_t(g, u, d, m, x, h, y)
    h2 = torch.empty_like(h)
    y2 = torch.empty_like(y)
    matmul_t_silu_gate(g, u, (m, k, f), x, h2)
    d.matmul_t((m, f, n), h2, y2)
    torch.cuda.synchronize()
    assert torch.equal(h, h2), f"h differs from silu_gate, dt={dt} m={m}"
    assert torch.equal(y, y2), f"y differs from silu_gate + matmul_t, dt={dt} m={m}"
    xh = x.cpu().numpy()
    want_h = _silu(orc.matmul(dt, xh, gb, f).astype(np.float64)) * orc.matmul(dt, xh, ub, f)
    assert_close(h.cpu().numpy(), want_h, f"mlp h dt={dt} m={m}")
    assert_close(y.cpu().numpy(), orc.matmul(down_dt, h.cpu().numpy(), db, n), f"mlp y dt={dt} m={m}")
