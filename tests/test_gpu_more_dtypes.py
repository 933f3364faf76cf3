"""GPU parity for the remaining GGUF dtypes (Q4_1, Q5_0, Q5_1, Q2_K, Q3_K,
Q5_K; mod.rs:444-455 supports them on the CPU), through the C ABI, against
the CPU oracle (oracle/xnq_oracle_more.c): raw_data round trips,
dequantization and the integer parts of every block dot bit-exact, matmul
outputs within the path's f32 tolerance.
"""
import numpy as np
import pytest
import torch

from tests import _formats as F
from tests.test_gpu_parity import assert_close, upload

pytestmark = pytest.mark.gpu

Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K = 3, 6, 7, 10, 11, 13
MORE = [Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K]


def _blocks(orc, dt, n, k, seed):
    rng = np.random.default_rng(seed)
    return orc.from_float(dt, rng.normal(0, 0.02, (n, k)))


@pytest.mark.parametrize("dt", MORE)
def test_raw_data_round_trip(orc, dev, dt):
    """raw_data returns the GGUF bytes (mod.rs:206-214), also for arbitrary bytes."""
    n, k = 7, 1024
    blocks = _blocks(orc, dt, n, k, 9000 + dt)
    assert upload(blocks, n, k, dt, dev).data() == blocks.tobytes()
    rnd = np.random.default_rng(9100 + dt).integers(0, 256, blocks.size).astype(np.uint8)
    assert upload(rnd, n, k, dt, dev).data() == rnd.tobytes()


@pytest.mark.parametrize("dt", MORE)
def test_dequantize_bit_exact(orc, dev, dt):
    n, k = 13, 1536
    blocks = _blocks(orc, dt, n, k, 9200 + dt)
    got = upload(blocks, n, k, dt, dev).dequantize().cpu().numpy().reshape(-1)
    want = orc.to_float(dt, blocks)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dt", MORE)
def test_block_ints_bit_exact(orc, dev, dt):
    """The integer parts of every block dot the matvec kernels scale equal the
    ones brute-forced from independently decoded quants (k_quants.rs:316-343,
    419-440, 513-544, 899-948, 1071-1152, 1524-1605)."""
    from xn_amd.quantized import block_ints, lhs_workspace, quantize_lhs

    rng = np.random.default_rng(9300 + dt)
    m, n, k = 3, 21, 1024
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    ws = lhs_workspace(qt.dtype(), m, k, dev)
    quantize_lhs(qt.dtype(), torch.from_numpy(x).to(dev), ws, m, k)
    got = block_ints(qt, m, ws).cpu().numpy().astype(np.int64)
    want = F.block_ints_bruteforce(dt, blocks, orc.quantize_lhs(dt, x), m, n, k)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", MORE)
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9, 17])
@pytest.mark.parametrize("entry", ["matmul_t", "matmul_t_split"])
def test_matmul(orc, dev, dt, m, entry):
    rng = np.random.default_rng(9300 + 7 * dt + m)
    n, k = 300, 2048
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    getattr(qt, entry)((m, k, n), torch.from_numpy(x).to(dev), dst)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} m={m} {entry}")


@pytest.mark.parametrize("dt", MORE)
@pytest.mark.parametrize("k,n", [(4096, 4096), (14336, 512)])
def test_matmul_model_shapes(orc, dev, dt, k, n):
    rng = np.random.default_rng(9400 + dt + k)
    blocks = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (1, k)).astype(np.float32)
    qt = upload(blocks, n, k, dt, dev)
    dst = torch.empty((1, n), dtype=torch.float32, device=dev)
    qt.matmul_t((1, k, n), torch.from_numpy(x).to(dev), dst)
    assert_close(dst.cpu().numpy(), orc.matmul(dt, x, blocks, n), f"dt={dt} k={k} n={n}")


@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1])
def test_odd_block_count_rejected(orc, dev, dt):
    """vec_dot_q4_1_q8_1 / q5_0_q8_0 / q5_1_q8_1 bail on an odd number of
    blocks (k_quants.rs:323-325, 413-415, 519-521)."""
    from xn_amd._lib import XnqError

    k, n = 96, 8
    qt = upload(_blocks(orc, dt, n, k, 9500), n, k, dt, dev)
    x = torch.zeros((1, k), dtype=torch.float32, device=dev)
    dst = torch.empty((1, n), dtype=torch.float32, device=dev)
    with pytest.raises(XnqError, match="nb is not divisible by 2"):
        qt.matmul_t((1, k, n), x, dst)


@pytest.mark.parametrize("dt", MORE)
def test_device_weight_quantizer_bit_exact(orc, dev, dt):
    """QTensor::quantize_f32 on the device (mod.rs:283-303) writes the bytes
    xn's from_float does (k_quants.rs:345-377, 442-476, 546-583, 951-1011,
    1170-1236, 1608-1679): N(0, 0.02) rows plus a zero row, a constant row,
    an all-positive row (min clamps to 0), a ramp, single outliers and
    magnitudes near the f16 subnormal range."""
    from xn_amd import GgmlDType, QTensor

    rng = np.random.default_rng(4100 + dt)
    n, k = 24, 2048
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    w[1] = 0.0
    w[2] = 0.125
    w[3, :256] = np.linspace(-1, 1, 256, dtype=np.float32)
    w[4] = np.abs(w[4]) + 0.01
    w[5, ::37] = 0.75
    w[6] *= 1e-4
    w[7, 5] = -0.9
    qt = QTensor.quantize_f32(torch.from_numpy(w).to(dev), (n, k), GgmlDType(dt))
    assert qt.data() == orc.from_float(dt, w).tobytes()


@pytest.mark.parametrize("dt", [Q4_1, Q5K])
def test_gate_and_group(orc, dev, dt):
    from xn_amd.quantized import matmul_t_group, matmul_t_silu_gate

    rng = np.random.default_rng(9600 + dt)
    k, n = 2048, 320
    bs = [orc.from_float(dt, rng.normal(0, 0.02, (n, k))) for _ in range(3)]
    qts = [upload(b, n, k, dt, dev) for b in bs]
    x = rng.normal(0, 1, (1, k)).astype(np.float32)
    xt = torch.from_numpy(x).to(dev)
    dst = torch.empty((1, n), dtype=torch.float32, device=dev)
    matmul_t_silu_gate(qts[0], qts[1], (1, k, n), xt, dst)
    g = orc.matmul(dt, x, bs[0], n).astype(np.float64)
    want = g / (1.0 + np.exp(-g)) * orc.matmul(dt, x, bs[1], n)
    assert_close(dst.cpu().numpy(), want, f"gate dt={dt}")
    outs = [torch.empty((1, n), dtype=torch.float32, device=dev) for _ in range(3)]
    matmul_t_group(qts, 1, k, xt, outs)
    for o, b in zip(outs, bs):
        assert_close(o.cpu().numpy(), orc.matmul(dt, x, b, n), f"group dt={dt}")
