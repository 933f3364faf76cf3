"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored byte and value.
GPU: the device path reproduces the stored weight blocks, activation blocks
and integer block dots bit for bit, and the f32 output within the tolerance
of the quantized-matmul contract (1e-3 relative L2, 2e-3 max relative error
per row)."""
import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "golden_*.npz")))
IDS = [os.path.basename(f)[7:-4] for f in FIXTURES]


def load(path):
    with np.load(path, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def test_fixtures_present():
    assert len(FIXTURES) == 10


@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_oracle_reproduces_golden(orc, path):
    g = load(path)
    dt, m, k, n = int(g["dtype"]), int(g["m"]), int(g["k"]), int(g["n"])
    wb = orc.from_float(dt, g["w"])
    assert np.array_equal(wb, g["w_blocks"])
    ab = orc.quantize_lhs(dt, g["x"])
    assert np.array_equal(ab, g["act_blocks"])
    assert np.array_equal(orc.block_ints(dt, wb, ab, m, n, k), g["block_ints"])
    assert np.array_equal(orc.matmul(dt, g["x"], wb, n), g["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_device_matches_golden(dev, path):
    import torch

    from xn_amd import GgmlDType, QTensor
    from xn_amd.quantized import block_ints, lhs_workspace, quantize_act_blocks, quantize_lhs

    from .test_gpu_parity import assert_close

    g = load(path)
    dt, m, k, n = int(g["dtype"]), int(g["m"]), int(g["k"]), int(g["n"])
    w = torch.from_numpy(g["w"]).to(dev)
    x = torch.from_numpy(g["x"]).to(dev)
    if dt in (GgmlDType.Q4_0, GgmlDType.Q8_0, GgmlDType.Q4K, GgmlDType.Q6K):
        # device weight quantizer
        qt = QTensor.quantize_f32(w, (n, k), GgmlDType(dt))
        assert qt.data() == g["w_blocks"].tobytes()
    else:
        # no device quantizer for this dtype (xn quantizes on the host): upload
        qt = QTensor.from_gguf_bytes(g["w_blocks"], (n, k), GgmlDType(dt), dev)
        assert qt.data() == g["w_blocks"].tobytes()
    # device activation quantizer, canonical blocks
    kq = dt in (GgmlDType.Q2K, GgmlDType.Q3K, GgmlDType.Q4K, GgmlDType.Q5K, GgmlDType.Q6K)
    act = GgmlDType.Q8K if kq else GgmlDType.Q8_0
    got_ab = quantize_act_blocks(act, x, m, k).cpu().numpy()
    if dt in (GgmlDType.Q4_1, GgmlDType.Q5_1):
        # Q8_1 blocks (d, s, qs): the device's Q8_0 blocks carry the same d and qs
        want = g["act_blocks"].reshape(-1, 36)
        got = got_ab.reshape(-1, 34)
        assert np.array_equal(got[:, :2], want[:, :2]) and np.array_equal(got[:, 2:], want[:, 4:])
    else:
        assert np.array_equal(got_ab.reshape(-1), g["act_blocks"].reshape(-1))
    # integer block dots
    ws = lhs_workspace(qt.dtype(), m, k, dev)
    quantize_lhs(qt.dtype(), x, ws, m, k)
    ints = block_ints(qt, m, ws).cpu().numpy().astype(np.int64)
    assert np.array_equal(ints.reshape(g["block_ints"].shape), g["block_ints"])
    # f32 output through matmul_t
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    qt.matmul_t((m, k, n), x, dst)
    assert_close(dst.cpu().numpy(), g["y"], f"golden {path}")
