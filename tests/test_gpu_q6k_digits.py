"""The Q6_K digit planes of the int8-MFMA kernels at the corners of their
range.

The skinny and tiled kernels contract w = sc * (q - 32) as two int8 digit
planes, hi = byte 1 and lo = byte 0 (top bit flipped) of w + 128, so that
w = 256 * hi + lo.  Random quantized weights rarely reach the corners of
sc (int8) and q (6 bits), so here every block is built from the extreme
values, and every activation row is one-hot: each output is then a single
product d_a * d_w * sc * (q - 32) * 127, and any digit error larger than a
rounding shows at the 1e-6 level, far below the f32 matmul bar.  The
decode matvec (m = 1 fused, forced at m = 4), which needs no digits, is
held to the same bar.

Reference semantics: BlockQ6K::vec_dot (k_quants.rs:1724-1905) through
k_quants::matmul (k_quants.rs:1996-2011); the oracle's matmul is the check.
"""
import numpy as np
import pytest
import torch

from tests import _formats as F

pytestmark = pytest.mark.gpu

Q6K = 14
SC_EXT = [-128, -127, -64, -1, 0, 1, 63, 126, 127]
Q_EXT = [0, 1, 2, 31, 32, 33, 61, 62, 63]
D_BITS = [0x3C00, 0x3800]  # f16 1.0 and 0.5, alternating by super-block


def crafted_weights(n: int, k: int) -> np.ndarray:
    nb = k // 256
    blocks = []
    for c in range(n):
        for b in range(nb):
            sc = [SC_EXT[(c + 3 * b + s) % len(SC_EXT)] for s in range(16)]
            q = [Q_EXT[(7 * c + 5 * b + i) % len(Q_EXT)] for i in range(256)]
            blocks.append(F.encode_q6k(D_BITS[b % 2], sc, q))
    return np.stack(blocks).reshape(n, nb * 210)


def one_hot_rows(m: int, k: int) -> np.ndarray:
    x = np.zeros((m, k), dtype=np.float32)
    for r in range(m):
        p = (37 * r + 5) % k  # spread over super-blocks, sub-blocks, dwords and bytes
        x[r, p] = 1.5 if r % 2 == 0 else -0.75
    return x


@pytest.mark.parametrize("m,route", [(1, 0), (4, 1), (16, 0), (16, 3), (16, 2), (40, 3), (128, 0), (128, 2)])
@pytest.mark.parametrize("k", [256, 512])
def test_q6k_digit_extremes(orc, dev, m, route, k):
    from xn_amd import GgmlDType, QTensor
    from xn_amd.quantized import set_route

    n = 96
    blocks = crafted_weights(n, k)
    x = one_hot_rows(m, k)
    qt = QTensor.from_gguf_bytes(blocks, (n, k), GgmlDType(Q6K), dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    set_route(route)
    try:
        qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    finally:
        set_route(0)
    got = dst.cpu().numpy().astype(np.float64)
    want = orc.matmul(Q6K, x, blocks, n).reshape(m, n).astype(np.float64)
    assert np.count_nonzero(want) > m * n // 2  # the crafted products are mostly nonzero
    err = np.abs(got - want)
    bad = err > 1e-6 * np.abs(want)
    assert not bad.any(), (
        f"m={m} route={route} k={k}: {bad.sum()} outputs off, first at {np.argwhere(bad)[0]}: "
        f"got {got[bad][0]!r} want {want[bad][0]!r}")
