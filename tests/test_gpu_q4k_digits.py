"""The Q4_K digit planes and min term of the int8-MFMA kernels at the
corners of their range.

The skinny, prefill and tiled kernels split each 6-bit sub-block scale as
sc = 8 * sh + sl and contract the digits sh * q and sl * q (each <= 105)
as int8 planes; the min term dmin * m_j * bsum_j runs on the bf16 matrix
cores with f32 operands split into bf16 high + remainder.  Blocks here are
built from the extreme scales, mins and levels, and every activation row
is one-hot, so each output is a single product:
  main term (dmin = 0):   d_a * d * sc * q * 127         (exact: 1e-6)
  min term (sc = 0):     -d_a * dmin * m * 127           (the bf16 split's
                                                          ~16 bits: 1e-4)
Reference semantics: BlockQ4K::vec_dot (k_quants.rs:1324-1416) through
k_quants::matmul (k_quants.rs:1996-2011); the oracle's matmul is the check.
"""
import numpy as np
import pytest
import torch

from tests import _formats as F

pytestmark = pytest.mark.gpu

Q4K = 12
SC_EXT = [0, 1, 7, 8, 9, 55, 56, 62, 63]
Q_EXT = [0, 1, 7, 8, 14, 15]
D_BITS = [0x3C00, 0x3800]  # f16 1.0 and 0.5, alternating by super-block


def crafted_weights(n: int, k: int, main: bool) -> np.ndarray:
    nb = k // 256
    blocks = []
    for c in range(n):
        for b in range(nb):
            ext = [SC_EXT[(c + 3 * b + j) % len(SC_EXT)] for j in range(8)]
            q = [Q_EXT[(7 * c + 5 * b + i) % len(Q_EXT)] for i in range(256)]
            if main:   # scales at the extremes, no min term
                blocks.append(F.encode_q4k(D_BITS[b % 2], 0, ext, [0] * 8, q))
            else:      # mins at the extremes, no main term
                blocks.append(F.encode_q4k(D_BITS[b % 2], D_BITS[(b + 1) % 2], [0] * 8, ext, q))
    return np.stack(blocks).reshape(n, nb * 144)


def one_hot_rows(m: int, k: int) -> np.ndarray:
    x = np.zeros((m, k), dtype=np.float32)
    for r in range(m):
        p = (37 * r + 5) % k  # spread over super-blocks, sub-blocks, dwords and nibbles
        x[r, p] = 1.5 if r % 2 == 0 else -0.75
    return x


# auto routes: m = 1 the fused matvec (quantize in LDS), 16 the
# wavefront-split skinny kernel, 40 and 128 the prefill kernel, 600 the
# tiled kernel; forced: 1 the matvec, 3 skinny (16- and 64-row tiles), 2
# the MFMA route
@pytest.mark.parametrize("m,route", [(1, 0), (4, 1), (16, 0), (16, 3), (16, 2), (40, 3), (40, 0), (128, 0), (600, 0)])
@pytest.mark.parametrize("term", ["main", "min"])
@pytest.mark.parametrize("k", [256, 512])
def test_q4k_digit_extremes(orc, dev, m, route, term, k):
    from xn_amd import GgmlDType, QTensor
    from xn_amd.quantized import set_route

    n = 96
    blocks = crafted_weights(n, k, term == "main")
    x = one_hot_rows(m, k)
    qt = QTensor.from_gguf_bytes(blocks, (n, k), GgmlDType(Q4K), dev)
    dst = torch.empty((m, n), dtype=torch.float32, device=dev)
    set_route(route)
    try:
        qt.matmul_t((m, k, n), torch.from_numpy(x).to(dev), dst)
    finally:
        set_route(0)
    got = dst.cpu().numpy().astype(np.float64)
    want = orc.matmul(Q4K, x, blocks, n).reshape(m, n).astype(np.float64)
    assert np.count_nonzero(want) > m * n // 2  # the crafted products are mostly nonzero
    tol = 1e-6 if term == "main" else 1e-4
    bad = np.abs(got - want) > tol * np.abs(want)
    assert not bad.any(), (
        f"m={m} route={route} term={term} k={k}: {bad.sum()} outputs off, first at {np.argwhere(bad)[0]}: "
        f"got {got[bad][0]!r} want {want[bad][0]!r}")
