"""Pins the oracle's restatement of the remaining GGUF types (Q4_1, Q5_0,
Q5_1 with their Q8_1 activations; Q2_K, Q3_K, Q5_K; oracle/xnq_oracle_more.c)
against computations that do not share its code: independent numpy codecs
written from the block layouts (tests/_formats.py), closed forms for the
block scales, brute-force integer dots, f64 dots of dequantized operands, and
round-trip error bounds.  The reference holds no test vectors for these types
(its tests cover Q8_0 only); the exact bits of the iterative weight
quantizers (make_qkx1_quants, make_q3_quants) versus a Rust build are "parity
unpinned" and covered by round-trip bounds only.
"""
import numpy as np
import pytest

from tests import _formats as F

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 2, 3, 6, 7, 8, 9
Q2K, Q3K, Q4K, Q5K, Q6K, Q8K = 10, 11, 12, 13, 14, 15
f16 = np.float16


def _h(v):
    return np.asarray(v, np.float32).astype(f16).astype(np.float32)


# --------------------------------------------------------- Q8_1
def test_q8_1_closed_form(orc):
    """k_quants.rs:847-873: d = f16(amax / 127), q = round(x / d) saturated,
    s = f16(f16(sum q) * d) (half's f16 product rounds once)."""
    rng = np.random.default_rng(100)
    x = rng.normal(0, 1, (64, 32)).astype(np.float32)
    x[3] = 0.0
    b = orc.from_float(Q8_1, x)
    d, s, q = F.decode_q8_1(b)
    amax = np.abs(x).max(axis=1)
    dd = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(d, _h(dd))
    assert np.all(np.abs(q) <= 127)
    idd = np.where(dd != 0, np.float32(1) / np.where(dd != 0, dd, 1), 0).astype(np.float32)
    want_q = np.trunc(np.abs(x * idd[:, None]) + np.float32(0.5)) * np.sign(x * idd[:, None])
    assert np.array_equal(q, want_q.astype(np.int64))
    want_s = (_h(q.sum(axis=1).astype(np.float32)).astype(f16) * d.astype(f16)).astype(np.float32)
    assert np.array_equal(s, want_s)


# ---------------------------------------------- 32-element types
@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1])
def test_small_block_scales_closed_form(orc, dt):
    rng = np.random.default_rng(101 + dt)
    x = rng.normal(0, 0.02, (64, 32)).astype(np.float32)
    b = orc.from_float(dt, x)
    if dt == Q5_0:
        d, q = F.decode_q5_0(b)
        first = np.argmax(np.abs(x) == np.abs(x).max(axis=1, keepdims=True), axis=1)
        mx = x[np.arange(64), first]
        assert np.array_equal(d, _h(mx / np.float32(-16)))
        assert q.min() >= -16 and q.max() <= 15
    else:
        dec = F.decode_q4_1 if dt == Q4_1 else F.decode_q5_1
        d, m, q = dec(b)
        nmax = 15 if dt == Q4_1 else 31
        lo, hi = x.min(axis=1), x.max(axis=1)
        assert np.array_equal(d, _h((hi - lo) / np.float32(nmax)))
        assert np.array_equal(m, _h(lo))
        assert q.min() >= 0 and q.max() <= nmax


@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1])
def test_small_block_to_float_closed_form(orc, dt):
    """to_float against the independent decoder: y = q*d (+ m), f32."""
    rng = np.random.default_rng(110 + dt)
    b = orc.from_float(dt, rng.normal(0, 0.02, (32, 32)))
    y = orc.to_float(dt, b).reshape(32, 32)
    if dt == Q5_0:
        d, q = F.decode_q5_0(b)
        want = (q.astype(np.float32) * d[:, None]).astype(np.float32)
    else:
        d, m, q = (F.decode_q4_1 if dt == Q4_1 else F.decode_q5_1)(b)
        want = ((q.astype(np.float32) * d[:, None]).astype(np.float32) + m[:, None]).astype(np.float32)
    assert np.array_equal(y, want)


@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K])
def test_round_trip_error_bound(orc, dt):
    rng = np.random.default_rng(120 + dt)
    x = rng.normal(0, 0.02, (16, 512)).astype(np.float32)
    b = orc.from_float(dt, x)
    y = orc.to_float(dt, b).reshape(x.shape)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    # relative L2 error of the quantization: bits per weight 2.6 .. 5.5
    bound = {Q4_1: 0.12, Q5_0: 0.06, Q5_1: 0.06, Q2K: 0.45, Q3K: 0.25, Q5K: 0.06}[dt]
    assert rel < bound, rel
    if dt in (Q4_1, Q5_1):
        d, m, q = (F.decode_q4_1 if dt == Q4_1 else F.decode_q5_1)(b)
        step = np.repeat(d, 32).reshape(x.shape)
        # half a step, plus what rounding d and m to f16 moves (<= nmax * 2^-11 steps)
        assert np.all(np.abs(y - x) <= step * 0.52 + 1e-6)


# ------------------------------------------------------ K types
def test_q2k_to_float_from_encoded_fields(orc):
    rng = np.random.default_rng(130)
    blocks, want = [], []
    sc_first = q_first = None
    for _ in range(12):
        db = int(f16(rng.uniform(1e-4, 1e-2)).view(np.uint16))
        mb = int(f16(rng.uniform(1e-4, 1e-2)).view(np.uint16))
        sc, mn, q = rng.integers(0, 16, 16), rng.integers(0, 16, 16), rng.integers(0, 4, 256)
        blocks.append(F.encode_q2k(db, mb, sc, mn, q))
        if sc_first is None:
            sc_first, q_first = sc, q
        d = np.uint16(db).view(f16).astype(np.float32)
        dm = np.uint16(mb).view(f16).astype(np.float32)
        dl = (d * sc.astype(np.float32)).astype(np.float32).repeat(16)
        ml = (dm * mn.astype(np.float32)).astype(np.float32).repeat(16)
        want.append(((dl * q.astype(np.float32)).astype(np.float32) - ml).astype(np.float32))
    b = np.concatenate(blocks)
    assert np.array_equal(orc.to_float(Q2K, b), np.concatenate(want))
    d, dmin, sc2, mn2, q2 = F.decode_q2k(b[:84])
    assert np.array_equal(sc2[0], sc_first) and np.array_equal(q2[0], q_first)


def test_q3k_to_float_from_encoded_fields(orc):
    rng = np.random.default_rng(131)
    blocks, want = [], []
    for _ in range(12):
        db = int(f16(rng.uniform(-1e-2, 1e-2)).view(np.uint16))
        sc, q = rng.integers(0, 64, 16), rng.integers(-4, 4, 256)
        blk = F.encode_q3k(db, sc, q)
        blocks.append(blk)
        d = np.uint16(db).view(f16).astype(np.float32)
        dl = (d * (sc - 32).astype(np.float32)).astype(np.float32).repeat(16)
        want.append((dl * q.astype(np.float32)).astype(np.float32))
        got_sc = np.zeros(16, np.uint8)
        orc.lib().orc_q3k_scales(np.ascontiguousarray(blk[96:108]).ctypes.data, got_sc.ctypes.data)
        assert np.array_equal(got_sc, sc), "KMASK scale shuffle vs independent unpacker"
        _, dsc, dq = F.decode_q3k(blk)
        assert np.array_equal(dsc[0], sc - 32) and np.array_equal(dq[0], q)
    assert np.array_equal(orc.to_float(Q3K, np.concatenate(blocks)), np.concatenate(want))


def test_q5k_to_float_from_encoded_fields(orc):
    rng = np.random.default_rng(132)
    blocks, want = [], []
    for _ in range(12):
        db = int(f16(rng.uniform(1e-4, 1e-2)).view(np.uint16))
        mb = int(f16(rng.uniform(1e-4, 1e-2)).view(np.uint16))
        sc, mn, q = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 32, 256)
        blk = F.encode_q5k(db, mb, sc, mn, q)
        blocks.append(blk)
        d = np.uint16(db).view(f16).astype(np.float32)
        dm = np.uint16(mb).view(f16).astype(np.float32)
        d1 = (d * sc.astype(np.float32)).astype(np.float32).repeat(32)
        m1 = (dm * mn.astype(np.float32)).astype(np.float32).repeat(32)
        want.append(((d1 * q.astype(np.float32)).astype(np.float32) - m1).astype(np.float32))
        _, _, s2, m2, q2 = F.decode_q5k(blk)
        assert np.array_equal(s2[0], sc) and np.array_equal(m2[0], mn) and np.array_equal(q2[0], q)
    assert np.array_equal(orc.to_float(Q5K, np.concatenate(blocks)), np.concatenate(want))


def test_make_q3_quants_degenerate_and_grid(orc):
    x = np.zeros(16, np.float32)
    ls = np.zeros(16, np.int8)
    assert orc.lib().orc_make_q3_quants(x.ctypes.data, 16, 4, 1, ls.ctypes.data) == 0.0
    # values on the grid -4..3 times s: the quantizer recovers the grid (rmse path)
    g = np.array([-4, -3, -2, -1, 0, 1, 2, 3] * 2, np.float32)
    x = g * np.float32(0.125)
    s = orc.lib().orc_make_q3_quants(x.ctypes.data, 16, 4, 1, ls.ctypes.data)
    assert np.allclose((ls.astype(np.float32) - 4) * s, x, atol=1e-6)


@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K])
def test_kquant_block_ints_bruteforce(orc, dt):
    rng = np.random.default_rng(140 + dt)
    m, n, k = 3, 5, 512
    w = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    a = orc.quantize_lhs(dt, rng.normal(0, 1, (m, k)))
    assert np.array_equal(orc.block_ints(dt, w, a, m, n, k), F.block_ints_bruteforce(dt, w, a, m, n, k))


@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K])
def test_vec_dot_vs_dequantized_f64(orc, dt):
    """vec_dot equals the f64 dot of the dequantized operands up to f32 rounding
    (Q8_1's s enters as its f16 value, as in the reference)."""
    rng = np.random.default_rng(150 + dt)
    m, n, k = 2, 7, 1024
    w = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    a = orc.quantize_lhs(dt, x)
    wd = orc.to_float(dt, w).reshape(n, k).astype(np.float64)
    vt = orc.vec_dot_type(dt)
    if vt == Q8_1:
        # sum_b [ d_w d_a sum q_w q_a + m_w s_a ] with y = q_w d_w + m_w
        da, sa, qa = F.decode_q8_1(a)
        dec = F.decode_q4_1 if dt == Q4_1 else F.decode_q5_1
        dw, mw, qw = dec(w)
        nb = k // 32
        da, sa, qa = da.reshape(m, nb), sa.reshape(m, nb), qa.reshape(m, nb, 32)
        dw, mw, qw = dw.reshape(n, nb), mw.reshape(n, nb), qw.reshape(n, nb, 32)
        ints = np.einsum("mbe,nbe->mnb", qa, qw).astype(np.float64)
        want = (ints * dw[None] * da[:, None] + mw[None] * sa[:, None]).sum(axis=2)
        scale = (np.abs(ints) * np.abs(dw[None] * da[:, None]) + np.abs(mw[None] * sa[:, None])).sum(axis=2)
    else:
        ad = orc.to_float(vt, a).reshape(m, k).astype(np.float64)
        want = ad @ wd.T
        scale = np.abs(ad) @ np.abs(wd).T
    got = orc.matmul(dt, x, w, n)
    assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-7)


@pytest.mark.parametrize("dt", [Q4_1, Q5_0, Q5_1])
def test_odd_block_count_is_rejected(orc, dt):
    """vec_dot_q4_1_q8_1 / q5_0_q8_0 / q5_1_q8_1 bail on an odd block count
    (k_quants.rs:323-325, 413-415, 519-521)."""
    rng = np.random.default_rng(160)
    w = orc.from_float(dt, rng.normal(0, 0.02, (2, 96)))
    x = rng.normal(0, 1, (1, 96)).astype(np.float32)
    with pytest.raises(AssertionError):
        orc.matmul(dt, x, w, 2)
