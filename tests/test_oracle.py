"""Pins the CPU oracle (oracle/xnq_oracle.c) before anything is compared with it.

Each oracle function is checked against something that does not share its
code: numpy's IEEE float16, the reference's own known-answer test
(k_quants.rs:2151-2210), integer brute force over decoded blocks, an
independent encoder of the block formats (tests/_formats.py), closed forms and
quantizer invariants.  The one thing none of these fixes is the exact bit
pattern of the iterative weight quantizers (make_qkx1_quants, make_qx_quants)
versus a Rust build -- "parity unpinned" for those bits; they are covered by
round-trip error bounds, and the device quantizer is held byte-equal to them.
"""
import numpy as np
import pytest

from tests import _formats as F

Q4_0, Q8_0, Q4K, Q6K, Q8K = 2, 8, 12, 14, 15


# --------------------------------------------------------------- f16
def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([orc.f16_bits_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.all(np.isinf(got[np.isinf(want)]))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(1)
    # random bit patterns over the whole f16 range incl. subnormals, plus exact ties
    ex = rng.integers(90, 160, size=20000)
    man = rng.integers(0, 1 << 23, size=20000)
    bits = ((ex << 23) | man).astype(np.uint32)
    sign = rng.integers(0, 2, size=20000).astype(np.uint32) << 31
    xs = (bits | sign).view(np.float32)
    h = np.arange(0, 0x7bff, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    ties = ((h[:-1] + h[1:]) / 2).astype(np.float32)  # exact midpoints are representable in f32
    xs = np.concatenate([xs, ties, -ties, np.float32([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8])])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16_bits(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------ the reference's own known-answer test
@pytest.mark.parametrize("m,k,n", [(1, 256, 64), (4, 128, 32), (7, 96, 12)])
def test_q8_0_matmul_matches_reference(orc, m, k, n):
    """k_quants.rs:2151-2210 q8_0_matmul_matches_reference_at_every_pool_size:
    deterministic weights ((i*37 % 211) - 105)/64, lhs ((i*53 % 173) - 86)/32,
    f64 dot of the quantized operands, tolerance 1e-4 * max(|want|, 1)."""
    raw = ((np.arange(n * k) * 37 % 211).astype(np.float32) - 105.0) / 64.0
    w = orc.from_float(Q8_0, raw)
    lhs = (((np.arange(m * k) * 53 % 173).astype(np.float32) - 86.0) / 32.0).reshape(m, k)
    a = orc.quantize_lhs(Q8_0, lhs)
    dw, qw = F.decode_q8_0(w)
    da, qa = F.decode_q8_0(a)
    kb = k // 32
    want = np.zeros((m, n))
    for r in range(m):
        for c in range(n):
            s = (qa[r * kb:(r + 1) * kb] * qw[c * kb:(c + 1) * kb]).sum(axis=1)
            want[r, c] = np.sum(s * da[r * kb:(r + 1) * kb].astype(np.float64) * dw[c * kb:(c + 1) * kb].astype(np.float64))
    for got in (orc.matmul(Q8_0, lhs, w, n), orc.cpu_matmul(Q8_0, lhs, w, n)):
        tol = 1e-4 * np.maximum(np.abs(want), 1.0)
        assert np.all(np.abs(got - want) <= tol)


# ---------------------------------------------------------- quantizers
def test_q8_0_quantizer_invariants(orc):
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (64, 32)).astype(np.float32)
    x[3] = 0.0
    b = orc.from_float(Q8_0, x)
    d, q = F.decode_q8_0(b)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.all(np.abs(q) <= 127)
    live = amax > 0
    # the largest |x| maps to +-127, and dequantization is within half a step
    idx = np.abs(x).argmax(axis=1)
    assert np.all(np.abs(q[np.arange(64), idx])[live] == 127)
    dd = amax / np.float32(127)
    assert np.all(np.abs(q * dd[:, None] - x)[live] <= dd[live, None] * 0.5 + 1e-6)
    assert np.all(q[3] == 0) and d[3] == 0


def test_q8k_quantizer_invariants(orc):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (16, 256)).astype(np.float32)
    x[2] = 0.0
    x[5, 10], x[5, 200] = -7.0, 7.0  # tie: the first one sets the sign
    b = orc.from_float(Q8K, x)
    d, q, bs = F.decode_q8k(b)
    assert np.array_equal(bs, q.reshape(16, 16, 16).sum(axis=2))
    assert np.all(q <= 127) and np.all(q >= -128)
    for r in range(16):
        if r == 2:
            assert d[r] == 0 and np.all(q[r] == 0)
            continue
        i = np.abs(x[r]).argmax()  # first index of the largest |x|
        assert q[r, i] == -128
        iscale = np.float32(-128.0) / x[r, i]
        assert d[r] == np.float32(1.0) / iscale
        ok = iscale * x[r] < np.float32(127.5)  # elements clamped to 127 are a full step off
        err = np.abs(q[r] * d[r] - x[r])[ok]
        assert np.all(err <= abs(d[r]) * 0.5 + 1e-6 * np.abs(x[r]).max())
    assert q[5, 10] == -128 and q[5, 200] == 127  # 7 * (-128 / -7) = 128 -> min(.,127)


def test_q4_0_quantizer_invariants(orc):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 0.02, (64, 32)).astype(np.float32)
    b = orc.from_float(Q4_0, x)
    d, q = F.decode_q4_0(b)
    # d = max / -8 where max is the signed value of largest |x|
    mx = x[np.arange(64), np.abs(x).argmax(axis=1)]
    assert np.array_equal(d, (mx / np.float32(-8)).astype(np.float16).astype(np.float32))
    assert np.all(np.abs(q * d[:, None] - x) <= np.abs(d)[:, None] * 1.0 + 1e-7)


@pytest.mark.parametrize("dt,tol_steps", [(Q4K, 1.0), (Q6K, 1.0)])
def test_kquant_round_trip(orc, dt, tol_steps):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 0.02, (32, 256)).astype(np.float32)
    b = orc.from_float(dt, x)
    y = orc.to_float(dt, b).reshape(x.shape)
    if dt == Q4K:
        d, dmin, sc, mn, q = F.decode_q4k(b)
        step = (d[:, None] * sc).repeat(32, axis=1)
    else:
        d, sc, q = F.decode_q6k(b)
        step = np.abs(d[:, None] * sc).repeat(16, axis=1)
    assert np.all(np.abs(y - x) <= tol_steps * step + 1e-6)
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < (0.12 if dt == Q4K else 0.03)


def test_make_qkx1_degenerate(orc):
    import ctypes
    x = np.full(32, 0.25, dtype=np.float32)
    nm = np.zeros(1, dtype=np.float32)
    s = orc.lib().orc_make_qkx1_quants(15, 5, x.ctypes.data, 32, nm.ctypes.data)
    assert s == 0.0 and nm[0] == 0.0
    # exactly representable ramp 0..15 * 0.5: scale 0.5, min 0
    x = (np.arange(32) % 16).astype(np.float32) * np.float32(0.5)
    s = orc.lib().orc_make_qkx1_quants(15, 5, x.ctypes.data, 32, nm.ctypes.data)
    assert s == np.float32(0.5) and nm[0] == 0.0
    del ctypes


def test_make_qx_quants_exact_grid(orc):
    # values on an integer grid -31..31 times s quantize to that grid with scale s
    x = (np.array(list(range(-8, 8)), dtype=np.float32) * np.float32(0.25))
    x[0] = -8 * 0.25
    ls = np.zeros(16, dtype=np.int8)
    s = orc.lib().orc_make_qx_quants(16, 32, x.ctypes.data, ls.ctypes.data, 1)
    assert np.allclose((ls.astype(np.float32) - 32) * s, x, atol=1e-6)


# ------------------------------------------------------- format decoding
def test_get_scale_min_two_forms(orc):
    """get_scale_min_k4 (utils.rs:53-63) and the KMASK unpacking
    (k_quants.rs:1375-1385) agree with the independent unpacker on random bytes."""
    rng = np.random.default_rng(6)
    for _ in range(500):
        b12 = rng.integers(0, 256, 12).astype(np.uint8)
        sc, mn = F.unpack_scales_k4(b12)
        s8 = np.zeros(8, np.uint8)
        m8 = np.zeros(8, np.uint8)
        orc.lib().orc_q4k_unpack_scales_kmask(b12.ctypes.data, s8.ctypes.data, m8.ctypes.data)
        assert np.array_equal(s8, sc) and np.array_equal(m8, mn)
        out2 = np.zeros(2, np.uint8)
        for j in range(8):
            orc.lib().orc_get_scale_min_k4(j, b12.ctypes.data, out2.ctypes.data)
            assert out2[0] == sc[j] and out2[1] == mn[j]
        # and the packer inverts the unpacker
        assert np.array_equal(F.pack_scales_k4(sc, mn), b12)


def test_q4k_to_float_from_encoded_fields(orc):
    rng = np.random.default_rng(7)
    blocks, want = [], []
    for _ in range(16):
        dbits = int(np.float16(rng.uniform(1e-4, 1e-2)).view(np.uint16))
        mbits = int(np.float16(rng.uniform(1e-4, 1e-2)).view(np.uint16))
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        blocks.append(F.encode_q4k(dbits, mbits, sc, mn, q))
        d = np.uint16(dbits).view(np.float16).astype(np.float32)
        dm = np.uint16(mbits).view(np.float16).astype(np.float32)
        # y = (d*sc)*q - (dmin*m), each product rounded to f32
        d1 = (d * sc.astype(np.float32)).astype(np.float32).repeat(32)
        m1 = (dm * mn.astype(np.float32)).astype(np.float32).repeat(32)
        want.append((d1 * q.astype(np.float32)).astype(np.float32) - m1)
    got = orc.to_float(Q4K, np.concatenate(blocks))
    assert np.array_equal(got, np.concatenate(want).astype(np.float32))


def test_q6k_to_float_from_encoded_fields(orc):
    rng = np.random.default_rng(8)
    blocks, want = [], []
    for _ in range(16):
        dbits = int(np.float16(rng.uniform(-1e-3, 1e-3)).view(np.uint16))
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, 256)
        blocks.append(F.encode_q6k(dbits, sc, q))
        d = np.uint16(dbits).view(np.float16).astype(np.float32)
        ds = (d * sc.astype(np.float32)).astype(np.float32).repeat(16)
        want.append((ds * (q - 32).astype(np.float32)).astype(np.float32))
    got = orc.to_float(Q6K, np.concatenate(blocks))
    assert np.array_equal(got, np.concatenate(want))


def test_q4_0_q8_0_to_float_closed_form(orc):
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (8, 32)).astype(np.float32)
    for dt, dec in ((Q4_0, F.decode_q4_0), (Q8_0, F.decode_q8_0)):
        b = orc.from_float(dt, x)
        d, q = dec(b)
        assert np.array_equal(orc.to_float(dt, b).reshape(8, 32), (q.astype(np.float32) * d[:, None]).astype(np.float32))


# -------------------------------------------------------- integer dots
@pytest.mark.parametrize("dt,k", [(Q4_0, 256), (Q8_0, 256), (Q4K, 512), (Q6K, 512)])
def test_block_ints_bruteforce(orc, dt, k):
    rng = np.random.default_rng(10 + dt)
    m, n = 3, 5
    w = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    a = orc.quantize_lhs(dt, rng.normal(0, 1, (m, k)))
    got = orc.block_ints(dt, w, a, m, n, k)
    want = F.block_ints_bruteforce(dt, w, a, m, n, k)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt,k", [(Q4_0, 512), (Q8_0, 512), (Q4K, 1024), (Q6K, 1024)])
def test_vec_dot_vs_dequantized_f64(orc, dt, k):
    """vec_dot equals the f64 dot of the dequantized operands up to f32 rounding."""
    rng = np.random.default_rng(20 + dt)
    m, n = 2, 7
    w = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    a = orc.quantize_lhs(dt, x)
    wd = orc.to_float(dt, w).reshape(n, k).astype(np.float64)
    ad = orc.to_float(orc.vec_dot_type(dt), a).reshape(m, k).astype(np.float64)
    want = ad @ wd.T
    got = orc.matmul(dt, x, w, n)
    scale = np.abs(ad) @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-7)


@pytest.mark.parametrize("dt", [Q4_0, Q8_0, Q4K, Q6K])
def test_avx2_baseline_agrees(orc, dt):
    rng = np.random.default_rng(30 + dt)
    m, k, n = 3, 1024, 300
    w = orc.from_float(dt, rng.normal(0, 0.02, (n, k)))
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    orc.cpu_pool_init(4)
    got = orc.cpu_matmul(dt, x, w, n)
    want = orc.matmul(dt, x, w, n)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())
