"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for xn's quantized matmul path.

ctypes wrappers over oracle/build/liboracle.so (xnq_oracle.c: scalar
restatement of xn-core/src/quantized/k_quants.rs + utils.rs; xnq_cpu_avx2.c:
the AVX2 baseline restating avx.rs).  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "build", "liboracle.so")

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 2, 3, 6, 7, 8, 9
Q2K, Q3K, Q4K, Q5K, Q6K, Q8K = 10, 11, 12, 13, 14, 15
TYPE_SIZE = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q8_1: 36,
             Q2K: 84, Q3K: 110, Q4K: 144, Q5K: 176, Q6K: 210, Q8K: 292}
BLOCK_SIZE = {t: (32 if t <= Q8_1 else 256) for t in TYPE_SIZE}

_lib = None


def build() -> None:
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        sz, vp, i = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        for name in ("orc_from_float", "orc_to_float"):
            getattr(L, name).restype = i
            getattr(L, name).argtypes = [i, vp, vp, sz]
        L.orc_vec_dot.restype = ctypes.c_float
        L.orc_vec_dot.argtypes = [i, sz, vp, vp]
        L.orc_quantize_lhs.restype = i
        L.orc_quantize_lhs.argtypes = [i, sz, sz, vp, vp]
        L.orc_matmul_preq.restype = i
        L.orc_matmul_preq.argtypes = [i, sz, sz, sz, vp, vp, vp]
        L.orc_matmul.restype = i
        L.orc_matmul.argtypes = [i, sz, sz, sz, vp, vp, vp]
        L.orc_q4k_block_ints.argtypes = [vp, vp, vp]
        L.orc_q2k_block_ints.argtypes = [vp, vp, vp]
        L.orc_q3k_block_ints.argtypes = [vp, vp, vp, vp]
        L.orc_q5k_block_ints.argtypes = [vp, vp, vp, vp]
        L.orc_q3k_scales.argtypes = [vp, vp]
        L.orc_make_q3_quants.restype = ctypes.c_float
        L.orc_make_q3_quants.argtypes = [vp, i, i, i, vp]
        L.orc_q6k_block_ints.argtypes = [vp, vp, vp]
        L.orc_get_scale_min_k4.argtypes = [i, vp, vp]
        L.orc_q4k_unpack_scales_kmask.argtypes = [vp, vp, vp]
        L.orc_make_qkx1_quants.restype = ctypes.c_float
        L.orc_make_qkx1_quants.argtypes = [i, i, vp, i, vp]
        L.orc_make_qx_quants.restype = ctypes.c_float
        L.orc_make_qx_quants.argtypes = [i, i, vp, vp, i]
        L.orc_make_qkx1_quants_ex.restype = ctypes.c_float
        L.orc_make_qkx1_quants_ex.argtypes = [i, i, vp, i, vp, vp, vp]
        L.orc_make_qx_quants_ex.restype = ctypes.c_float
        L.orc_make_qx_quants_ex.argtypes = [i, i, vp, vp, i, vp, vp]
        L.orc_make_q3_quants_ex.restype = ctypes.c_float
        L.orc_make_q3_quants_ex.argtypes = [vp, i, i, i, vp, vp]
        L.cpu_pool_init.restype = i
        L.cpu_pool_init.argtypes = [sz]
        L.cpu_matmul.restype = i
        L.cpu_matmul.argtypes = [i, sz, sz, sz, vp, vp, vp, vp]
        L.cpu_matmul_preq.restype = i
        L.cpu_matmul_preq.argtypes = [i, sz, sz, sz, vp, vp, vp]
        for name in ("cpu_vec_dot_q4_0", "cpu_vec_dot_q8_0", "cpu_vec_dot_q4k", "cpu_vec_dot_q6k"):
            getattr(L, name).restype = ctypes.c_float
            getattr(L, name).argtypes = [sz, vp, vp]
        _lib = L
    return _lib


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def nbytes(dt: int, nelem: int) -> int:
    return nelem // BLOCK_SIZE[dt] * TYPE_SIZE[dt]


def vec_dot_type(dt: int) -> int:
    """k_quants.rs: the VecDotType of each weight type."""
    if dt in (Q4_0, Q5_0, Q8_0):
        return Q8_0
    if dt in (Q4_1, Q5_1):
        return Q8_1
    return Q8K


def from_float(dt: int, x) -> np.ndarray:
    """GgmlType::from_float -> canonical block bytes (uint8)."""
    x = _f32(x).reshape(-1)
    out = np.zeros(nbytes(dt, x.size), dtype=np.uint8)
    assert lib().orc_from_float(dt, x.ctypes.data, out.ctypes.data, x.size // BLOCK_SIZE[dt]) == 0
    return out


def to_float(dt: int, blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = blocks.size // TYPE_SIZE[dt]
    out = np.zeros(nb * BLOCK_SIZE[dt], dtype=np.float32)
    assert lib().orc_to_float(dt, blocks.ctypes.data, out.ctypes.data, nb) == 0
    return out


def vec_dot(dt: int, k: int, w_row: np.ndarray, a_row: np.ndarray) -> float:
    return lib().orc_vec_dot(dt, k, w_row.ctypes.data, a_row.ctypes.data)


def quantize_lhs(dt: int, lhs) -> np.ndarray:
    lhs = _f32(lhs)
    m, k = lhs.shape
    vt = vec_dot_type(dt)
    out = np.zeros(m * nbytes(vt, k), dtype=np.uint8)
    assert lib().orc_quantize_lhs(dt, m, k, lhs.ctypes.data, out.ctypes.data) == 0
    return out


def matmul(dt: int, lhs, w_blocks: np.ndarray, n: int) -> np.ndarray:
    """k_quants::matmul: (m, k) f32 x W[n, k]^T -> (m, n) f32 (scalar vec_dot_unopt path)."""
    lhs = _f32(lhs)
    m, k = lhs.shape
    w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    dst = np.zeros((m, n), dtype=np.float32)
    assert lib().orc_matmul(dt, m, k, n, lhs.ctypes.data, w_blocks.ctypes.data, dst.ctypes.data) == 0
    return dst


def matmul_preq(dt: int, lhs_blocks: np.ndarray, w_blocks: np.ndarray, m: int, k: int, n: int) -> np.ndarray:
    dst = np.zeros((m, n), dtype=np.float32)
    assert lib().orc_matmul_preq(dt, m, k, n, lhs_blocks.ctypes.data, w_blocks.ctypes.data,
                                 dst.ctypes.data) == 0
    return dst


def block_ints(dt: int, w_blocks: np.ndarray, a_blocks: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    """int64 [m, n, nb, 2]: the integer parts of every block dot, as the CPU
    vec_dot forms them (the K types through orc_q*k_block_ints; the 32-element
    types as their block integer sums, restated here)."""
    bs = BLOCK_SIZE[dt]
    nb = k // bs
    vt = vec_dot_type(dt)
    out = np.zeros((m, n, nb, 2), dtype=np.int64)
    wv = w_blocks.reshape(n, nb, TYPE_SIZE[dt])
    if dt in (Q2K, Q3K, Q4K, Q5K, Q6K):
        av = a_blocks.reshape(m, nb, TYPE_SIZE[vt])
        L = lib()
        fn = {Q2K: L.orc_q2k_block_ints, Q4K: L.orc_q4k_block_ints, Q6K: L.orc_q6k_block_ints,
              Q3K: lambda w, a, o: L.orc_q3k_block_ints(w, a, o, None),
              Q5K: lambda w, a, o: L.orc_q5k_block_ints(w, a, o, None)}[dt]
        tmp = np.zeros(2, dtype=np.int64)
        for r in range(m):
            for c in range(n):
                for b in range(nb):
                    wb = np.ascontiguousarray(wv[c, b])
                    ab = np.ascontiguousarray(av[r, b])
                    tmp[:] = 0
                    fn(wb.ctypes.data, ab.ctypes.data, tmp.ctypes.data)
                    out[r, c, b] = tmp
        return out
    if dt in (Q4_1, Q5_0, Q5_1):
        # k_quants.rs:316-343 / 419-440 / 513-544: sum_i q_i * a_i per 32-block,
        # q from the nibble (and Q5's fifth bit qh >> i), Q5_0 offset by -16
        vb = TYPE_SIZE[vt]  # Q8_1 (36 B: d, s, qs) or Q8_0 (34 B: d, qs)
        aq = a_blocks.reshape(m, nb, vb)[:, :, vb - 32:].view(np.int8).astype(np.int64)
        ts = TYPE_SIZE[dt]
        qs_off = {Q4_1: 4, Q5_0: 6, Q5_1: 8}[dt]
        qs = wv[:, :, qs_off:qs_off + 16].astype(np.int64)
        wq = np.concatenate([qs & 0xF, qs >> 4], axis=2)
        if dt != Q4_1:
            qh_off = 2 if dt == Q5_0 else 4
            qh = wv[:, :, qh_off:qh_off + 4].copy().view(np.uint32)[:, :, 0].astype(np.int64)
            wq = wq | (((qh[:, :, None] >> np.arange(32)[None, None, :]) & 1) << 4)
            if dt == Q5_0:
                wq = wq - 16
        assert ts == wv.shape[2]
        out[..., 0] = np.einsum("mbe,nbe->mnb", aq, wq)
        return out
    # Q4_0 / Q8_0: integer block sums, vectorised
    av = a_blocks.reshape(m, nb, 34)
    aq = av[:, :, 2:].view(np.int8).astype(np.int64)  # [m, nb, 32]
    if dt == Q8_0:
        wq = wv[:, :, 2:].view(np.int8).astype(np.int64)
    else:
        qs = wv[:, :, 2:].astype(np.int64)
        wq = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], axis=2)
    out[..., 0] = np.einsum("mbe,nbe->mnb", aq, wq)
    return out


def make_qkx1_quants(nmax: int, ntry: int, x) -> tuple:
    """utils.rs:205-254 -> (scale, -min, levels of the last pass,
    passes run, iscale and min that pass assigned the levels with)."""
    x = _f32(x).reshape(-1)
    nm = np.zeros(1, np.float32)
    lv = np.zeros(x.size, np.uint8)
    info = np.zeros(3, np.float32)
    s = lib().orc_make_qkx1_quants_ex(nmax, ntry, x.ctypes.data, x.size, nm.ctypes.data, lv.ctypes.data,
                                      info.ctypes.data)
    return np.float32(s), nm[0], lv, int(info[0]), info[1], info[2]


def make_qx_quants(nmax: int, x, rmse_type: int, mid: bool = False) -> tuple:
    """utils.rs:65-202 -> (scale, levels (stored, 0..2*nmax-1), info:
    [whole-block passes, per-element passes, changes in the last pass,
    whole-block passes kept]) and, with mid, the stored levels the
    whole-block loop left."""
    x = _f32(x).reshape(-1)
    ls = np.zeros(x.size, np.int8)
    ls_mid = np.zeros(x.size, np.int8)
    info = np.zeros(4, np.int32)
    s = lib().orc_make_qx_quants_ex(x.size, nmax, x.ctypes.data, ls.ctypes.data, rmse_type, info.ctypes.data,
                                    ls_mid.ctypes.data)
    return (np.float32(s), ls, info, ls_mid) if mid else (np.float32(s), ls, info)


def make_q3_quants(nmax: int, x, do_rmse: bool) -> tuple:
    """utils.rs:257-322 -> (scale, levels (stored, 0..2*nmax-1), info:
    [per-element passes, changes in the last pass])."""
    x = _f32(x).reshape(-1)
    ls = np.zeros(x.size, np.int8)
    info = np.zeros(2, np.int32)
    s = lib().orc_make_q3_quants_ex(x.ctypes.data, x.size, nmax, int(do_rmse), ls.ctypes.data, info.ctypes.data)
    return np.float32(s), ls, info


def cpu_pool_init(threads: int) -> int:
    return lib().cpu_pool_init(threads)


def cpu_matmul(dt: int, lhs: np.ndarray, w_blocks: np.ndarray, n: int, scratch: np.ndarray | None = None) -> np.ndarray:
    """The AVX2 baseline: serial quantize_lhs then the threaded kernel."""
    lhs = _f32(lhs)
    m, k = lhs.shape
    if scratch is None:
        scratch = np.zeros(m * nbytes(vec_dot_type(dt), k), dtype=np.uint8)
    dst = np.zeros((m, n), dtype=np.float32)
    assert lib().cpu_matmul(dt, m, k, n, lhs.ctypes.data, w_blocks.ctypes.data, dst.ctypes.data,
                            scratch.ctypes.data) == 0
    return dst


def cpu_matmul_preq(dt: int, lhs_blocks: np.ndarray, w_blocks: np.ndarray, m: int, k: int, n: int) -> np.ndarray:
    """The AVX2 baseline on an already-quantized lhs (threaded kernel only)."""
    dst = np.zeros((m, n), dtype=np.float32)
    assert lib().cpu_matmul_preq(dt, m, k, n, lhs_blocks.ctypes.data, w_blocks.ctypes.data,
                                 dst.ctypes.data) == 0
    return dst


def f32_to_f16_bits(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def f16_bits_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)
