"""Independent numpy codecs of the GGUF block formats, written from the format
description (k_quants.rs:92-205 struct layouts; the bit layouts of
utils.rs:53-63 and k_quants.rs:1759-1771), used to check the oracle and the
device kernels from a second direction: these pack known integers into
bytes and unpack bytes into integers, whereas the oracle quantizes floats.
"""
from __future__ import annotations

import numpy as np

F16 = np.float16


def _f16_from_bits(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(F16).astype(np.float32)


# ----------------------------------------------------------------- Q8_0
def decode_q8_0(blocks: np.ndarray):
    """-> d f32 [nb], q int64 [nb, 32]"""
    b = blocks.reshape(-1, 34)
    d = _f16_from_bits(b[:, 0:2].copy().view(np.uint16)[:, 0])
    q = b[:, 2:].view(np.int8).astype(np.int64)
    return d, q


# ----------------------------------------------------------------- Q4_0
def decode_q4_0(blocks: np.ndarray):
    """-> d f32 [nb], q int64 [nb, 32] in -8..7"""
    b = blocks.reshape(-1, 18)
    d = _f16_from_bits(b[:, 0:2].copy().view(np.uint16)[:, 0])
    qs = b[:, 2:].astype(np.int64)
    q = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], axis=1)
    return d, q


# ----------------------------------------------------------------- Q8_K
def decode_q8k(blocks: np.ndarray):
    """-> d f32 [nb], q int64 [nb, 256], bsums int64 [nb, 16]"""
    b = blocks.reshape(-1, 292)
    d = b[:, 0:4].copy().view(np.float32)[:, 0]
    q = b[:, 4:260].view(np.int8).astype(np.int64)
    bs = b[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, q, bs


# ----------------------------------------------------------------- Q4_K
def pack_scales_k4(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """8 six-bit scales and mins -> the 12 packed bytes.
    Bytes 0-3: sc[0..4] low 6 bits, top 2 bits carry sc[4..8] >> 4.
    Bytes 4-7: mn[0..4] low 6 bits, top 2 bits carry mn[4..8] >> 4.
    Bytes 8-11: low nibble sc[4..8] & 15, high nibble mn[4..8] & 15."""
    out = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return out


def unpack_scales_k4(b12: np.ndarray):
    sc = np.zeros(8, dtype=np.int64)
    mn = np.zeros(8, dtype=np.int64)
    b = b12.astype(np.int64)
    for j in range(4):
        sc[j] = b[j] & 63
        mn[j] = b[j + 4] & 63
        sc[j + 4] = (b[j + 8] & 15) | ((b[j] >> 6) << 4)
        mn[j + 4] = (b[j + 8] >> 4) | ((b[j + 4] >> 6) << 4)
    return sc, mn


def encode_q4k(d_bits: int, dmin_bits: int, sc, mn, q) -> np.ndarray:
    """One BlockQ4K from integer fields: q[256] in 0..15 in element order.
    qs byte 32*p + l holds element 64p+l (low nibble) and 64p+32+l (high)."""
    q = np.asarray(q, dtype=np.int64)
    out = np.zeros(144, dtype=np.uint8)
    out[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    out[2:4] = np.array([dmin_bits], dtype=np.uint16).view(np.uint8)
    out[4:16] = pack_scales_k4(np.asarray(sc, np.int64), np.asarray(mn, np.int64))
    for p in range(4):
        for l in range(32):
            out[16 + 32 * p + l] = q[64 * p + l] | (q[64 * p + 32 + l] << 4)
    return out


def decode_q4k(blocks: np.ndarray):
    """-> d, dmin f32 [nb]; sc, mn int64 [nb, 8]; q int64 [nb, 256] in 0..15"""
    b = blocks.reshape(-1, 144)
    nb = b.shape[0]
    d = _f16_from_bits(b[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = _f16_from_bits(b[:, 2:4].copy().view(np.uint16)[:, 0])
    sc = np.zeros((nb, 8), np.int64)
    mn = np.zeros((nb, 8), np.int64)
    for i in range(nb):
        sc[i], mn[i] = unpack_scales_k4(b[i, 4:16])
    qs = b[:, 16:].astype(np.int64).reshape(nb, 4, 32)
    q = np.concatenate([np.stack([qs[:, p] & 0xF, qs[:, p] >> 4], axis=1) for p in range(4)], axis=1)
    return d, dmin, sc, mn, q.reshape(nb, 256)


# ----------------------------------------------------------------- Q6_K
def encode_q6k(d_bits: int, sc, q) -> np.ndarray:
    """One BlockQ6K: q[256] in 0..63 (value + 32), sc[16] int8.
    For half h, l < 32: ql[64h+l] = q(128h+l) | q(128h+64+l) << 4 (low 4 bits),
    ql[64h+32+l] = q(128h+32+l) | q(128h+96+l) << 4, qh[32h+l] packs the top
    2 bits of q(128h+l), q(+32), q(+64), q(+96) at bits 0, 2, 4, 6."""
    q = np.asarray(q, dtype=np.int64)
    out = np.zeros(210, dtype=np.uint8)
    for h in range(2):
        for l in range(32):
            e = 128 * h + l
            out[64 * h + l] = (q[e] & 15) | ((q[e + 64] & 15) << 4)
            out[64 * h + 32 + l] = (q[e + 32] & 15) | ((q[e + 96] & 15) << 4)
            out[128 + 32 * h + l] = (q[e] >> 4) | ((q[e + 32] >> 4) << 2) | ((q[e + 64] >> 4) << 4) | (
                (q[e + 96] >> 4) << 6)
    out[192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    out[208:210] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    return out


def decode_q6k(blocks: np.ndarray):
    """-> d f32 [nb], sc int64 [nb, 16], q int64 [nb, 256] in -32..31"""
    b = blocks.reshape(-1, 210)
    nb = b.shape[0]
    ql = b[:, :128].astype(np.int64)
    qh = b[:, 128:192].astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = _f16_from_bits(b[:, 208:210].copy().view(np.uint16)[:, 0])
    q = np.zeros((nb, 256), np.int64)
    for h in range(2):
        for l in range(32):
            e = 128 * h + l
            lo0, lo1 = ql[:, 64 * h + l], ql[:, 64 * h + 32 + l]
            hb = qh[:, 32 * h + l]
            q[:, e] = (lo0 & 15) | ((hb & 3) << 4)
            q[:, e + 32] = (lo1 & 15) | (((hb >> 2) & 3) << 4)
            q[:, e + 64] = (lo0 >> 4) | (((hb >> 4) & 3) << 4)
            q[:, e + 96] = (lo1 >> 4) | (((hb >> 6) & 3) << 4)
    return d, sc, q - 32


# ------------------------------------------------- brute-force integer dots
def block_ints_bruteforce(dt: int, w_blocks: np.ndarray, a_blocks: np.ndarray, m: int, n: int, k: int):
    """int64 [m, n, nb, 2] from decoded integers (see xnq.h block_ints).

    a_blocks are the weight type's vec-dot blocks: Q8_0 for Q4_0, Q8_0 and
    Q5_0, Q8_1 for Q4_1 and Q5_1, Q8_K for the K types."""
    if dt in (3, 6, 7):  # Q4_1, Q5_0, Q5_1: [sum q*a, 0] per 32-block
        nb = k // 32
        qa = (decode_q8_0(a_blocks)[1] if dt == 6 else decode_q8_1(a_blocks)[2]).reshape(m, nb, 32)
        qw = {3: lambda b: decode_q4_1(b)[2], 6: lambda b: decode_q5_0(b)[1],
              7: lambda b: decode_q5_1(b)[2]}[dt](w_blocks).reshape(n, nb, 32)
        out = np.zeros((m, n, nb, 2), np.int64)
        out[..., 0] = np.einsum("mbe,nbe->mnb", qa, qw)
        return out
    if dt in (10, 11, 13):  # Q2K, Q3K, Q5K
        nb = k // 256
        _, qa, bsums = decode_q8k(a_blocks)
        qa = qa.reshape(m, nb, 256)
        bsums = bsums.reshape(m, nb, 16)
        out = np.zeros((m, n, nb, 2), np.int64)
        if dt == 10:
            _, _, sc, mn, q = decode_q2k(w_blocks)
            sc, mn, q = sc.reshape(n, nb, 16), mn.reshape(n, nb, 16), q.reshape(n, nb, 16, 16)
            sub = np.einsum("mbge,nbge->mnbg", qa.reshape(m, nb, 16, 16), q)
            out[..., 0] = np.einsum("mnbg,nbg->mnb", sub, sc)
            out[..., 1] = np.einsum("mbg,nbg->mnb", bsums, mn)
        elif dt == 11:
            _, sc, q = decode_q3k(w_blocks)
            sc, q = sc.reshape(n, nb, 16), q.reshape(n, nb, 16, 16)
            sub = np.einsum("mbge,nbge->mnbg", qa.reshape(m, nb, 16, 16), q)
            out[..., 0] = np.einsum("mnbg,nbg->mnb", sub, sc)
        else:
            _, _, sc, mn, q = decode_q5k(w_blocks)
            sc, mn, q = sc.reshape(n, nb, 8), mn.reshape(n, nb, 8), q.reshape(n, nb, 8, 32)
            sub = np.einsum("mbje,nbje->mnbj", qa.reshape(m, nb, 8, 32), q)
            out[..., 0] = np.einsum("mnbj,nbj->mnb", sub, sc)
            s32 = bsums.reshape(m, nb, 8, 2).sum(axis=3)
            out[..., 1] = np.einsum("mbj,nbj->mnb", s32, mn)
        return out
    if dt in (2, 8):
        nb = k // 32
        da, qa = decode_q8_0(a_blocks)
        qa = qa.reshape(m, nb, 32)
        _, qw = (decode_q8_0 if dt == 8 else decode_q4_0)(w_blocks)
        qw = qw.reshape(n, nb, 32)
        out = np.zeros((m, n, nb, 2), np.int64)
        out[..., 0] = np.einsum("mbe,nbe->mnb", qa, qw)
        return out
    nb = k // 256
    _, qa, bsums = decode_q8k(a_blocks)
    qa = qa.reshape(m, nb, 256)
    out = np.zeros((m, n, nb, 2), np.int64)
    if dt == 12:
        _, _, sc, mn, q = decode_q4k(w_blocks)
        sc = sc.reshape(n, nb, 8)
        mn = mn.reshape(n, nb, 8)
        q = q.reshape(n, nb, 8, 32)
        qa8 = qa.reshape(m, nb, 8, 32)
        sub = np.einsum("mbje,nbje->mnbj", qa8, q)  # per sub-block integer dots
        out[..., 0] = np.einsum("mnbj,nbj->mnb", sub, sc)
        s32 = qa8.sum(axis=3)  # [m, nb, 8]
        out[..., 1] = np.einsum("mbj,nbj->mnb", s32, mn)
    else:
        _, sc, q = decode_q6k(w_blocks)
        sc = sc.reshape(n, nb, 16)
        q = q.reshape(n, nb, 16, 16)
        qa16 = qa.reshape(m, nb, 16, 16)
        sub = np.einsum("mbje,nbje->mnbj", qa16, q)
        out[..., 0] = np.einsum("mnbj,nbj->mnb", sub, sc)
    return out


# --------------------------------------------- Q4_1, Q5_0, Q5_1, Q8_1
def _f16_field(b: np.ndarray, off: int) -> np.ndarray:
    return _f16_from_bits(b[:, off:off + 2].copy().view(np.uint16)[:, 0])


def decode_q4_1(blocks: np.ndarray):
    """-> d, m f32 [nb], q int64 [nb, 32] in 0..15; y = q*d + m"""
    b = blocks.reshape(-1, 20)
    qs = b[:, 4:].astype(np.int64)
    return _f16_field(b, 0), _f16_field(b, 2), np.concatenate([qs & 0xF, qs >> 4], axis=1)


def _fifth_bits(qh_bytes: np.ndarray) -> np.ndarray:
    """u32 little endian qh -> bit e of it for e = 0..31, as int64 [nb, 32]."""
    qh = qh_bytes.copy().view(np.uint32)[:, 0].astype(np.int64)
    return (qh[:, None] >> np.arange(32)[None, :]) & 1


def decode_q5_0(blocks: np.ndarray):
    """-> d f32 [nb], q int64 [nb, 32] in -16..15"""
    b = blocks.reshape(-1, 22)
    qs = b[:, 6:].astype(np.int64)
    lo = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    return _f16_field(b, 0), (lo | (_fifth_bits(b[:, 2:6]) << 4)) - 16


def decode_q5_1(blocks: np.ndarray):
    """-> d, m f32 [nb], q int64 [nb, 32] in 0..31"""
    b = blocks.reshape(-1, 24)
    qs = b[:, 8:].astype(np.int64)
    lo = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    return _f16_field(b, 0), _f16_field(b, 2), lo | (_fifth_bits(b[:, 4:8]) << 4)


def decode_q8_1(blocks: np.ndarray):
    """-> d, s f32 [nb], q int64 [nb, 32]"""
    b = blocks.reshape(-1, 36)
    return _f16_field(b, 0), _f16_field(b, 2), b[:, 4:].view(np.int8).astype(np.int64)


# --------------------------------------------------------- Q2_K, Q3_K, Q5_K
# Element e of a super-block, e = 128*h + 32*t + l (h half, t 2-bit plane):
#   Q2K / Q3K low bits: qs[32*h + l] >> 2t & 3; Q3K high bit: hmask[l] bit 4h + t.
#   Q5K: e = 64*i + 32*s + l: low nibble of qs[32*i + l] (s = 0) or high (s = 1),
#   fifth bit qh[l] bit 2i + s.
def encode_q2k(d_bits: int, dmin_bits: int, sc, mn, q) -> np.ndarray:
    """sc, mn [16] in 0..15; q [256] in 0..3."""
    q = np.asarray(q, np.int64)
    out = np.zeros(84, np.uint8)
    out[0:16] = (np.asarray(sc, np.int64) & 15) | ((np.asarray(mn, np.int64) & 15) << 4)
    for e in range(256):
        h, t, l = e // 128, (e % 128) // 32, e % 32
        out[16 + 32 * h + l] |= (q[e] & 3) << (2 * t)
    out[80:82] = np.array([d_bits], np.uint16).view(np.uint8)
    out[82:84] = np.array([dmin_bits], np.uint16).view(np.uint8)
    return out


def decode_q2k(blocks: np.ndarray):
    """-> d, dmin f32 [nb]; sc, mn int64 [nb, 16]; q int64 [nb, 256] in 0..3"""
    b = blocks.reshape(-1, 84)
    nb = b.shape[0]
    sc = b[:, 0:16].astype(np.int64)
    q = np.zeros((nb, 256), np.int64)
    qs = b[:, 16:80].astype(np.int64)
    for e in range(256):
        h, t, l = e // 128, (e % 128) // 32, e % 32
        q[:, e] = (qs[:, 32 * h + l] >> (2 * t)) & 3
    return _f16_field(b, 80), _f16_field(b, 82), sc & 15, sc >> 4, q


def pack_scales_q3k(sc) -> np.ndarray:
    """16 six-bit scales (0..63) -> 12 bytes: low nibbles of scales j and j + 8
    in byte j (j < 8), the top 2 bits of scale j in byte 8 + j % 4 at bit 2*(j // 4)."""
    sc = np.asarray(sc, np.int64)
    out = np.zeros(12, np.int64)
    for j in range(16):
        if j < 8:
            out[j] |= sc[j] & 15
        else:
            out[j - 8] |= (sc[j] & 15) << 4
        out[8 + j % 4] |= (sc[j] >> 4) << (2 * (j // 4))
    return out.astype(np.uint8)


def unpack_scales_q3k(b12: np.ndarray) -> np.ndarray:
    b = b12.astype(np.int64)
    sc = np.zeros(16, np.int64)
    for j in range(16):
        lo = (b[j] & 15) if j < 8 else (b[j - 8] >> 4)
        sc[j] = lo | (((b[8 + j % 4] >> (2 * (j // 4))) & 3) << 4)
    return sc


def encode_q3k(d_bits: int, sc, q) -> np.ndarray:
    """sc [16] in 0..63 (scale + 32); q [256] in -4..3."""
    q = np.asarray(q, np.int64) + 4  # 0..7
    out = np.zeros(110, np.uint8)
    for e in range(256):
        h, t, l = e // 128, (e % 128) // 32, e % 32
        out[32 + 32 * h + l] |= (q[e] & 3) << (2 * t)
        if q[e] & 4:
            out[l] |= 1 << (4 * h + t)
    out[96:108] = pack_scales_q3k(sc)
    out[108:110] = np.array([d_bits], np.uint16).view(np.uint8)
    return out


def decode_q3k(blocks: np.ndarray):
    """-> d f32 [nb]; sc int64 [nb, 16] in -32..31; q int64 [nb, 256] in -4..3"""
    b = blocks.reshape(-1, 110)
    nb = b.shape[0]
    sc = np.stack([unpack_scales_q3k(b[i, 96:108]) for i in range(nb)]) - 32
    q = np.zeros((nb, 256), np.int64)
    hm = b[:, 0:32].astype(np.int64)
    qs = b[:, 32:96].astype(np.int64)
    for e in range(256):
        h, t, l = e // 128, (e % 128) // 32, e % 32
        q[:, e] = ((qs[:, 32 * h + l] >> (2 * t)) & 3) | (((hm[:, l] >> (4 * h + t)) & 1) << 2)
    return _f16_field(b, 108), sc, q - 4


def encode_q5k(d_bits: int, dmin_bits: int, sc, mn, q) -> np.ndarray:
    """sc, mn [8] in 0..63; q [256] in 0..31."""
    q = np.asarray(q, np.int64)
    out = np.zeros(176, np.uint8)
    out[0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    out[2:4] = np.array([dmin_bits], np.uint16).view(np.uint8)
    out[4:16] = pack_scales_k4(np.asarray(sc, np.int64), np.asarray(mn, np.int64))
    for e in range(256):
        i, s, l = e // 64, (e % 64) // 32, e % 32
        out[48 + 32 * i + l] |= (q[e] & 15) << (4 * s)
        if q[e] & 16:
            out[16 + l] |= 1 << (2 * i + s)
    return out


def decode_q5k(blocks: np.ndarray):
    """-> d, dmin f32 [nb]; sc, mn int64 [nb, 8]; q int64 [nb, 256] in 0..31"""
    b = blocks.reshape(-1, 176)
    nb = b.shape[0]
    sc = np.zeros((nb, 8), np.int64)
    mn = np.zeros((nb, 8), np.int64)
    for i in range(nb):
        sc[i], mn[i] = unpack_scales_k4(b[i, 4:16])
    qh = b[:, 16:48].astype(np.int64)
    qs = b[:, 48:176].astype(np.int64)
    q = np.zeros((nb, 256), np.int64)
    for e in range(256):
        i, s, l = e // 64, (e % 64) // 32, e % 32
        q[:, e] = ((qs[:, 32 * i + l] >> (4 * s)) & 15) | (((qh[:, l] >> (2 * i + s)) & 1) << 4)
    return _f16_field(b, 0), _f16_field(b, 2), sc, mn, q
