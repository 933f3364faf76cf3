// GGUF block bytes <-> the repacked device planes, and dequantization.
//
// repack   : canonical GGUF blocks (as read from a file) -> planes
// unrepack : planes -> canonical GGUF blocks (QuantizedType::raw_data must
//            return the on-disk format, xn mod.rs:206-214)
// dequant  : planes -> f32, the same f32 operations as GgmlType::to_float
// The planar layout is described in xnq_internal.h.
#pragma clang fp contract(off)

#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

__device__ __forceinline__ uint16_t ld16(const uint8_t* p) {
    return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

// 6-bit value of element E (0..255) of a canonical BlockQ6K
// (the ql/qh layout of k_quants.rs:1759-1771).
__device__ __forceinline__ uint32_t q6_canon(const uint8_t* ql, const uint8_t* qh, int E) {
    const int hh = E >> 7, r = (E >> 5) & 3, l = E & 31;
    const uint8_t lo = ql[64 * hh + 32 * (r & 1) + l];
    const uint32_t nib = (r >= 2) ? (lo >> 4) : (lo & 0xF);
    const uint32_t hi = (qh[32 * hh + l] >> (2 * r)) & 3u;
    return nib | (hi << 4);
}

// 4-bit value of element E (0..255) of a canonical BlockQ4K qs array.
__device__ __forceinline__ uint32_t q4k_canon(const uint8_t* qs, int E) {
    const int p = E >> 6, h = (E >> 5) & 1, l = E & 31;
    return (qs[32 * p + l] >> (4 * h)) & 0xFu;
}

// One thread per (row, block) for Q4_0 / Q8_0; per (row, super-block, chunk)
// for Q4K / Q6K.
__global__ void repack_kernel(WView w, const uint8_t* __restrict__ src, uint8_t* __restrict__ q,
                              uint8_t* __restrict__ h, uint8_t* __restrict__ s,
                              uint8_t* __restrict__ d, uint8_t* __restrict__ st, uint8_t* __restrict__ dt,
                              size_t total) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    if (w.dtype == XNQ_Q8_0 || w.dtype == XNQ_Q4_0) {
        const size_t row = t / w.nb, b = t % w.nb;
        const bool q8 = w.dtype == XNQ_Q8_0;
        const size_t tsz = q8 ? 34 : 18, qb = q8 ? 32 : 16;
        const uint8_t* blk = src + t * tsz;
        uint8_t* qo = q + row * w.q_row + b * qb;
        for (size_t i = 0; i < qb; i++) qo[i] = blk[2 + i];
        uint8_t* dp = d + row * w.d_row + b * 2;
        dp[0] = blk[0];
        dp[1] = blk[1];
        return;
    }
    const size_t c = t & 7, sbg = t >> 3;  // global super-block index
    const size_t row = sbg / w.nb, sb = sbg % w.nb;
    if (w.dtype == XNQ_Q4K) {
        const uint8_t* blk = src + sbg * 144;
        uint32_t out[4];
        for (int dw = 0; dw < 4; dw++) {
            uint32_t v = 0;
            for (int p = 0; p < 4; p++) {
                const int e = 4 * dw + p;
                const uint32_t lo = q4k_canon(blk + 16, (int)(32 * c) + e);
                const uint32_t hi = q4k_canon(blk + 16, (int)(32 * c) + 16 + e);
                v |= (lo | (hi << 4)) << (8 * p);
            }
            out[dw] = v;
        }
        *reinterpret_cast<uint4*>(q + row * w.q_row + sb * 128 + c * 16) =
            make_uint4(out[0], out[1], out[2], out[3]);
        if (c == 0) {
            uint8_t* so = s + row * w.s_row + sb * 16;
            uint8_t* sto = st + kq_tile_off(w.nb, (uint32_t)row, (uint32_t)sb, 16);
            for (int i = 0; i < 16; i++) so[i] = sto[i] = blk[i];
        }
        return;
    }
    // Q6K
    const uint8_t* blk = src + sbg * 210;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    uint32_t lo4[4], hi2[2] = {0u, 0u};
    for (int dw = 0; dw < 4; dw++) {
        uint32_t v = 0;
        for (int p = 0; p < 4; p++) {
            const int e = 4 * dw + p;
            const uint32_t a = q6_canon(ql, qh, (int)(32 * c) + e);
            const uint32_t b2 = q6_canon(ql, qh, (int)(32 * c) + 16 + e);
            v |= ((a & 0xF) | ((b2 & 0xF) << 4)) << (8 * p);
        }
        lo4[dw] = v;
    }
    for (int g = 0; g < 8; g++) {
        for (int p = 0; p < 4; p++) {
            const uint32_t v = q6_canon(ql, qh, (int)(32 * c) + 4 * g + p) >> 4;
            hi2[g >> 2] |= v << (8 * p + 2 * (g & 3));
        }
    }
    *reinterpret_cast<uint4*>(q + row * w.q_row + sb * 128 + c * 16) =
        make_uint4(lo4[0], lo4[1], lo4[2], lo4[3]);
    *reinterpret_cast<uint2*>(h + row * w.h_row + sb * 64 + c * 8) = make_uint2(hi2[0], hi2[1]);
    if (c == 0) {
        uint8_t* so = s + row * w.s_row + sb * 16;
        uint8_t* sto = st + kq_tile_off(w.nb, (uint32_t)row, (uint32_t)sb, 16);
        for (int i = 0; i < 16; i++) so[i] = sto[i] = blk[192 + i];
        uint8_t* dp = d + row * w.d_row + sb * 2;
        dp[0] = blk[208];
        dp[1] = blk[209];
        uint8_t* dtp = dt + kq_tile_off((w.nb + 1) / 2, (uint32_t)row, (uint32_t)(sb >> 1), 4) + (sb & 1) * 2;
        dtp[0] = blk[208];
        dtp[1] = blk[209];
    }
}

// 4-bit value of element e (0..31) of a repacked nibble chunk.
__device__ __forceinline__ uint32_t nib_rep(const uint8_t* chunk, int e) {
    return e < 16 ? (chunk[e] & 0xFu) : (chunk[e - 16] >> 4);
}
// 6-bit value of element e (0..31) of a repacked Q6K chunk.
__device__ __forceinline__ uint32_t q6_rep(const uint8_t* ql, const uint8_t* qh, int e) {
    const int g = e >> 2, p = e & 3;
    const uint32_t hi = (qh[4 * (g >> 2) + p] >> (2 * (g & 3))) & 3u;
    return nib_rep(ql, e) | (hi << 4);
}

// One thread per (row, block): rebuild the canonical block bytes.
__global__ void unrepack_kernel(WView w, uint8_t* __restrict__ dst, size_t total) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const size_t row = t / w.nb, b = t % w.nb;
    if (w.dtype == XNQ_Q8_0 || w.dtype == XNQ_Q4_0) {
        const bool q8 = w.dtype == XNQ_Q8_0;
        const size_t tsz = q8 ? 34 : 18, qb = q8 ? 32 : 16;
        uint8_t* o = dst + t * tsz;
        const uint8_t* dp = w.d + row * w.d_row + b * 2;
        o[0] = dp[0];
        o[1] = dp[1];
        const uint8_t* qi = w.q + row * w.q_row + b * qb;
        for (size_t i = 0; i < qb; i++) o[2 + i] = qi[i];
        return;
    }
    const uint8_t* qrow = w.q + row * w.q_row + b * 128;
    if (w.dtype == XNQ_Q4K) {
        uint8_t* o = dst + t * 144;
        const uint8_t* si = w.s + row * w.s_row + b * 16;
        for (int i = 0; i < 16; i++) o[i] = si[i];
        // canonical qs[32p + l] = elem(64p + l) | elem(64p + 32 + l) << 4
        for (int p = 0; p < 4; p++)
            for (int l = 0; l < 32; l++) {
                const uint32_t lo = nib_rep(qrow + 16 * (2 * p), l);
                const uint32_t hi = nib_rep(qrow + 16 * (2 * p + 1), l);
                o[16 + 32 * p + l] = (uint8_t)(lo | (hi << 4));
            }
        return;
    }
    uint8_t* o = dst + t * 210;
    const uint8_t* hrow = w.h + row * w.h_row + b * 64;
    for (int hh = 0; hh < 2; hh++)
        for (int l = 0; l < 32; l++) {
            uint32_t v[4];
            for (int r = 0; r < 4; r++) {
                const int E = 128 * hh + 32 * r + l;
                v[r] = q6_rep(qrow + 16 * (E >> 5), hrow + 8 * (E >> 5), E & 31);
            }
            o[64 * hh + l] = (uint8_t)((v[0] & 0xF) | ((v[2] & 0xF) << 4));
            o[64 * hh + 32 + l] = (uint8_t)((v[1] & 0xF) | ((v[3] & 0xF) << 4));
            o[128 + 32 * hh + l] =
                (uint8_t)((v[0] >> 4) | ((v[1] >> 4) << 2) | ((v[2] >> 4) << 4) | ((v[3] >> 4) << 6));
        }
    const uint8_t* si = w.s + row * w.s_row + b * 16;
    for (int i = 0; i < 16; i++) o[192 + i] = si[i];
    const uint8_t* dp = w.d + row * w.d_row + b * 2;
    o[208] = dp[0];
    o[209] = dp[1];
}

// One thread per chunk of 32 outputs; same f32 operations as to_float.
__global__ void dequant_kernel(WView w, float* __restrict__ y, size_t total) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const size_t cpr = w.k / 32;  // chunks per row
    const size_t row = t / cpr, c = t % cpr;
    float* out = y + row * (size_t)w.k + c * 32;
    if (w.dtype == XNQ_Q8_0) {  // k_quants.rs:618-634
        const float d = f16_bits_to_f32(ld16(w.d + row * w.d_row + c * 2));
        const int8_t* qi = reinterpret_cast<const int8_t*>(w.q + row * w.q_row + c * 32);
        for (int j = 0; j < 32; j++) out[j] = (float)qi[j] * d;
        return;
    }
    if (w.dtype == XNQ_Q4_0) {  // k_quants.rs:213-233
        const float d = f16_bits_to_f32(ld16(w.d + row * w.d_row + c * 2));
        const uint8_t* qi = w.q + row * w.q_row + c * 16;
        for (int j = 0; j < 32; j++) out[j] = (float)((int)nib_rep(qi, j) - 8) * d;
        return;
    }
    const size_t sb = c / 8, j = c % 8;
    const uint8_t* qi = w.q + row * w.q_row + sb * 128 + j * 16;
    if (w.dtype == XNQ_Q4K) {  // k_quants.rs:1475-1503
        const uint8_t* si = w.s + row * w.s_row + sb * 16;
        const float d = f16_bits_to_f32(ld16(si)), mn = f16_bits_to_f32(ld16(si + 2));
        const uint32_t* sc = reinterpret_cast<const uint32_t*>(si + 4);
        int scv, mv;
        q4k_scale_min(sc[0], sc[1], sc[2], (int)j, scv, mv);
        const float d1 = d * (float)scv, m1 = mn * (float)mv;
        for (int e = 0; e < 32; e++) out[e] = d1 * (float)nib_rep(qi, e) - m1;
        return;
    }
    // Q6K, k_quants.rs:1874-1904
    const uint8_t* hi = w.h + row * w.h_row + sb * 64 + j * 8;
    const int8_t* sc = reinterpret_cast<const int8_t*>(w.s + row * w.s_row + sb * 16);
    const float d = f16_bits_to_f32(ld16(w.d + row * w.d_row + sb * 2));
    for (int e = 0; e < 32; e++) {
        const int q = (int)q6_rep(qi, hi, e) - 32;
        out[e] = d * (float)sc[2 * j + (e >> 4)] * (float)q;
    }
}

// ---- the padded-block types (Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K) ----

// Where the padded block's bytes come from: bytes [0, a) are GGUF bytes
// [0, a), bytes [a, a + h) are zero, byte i >= a + h is GGUF byte i - h, and
// bytes past the GGUF block are zero. Q5_0 inserts 2 zero bytes after d
// (a = 2, h = 2); Q3K appends 2 (a = stride, h = 0); the others copy.
// The map is plain arithmetic on host-computed (a, h): a per-dtype branch
// chain here was miscompiled by hipcc 7.2 for dtypes above Q3K (the byte
// index stayed at its entry value), which zeroed every Q5K block past d/dmin.
struct RawMap {
    uint32_t a, h, tsz, stride;
};
inline RawMap raw_map(uint32_t dt) {
    const uint32_t tsz = (uint32_t)type_size(dt), stride = raw_stride(dt);
    return dt == XNQ_Q5_0 ? RawMap{2, 2, tsz, stride} : RawMap{stride, 0, tsz, stride};
}
__device__ __forceinline__ int raw_src(const RawMap& r, uint32_t i) {
    const uint32_t j = i < r.a ? i : i - r.h;
    return (i >= r.a && i < r.a + r.h) || j >= r.tsz ? -1 : (int)j;
}

// One thread per (row, block).
__global__ void pad_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ q, size_t total, RawMap r) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const uint8_t* in = src + t * r.tsz;
    uint8_t* out = q + t * r.stride;  // rows are nb * stride bytes, blocks back to back
    for (uint32_t i = 0; i < r.stride; i++) {
        const int j = raw_src(r, i);
        out[i] = j < 0 ? 0 : in[j];
    }
}

__global__ void unpad_kernel(const uint8_t* __restrict__ q, uint8_t* __restrict__ dst, size_t total, RawMap r) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const uint8_t* in = q + t * r.stride;
    uint8_t* out = dst + t * r.tsz;
    for (uint32_t i = 0; i < r.stride; i++) {
        const int j = raw_src(r, i);
        if (j >= 0) out[j] = in[i];
    }
}

// One thread per chunk of 32 outputs; the f32 operations of to_float
// (k_quants.rs:379-399, 478-502, 585-609, 1014-1053, 1240-1315, 1682-1721).
template <uint32_t dt>
__global__ void dequant_raw_kernel(WView w, float* __restrict__ y, size_t total) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const size_t cpr = w.k / 32;
    const size_t row = t / cpr, c = t % cpr;
    float* out = y + row * (size_t)w.k + c * 32;
    const uint32_t stride = raw_stride(dt);
    if (!is_kquant(dt)) {
        const uint8_t* b = w.q + row * w.q_row + c * stride;
        const float d = f16_bits_to_f32(ld16(b));
        if (dt == XNQ_Q4_1) {
            const float m = f16_bits_to_f32(ld16(b + 2));
            for (int j = 0; j < 16; j++) {
                out[j] = (float)(b[4 + j] & 0x0F) * d + m;
                out[j + 16] = (float)(b[4 + j] >> 4) * d + m;
            }
            return;
        }
        const uint32_t qh = *reinterpret_cast<const uint32_t*>(b + 4);
        for (int j = 0; j < 16; j++) {
            const uint32_t x0 = (b[8 + j] & 0x0Fu) | (((qh >> j) << 4) & 0x10u);
            const uint32_t x1 = (b[8 + j] >> 4) | ((qh >> (j + 12)) & 0x10u);
            if (dt == XNQ_Q5_0) {
                out[j] = (float)((int)x0 - 16) * d;
                out[j + 16] = (float)((int)x1 - 16) * d;
            } else {
                const float m = f16_bits_to_f32(ld16(b + 2));
                out[j] = (float)x0 * d + m;
                out[j + 16] = (float)x1 * d + m;
            }
        }
        return;
    }
    const size_t sb = c / 8;
    const int j = (int)(c % 8);
    const uint8_t* b = w.q + row * w.q_row + sb * stride;
    if (dt == XNQ_Q2K) {
        const int h = j >> 2, sh = 2 * (j & 3);
        const float d = f16_bits_to_f32(ld16(b + 80)), mn = f16_bits_to_f32(ld16(b + 82));
        for (int g = 0; g < 2; g++) {
            const uint8_t sc = b[2 * j + g];
            const float dl = d * (float)(sc & 0xF), ml = mn * (float)(sc >> 4);
            for (int l = 0; l < 16; l++) out[16 * g + l] = dl * (float)((b[16 + 32 * h + 16 * g + l] >> sh) & 3) - ml;
        }
        return;
    }
    if (dt == XNQ_Q3K) {
        const int h = j >> 2, sh = 2 * (j & 3);
        const uint32_t* s3 = reinterpret_cast<const uint32_t*>(b + 96);
        const float d_all = f16_bits_to_f32(ld16(b + 108));
        const uint32_t bit = 1u << (4 * h + (j & 3));
        for (int g = 0; g < 2; g++) {
            const float dl = d_all * ((float)(int8_t)q3k_scale(s3[0], s3[1], s3[2], 2 * j + g) - 32.0f);
            for (int l = 16 * g; l < 16 * g + 16; l++) {
                const int v = (int)((b[32 + 32 * h + l] >> sh) & 3) - ((b[l] & bit) == 0 ? 4 : 0);
                out[l] = dl * (float)v;
            }
        }
        return;
    }
    // Q5K
    const int i = j >> 1, s = j & 1;
    const float d = f16_bits_to_f32(ld16(b)), mn = f16_bits_to_f32(ld16(b + 2));
    const uint32_t* sc = reinterpret_cast<const uint32_t*>(b + 4);
    int scv, mv;
    q4k_scale_min(sc[0], sc[1], sc[2], j, scv, mv);
    const float d1 = d * (float)scv, m1 = mn * (float)mv;
    const uint32_t u = 1u << (2 * i + s);
    for (int l = 0; l < 32; l++) {
        const uint8_t ql = b[48 + 32 * i + l];
        const float nib = (float)(s ? (ql >> 4) : (ql & 0xF));
        out[l] = d1 * (nib + ((b[16 + l] & u) ? 16.0f : 0.0f)) - m1;
    }
}

inline unsigned blocks_for(size_t total, unsigned threads) {
    return (unsigned)((total + threads - 1) / threads);
}

}  // namespace

hipError_t launch_repack(const WLayout& L, const void* gguf_dev, void* dst_dev, hipStream_t s) {
    WView w = make_wview(L, dst_dev);
    uint8_t* base = static_cast<uint8_t*>(dst_dev);
    if (is_raw_layout(L.dtype)) {
        const size_t total = L.n * L.nb;
        if (total == 0) return hipSuccess;
        pad_kernel<<<blocks_for(total, 128), 128, 0, s>>>(static_cast<const uint8_t*>(gguf_dev), base + L.off_q, total,
                                                          raw_map(L.dtype));
        return hipGetLastError();
    }
    const bool kq = is_kquant(L.dtype);
    const size_t total = L.n * L.nb * (kq ? 8 : 1);
    if (total == 0) return hipSuccess;
    repack_kernel<<<blocks_for(total, 256), 256, 0, s>>>(
        w, static_cast<const uint8_t*>(gguf_dev), base + L.off_q, base + L.off_h, base + L.off_s,
        base + L.off_d, base + L.off_st, base + L.off_dt, total);
    return hipGetLastError();
}

hipError_t launch_unrepack(const WLayout& L, const void* src_dev, void* gguf_dev, hipStream_t s) {
    WView w = make_wview(L, src_dev);
    const size_t total = L.n * L.nb;
    if (total == 0) return hipSuccess;
    if (is_raw_layout(L.dtype)) {
        unpad_kernel<<<blocks_for(total, 128), 128, 0, s>>>(w.q, static_cast<uint8_t*>(gguf_dev), total,
                                                            raw_map(L.dtype));
        return hipGetLastError();
    }
    unrepack_kernel<<<blocks_for(total, 128), 128, 0, s>>>(w, static_cast<uint8_t*>(gguf_dev), total);
    return hipGetLastError();
}

hipError_t launch_dequant(const WLayout& L, const void* src_dev, float* y, hipStream_t s) {
    WView w = make_wview(L, src_dev);
    const size_t total = L.n * (L.k / 32);
    if (total == 0) return hipSuccess;
    if (is_raw_layout(L.dtype)) {
        const unsigned g = blocks_for(total, 256);
        switch (L.dtype) {
        case XNQ_Q4_1: dequant_raw_kernel<XNQ_Q4_1><<<g, 256, 0, s>>>(w, y, total); break;
        case XNQ_Q5_0: dequant_raw_kernel<XNQ_Q5_0><<<g, 256, 0, s>>>(w, y, total); break;
        case XNQ_Q5_1: dequant_raw_kernel<XNQ_Q5_1><<<g, 256, 0, s>>>(w, y, total); break;
        case XNQ_Q2K: dequant_raw_kernel<XNQ_Q2K><<<g, 256, 0, s>>>(w, y, total); break;
        case XNQ_Q3K: dequant_raw_kernel<XNQ_Q3K><<<g, 256, 0, s>>>(w, y, total); break;
        default: dequant_raw_kernel<XNQ_Q5K><<<g, 256, 0, s>>>(w, y, total); break;
        }
        return hipGetLastError();
    }
    dequant_kernel<<<blocks_for(total, 256), 256, 0, s>>>(w, y, total);
    return hipGetLastError();
}

}  // namespace xnq
