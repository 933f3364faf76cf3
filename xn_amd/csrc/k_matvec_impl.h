// Decode-path matmul for m <= 8 activation rows (template; instantiated per
// weight dtype in k_matvec_<dtype>.hip).
//
// Work split: a wavefront owns R consecutive weight rows ("row group") and,
// for each row, CPL 32-element chunks per lane (chunk c = lane + 64*v), i.e.
// every dwordx4 load instruction of the wavefront covers 1 KiB of one plane.
// All R*CPL loads of a row group are issued before anything else happens, so
// the whole weight stream is in flight while the activations are staged; the
// grid is sized so every row group of the common shapes is resident at once.
//
// Activations live in LDS: either quantized there by the workgroup itself
// from the f32 rows (FUSED, m == 1: one kernel per matmul call, no
// workspace) or copied from a Q8 workspace produced by the quantize kernel.
// Integer dot products use v_dot4_i32_i8; block scales are applied in f32.
#pragma once

#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>

#include "xnq_device.h"
#include "xnq_internal.h"
#include "xnq_quant_dev.h"

namespace xnq {
namespace mv {

constexpr int kWave = 64;
constexpr uint32_t kMaxLds = 160 * 1024;

// LDS holds MB consecutive activation row images (ActImg in xnq_internal.h),
// the same bytes as the quantized workspace, so staging is a flat copy.
// LDS bytes of MB staged rows: flat row images, or the interleaved layout of
// the multi-row workspace path when that is larger
__host__ __device__ inline uint32_t lds_bytes(int mb, uint32_t k, bool kquant);

// Sum over the 64 lanes with DPP: row_shr 1/2/4/8 build each 16-lane row's
// total in its last lane, row_bcast 15/31 carry it across rows; lane 63 ends
// up with the wavefront total, which readlane broadcasts.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true);
    return v + __int_as_float(t);
}
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0x111, 0xf>(v);  // row_shr:1
    v = dpp_add<0x112, 0xf>(v);  // row_shr:2
    v = dpp_add<0x114, 0xf>(v);  // row_shr:4
    v = dpp_add<0x118, 0xf>(v);  // row_shr:8
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Copy MB row images of the quantized workspace into LDS; rows past mcount
// are zero.  Loads are issued in batches of kBatch before any LDS write so one
// memory round trip covers the whole batch.
template <int MB, int NW>
__device__ void stage_activations(const AView& a, uint32_t m0, uint32_t mcount, uint8_t* lds) {
    constexpr int kBatch = 8;
    constexpr int kThreads = NW * kWave;
    const uint32_t rb = a.A.row_bytes;
    const uint32_t total = (uint32_t)MB * rb / 16, live = (mcount < (uint32_t)MB ? mcount : MB) * rb / 16;
    const uint4* src = reinterpret_cast<const uint4*>(a.img + (size_t)m0 * rb);
    uint4* dst = reinterpret_cast<uint4*>(lds);
    for (uint32_t base = 0; base < total; base += kBatch * kThreads) {
        uint4 v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; j++) {
            const uint32_t i = base + j * kThreads + threadIdx.x;
            v[j] = i < live ? src[i] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < kBatch; j++) {
            const uint32_t i = base + j * kThreads + threadIdx.x;
            if (i < total) dst[i] = v[j];
        }
    }
}

// Quantize MB f32 rows straight into the LDS images (the same bytes as the
// standalone quantize kernel: both go through q8k/q80 quant + store).
// Work is cut in rounds of kBatch blocks per wavefront; `load` issues one
// round's f32 loads and `quant` turns them into LDS bytes.  The kernel loads
// the first round before it issues any weight load: loads complete in order
// (one vmcnt counter), so x loaded after the weights would wait for the HBM
// weight stream.
template <int DT, int MB, int kNW, int kBatch>
struct XQuant {
    static constexpr bool kq = is_kquant(DT);
    float4 v[kBatch];
    // first block of round 0 for this wavefront, and the block step between rounds
    __device__ __forceinline__ static uint32_t first(uint32_t wave) { return kq ? wave : wave * 8; }
    __device__ __forceinline__ static uint32_t step() { return kq ? kBatch * kNW : kBatch * kNW * 8; }
    __device__ __forceinline__ static uint32_t total(uint32_t k) { return MB * (kq ? k / 256 : k / 32); }

    __device__ __forceinline__ void load(const float* __restrict__ x, uint32_t k, uint32_t m0, uint32_t mcount,
                                         uint32_t b0, uint32_t lane) {
#pragma unroll
        for (int j = 0; j < kBatch; j++) {
            // unconditional loads, clamped to the last live block (rows past
            // mcount quantize copies of it; their outputs are never stored)
            const uint32_t live = (mcount < (uint32_t)MB ? mcount : MB) * (kq ? k / 256 : k / 32);
            if (kq) {
                const uint32_t nb = k / 256, b = b0 + j * kNW, bc = min(b, live - 1);
                const float4 t = reinterpret_cast<const float4*>(x + (size_t)(m0 + bc / nb) * k + (bc % nb) * 256)[lane];
                v[j] = t;
            } else {
                const uint32_t nb = k / 32, b = b0 + j * kNW * 8 + (lane >> 3), bc = min(b, live - 1);
                const float4 t = reinterpret_cast<const float4*>(x + (size_t)(m0 + bc / nb) * k + (bc % nb) * 32)[lane & 7];
                v[j] = t;
            }
        }
    }
    // Every block slot is quantized, also past the end (on clamped copies),
    // and only the store is conditional: a loaded value used only under a
    // condition would have its load moved behind the weight loads.
    __device__ __forceinline__ void quant(uint8_t* lds, const ActImg& A, uint32_t k, uint32_t b0, uint32_t lane) {
        const uint32_t tot = total(k);
#pragma unroll
        for (int j = 0; j < kBatch; j++) {
            if (kq) {
                const uint32_t nb = k / 256, b = b0 + j * kNW;
                const Q8KLane r = q8k_quant_wave(v[j], (int)lane);
                if (b < tot) q8k_store(lds + (b / nb) * A.row_bytes, A, b % nb, (int)lane, r);  // uniform
            } else {
                const uint32_t nb = k / 32, b = b0 + j * kNW * 8 + (lane >> 3);
                const Q80Lane r = q80_quant_8lanes(v[j]);
                if (b < tot) q80_store(lds + (b / nb) * A.row_bytes, A, b % nb, (int)(lane & 7), r);
            }
        }
    }
    // the rounds after the first
    __device__ __forceinline__ void rest(const float* __restrict__ x, uint32_t k, uint32_t m0, uint32_t mcount,
                                         uint8_t* lds, const ActImg& A, uint32_t wave, uint32_t lane) {
        for (uint32_t b0 = first(wave) + step(); b0 < total(k); b0 += step()) {
            load(x, k, m0, mcount, b0, lane);
            quant(lds, A, k, b0, lane);
        }
    }
};

// Per-chunk weight data held in registers between the load and the compute.
struct Chunk {
    uint4 q;
    uint4 x;  // Q8_0: second 16 bytes; Q4K: {d|dmin, scales}; Q6K: qh in .x/.y, scale pair in .z
    float dw;
    // the padded-block types: the chunk's low bits (Q2K/Q3K/Q5K: 32 bytes in
    // q, e0), its high bits (Q3K hmask / Q5K qh: 32 bytes in e1, e2)
    uint4 e0, e1, e2;
};

// Byte offsets are 32-bit (every plane is < 4 GiB, checked at upload), so the
// loads use a uniform 64-bit base plus one VGPR offset.
// Weight stream loads: each weight byte is read once per call, so the loads
// are marked non-temporal and the stream does not displace the activation
// data in L2.
typedef unsigned int nt_u4 __attribute__((ext_vector_type(4)));
typedef unsigned int nt_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ldw(const uint4* p) {
    const nt_u4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldw(const uint2* p) {
    const nt_u2 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u2*>(p));
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint16_t ldw(const uint16_t* p) { return __builtin_nontemporal_load(p); }

template <int DT>
__device__ __forceinline__ void load_chunk(const WView& w, uint32_t row, uint32_t c, Chunk& ch) {
    if (DT == XNQ_Q8_0) {
        const uint32_t o = row * w.q_row + c * 32;
        ch.q = ldw(reinterpret_cast<const uint4*>(w.q + o));
        ch.x = ldw(reinterpret_cast<const uint4*>(w.q + o + 16));
        ch.dw = f16_bits_to_f32(ldw(reinterpret_cast<const uint16_t*>(w.d + (row * w.d_row + c * 2))));
    } else if (DT == XNQ_Q4_0) {
        ch.q = ldw(reinterpret_cast<const uint4*>(w.q + (row * w.q_row + c * 16)));
        ch.dw = f16_bits_to_f32(ldw(reinterpret_cast<const uint16_t*>(w.d + (row * w.d_row + c * 2))));
    } else if (DT == XNQ_Q4K) {
        ch.q = ldw(reinterpret_cast<const uint4*>(w.q + (row * w.q_row + c * 16)));
        ch.x = ldw(reinterpret_cast<const uint4*>(w.s + (row * w.s_row + (c >> 3) * 16)));
    } else if (DT == XNQ_Q6K) {
        const uint32_t sb = c >> 3, j = c & 7;
        ch.q = ldw(reinterpret_cast<const uint4*>(w.q + (row * w.q_row + c * 16)));
        const uint2 h = ldw(reinterpret_cast<const uint2*>(w.h + (row * w.h_row + c * 8)));
        ch.x.x = h.x;
        ch.x.y = h.y;
        ch.x.z = ldw(reinterpret_cast<const uint16_t*>(w.s + (row * w.s_row + sb * 16 + 2 * j)));
        ch.dw = f16_bits_to_f32(ldw(reinterpret_cast<const uint16_t*>(w.d + (row * w.d_row + sb * 2))));
    } else {
        // padded GGUF blocks: every field is dword aligned (raw_stride), the
        // loads are dword loads
        const uint32_t* b;
        if (!is_kquant(DT)) {
            b = reinterpret_cast<const uint32_t*>(w.q + row * w.q_row + c * raw_stride(DT));
            ch.x.x = b[0];  // d | m (Q4_1, Q5_1) or d (Q5_0)
            const uint32_t o = DT == XNQ_Q4_1 ? 1 : 2;
            if (DT != XNQ_Q4_1) ch.x.y = b[1];  // qh
            ch.q = make_uint4(b[o], b[o + 1], b[o + 2], b[o + 3]);
            return;
        }
        const uint32_t j = c & 7;
        b = reinterpret_cast<const uint32_t*>(w.q + row * w.q_row + (c >> 3) * raw_stride(DT));
        auto ld8 = [&](uint32_t dw0, uint4& lo, uint4& hi) {
            lo = make_uint4(b[dw0], b[dw0 + 1], b[dw0 + 2], b[dw0 + 3]);
            hi = make_uint4(b[dw0 + 4], b[dw0 + 5], b[dw0 + 6], b[dw0 + 7]);
        };
        if (DT == XNQ_Q2K) {
            ld8(4 + 8 * (j >> 2), ch.q, ch.e0);  // qs[32h .. 32h+32)
            ch.x.x = b[20];                        // d | dmin
            ch.x.y = b[j >> 1];                    // scales 2j, 2j+1 in half (j & 1)
        } else if (DT == XNQ_Q3K) {
            ld8(8 + 8 * (j >> 2), ch.q, ch.e0);  // qs[32h .. 32h+32)
            ld8(0, ch.e1, ch.e2);                 // hmask
            ch.x = make_uint4(b[24], b[25], b[26], b[27]);  // scales[12], d
        } else {  // Q5K
            ld8(12 + 8 * (j >> 1), ch.q, ch.e0);  // qs[32i .. 32i+32)
            ld8(4, ch.e1, ch.e2);                  // qh
            ch.x = make_uint4(b[0], b[1], b[2], b[3]);  // d | dmin, scales[12]
        }
    }
}

// Bytes 4w .. 4w+3 of a 32-byte run held as two uint4.
__device__ __forceinline__ uint32_t dw_of(const uint4& lo, const uint4& hi, int w) {
    const uint4& v = w < 4 ? lo : hi;
    const int i = w & 3;
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
// The 4 bits at 4w .. 4w+3 of x spread to bit 0 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t x, int w) {
    const uint32_t v = (x >> (4 * w)) & 0xFu;
    return (v & 1u) | ((v & 2u) << 7) | ((v & 4u) << 14) | ((v & 8u) << 21);
}

// Integer parts of one chunk's dot for the padded-block types: a[8] the
// chunk's 32 int8 activations (elements 0-15 in a[0..3], 16-31 in a[4..7]),
// sv the chunk's side word (Q8K: bsum of elements 0-15 | bsum of 16-31 << 16;
// Q8_0: the block sum):
//   Q4_1, Q5_1: r0 = sum q*a;  Q5_0: r0 = sum (q - 16)*a;  r1 = 0
//   Q2K: r0 = sum_g (sc_g & 15) * sum q2*a,  r1 = sum_g (sc_g >> 4) * bsum_g
//   Q3K: r0 = sum_g (sc_g - 32) * sum (q3 - 4 * !hbit)*a,  r1 = 0
//   Q5K: r0 = sc_j * sum q5*a,  r1 = m_j * bsum32_j
// Summed over a block's chunks these are the block integers of the CPU
// vec_dot (k_quants.rs:316-343, 419-440, 513-544, 899-948, 1071-1152, 1524-1605).
template <int DT>
__device__ __forceinline__ void chunk_ints(const Chunk& ch, uint32_t c, const int* a, int32_t sv, int& r0, int& r1) {
    const int bs0 = (int)(int16_t)(sv & 0xffff), bs1 = (int)(int16_t)(sv >> 16);
    r1 = 0;
    if (DT == XNQ_Q4_1) {
        int lo, hi;
        nib_dot2(ch.q, a, lo, hi);
        r0 = lo + hi;
    } else if (DT == XNQ_Q5_0 || DT == XNQ_Q5_1) {
        const uint32_t q4[4] = {ch.q.x, ch.q.y, ch.q.z, ch.q.w};
        int sumi = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t lo = (q4[w] & 0x0F0F0F0Fu) | (spread4(ch.x.y, w) << 4);
            const uint32_t hi = ((q4[w] >> 4) & 0x0F0F0F0Fu) | (spread4(ch.x.y >> 16, w) << 4);
            sumi = dot4((int)lo, a[w], sumi);
            sumi = dot4((int)hi, a[4 + w], sumi);
        }
        r0 = DT == XNQ_Q5_0 ? sumi - 16 * sv : sumi;
    } else if (DT == XNQ_Q2K) {
        const uint32_t sh = 2 * (c & 3);
        int i0 = 0, i1 = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            i0 = dot4((int)((dw_of(ch.q, ch.e0, w) >> sh) & 0x03030303u), a[w], i0);
            i1 = dot4((int)((dw_of(ch.q, ch.e0, w + 4) >> sh) & 0x03030303u), a[4 + w], i1);
        }
        const uint32_t scw = (ch.x.y >> (16 * (c & 1))) & 0xffffu;
        const int s0 = (int)(scw & 0xff), s1 = (int)(scw >> 8);
        r0 = __mul24(s0 & 15, i0) + __mul24(s1 & 15, i1);  // |i| <= 16*3*128
        r1 = bs0 * (s0 >> 4) + bs1 * (s1 >> 4);
    } else if (DT == XNQ_Q3K) {
        // (q3 & 3) - (hmask bit ? 0 : 4), 16-element groups of scale sc - 32
        const uint32_t sh = 2 * (c & 3), hb = 4 * ((c & 7) >> 2) + (c & 3);
        int u0 = 0, u1 = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t l0 = ((dw_of(ch.q, ch.e0, w) >> sh) & 0x03030303u) |
                                (((dw_of(ch.e1, ch.e2, w) >> hb) & 0x01010101u) << 2);
            const uint32_t l1 = ((dw_of(ch.q, ch.e0, w + 4) >> sh) & 0x03030303u) |
                                (((dw_of(ch.e1, ch.e2, w + 4) >> hb) & 0x01010101u) << 2);
            u0 = dot4((int)l0, a[w], u0);
            u1 = dot4((int)l1, a[4 + w], u1);
        }
        const int g = 2 * (int)(c & 7);
        const int sc0 = (int)(int8_t)q3k_scale(ch.x.x, ch.x.y, ch.x.z, g) - 32;
        const int sc1 = (int)(int8_t)q3k_scale(ch.x.x, ch.x.y, ch.x.z, g + 1) - 32;
        r0 = __mul24(sc0, u0 - 4 * bs0) + __mul24(sc1, u1 - 4 * bs1);  // |u - 4 bs| < 2^16
    } else {  // Q5K
        const uint32_t j = c & 7, s = j & 1, hb = 2 * (j >> 1) + s;
        int v = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            const uint32_t nib = (dw_of(ch.q, ch.e0, w) >> (4 * s)) & 0x0F0F0F0Fu;
            const uint32_t h5 = ((dw_of(ch.e1, ch.e2, w) >> hb) & 0x01010101u) << 4;
            v = dot4((int)(nib | h5), a[w], v);
        }
        int sc, mn;
        q4k_scale_min(ch.x.y, ch.x.z, ch.x.w, (int)j, sc, mn);
        r0 = __mul24(sc, v);  // |v| <= 32*31*128 < 2^23
        r1 = mn * (bs0 + bs1);
    }
}

// f32 combine of one weight chunk c against one activation chunk (a, sv as
// for chunk_ints), da the activation block scale.  Integer parts are exact; the f32
// combine follows each type's vec_dot per block.
template <int DT>
__device__ __forceinline__ void chunk_fma(const Chunk& ch, uint32_t c, const int* a, int32_t sv, float da,
                                          float& acc) {
    const int bs0 = (int)(int16_t)(sv & 0xffff), bs1 = (int)(int16_t)(sv >> 16);
    if (DT == XNQ_Q4K) {
        int sc, mn;
        const float dw = f16_bits_to_f32(ch.x.x), dmin = f16_bits_to_f32(ch.x.x >> 16);
        q4k_scale_min(ch.x.y, ch.x.z, ch.x.w, (int)(c & 7), sc, mn);
        const int raw = nib_dot(ch.q, a);  // |raw| <= 32*15*128
        // dw * (sc * raw) with the integer product formed in f32: d (an
        // f16, 11 significant bits) times sc (6 bits) is exact, and so is
        // the integer |sc * raw| < 2^24, so cw * raw rounds the same
        // exact product once, as the integer form does; the same holds for
        // the min term.  cw and cm depend only on the chunk, so with several
        // activation rows they are formed once.
        const float cw = dw * (float)sc, cm = dmin * (float)mn;
        acc = fmaf(da, fmaf(cw, (float)raw, -(cm * (float)(bs0 + bs1))), acc);
    } else if (DT == XNQ_Q6K) {
        const int sc0 = (int)(int8_t)(ch.x.z & 0xff), sc1 = (int)(int8_t)((ch.x.z >> 8) & 0xff);
        const int v = q6k_chunk_int(ch.q, make_uint2(ch.x.x, ch.x.y), a, sc0, sc1, bs0, bs1);
        acc += (ch.dw * da) * (float)v;
    } else if (DT == XNQ_Q4_0) {
        int lo, hi;
        nib_dot2(ch.q, a, lo, hi);
        acc += (ch.dw * da) * (float)(lo + hi - 8 * sv);
    } else if (DT == XNQ_Q8_0) {
        acc += (ch.dw * da) * (float)i8_dot32(ch.q, ch.x, a);
    } else if (DT == XNQ_Q4_1 || DT == XNQ_Q5_0 || DT == XNQ_Q5_1) {
        // k_quants.rs:316-343, 419-440, 513-544
        int sumi, unused;
        chunk_ints<DT>(ch, c, a, sv, sumi, unused);
        const float dw = f16_bits_to_f32(ch.x.x);
        float r = (float)sumi * dw * da;
        if (DT != XNQ_Q5_0) {
            // Q8_1's s = f16(f16(sum) * d) (k_quants.rs:871), times the weight's m
            const float s = f16_bits_to_f32(
                f32_to_f16_bits(f16_bits_to_f32(f32_to_f16_bits((float)sv)) * da));
            r = r + f16_bits_to_f32(ch.x.x >> 16) * s;
        }
        acc += r;
    } else if (DT == XNQ_Q2K) {
        // k_quants.rs:899-948: dall * sum_g (sc_g & 15) isum_g - dmin * sum_g (sc_g >> 4) bsum_g
        int isum, summs;
        chunk_ints<DT>(ch, c, a, sv, isum, summs);
        const float dall = da * f16_bits_to_f32(ch.x.x), dmin = da * f16_bits_to_f32(ch.x.x >> 16);
        acc += dall * (float)isum - dmin * (float)summs;
    } else if (DT == XNQ_Q3K) {
        // k_quants.rs:1071-1152
        int isum, unused;
        chunk_ints<DT>(ch, c, a, sv, isum, unused);
        acc += (f16_bits_to_f32(ch.x.w) * da) * (float)isum;
    } else {  // Q5K, k_quants.rs:1524-1605
        int isum, msum;
        chunk_ints<DT>(ch, c, a, sv, isum, msum);
        const float d = f16_bits_to_f32(ch.x.x) * da, dmin = f16_bits_to_f32(ch.x.x >> 16) * da;
        acc += d * (float)isum - dmin * (float)msum;
    }
}

template <int DT, int MB>
__device__ __forceinline__ void compute_chunk(const Chunk& ch, uint32_t c, uint32_t k,
                                              const uint8_t* lds, const ActImg& A, float* acc) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const uint8_t* row = lds + mb * A.row_bytes;
        const uint4 a0 = *reinterpret_cast<const uint4*>(row + c * 16);
        const uint4 a1 = *reinterpret_cast<const uint4*>(row + k / 2 + c * 16);
        const int a[8] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                          (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        const int32_t sv = reinterpret_cast<const int32_t*>(row + A.s_off)[c];
        const float* ld = reinterpret_cast<const float*>(row + A.d_off);
        chunk_fma<DT>(ch, c, a, sv, ld[is_kquant(DT) ? c >> 3 : c], acc[mb]);
    }
}

// Q4_K with several activation rows (MB >= 4, workspace path): the staged
// Q8K image is interleaved by row in groups of 64 chunks (a wavefront's chunks of one
// load instruction), so one chunk's reads for all MB rows sit at fixed
// distances (immediate ds_read offsets, no per-row address arithmetic) and
// the 64 lanes of one read still cover 64 consecutive slots (no bank
// conflicts).  With chunk c = 64u + l, NU = ceil(nch / 64):
//   [half 2][u NU][row MB][l 64][16]  quants: bytes 16h .. 16h+15 of chunk c
//   [u NU][row MB][l 64] f32           chunk c's bsum (both 16-element halves)
//   [block nb][row MB] f32             d_a of block b (256 elements)
struct IlLay {
    uint32_t nu, sv, da, bytes;
};
__host__ __device__ inline IlLay il_lay(int mb, uint32_t k) {
    IlLay L;
    L.nu = (k / 32 + 63) / 64;
    L.sv = 2 * L.nu * (uint32_t)mb * 1024;
    L.da = L.sv + L.nu * (uint32_t)mb * 256;
    L.bytes = L.da + (k / 256) * (uint32_t)mb * 4;
    return L;
}

__host__ __device__ inline uint32_t lds_bytes(int mb, uint32_t k, bool kquant) {
    const uint32_t flat = (uint32_t)mb * act_img(k, kquant).row_bytes;
    if (mb == 1) return flat;
    const uint32_t il = kquant ? il_lay(mb, k).bytes : 0u;
    return il > flat ? il : flat;
}

template <int DT, int MB>
__device__ __forceinline__ void compute_chunk_il(const Chunk& ch, uint32_t c, const IlLay& L,
                                                 const uint8_t* lds, float* acc) {
    static_assert(DT == XNQ_Q4K, "the interleaved staging holds Q4_K's f32 chunk bsums");
    int sc, mn;
    q4k_scale_min(ch.x.y, ch.x.z, ch.x.w, (int)(c & 7), sc, mn);
    const float cw = f16_bits_to_f32(ch.x.x) * (float)sc, cm = f16_bits_to_f32(ch.x.x >> 16) * (float)mn;
    const uint32_t u = c / 64, l = c % 64;
    const uint8_t* q0 = lds + (u * MB * 64 + l) * 16;
    const uint8_t* q1 = q0 + L.nu * (MB * 1024);
    const float* sv = reinterpret_cast<const float*>(lds + L.sv) + u * MB * 64 + l;
    const float* da = reinterpret_cast<const float*>(lds + L.da) + (c >> 3) * MB;
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const uint4 a0 = *reinterpret_cast<const uint4*>(q0 + mb * 1024);
        const uint4 a1 = *reinterpret_cast<const uint4*>(q1 + mb * 1024);
        const int a[8] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                          (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        // chunk_fma's Q4K combine with the bsum already summed in f32
        const int raw = nib_dot(ch.q, a);
        acc[mb] = fmaf(da[mb], fmaf(cw, (float)raw, -(cm * sv[mb * 64])), acc[mb]);
    }
}

// First staging batch of the quantized workspace, loaded into registers before
// the weight loads are issued so its (L2) latency overlaps them.
template <int MB, int NW>
struct StagePrefetch {
    static constexpr int kPer = 2;
    uint4 v[kPer];
    __device__ __forceinline__ void load(const AView& a, uint32_t m0, uint32_t mcount) {
        const uint32_t rb = a.A.row_bytes;
        const uint32_t live = (mcount < (uint32_t)MB ? mcount : MB) * rb / 16;
        const uint32_t total = (uint32_t)MB * rb / 16;
        const uint4* src = reinterpret_cast<const uint4*>(a.img + (size_t)m0 * rb);
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const uint32_t i = j * NW * kWave + threadIdx.x;
            v[j] = src[min(min(i, total - 1), live - 1)];
        }
    }
    // 16-byte piece i of the flat MB-row image, written to its place in the
    // interleaved layout (compute_chunk_il)
    __device__ __forceinline__ static void put_il(uint8_t* lds, const ActImg& A, const IlLay& L, uint32_t r,
                                                  uint32_t o, uint4 v) {
        if (o < A.k) {
            const uint32_t h = o >= A.k / 2 ? 1u : 0u;
            const uint32_t c = (o - h * (A.k / 2)) / 16;
            *reinterpret_cast<uint4*>(lds + (((h * L.nu + c / 64) * MB + r) * 64 + c % 64) * 16) = v;
            return;
        }
        // side words and d_a, dword by dword
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        const uint32_t nb = A.k / 256;
        uint32_t* sv = reinterpret_cast<uint32_t*>(lds + L.sv);
        uint32_t* da = reinterpret_cast<uint32_t*>(lds + L.da);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t ob = o + 4 * j;
            if (ob < A.d_off) {
                const uint32_t c = (ob - A.s_off) / 4;
                // the chunk's two 16-element bsums, summed, as f32 (exact)
                const float bsum = (float)((int)(int16_t)(w[j] & 0xffffu) + (int)(int16_t)(w[j] >> 16));
                sv[((c / 64) * MB + r) * 64 + c % 64] = __float_as_uint(bsum);
            } else {
                const uint32_t b = (ob - A.d_off) / 4;
                if (b < nb) da[b * MB + r] = w[j];
            }
        }
    }
    // Write the prefetched batch and copy whatever it did not cover, into the
    // interleaved layout.
    __device__ __forceinline__ void store_il(const AView& a, uint32_t m0, uint32_t mcount, const IlLay& L,
                                             uint8_t* lds) {
        const uint32_t rb = a.A.row_bytes, rb16 = rb / 16;
        const uint32_t total = (uint32_t)MB * rb16;
        const uint32_t live = (mcount < (uint32_t)MB ? mcount : MB) * rb16;
        constexpr uint32_t kStep = NW * kWave;
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const uint32_t i = j * kStep + threadIdx.x;
            // the prefetch clamped past-the-end lanes to the last live piece:
            // rows past mcount only ever hold copies, never read for output
            if (i < total) {
                const uint32_t r = i / rb16;
                put_il(lds, a.A, L, r, (i - r * rb16) * 16, i < live ? v[j] : make_uint4(0u, 0u, 0u, 0u));
            }
        }
        // the rest in batches of kBatch loads (one memory round trip per
        // batch), walking (row, piece) without a division per piece
        constexpr int kBatch = 4;
        const uint4* src = reinterpret_cast<const uint4*>(a.img + (size_t)m0 * rb);
        uint32_t i = kPer * kStep + threadIdx.x;
        uint32_t r = i / rb16, p = i - r * rb16;
        for (; i < total; i += kBatch * kStep) {
            uint4 vb[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; j++) vb[j] = src[min(i + j * kStep, live - 1)];
#pragma unroll
            for (int j = 0; j < kBatch; j++) {
                const uint32_t ij = i + j * kStep;
                if (ij < total) put_il(lds, a.A, L, r, p * 16, ij < live ? vb[j] : make_uint4(0u, 0u, 0u, 0u));
                p += kStep;
                while (p >= rb16) {
                    p -= rb16;
                    r++;
                }
            }
        }
    }
    // Write the prefetched batch and copy whatever it did not cover.
    __device__ __forceinline__ void store(const AView& a, uint32_t m0, uint32_t mcount, uint8_t* lds) {
        const uint32_t rb = a.A.row_bytes;
        const uint32_t total = (uint32_t)MB * rb / 16;
        const uint32_t live = (mcount < (uint32_t)MB ? mcount : MB) * rb / 16;
        uint4* dst = reinterpret_cast<uint4*>(lds);
        // Unconditional stores of unconditional loads (a load whose value is
        // used only under a condition gets moved behind the weight loads by
        // the compiler).  Lanes past the end rewrite the last slot with the
        // value it gets anyway; rows past mcount hold copies of the last live
        // data, whose outputs are never stored.
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const uint32_t i = min(j * NW * kWave + threadIdx.x, total - 1);
            dst[i] = v[j];
        }
        const uint4* src = reinterpret_cast<const uint4*>(a.img + (size_t)m0 * rb);
        for (uint32_t i = kPer * NW * kWave + threadIdx.x; i < total; i += NW * kWave)
            dst[i] = i < live ? src[i] : make_uint4(0u, 0u, 0u, 0u);
    }
};

// One wavefront per row group of R rows, NW wavefronts per workgroup.
template <int DT, int MB, int R, int CPL, int NW, bool FUSED>
__global__ __launch_bounds__(NW * 64) void matvec_kernel(WView w, AView a, const float* __restrict__ x,
                                                         uint32_t m0, uint32_t mcount,
                                                         float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool kq = is_kquant(DT);
    // interleaved staging (compute_chunk_il): Q4_K from 4 rows (4096 -> 14336
    // at m = 4: 14.0 against 14.7 us; 8192 -> 28672: 35 against 43).  At 2
    // rows, and for Q6_K, its per-chunk address work outweighs the per-row
    // savings (Q6_K 14336 -> 4096 at m = 2: 16.5 against 15.7).
    constexpr bool kIL = MB >= 4 && !FUSED && DT == XNQ_Q4K;
    const ActImg A = act_img(w.k, kq);
    const IlLay IL = il_lay(MB, w.k);
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t nchunks = w.k / 32;
    const uint32_t npass = (nchunks + 64 * CPL - 1) / (64 * CPL);
    const uint32_t ngroups = (w.n + R - 1) / R;
    const uint32_t gstride = gridDim.x * NW;
    // The fused Q4_K kernel runs one workgroup per CU (launch_one): there its
    // row groups go wave-major (g = wave * grid + block), so when they do not
    // divide evenly every CU and SIMD gets the same share of the extra ones
    // (4096 -> 14336: 56 rows per CU, where block-major order gave the first
    // 128 workgroups 64 and the rest 48).  Grids of several workgroups per
    // CU keep block-major order, which spreads them already.
    constexpr bool kWaveMajor = FUSED && DT == XNQ_Q4K;
    uint32_t g = kWaveMajor ? wave * gridDim.x + blockIdx.x : blockIdx.x * NW + wave;

    // Loads are unconditional (row and chunk clamped to the last valid one,
    // results past the end are never used): with no branches around them the
    // compiler counts outstanding loads exactly and waits for the activation
    // data without waiting for the weight stream behind it.
    Chunk ch[R][CPL];
    auto issue = [&](uint32_t grp, uint32_t pass) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = min(grp * R + r, w.n - 1);
#pragma unroll
            for (int v = 0; v < CPL; v++) {
                const uint32_t c = min(lane + 64 * (v + CPL * pass), nchunks - 1);
                load_chunk<DT>(w, row, c, ch[r][v]);
            }
        }
    };

    // Activation loads first (short, L2-resident), then this wavefront's
    // whole first row group; the activation image is built while the weight
    // loads travel.
    StagePrefetch<MB, NW> pre;
    // one round of the fused quantizer covers the row length one pass of
    // the weight loads covers (64 * CPL chunks): 64 * CPL * 32 / 256 blocks
    // over NW wavefronts (further rounds, for longer rows, in xq.rest)
    XQuant<DT, MB, NW, (CPL * 8 + NW - 1) / NW> xq;
    if (FUSED) xq.load(x, w.k, m0, mcount, xq.first(wave), lane);
    else pre.load(a, m0, mcount);
    issue(min(g, ngroups - 1), 0);
    if (FUSED) {
        xq.quant(lds, A, w.k, xq.first(wave), lane);
        xq.rest(x, w.k, m0, mcount, lds, A, wave, lane);
    } else if constexpr (kIL) {
        pre.store_il(a, m0, mcount, IL, lds);
    } else {
        pre.store(a, m0, mcount, lds);
    }
    __syncthreads();

    for (; g < ngroups; g += gstride) {
        float acc[R][MB];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < MB; i++) acc[r][i] = 0.0f;
        for (uint32_t p = 0; p < npass; p++) {
            if (p > 0) issue(g, p);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = g * R + r;
#pragma unroll
                for (int v = 0; v < CPL; v++) {
                    const uint32_t c = lane + 64 * (v + CPL * p);
                    if (row < w.n && c < nchunks) {
                        if constexpr (kIL) compute_chunk_il<DT, MB>(ch[r][v], c, IL, lds, acc[r]);
                        else compute_chunk<DT, MB>(ch[r][v], c, w.k, lds, A, acc[r]);
                    }
                }
            }
        }
        const uint32_t gn = g + gstride;
        if (gn < ngroups) issue(gn, 0);
        float out = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const float s = wave_sum(acc[r][i]);
                if (lane == (uint32_t)(r * MB + i)) out = s;
            }
        const uint32_t r = lane / MB, i = lane % MB;
        if (lane < (uint32_t)(R * MB) && i < mcount && g * R + r < w.n)
            y[(size_t)(m0 + i) * w.n + g * R + r] = out;
    }
}

// One activation row (m == 1, the decode step), f32 activation quantized in
// LDS by every workgroup, over a group of weights that share it:
//   plain / grouped: the rows of up to kMaxGroup weights (same dtype and K,
//     e.g. the q, k and v projections, llama.rs:156-158) form one row space;
//     each output row goes to its own weight's destination;
//   GATE: two weights of the same shape (gate, up), one output
//     y = silu(x . gate) * (x . up), the SwiGLU of llama.rs:258-264 with
//     silu(s) = s / (1 + exp(0 - s)) (cpu_backend.rs:354-356).
// Every wavefront owns R rows at a time (GATE: R rows of each weight): the
// activation loads, then every weight load of the wavefront's rows (K <= 64 *
// CPL * 32; longer rows take further passes), then the activation image is
// built in LDS while the weight stream is in flight.  The grid is capped at
// the workgroups resident at once; past that the wavefronts stride over the
// remaining row groups, each group's loads issued before the previous
// group's reduction.
template <int DT, int R, int CPL, int NW, bool GATE>
__global__ __launch_bounds__(NW * 64) void group_kernel(WGroup G, const float* __restrict__ x) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool kq = is_kquant(DT);
    constexpr int RR = GATE ? 2 * R : R;  // rows loaded per wavefront
    const uint32_t k = G.w[0].k;
    const ActImg A = act_img(k, kq);
    const uint32_t lane = threadIdx.x & (kWave - 1);
    // wavefront-uniform in an SGPR: the weight view G.w[t] of a row is then
    // read with scalar loads; indexed by a VGPR it is read with vector loads,
    // whose in-order wait would also wait for the activation load issued
    // before them and hold back the whole weight stream
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t nchunks = k / 32;
    const uint32_t npass = (nchunks + 64 * CPL - 1) / (64 * CPL);
    // row groups of R rows, grid-strided when the grid is smaller than the
    // group count (the launch caps it at the workgroups resident at once)
    const uint32_t ngroups = (G.rows + R - 1) / R, gstride = gridDim.x * NW;
    uint32_t grp = blockIdx.x * NW + wave;
    uint32_t row0 = grp * R;

    // weight t and local row of loaded row r (wavefront-uniform)
    auto locate = [&](int r, uint32_t& t, uint32_t& lr) {
        if (GATE) {
            t = r < R ? 0u : 1u;
            lr = min(row0 + (uint32_t)(r % R), G.rows - 1);
            return;
        }
        const uint32_t gr = min(row0 + (uint32_t)r, G.rows - 1);
        t = 0;
        lr = gr;
        if (G.count > 1 && gr >= G.row_end[0]) {
            t = 1;
            lr = gr - G.row_end[0];
            if (G.count > 2 && gr >= G.row_end[1]) {
                t = 2;
                lr = gr - G.row_end[1];
            }
        }
    };

    Chunk ch[RR][CPL];
    auto issue = [&](uint32_t pass) {
#pragma unroll
        for (int r = 0; r < RR; r++) {
            uint32_t t, lr;
            locate(r, t, lr);
            const WView& w = G.w[t];
#pragma unroll
            for (int v = 0; v < CPL; v++)
                load_chunk<DT>(w, lr, min(lane + 64 * (v + CPL * pass), nchunks - 1), ch[r][v]);
        }
    };

    XQuant<DT, 1, NW, (CPL * 64 + NW * 128 - 1) / (NW * 128)> xq;  // one round covers K = 64 * CPL * 32
    xq.load(x, k, 0, 1, xq.first(wave), lane);
    issue(0);
    // every weight load is issued before the quantizer's first use of x
    __builtin_amdgcn_sched_barrier(0);
    xq.quant(lds, A, k, xq.first(wave), lane);
    xq.rest(x, k, 0, 1, lds, A, wave, lane);
    __syncthreads();

    for (;;) {
        float acc[RR][1];
#pragma unroll
        for (int r = 0; r < RR; r++) acc[r][0] = 0.0f;
        for (uint32_t p = 0; p < npass; p++) {
            if (p > 0) issue(p);
#pragma unroll
            for (int r = 0; r < RR; r++)
#pragma unroll
                for (int v = 0; v < CPL; v++) {
                    const uint32_t c = lane + 64 * (v + CPL * p);
                    if (c < nchunks) compute_chunk<DT, 1>(ch[r][v], c, k, lds, A, acc[r]);
                }
        }
        // the next group's loads go out before this group's reduction
        const uint32_t cur = row0, next = grp + gstride;
        if (next < ngroups) {
            grp = next;
            row0 = next * R;
            issue(0);
        }
        float out = 0.0f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            float t = wave_sum(acc[r][0]);
            if (GATE) {
                const float u = wave_sum(acc[R + r][0]);
                t = t / (1.0f + expf(0.0f - t)) * u;
            }
            if (lane == (uint32_t)r) out = t;
        }
        const uint32_t gr = cur + lane;
        if (lane < (uint32_t)R && gr < G.rows) {
            if (GATE) {
                G.y[0][gr] = out;
            } else {
                uint32_t t = 0, lr = gr;
                if (G.count > 1 && gr >= G.row_end[0]) {
                    t = 1;
                    lr = gr - G.row_end[0];
                    if (G.count > 2 && gr >= G.row_end[1]) {
                        t = 2;
                        lr = gr - G.row_end[1];
                    }
                }
                G.y[t][lr] = out;
            }
        }
        if (next >= ngroups) break;
    }
}

// Occupancy (workgroups per CU) of one kernel at one LDS size, cached.
inline int wg_per_cu(const void* fn, int threads, uint32_t lds_bytes, int* num_cu) {
    static std::mutex mu;
    static std::map<std::pair<const void*, uint32_t>, int> cache;
    static int ncu = 0;
    std::lock_guard<std::mutex> lock(mu);
    if (ncu == 0) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        if (ncu <= 0) ncu = 1;
    }
    *num_cu = ncu;
    auto key = std::make_pair(fn, lds_bytes);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), threads,
                                                     lds_bytes) != hipSuccess || occ < 1)
        occ = 1;
    cache[key] = occ;
    return occ;
}

template <int DT, int MB, int R, int CPL, int NW, bool FUSED>
hipError_t launch_one(const WView& w, const AView& a, const float* x, uint32_t m0, uint32_t mc,
                      float* y, hipStream_t s) {
    static_assert(R * MB <= 64, "one output per lane");
    constexpr bool kq = is_kquant(DT);
    const uint32_t lds = lds_bytes(MB, w.k, kq);
    auto fn = matvec_kernel<DT, MB, R, CPL, NW, FUSED>;
    int ncu = 1;
    const int occ = wg_per_cu(reinterpret_cast<const void*>(fn), NW * kWave, lds, &ncu);
    const uint32_t ngroups = (w.n + R - 1) / R;
    const uint32_t need = (ngroups + NW - 1) / NW;
    // the fused Q4_K kernel runs one 16-wavefront workgroup per CU: each CU
    // then quantizes the row once, not twice (4096 -> 14336 step 9.27 ->
    // 8.82 us); Q4_0 (7.7 -> 9.4) and Q6_K (69.1 -> 69.7 on the lm_head)
    // keep the full occupancy.
    const int wg_cu = FUSED && DT == XNQ_Q4K ? 1 : occ;
    const uint32_t cap = (uint32_t)(wg_cu * ncu);
    const uint32_t grid = need < cap ? need : cap;
    hipLaunchKernelGGL(fn, dim3(grid), dim3(NW * kWave), lds, s, w, a, x, m0, mc, y);
    return hipGetLastError();
}

template <int DT, int R, int CPL, bool GATE>
hipError_t launch_group_one(const WGroup& g, const float* x, hipStream_t s) {
    constexpr bool kq = is_kquant(DT);
    constexpr int NW = 16;
    const uint32_t lds = lds_bytes(1, g.w[0].k, kq);
    auto fn = group_kernel<DT, R, CPL, NW, GATE>;
    int ncu = 1;
    const int occ = wg_per_cu(reinterpret_cast<const void*>(fn), NW * kWave, lds, &ncu);
    const uint32_t need = (g.rows + R * NW - 1) / (R * NW);
    const uint32_t cap = (uint32_t)(occ * ncu);
    const uint32_t grid = need < cap ? need : cap;
    hipLaunchKernelGGL(fn, dim3(grid), dim3(NW * kWave), lds, s, g, x);
    return hipGetLastError();
}

// Rows * chunks per lane are bounded so the weight registers fit without
// spilling (128 VGPRs at 16 wavefronts per workgroup): loaded rows x CPL <= 10.
template <int DT, int R, bool GATE>
hipError_t launch_group_r(int cpl, const WGroup& g, const float* x, hipStream_t s) {
    constexpr int kRows = GATE ? 2 * R : R;
    constexpr int kMaxCpl = kRows == 1 ? 8 : kRows == 2 ? 5 : 2;
    switch (cpl) {
    case 1: return launch_group_one<DT, R, 1, GATE>(g, x, s);
    case 2: return launch_group_one<DT, R, 2, GATE>(g, x, s);
    }
    if constexpr (kMaxCpl >= 5) {
        switch (cpl) {
        case 3: return launch_group_one<DT, R, 3, GATE>(g, x, s);
        case 4: return launch_group_one<DT, R, 4, GATE>(g, x, s);
        case 5: return launch_group_one<DT, R, 5, GATE>(g, x, s);
        }
    }
    if constexpr (kMaxCpl >= 8) {
        switch (cpl) {
        case 6: return launch_group_one<DT, R, 6, GATE>(g, x, s);
        case 7: return launch_group_one<DT, R, 7, GATE>(g, x, s);
        default: return launch_group_one<DT, R, 8, GATE>(g, x, s);
        }
    }
    return hipErrorInvalidValue;
}

// m == 1 over a weight group: chunks per lane cover the row in one pass up
// to K = 16384.  One row (GATE: one row of each weight) per wavefront: with
// the weight loads issued ahead of the quantizer, that measured fastest
// (decode step 1432 -> 1376 us against two rows per wavefront, which uses
// fewer workgroups and so quantizes the activation fewer times).
// Returns hipErrorNotSupported for a GATE shape past the register bound.
template <int DT, bool GATE>
hipError_t launch_group(const WGroup& g, const float* x, hipStream_t s) {
    const uint32_t nchunks = g.w[0].k / 32;
    const int cpl = (int)std::min<uint32_t>(8, (nchunks + 63) / 64);
    if (GATE && cpl > 5) return hipErrorNotSupported;
    return launch_group_r<DT, 1, GATE>(cpl, g, x, s);
}

inline int pick_cpl(uint32_t nchunks) {
    return nchunks <= 64 ? 1 : nchunks <= 128 ? 2 : nchunks <= 256 ? 4 : 8;
}

// One weight row per wavefront (more rows per wavefront cost occupancy and
// measured slower for every shape).  Wavefronts per workgroup: the fused
// kernels 16 (the workgroup shares the row's quantization); the workspace
// kernels at one row 8 for rows of 8 chunks per lane (K > 8192: 14336 ->
// 4096 Q4_K 8.25 against 8.87 us, Q4_0 7.97 against 8.97) and 4 for shorter
// rows (8192 -> 28672: 22.5 against 23.3), and at 2..8 rows 8, which stage
// the rows into LDS half as often (4096 -> 14336 at m = 4: 11.9 against
// 12.5 us).
template <int DT, int MB, int NW, bool FUSED>
hipError_t launch_by_cpl(int cpl, const WView& w, const AView& a, const float* x, uint32_t m0, uint32_t mc,
                         float* y, hipStream_t s) {
    switch (cpl) {
    case 1: return launch_one<DT, MB, 1, 1, NW, FUSED>(w, a, x, m0, mc, y, s);
    case 2: return launch_one<DT, MB, 1, 2, NW, FUSED>(w, a, x, m0, mc, y, s);
    case 4: return launch_one<DT, MB, 1, 4, NW, FUSED>(w, a, x, m0, mc, y, s);
    case 8: return launch_one<DT, MB, 1, 8, NW, FUSED>(w, a, x, m0, mc, y, s);
    }
    return hipErrorInvalidValue;
}

template <int DT, int MB, bool FUSED>
hipError_t launch_cpl(int cpl, const WView& w, const AView& a, const float* x, uint32_t m0, uint32_t mc, float* y,
                      hipStream_t s) {
    if constexpr (FUSED) return launch_by_cpl<DT, MB, 16, true>(cpl, w, a, x, m0, mc, y, s);
    if constexpr (MB > 1) return launch_by_cpl<DT, MB, 8, false>(cpl, w, a, x, m0, mc, y, s);
    if (cpl == 8) return launch_one<DT, 1, 1, 8, 8, false>(w, a, x, m0, mc, y, s);
    switch (cpl) {
    case 1: return launch_one<DT, 1, 1, 1, 4, false>(w, a, x, m0, mc, y, s);
    case 2: return launch_one<DT, 1, 1, 2, 4, false>(w, a, x, m0, mc, y, s);
    case 4: return launch_one<DT, 1, 1, 4, 4, false>(w, a, x, m0, mc, y, s);
    }
    return hipErrorInvalidValue;
}

// y[m x n] for all m rows, in launches of up to 8 rows: `fused` nonzero
// quantizes each launch's rows from f32 `x` in LDS (kFusedOneShot: at m == 1
// the one-shot group kernel, one wavefront per row, for small weights; else
// the persistent matvec kernel with 16-wavefront workgroups), zero reads the
// Q8 workspace `a`.
template <int DT>
hipError_t launch_dtype(const WView& w, const AView& a, const float* x, size_t m, float* y,
                        hipStream_t s, int fused) {
    constexpr bool kq = is_kquant(DT);
    int gmax = 8;
    while (gmax > 1 && lds_bytes(gmax, w.k, kq) > kMaxLds) gmax >>= 1;
    if (lds_bytes(gmax, w.k, kq) > kMaxLds) return hipErrorInvalidConfiguration;
    const int cpl = pick_cpl(w.k / 32);
    for (size_t m0 = 0; m0 < m; m0 += gmax) {
        const uint32_t mc = (uint32_t)((m - m0) < (size_t)gmax ? (m - m0) : (size_t)gmax);
        hipError_t e;
        if (mc == 1 && m == 1 && fused == kFusedOneShot) {
            WGroup g{};
            g.w[0] = w;
            g.y[0] = y;
            g.row_end[0] = w.n;
            g.count = 1;
            g.rows = w.n;
            e = launch_group<DT, false>(g, x, s);
        } else if (fused) {
            if (mc == 1) e = launch_cpl<DT, 1, true>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
            else if (mc == 2) e = launch_cpl<DT, 2, true>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
            else if (mc <= 4) e = launch_cpl<DT, 4, true>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
            else e = launch_cpl<DT, 8, true>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
        } else {
            if (mc == 1) e = launch_cpl<DT, 1, false>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
            else if (mc == 2) e = launch_cpl<DT, 2, false>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
            else if (mc <= 4) e = launch_cpl<DT, 4, false>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
            else e = launch_cpl<DT, 8, false>(cpl, w, a, x, (uint32_t)m0, mc, y, s);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace mv

template <int DT>
hipError_t launch_group_dt(const WGroup& g, const float* x, bool gate, hipStream_t s) {
    return gate ? mv::launch_group<DT, true>(g, x, s) : mv::launch_group<DT, false>(g, x, s);
}

hipError_t launch_matvec_q4_0(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q8_0(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q4k(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q6k(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q4_1(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q5_0(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q5_1(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q2k(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q3k(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_matvec_q5k(const WView&, const AView&, const float*, size_t, float*, hipStream_t, int);
hipError_t launch_group_q4_1(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q5_0(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q5_1(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q2k(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q3k(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q5k(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q4_0(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q8_0(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q4k(const WGroup&, const float*, bool, hipStream_t);
hipError_t launch_group_q6k(const WGroup&, const float*, bool, hipStream_t);

}  // namespace xnq
