// Device-side helpers shared by the libxnq kernels: Rust cast semantics,
// f16 conversion, and the per-chunk integer dot products of each GGML type.
// A chunk is 32 consecutive elements of one weight row (see xnq_internal.h).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace xnq {

// ---- scalar semantics of the reference (Rust) -----------------------------

// f32 `as i8`: saturating, NaN -> 0, else truncated toward zero.  Branch
// free: NaN replaced by 0, clamped to [-128, 127] with med3, then converted.
__device__ __forceinline__ int8_t f_as_i8(float v) {
    const float c = __builtin_amdgcn_fmed3f(v == v ? v : 0.0f, -128.0f, 127.0f);
    return (int8_t)(int)c;
}
__device__ __forceinline__ uint8_t f_as_u8(float v) {
    if (v != v) return 0;
    if (v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)(int)v;
}
__device__ __forceinline__ int32_t f_as_i32(float v) {
    if (v != v) return 0;
    if (v <= -2147483648.0f) return INT32_MIN;
    if (v >= 2147483647.0f) return INT32_MAX;
    return (int32_t)v;
}
// utils.rs:3-5 nearest_int: f32::round (half away from zero) then `as i32`.
__device__ __forceinline__ int32_t nearest_int(float v) { return f_as_i32(roundf(v)); }
__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// IEEE binary16 conversions (round to nearest even on the way down).
// The empty asm keeps the compiler from fusing the conversion with the
// multiply that produced `f` (a mixed-precision fma with a +0 addend, which
// would turn a -0 product into +0).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    __asm__ volatile("" : "+v"(f));
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
    return (float)h;
}

// Four f32 values as bf16 high parts (round to nearest even) and bf16
// remainders (v - hi, so hi + lo carries ~16 significant bits), packed as
// 16 bytes: the 4 high parts, then the 4 remainders.
__device__ __forceinline__ uint4 bf16_hilo4(const float* v) {
    typedef __bf16 v4bf_t __attribute__((ext_vector_type(4)));
    v4bf_t h, l;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const __bf16 hb = (__bf16)v[t];
        h[t] = hb;
        l[t] = (__bf16)(v[t] - (float)hb);
    }
    const uint2 hu = __builtin_bit_cast(uint2, h), lu = __builtin_bit_cast(uint2, l);
    return make_uint4(hu.x, hu.y, lu.x, lu.y);
}

// ---- packed integer dots ---------------------------------------------------

__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Sum over 32 elements of nibble * q8, with the nibble order
//   dword w of q: low nibbles = elements 4w..4w+3, high = elements 16+4w..16+4w+3
// and a[0..7] the 32 activation bytes as 8 dwords.
__device__ __forceinline__ void nib_dot2(uint4 q, const int* a, int& lo, int& hi) {
    const uint32_t M = 0x0F0F0F0Fu;
    int l = 0, h = 0;
    l = dot4((int)(q.x & M), a[0], l);
    l = dot4((int)(q.y & M), a[1], l);
    l = dot4((int)(q.z & M), a[2], l);
    l = dot4((int)(q.w & M), a[3], l);
    h = dot4((int)((q.x >> 4) & M), a[4], h);
    h = dot4((int)((q.y >> 4) & M), a[5], h);
    h = dot4((int)((q.z >> 4) & M), a[6], h);
    h = dot4((int)((q.w >> 4) & M), a[7], h);
    lo = l;
    hi = h;
}

// sum of q*a over the 32 nibbles of q (low nibbles against a[0..3], high
// against a[4..7]) in one dependency chain
__device__ __forceinline__ int nib_dot(uint4 q, const int* a) {
    const uint32_t M = 0x0F0F0F0Fu;
    int s = dot4((int)(q.x & M), a[0], 0);
    s = dot4((int)(q.y & M), a[1], s);
    s = dot4((int)(q.z & M), a[2], s);
    s = dot4((int)(q.w & M), a[3], s);
    s = dot4((int)((q.x >> 4) & M), a[4], s);
    s = dot4((int)((q.y >> 4) & M), a[5], s);
    s = dot4((int)((q.z >> 4) & M), a[6], s);
    return dot4((int)((q.w >> 4) & M), a[7], s);
}

// Q4K: 6-bit scale and min of sub-block j from the 12 packed bytes
// (utils.rs:53-63 get_scale_min_k4); s0,s1,s2 = scales bytes 0-3, 4-7, 8-11.
// Branch-free: both cases are "a nibble of one byte | the top 2 bits of
// another << 4" on byte jj = j & 3 of one of the three dwords:
//   j < 4:  sc = q[j] & 63          = nib(s0, 0) | top2(s0, 4)
//           m  = q[j + 4] & 63      = nib(s1, 0) | top2(s1, 4)
//   j >= 4: sc = (q[j + 4] & 15) | (q[j - 4] >> 6) << 4 = nib(s2, 0) | top2(s0, 6)
//           m  = (q[j + 4] >> 4) | (q[j] >> 6) << 4     = nib(s2, 4) | top2(s1, 6)
// so a lane-dependent j costs two selects and four bit-field extracts, not
// both sides of a divergent branch.
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              int& sc, int& m) {
    const bool hi = j >= 4;
    const uint32_t b = 8u * (uint32_t)(j & 3), o = hi ? 6u : 4u;
    const uint32_t xs = hi ? s2 : s0, xm = hi ? s2 : s1, om = hi ? 4u : 0u;
    sc = (int)(__builtin_amdgcn_ubfe(xs, b, 4) | (__builtin_amdgcn_ubfe(s0, b + o, 2) << 4));
    m = (int)(__builtin_amdgcn_ubfe(xm, b + om, 4) | (__builtin_amdgcn_ubfe(s1, b + o, 2) << 4));
}

// All eight 6-bit scales and mins of a Q4K block header at once, four per
// dword: byte r of sc_lo / sc_hi is the scale of sub-block r / 4 + r, the
// same for m_lo / m_hi (the get_scale_min_k4 cases of utils.rs:53-63 applied
// bytewise: j < 4 takes the low 6 bits of q[j] and q[j + 4]; j >= 4 takes a
// nibble of q[j + 4] and the top 2 bits of q[j - 4] resp. q[j]).
struct Q4KScales {
    uint32_t sc_lo, sc_hi, m_lo, m_hi;
};
__host__ __device__ __forceinline__ Q4KScales q4k_scales(uint32_t s0, uint32_t s1, uint32_t s2) {
    Q4KScales q;
    q.sc_lo = s0 & 0x3f3f3f3fu;
    q.sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    q.m_lo = s1 & 0x3f3f3f3fu;
    q.m_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    return q;
}

// The 16 six-bit Q3K scales (0..63): byte g of the aux words that
// k_quants.rs:1252-1258 builds from the 12 packed bytes s0, s1, s2.
__device__ __forceinline__ int q3k_scale(uint32_t s0, uint32_t s1, uint32_t s2, int g) {
    const uint32_t K1 = 0x03030303u, K2 = 0x0f0f0f0fu;
    uint32_t a;
    switch (g >> 2) {
    case 0: a = (s0 & K2) | ((s2 & K1) << 4); break;
    case 1: a = (s1 & K2) | (((s2 >> 2) & K1) << 4); break;
    case 2: a = ((s0 >> 4) & K2) | (((s2 >> 4) & K1) << 4); break;
    default: a = ((s1 >> 4) & K2) | (((s2 >> 6) & K1) << 4); break;
    }
    return (int)((a >> (8 * (g & 3))) & 0xffu);
}

// Q6K: the 8 dwords of 6-bit values (0..63) of one chunk.
__device__ __forceinline__ void q6k_unpack(uint4 ql, uint2 qh, int* b) {
    const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x03030303u;
    b[0] = (int)((ql.x & M4) | ((qh.x & M2) << 4));
    b[1] = (int)((ql.y & M4) | (((qh.x >> 2) & M2) << 4));
    b[2] = (int)((ql.z & M4) | (((qh.x >> 4) & M2) << 4));
    b[3] = (int)((ql.w & M4) | (((qh.x >> 6) & M2) << 4));
    b[4] = (int)(((ql.x >> 4) & M4) | ((qh.y & M2) << 4));
    b[5] = (int)(((ql.y >> 4) & M4) | (((qh.y >> 2) & M2) << 4));
    b[6] = (int)(((ql.z >> 4) & M4) | (((qh.y >> 4) & M2) << 4));
    b[7] = (int)(((ql.w >> 4) & M4) | (((qh.y >> 6) & M2) << 4));
}

// ---- LDS DMA (the int8-MFMA kernels) ---------------------------------------

// global_load_lds: uniform 64-bit base + 32-bit per-lane byte offset; m0
// holds the LDS address lane 0 writes (lane i writes i * size beyond it).
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr),
                 "v"(off), "s"(base)
                 : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_addr),
                 "v"(off), "s"(base)
                 : "memory");
}

// s_waitcnt vmcnt(N) for a compile-time N
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// bytes of d (each <= 15) times s (<= 7): every product is <= 105, so no
// carry leaves its byte and one packed 16-bit multiply does all four
__device__ __forceinline__ uint32_t mul_bytes(uint32_t d, uint32_t s) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 s2 = {(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, d) * s2);
}

// Q6K digit planes of 4 six-bit values (bytes of q) times a signed scale,
// for the int8 matrix cores (the skinny and tiled kernels):
// w = sc * (q - 32) in [-3968, 4096]; w + 128 = 256 * hi + u with u in
// [0, 255], so w = 256 * hi + lo with hi = byte 1 of w + 128 (in [-15, 16])
// and lo = u - 128 (byte 0 of w + 128 with its top bit flipped).
__device__ __forceinline__ void q6_digits(uint32_t q, int sc, uint32_t& lo, uint32_t& hi) {
    typedef short s16x2 __attribute__((ext_vector_type(2)));
    // bytes 0, 1 and 2, 3 of q zero-extended to 16-bit lanes
    const s16x2 x01 = __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, q, 0x0C010C00u));
    const s16x2 x23 = __builtin_bit_cast(s16x2, __builtin_amdgcn_perm(0u, q, 0x0C030C02u));
    // (q - 32) * sc + 128 as q * sc + (128 - 32 sc): one packed multiply-add per pair
    const s16x2 s2 = {(short)sc, (short)sc};
    const s16x2 c2 = {(short)(128 - 32 * sc), (short)(128 - 32 * sc)};
    const uint32_t w01 = __builtin_bit_cast(uint32_t, x01 * s2 + c2);
    const uint32_t w23 = __builtin_bit_cast(uint32_t, x23 * s2 + c2);
    lo = __builtin_amdgcn_perm(w23, w01, 0x06040200u) ^ 0x80808080u;
    hi = __builtin_amdgcn_perm(w23, w01, 0x07050301u);
}

// Integer dot of one Q6K chunk: sc0 * sum_{16}(q6-32)*q8 + sc1 * (next 16),
// using sum (q-32)*a = sum q*a - 32*sum a with the Q8K block sums.
__device__ __forceinline__ int q6k_chunk_int(uint4 ql, uint2 qh, const int* a, int sc0, int sc1,
                                             int bs0, int bs1) {
    int b[8];
    q6k_unpack(ql, qh, b);
    int lo = 0, hi = 0;
    lo = dot4(b[0], a[0], lo);
    lo = dot4(b[1], a[1], lo);
    lo = dot4(b[2], a[2], lo);
    lo = dot4(b[3], a[3], lo);
    hi = dot4(b[4], a[4], hi);
    hi = dot4(b[5], a[5], hi);
    hi = dot4(b[6], a[6], hi);
    hi = dot4(b[7], a[7], hi);
    // |lo - 32*bs0| <= 16*63*128 + 32*16*128 < 2^23: the 24-bit multiply is exact
    return __mul24(sc0, lo - 32 * bs0) + __mul24(sc1, hi - 32 * bs1);
}

// Sum of 32 signed bytes x signed bytes.
__device__ __forceinline__ int i8_dot32(uint4 w0, uint4 w1, const int* a) {
    int s = 0;
    s = dot4((int)w0.x, a[0], s);
    s = dot4((int)w0.y, a[1], s);
    s = dot4((int)w0.z, a[2], s);
    s = dot4((int)w0.w, a[3], s);
    s = dot4((int)w1.x, a[4], s);
    s = dot4((int)w1.y, a[5], s);
    s = dot4((int)w1.z, a[6], s);
    s = dot4((int)w1.w, a[7], s);
    return s;
}

}  // namespace xnq
