// Wavefront-level activation quantizers shared by the standalone quantize
// kernels and the fused matvec prologue, so both produce identical bytes.
// They restate BlockQ8K::from_float (k_quants.rs:1942-1979) and
// BlockQ8_0::from_float (k_quants.rs:636-661); no multiply-add is contracted.
#pragma once

#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

// Cross-lane steps on the DPP path (no LDS round trip).  Controls:
// quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E, row_half_mirror = 0x141,
// row_shr:n = 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, true);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL, ROW_MASK>(__float_as_int(v)));
}

// Largest value over the wavefront (lanes shifted in from outside a row read
// 0, the identity here).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0x111>((int)v));
    v = max(v, (uint32_t)dpp_i<0x112>((int)v));
    v = max(v, (uint32_t)dpp_i<0x114>((int)v));
    v = max(v, (uint32_t)dpp_i<0x118>((int)v));
    v = max(v, (uint32_t)dpp_i<0x142, 0xa>((int)v));
    v = max(v, (uint32_t)dpp_i<0x143, 0xc>((int)v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// One 256-element Q8_K block per wavefront, elements 4*lane .. 4*lane+3 in `v`.
struct Q8KLane {
    uint32_t packed;  // this lane's 4 quants, little-endian bytes
    float d;          // block scale (same in every lane)
    int bsum;         // sum of the 16 quants of group lane/4 (same in lanes 4g..4g+3)
};

__device__ __forceinline__ Q8KLane q8k_quant_wave(float4 v, int lane) {
#pragma clang fp contract(off)
    (void)lane;
    const float xs[4] = {v.x, v.y, v.z, v.w};
    // Largest |x|; the reference keeps the first index on ties (strict
    // `amax < |x|`), so its signed value is taken from the lowest lane, and
    // the lowest element in that lane, holding an |x| equal to the maximum.
    // as bit patterns: non-negative floats order like their bits, and a NaN
    // (above the infinity pattern) is dropped as 0, as fmaxf drops it
    uint32_t lmax = 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t a = __float_as_uint(xs[i]) & 0x7fffffffu;
        lmax = max(lmax, a > 0x7f800000u ? 0u : a);
    }
    const float amax = __uint_as_float(wave_max_u32(lmax));
    int8_t q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (amax != 0.0f) {
        float cand = 0.0f;
        bool hit = false;
#pragma unroll
        for (int i = 3; i >= 0; i--)
            if (fabsf(xs[i]) == amax) {
                cand = xs[i];
                hit = true;
            }
        const unsigned long long mask = __ballot(hit);
        const int first = __builtin_ctzll(mask);
        const float max = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cand), first));
        const float iscale = -128.0f / max;
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = f_as_i8(fminf(roundf(iscale * xs[i]), 127.0f));
        d = 1.0f / iscale;
    }
    int s = (int)q[0] + q[1] + q[2] + q[3];
    s += dpp_i<0xB1>(s);
    s += dpp_i<0x4E>(s);
    Q8KLane r;
    r.packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
               ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
    r.d = d;
    r.bsum = s;
    return r;
}

// One 32-element Q8_0 block per 8 consecutive lanes; `sub` = lane & 7 holds
// elements 4*sub .. 4*sub+3.  Every lane of the 8 must call this together.
struct Q80Lane {
    uint32_t packed;
    uint16_t dh;  // f16 bits of the block scale
    int sum;      // sum of the 32 quants
};

__device__ __forceinline__ Q80Lane q80_quant_8lanes(float4 v) {
#pragma clang fp contract(off)
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, 0.0f);
    amax = fmaxf(amax, dpp_f<0xB1>(amax));
    amax = fmaxf(amax, dpp_f<0x4E>(amax));
    amax = fmaxf(amax, dpp_f<0x141>(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int8_t q0 = f_as_i8(roundf(v.x * id)), q1 = f_as_i8(roundf(v.y * id)),
                 q2 = f_as_i8(roundf(v.z * id)), q3 = f_as_i8(roundf(v.w * id));
    int s = (int)q0 + q1 + q2 + q3;
    s += dpp_i<0xB1>(s);
    s += dpp_i<0x4E>(s);
    s += dpp_i<0x141>(s);
    Q80Lane r;
    r.packed = (uint32_t)(uint8_t)q0 | ((uint32_t)(uint8_t)q1 << 8) | ((uint32_t)(uint8_t)q2 << 16) |
               ((uint32_t)(uint8_t)q3 << 24);
    r.dh = f32_to_f16_bits(d);
    r.sum = s;
    return r;
}

// Store one lane's share of a quantized Q8K block `bb` into a row image.
__device__ __forceinline__ void q8k_store(uint8_t* row, const ActImg& A, uint32_t bb, int lane,
                                          const Q8KLane& r) {
    *reinterpret_cast<uint32_t*>(row + act_q_off(A.k, bb * 256 + 4 * lane)) = r.packed;
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(row + A.s_off)[bb * 16 + (lane >> 2)] = (int16_t)r.bsum;
    if (lane == 0) reinterpret_cast<float*>(row + A.d_off)[bb] = r.d;
}

// Store one lane's share (sub = lane & 7) of quantized Q8_0 block `c` into a row image.
__device__ __forceinline__ void q80_store(uint8_t* row, const ActImg& A, uint32_t c, int sub,
                                          const Q80Lane& r) {
    *reinterpret_cast<uint32_t*>(row + act_q_off(A.k, c * 32 + 4 * sub)) = r.packed;
    if (sub == 0) {
        reinterpret_cast<int32_t*>(row + A.s_off)[c] = r.sum;
        reinterpret_cast<float*>(row + A.d_off)[c] = f16_bits_to_f32(r.dh);
    }
}

}  // namespace xnq
