// Wavefront-level activation quantizers shared by the standalone quantize
// kernels and the fused matvec prologue, so both produce identical bytes.
// They restate BlockQ8K::from_float (k_quants.rs:1942-1979) and
// BlockQ8_0::from_float (k_quants.rs:636-661); no multiply-add is contracted.
#pragma once

#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

// One 256-element Q8_K block per wavefront, elements 4*lane .. 4*lane+3 in `v`.
struct Q8KLane {
    uint32_t packed;  // this lane's 4 quants, little-endian bytes
    float d;          // block scale (same in every lane)
    int bsum;         // sum of the 16 quants of group lane/4 (same in lanes 4g..4g+3)
};

__device__ __forceinline__ Q8KLane q8k_quant_wave(float4 v, int lane) {
#pragma clang fp contract(off)
    const float xs[4] = {v.x, v.y, v.z, v.w};
    // Largest |x|, first index on ties (the reference's strict `amax < |x|`).
    float amax = 0.0f, max = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(xs[i]);
        if (amax < a) {
            amax = a;
            max = xs[i];
            idx = lane * 4 + i;
        }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float oa = __shfl_xor(amax, off);
        const int oi = __shfl_xor(idx, off);
        const float om = __shfl_xor(max, off);
        if ((oa > amax) || (oa == amax && oi < idx)) {
            amax = oa;
            idx = oi;
            max = om;
        }
    }
    int8_t q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -128.0f / max;
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = f_as_i8(fminf(roundf(iscale * xs[i]), 127.0f));
        d = 1.0f / iscale;
    }
    int s = (int)q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
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
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int8_t q0 = f_as_i8(roundf(v.x * id)), q1 = f_as_i8(roundf(v.y * id)),
                 q2 = f_as_i8(roundf(v.z * id)), q3 = f_as_i8(roundf(v.w * id));
    int s = (int)q0 + q1 + q2 + q3;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
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
