// Quantizers on the device, bit-identical to xn's CPU quantizers:
//   * activations ("lhs") to Q8_0 / Q8_K, into the private planar workspace
//     used by the matmul kernels or into canonical GGUF blocks;
//   * weights (QTensor::quantize_f32) to GGUF blocks of every device dtype.
// No multiply-add is fused in this file, so every f32 operation rounds exactly
// where the reference's does.
#pragma clang fp contract(off)

#include "xnq_device.h"
#include "xnq_internal.h"
#include "xnq_quant_dev.h"

namespace xnq {

namespace {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Q8_K activations, k_quants.rs:1942-1979.  One wavefront per 256-element
// block, four consecutive elements per lane.
// ---------------------------------------------------------------------------
template <bool CANONICAL>
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float* __restrict__ x,
                                                            size_t nblocks, ActImg A,
                                                            uint8_t* __restrict__ out) {
    const int lane = threadIdx.x & (kWave - 1);
    const size_t blk = (size_t)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave);
    if (blk >= nblocks) return;  // uniform over the wavefront
    const float4 v = reinterpret_cast<const float4*>(x + blk * 256)[lane];
    const Q8KLane r = q8k_quant_wave(v, lane);
    if (CANONICAL) {
        // BlockQ8K: f32 d; i8 qs[256]; i16 bsums[16]  (292 bytes, 4-byte aligned)
        uint8_t* b = out + blk * 292;
        reinterpret_cast<uint32_t*>(b + 4)[lane] = r.packed;
        if (lane == 0) *reinterpret_cast<float*>(b) = r.d;
        if ((lane & 3) == 0) reinterpret_cast<int16_t*>(b + 260)[lane >> 2] = (int16_t)r.bsum;
    } else {
        const size_t bpr = A.k / 256;
        const size_t row = blk / bpr, sb = blk % bpr;
        q8k_store(out + row * A.row_bytes, A, (uint32_t)sb, lane, r);
    }
}

// Q8_K activations for the prefill kernel: the row image plus its row-tiled
// copy.  One workgroup of R wavefronts per (64-row block, super-block, R-row
// group); wavefront w quantizes row w of the group.  Every R x 16-byte run of
// the tiled copy (whole cache lines for R >= 8) is assembled in LDS and stored
// by one workgroup, so no cache line of the copy is written piecewise from
// workgroups that sit on different XCDs (different L2s).  Rows past m (the
// padding of the last 64-row block) are stored as zeros.
template <int R>
__global__ __launch_bounds__(64 * R) void quantize_q8k_tiled_kernel(const float* __restrict__ x, uint32_t m,
                                                                     ActImg A, uint8_t* __restrict__ out,
                                                                     uint8_t* __restrict__ tile, TileImg T) {
    static_assert(R == 8 || R == 16, "8 or 16 rows per workgroup");
    constexpr uint32_t kGroups = 64 / R, kPitch = R * 16 + 16;  // + 16 bytes against LDS bank conflicts
    __shared__ __align__(16) uint8_t sq[16 * kPitch];  // [stage * 4 + piece][row][16]
    __shared__ __align__(16) float sd[R];              // d by row
    __shared__ __align__(16) int16_t ss[2][R][8];      // bsums [half][row][g & 7]
    const int lane = threadIdx.x & (kWave - 1), rr = threadIdx.x / kWave;
    const uint32_t bpr = A.k / 256;
    const uint32_t grp = blockIdx.x % kGroups, rest = blockIdx.x / kGroups;
    const uint32_t sb = rest % bpr, rb = rest / bpr;
    const uint32_t row = rb * 64 + grp * R + rr;
    const float4 v = row < m ? reinterpret_cast<const float4*>(x + (size_t)row * A.k + (size_t)sb * 256)[lane]
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    const Q8KLane r = q8k_quant_wave(v, lane);
    if (row < m) q8k_store(out + (size_t)row * A.row_bytes, A, sb, lane, r);
    // lane's 4 quants: stage lane / 16, piece (lane / 4) & 3, bytes 4 * (lane & 3)
    *reinterpret_cast<uint32_t*>(sq + (lane >> 2) * kPitch + rr * 16 + 4 * (lane & 3)) = r.packed;
    if (lane == 0) sd[rr] = r.d;
    if ((lane & 3) == 0) ss[lane >> 5][rr][(lane >> 2) & 7] = (int16_t)r.bsum;
    __syncthreads();
    const uint32_t t = threadIdx.x;
    const size_t rs = (size_t)rb * bpr + sb;
    const uint32_t r64 = grp * R;  // first row of the group in its 64-row block
    if (t < 16 * R) {
        const uint32_t seg = t / R, i = t % R;
        const uint4 val = *reinterpret_cast<const uint4*>(sq + seg * kPitch + i * 16);
        *reinterpret_cast<uint4*>(tile + (size_t)rb * 64 * A.k + (size_t)(4 * sb + (seg >> 2)) * 4096 +
                                  (seg & 3) * 1024 + (r64 + i) * 16) = val;
    } else if (t < 16 * R + R / 4) {
        const uint32_t i = t - 16 * R;
        reinterpret_cast<uint4*>(tile + T.d_off + rs * 256 + r64 * 4)[i] = reinterpret_cast<const uint4*>(sd)[i];
    } else if (t >= 16 * R + 64 && t < 18 * R + 64) {  // the bsums from a wavefront of their own
        const uint32_t i = t - (16 * R + 64), half = i / R, j = i % R;
        *reinterpret_cast<uint4*>(tile + T.s_off + (rs * 2 + (r64 >> 5)) * 1024 + half * 512 + ((r64 & 31) + j) * 16) =
            *reinterpret_cast<const uint4*>(&ss[half][j][0]);
    } else if (t >= 18 * R + 64 && t < 20 * R + 64) {  // the Q4K min-term operand
        const uint32_t i = t - (18 * R + 64), half = i / R, j = i % R;
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = -sd[j] * (float)((int)ss[half][j][2 * u] + (int)ss[half][j][2 * u + 1]);
        *reinterpret_cast<uint4*>(tile + T.x_off + (rs * 2 + (r64 >> 5)) * 1024 + half * 512 + ((r64 & 31) + j) * 16) =
            bf16_hilo4(v);
    }
}

// ---------------------------------------------------------------------------
// Q8_0 activations, k_quants.rs:636-661.  Eight lanes per 32-element block.
// ---------------------------------------------------------------------------
template <bool CANONICAL>
__global__ __launch_bounds__(256) void quantize_q80_kernel(const float* __restrict__ x,
                                                            size_t nblocks, ActImg A,
                                                            uint8_t* __restrict__ out) {
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t blk = t / 8;
    const int sub = (int)(t & 7);
    const bool live = blk < nblocks;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = reinterpret_cast<const float4*>(x + blk * 32)[sub];
    const Q80Lane r = q80_quant_8lanes(v);
    if (!live) return;
    if (CANONICAL) {
        // BlockQ8_0: f16 d; i8 qs[32]  (34 bytes, 2-byte aligned)
        uint8_t* b = out + blk * 34;
        uint16_t* w = reinterpret_cast<uint16_t*>(b + 2 + 4 * sub);
        w[0] = (uint16_t)(r.packed & 0xffffu);
        w[1] = (uint16_t)(r.packed >> 16);
        if (sub == 0) *reinterpret_cast<uint16_t*>(b) = r.dh;
    } else {
        const size_t bpr = A.k / 32;
        q80_store(out + (blk / bpr) * A.row_bytes, A, (uint32_t)(blk % bpr), sub, r);
    }
}

// ---------------------------------------------------------------------------
// Weight quantizers (one thread per GGUF block), restating the CPU code path
// of QTensor::quantize_f32.
// ---------------------------------------------------------------------------

// k_quants.rs:636-661
__global__ void w_q80_kernel(const float* __restrict__ x, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float* xs = x + i * 32;
    uint8_t* b = out + i * 34;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xs[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_bits(d);
    b[0] = (uint8_t)dh;
    b[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)f_as_i8(roundf(xs[j] * id));
}

// k_quants.rs:235-270
__global__ void w_q40_kernel(const float* __restrict__ x, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float* xs = x + i * 32;
    uint8_t* b = out + i * 18;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; j++) {
        if (amax < fabsf(xs[j])) {
            amax = fabsf(xs[j]);
            max = xs[j];
        }
    }
    const float d = max / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_bits(d);
    b[0] = (uint8_t)dh;
    b[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 16; j++) {
        const float x0 = xs[j] * id;
        const float x1 = xs[16 + j] * id;
        uint8_t xi0 = f_as_u8(x0 + 8.5f);
        uint8_t xi1 = f_as_u8(x1 + 8.5f);
        if (xi0 > 15) xi0 = 15;
        if (xi1 > 15) xi1 = 15;
        b[2 + j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

// Rust's f32::total_cmp order as an integer key.
__device__ __forceinline__ int32_t total_key(float f) {
    int32_t i = __builtin_bit_cast(int32_t, f);
    return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

// utils.rs:205-254 make_qkx1_quants(nmax, ntry, x[0..N]); returns scale, -min.
template <int N>
__device__ float make_qkx1_quants(int nmax, int ntry, const float* x, float* neg_min) {
    uint8_t l[N];
    for (int i = 0; i < N; i++) l[i] = 0;
    float mn = x[0], mx = x[0];
    for (int i = 1; i < N; i++) {
        if (total_key(x[i]) < total_key(mn)) mn = x[i];
        if (total_key(x[i]) >= total_key(mx)) mx = x[i];
    }
    if (mx == mn) {
        *neg_min = 0.0f;
        return 0.0f;
    }
    float min = fminf(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int t = 0; t < ntry; t++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        bool did_change = false;
        for (int i = 0; i < N; i++) {
            const float value = x[i];
            const int32_t li = clampi(nearest_int(iscale * (value - min)), 0, nmax);
            const uint8_t cl = (uint8_t)li;
            if (cl != l[i]) {
                l[i] = cl;
                did_change = true;
            }
            sumlx += (value - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < N; i++) sum += x[i] - scale * (float)l[i];
        min = sum / (float)N;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *neg_min = -min;
    return scale;
}

__device__ __forceinline__ void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// k_quants.rs:1418-1473
__global__ void w_q4k_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const float* x = xin + bi * 256;
    uint8_t sc12[12];
    for (int i = 0; i < 12; i++) sc12[i] = 0;
    float mins[8], scales[8];
    for (int j = 0; j < 8; j++) scales[j] = make_qkx1_quants<32>(15, 5, x + 32 * j, &mins[j]);
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        max_scale = fmaxf(scales[j], max_scale);
        max_min = fmaxf(mins[j], max_min);
    }
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 8; j++) {
        int32_t a = nearest_int(inv_scale * scales[j]);
        if (a > 63) a = 63;
        int32_t b = nearest_int(inv_min * mins[j]);
        if (b > 63) b = 63;
        const uint8_t ls = (uint8_t)a, lm = (uint8_t)b;
        if (j < 4) {
            sc12[j] = ls;
            sc12[j + 4] = lm;
        } else {
            sc12[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc12[j - 4] |= (uint8_t)((ls >> 4) << 6);
            sc12[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t dh = f32_to_f16_bits(max_scale / 63.0f);
    const uint16_t mh = f32_to_f16_bits(max_min / 63.0f);
    uint8_t* blk = out + bi * 144;
    blk[0] = (uint8_t)dh;
    blk[1] = (uint8_t)(dh >> 8);
    blk[2] = (uint8_t)mh;
    blk[3] = (uint8_t)(mh >> 8);
    for (int i = 0; i < 12; i++) blk[4 + i] = sc12[i];
    const float df = f16_bits_to_f32(dh), mf = f16_bits_to_f32(mh);
    // Quantize one 64-element half-pair at a time and pack straight into qs.
    for (int p = 0; p < 4; p++) {
        uint8_t sc0, m0, sc1, m1;
        get_scale_min_k4(2 * p, sc12, &sc0, &m0);
        get_scale_min_k4(2 * p + 1, sc12, &sc1, &m1);
        const float d0 = df * (float)sc0, d1 = df * (float)sc1;
        const float dm0 = mf * (float)m0, dm1 = mf * (float)m1;
        for (int lv = 0; lv < 32; lv++) {
            uint8_t lo = 0, hi = 0;
            if (d0 != 0.0f) lo = (uint8_t)clampi(nearest_int((x[64 * p + lv] + dm0) / d0), 0, 15);
            if (d1 != 0.0f) hi = (uint8_t)clampi(nearest_int((x[64 * p + 32 + lv] + dm1) / d1), 0, 15);
            blk[16 + 32 * p + lv] = (uint8_t)(lo | (hi << 4));
        }
    }
}

// utils.rs:65-202 make_qx_quants(16, nmax, x, ls, rmse_type = 1)
__device__ float make_qx_quants16(int nmax, const float* x, int8_t* ls) {
    const int n = 16;
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) ls[i] = 0;
        return 0.0f;
    }
    const float iscale = -(float)nmax / max;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        const float xi = x[i];
        const int32_t l = clampi(nearest_int(iscale * xi), -nmax, nmax - 1);
        ls[i] = (int8_t)(l + nmax);
        const float w = xi * xi;
        const float lf = (float)l;
        sumlx += w * xi * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        const float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        bool changed = false;
        for (int i = 0; i < n; i++) {
            const float xi = x[i];
            const int32_t l = clampi(nearest_int(is2 * xi), -nmax, nmax - 1);
            if (l + nmax != (int32_t)ls[i]) changed = true;
            const float w = xi * xi;
            const float lf = (float)l;
            slx += w * xi * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            const int32_t l = nearest_int(is2 * x[i]);
            ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
    }
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
        for (int i = 0; i < n; i++) {
            const float xi = x[i];
            const float w = xi * xi;
            const int32_t l = (int32_t)ls[i] - nmax;
            float slx = sumlx - w * xi * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                const int32_t new_l = clampi(nearest_int(xi * sl2 / slx), -nmax, nmax - 1);
                if (new_l != l) {
                    slx += w * xi * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        ls[i] = (int8_t)(nmax + new_l);
                        sumlx = slx;
                        suml2 = sl2;
                        scale = sumlx / suml2;
                        best = scale * sumlx;
                        n_changed++;
                    }
                }
            }
        }
        if (n_changed == 0) break;
    }
    (void)best;
    return scale;
}

// k_quants.rs:1801-1871
__global__ void w_q6k_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const float* x = xin + bi * 256;
    int8_t L[256];
    float scales[16];
    float max_scale = 0.0f, max_abs_scale = 0.0f;
    for (int ib = 0; ib < 16; ib++) {
        const float scale = make_qx_quants16(32, x + 16 * ib, L + 16 * ib);
        scales[ib] = scale;
        const float abs_scale = fabsf(scale);
        if (abs_scale > max_abs_scale) {
            max_abs_scale = abs_scale;
            max_scale = scale;
        }
    }
    const float iscale = -128.0f / max_scale;
    const uint16_t dh = f32_to_f16_bits(1.0f / iscale);
    uint8_t* y = out + bi * 210;
    int8_t ysc[16];
    for (int j = 0; j < 16; j++) {
        int32_t v = nearest_int(iscale * scales[j]);
        if (v > 127) v = 127;
        ysc[j] = (int8_t)v;
        y[192 + j] = (uint8_t)ysc[j];
    }
    y[208] = (uint8_t)dh;
    y[209] = (uint8_t)(dh >> 8);
    const float df = f16_bits_to_f32(dh);
    for (int j = 0; j < 16; j++) {
        const float d = df * (float)ysc[j];
        if (d == 0.0f) continue;
        for (int ii = 0; ii < 16; ii++) {
            const int32_t ll = clampi(nearest_int(x[16 * j + ii] / d), -32, 31);
            L[16 * j + ii] = (int8_t)(ll + 32);
        }
    }
    for (int j = 0; j < 256; j += 128) {
        uint8_t* ql = y + (j / 128) * 64;
        uint8_t* qh = y + 128 + (j / 128) * 32;
        for (int l = 0; l < 32; l++) {
            const uint8_t q1 = (uint8_t)(L[j + l] & 0xF), q2 = (uint8_t)(L[j + l + 32] & 0xF);
            const uint8_t q3 = (uint8_t)(L[j + l + 64] & 0xF), q4 = (uint8_t)(L[j + l + 96] & 0xF);
            ql[l] = (uint8_t)(q1 | (q3 << 4));
            ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
            qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                              ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
        }
    }
}

// ---------------------------------------------------------------------------
// The other GGUF weight types, one thread per block, step for step as xn's
// from_float.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
__device__ __forceinline__ void put32(uint8_t* p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}

// k_quants.rs:345-377 BlockQ4_1::from_float: {d, m, qs[16]}
__global__ void w_q41_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float* x = xin + i * 32;
    uint8_t* b = out + i * 20;
    float min = INFINITY, max = -INFINITY;
    for (int j = 0; j < 32; j++) {
        min = fminf(x[j], min);
        max = fmaxf(x[j], max);
    }
    const float d = (max - min) / 15.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(b, f32_to_f16_bits(d));
    put16(b + 2, f32_to_f16_bits(min));
    for (int j = 0; j < 16; j++) {
        uint8_t xi0 = f_as_u8((x[j] - min) * id + 0.5f), xi1 = f_as_u8((x[16 + j] - min) * id + 0.5f);
        if (xi0 > 15) xi0 = 15;
        if (xi1 > 15) xi1 = 15;
        b[4 + j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

// k_quants.rs:442-476 BlockQ5_0::from_float: {d, qh[4], qs[16]}
__global__ void w_q50_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float* x = xin + i * 32;
    uint8_t* b = out + i * 22;
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; j++)
        if (amax < fabsf(x[j])) {
            amax = fabsf(x[j]);
            max = x[j];
        }
    const float d = max / -16.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(b, f32_to_f16_bits(d));
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        const int8_t a0 = f_as_i8(x[j] * id + 16.5f), a1 = f_as_i8(x[j + 16] * id + 16.5f);
        const uint8_t xi0 = (uint8_t)(a0 < 31 ? a0 : 31), xi1 = (uint8_t)(a1 < 31 ? a1 : 31);
        b[6 + j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
        qh |= (((uint32_t)xi0 & 0x10) >> 4) << j;
        qh |= (((uint32_t)xi1 & 0x10) >> 4) << (j + 16);
    }
    put32(b + 2, qh);
}

// k_quants.rs:546-583 BlockQ5_1::from_float: {d, m, qh[4], qs[16]}
__global__ void w_q51_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float* x = xin + i * 32;
    uint8_t* b = out + i * 24;
    float min = INFINITY, max = -INFINITY;
    for (int j = 0; j < 32; j++) {
        min = fminf(x[j], min);
        max = fmaxf(x[j], max);
    }
    const float d = (max - min) / 31.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    put16(b, f32_to_f16_bits(d));
    put16(b + 2, f32_to_f16_bits(min));
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        const uint8_t xi0 = f_as_u8((x[j] - min) * id + 0.5f), xi1 = f_as_u8((x[16 + j] - min) * id + 0.5f);
        b[8 + j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
        qh |= (((uint32_t)xi0 & 0x10) >> 4) << j;
        qh |= (((uint32_t)xi1 & 0x10) >> 4) << (j + 16);
    }
    put32(b + 4, qh);
}

// k_quants.rs:951-1011 BlockQ2K::from_float: {scales[16], qs[64], d, dmin}
__global__ void w_q2k_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const float* x = xin + bi * 256;
    uint8_t* b = out + bi * 84;
    uint8_t* sc = b;
    const float q4scale = 15.0f;
    float mins[16], scales[16];
    for (int j = 0; j < 16; j++) scales[j] = make_qkx1_quants<16>(3, 5, x + 16 * j, &mins[j]);
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 16; j++) max_scale = fmaxf(scales[j], max_scale);
    for (int j = 0; j < 16; j++) max_min = fmaxf(mins[j], max_min);
    uint16_t dh, mh;
    if (max_scale > 0.0f) {
        const float iscale = q4scale / max_scale;
        for (int j = 0; j < 16; j++) sc[j] = (uint8_t)nearest_int(iscale * scales[j]);
        dh = f32_to_f16_bits(max_scale / q4scale);
    } else {
        for (int j = 0; j < 16; j++) sc[j] = 0;
        dh = f32_to_f16_bits(0.0f);
    }
    if (max_min > 0.0f) {
        const float iscale = q4scale / max_min;
        for (int j = 0; j < 16; j++) sc[j] = (uint8_t)(sc[j] | (uint8_t)((uint8_t)nearest_int(iscale * mins[j]) << 4));
        mh = f32_to_f16_bits(max_min / q4scale);
    } else {
        mh = f32_to_f16_bits(0.0f);
    }
    put16(b + 80, dh);
    put16(b + 82, mh);
    uint8_t L[256];
    for (int e = 0; e < 256; e++) L[e] = 0;
    const float df = f16_bits_to_f32(dh), mf = f16_bits_to_f32(mh);
    for (int j = 0; j < 16; j++) {
        const float d = df * (float)(sc[j] & 0xF);
        if (d == 0.0f) continue;
        const float dm = mf * (float)(sc[j] >> 4);
        for (int ii = 0; ii < 16; ii++) L[16 * j + ii] = (uint8_t)clampi(nearest_int((x[16 * j + ii] + dm) / d), 0, 3);
    }
    for (int j = 0; j < 256; j += 128)
        for (int l = 0; l < 32; l++)
            b[16 + j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
}

// utils.rs:257-320 make_q3_quants(x[0..16], nmax, do_rmse = true): scale of levels -nmax..nmax-1
__device__ float make_q3_quants16(int nmax, const float* x) {
    int8_t l[16];
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < 16; i++) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax == 0.0f) return 0.0f;
    const float iscale = -(float)nmax / max;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < 16; i++) {
        const int32_t li = clampi(f_as_i32(roundf(iscale * x[i])), -nmax, nmax - 1);
        l[i] = (int8_t)li;
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)li;
        suml2 += w * (float)(li * li);
    }
    for (int it = 0; it < 5; it++) {
        int n_changed = 0;
        for (int i = 0; i < 16; i++) {
            const float w = x[i] * x[i];
            float slx = sumlx - w * x[i] * (float)l[i];
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)((int32_t)l[i] * (int32_t)l[i]);
                const int32_t new_l = clampi(f_as_i32(roundf(x[i] * sl2 / slx)), -nmax, nmax - 1);
                if (new_l != (int32_t)l[i]) {
                    slx += w * x[i] * (float)new_l;
                    sl2 += w * (float)(new_l * new_l);
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        l[i] = (int8_t)new_l;
                        sumlx = slx;
                        suml2 = sl2;
                        n_changed++;
                    }
                }
            }
        }
        if (n_changed == 0) break;
    }
    return sumlx / suml2;
}

// k_quants.rs:1170-1236 BlockQ3K::from_float: {hmask[32], qs[64], scales[12], d}
__global__ void w_q3k_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const float* x = xin + bi * 256;
    uint8_t* b = out + bi * 110;
    uint8_t* hmask = b;
    uint8_t* qs = b + 32;
    uint8_t* sc = b + 96;
    float scales[16];
    for (int j = 0; j < 16; j++) scales[j] = make_q3_quants16(4, x + 16 * j);
    float max_scale = 0.0f;
    for (int j = 0; j < 16; j++)
        if (fabsf(scales[j]) > fabsf(max_scale)) max_scale = scales[j];
    for (int j = 0; j < 12; j++) sc[j] = 0;
    uint16_t dh;
    if (max_scale != 0.0f) {
        const float iscale = -32.0f / max_scale;
        for (int j = 0; j < 16; j++) {
            int32_t l = clampi(nearest_int(iscale * scales[j]), -32, 31) + 32;
            if (j < 8) sc[j] = (uint8_t)(l & 0xF);
            else sc[j - 8] = (uint8_t)(sc[j - 8] | (uint8_t)((l & 0xF) << 4));
            l >>= 4;
            sc[j % 4 + 8] = (uint8_t)(sc[j % 4 + 8] | (uint8_t)(l << (2 * (j / 4))));
        }
        dh = f32_to_f16_bits(1.0f / iscale);
    } else {
        dh = f32_to_f16_bits(0.0f);
    }
    put16(b + 108, dh);
    int8_t L[256];
    for (int e = 0; e < 256; e++) L[e] = 0;
    const float df = f16_bits_to_f32(dh);
    for (int j = 0; j < 16; j++) {
        const uint8_t s4 = j < 8 ? (uint8_t)(sc[j] & 0xF) : (uint8_t)(sc[j - 8] >> 4);
        const int8_t sci = (int8_t)((int8_t)(uint8_t)(s4 | (((sc[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32);
        const float d = df * (float)sci;
        if (d != 0.0f)
            for (int ii = 0; ii < 16; ii++) L[16 * j + ii] = (int8_t)(clampi(nearest_int(x[16 * j + ii] / d), -4, 3) + 4);
    }
    for (int j = 0; j < 32; j++) hmask[j] = 0;
    int m = 0;
    uint8_t hm = 1;
    for (int e = 0; e < 256; e++) {
        if (L[e] > 3) {
            hmask[m] |= hm;
            L[e] = (int8_t)(L[e] - 4);
        }
        if (++m == 32) {
            m = 0;
            hm = (uint8_t)(hm << 1);
        }
    }
    for (int j = 0; j < 256; j += 128)
        for (int l = 0; l < 32; l++)
            qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
}

// k_quants.rs:1608-1679 BlockQ5K::from_float: {d, dmin, scales[12], qh[32], qs[128]}
__global__ void w_q5k_kernel(const float* __restrict__ xin, size_t nblocks, uint8_t* __restrict__ out) {
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const float* x = xin + bi * 256;
    uint8_t* b = out + bi * 176;
    uint8_t* sc = b + 4;
    uint8_t* qh = b + 16;
    uint8_t* qs = b + 48;
    float mins[8], scales[8];
    for (int j = 0; j < 8; j++) scales[j] = make_qkx1_quants<32>(31, 5, x + 32 * j, &mins[j]);
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) max_scale = fmaxf(scales[j], max_scale);
    for (int j = 0; j < 8; j++) max_min = fmaxf(mins[j], max_min);
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    for (int j = 0; j < 12; j++) sc[j] = 0;
    for (int j = 0; j < 8; j++) {
        const int32_t ls0 = nearest_int(inv_scale * scales[j]), lm0 = nearest_int(inv_min * mins[j]);
        const uint8_t ls = (uint8_t)(ls0 < 63 ? ls0 : 63), lm = (uint8_t)(lm0 < 63 ? lm0 : 63);
        if (j < 4) {
            sc[j] = ls;
            sc[j + 4] = lm;
        } else {
            sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            sc[j - 4] = (uint8_t)(sc[j - 4] | ((ls >> 4) << 6));
            sc[j] = (uint8_t)(sc[j] | ((lm >> 4) << 6));
        }
    }
    const uint16_t dh = f32_to_f16_bits(max_scale / 63.0f), mh = f32_to_f16_bits(max_min / 63.0f);
    put16(b, dh);
    put16(b + 2, mh);
    uint8_t L[256];
    for (int e = 0; e < 256; e++) L[e] = 0;
    const float df = f16_bits_to_f32(dh), mf = f16_bits_to_f32(mh);
    for (int j = 0; j < 8; j++) {
        uint8_t s, m;
        get_scale_min_k4(j, sc, &s, &m);
        const float d = df * (float)s;
        if (d == 0.0f) continue;
        const float dm = mf * (float)m;
        for (int ii = 0; ii < 32; ii++) L[32 * j + ii] = (uint8_t)clampi(nearest_int((x[32 * j + ii] + dm) / d), 0, 31);
    }
    for (int j = 0; j < 32; j++) qh[j] = 0;
    uint8_t m1 = 1, m2 = 2;
    for (int nn = 0; nn < 256; nn += 64) {
        const int off = (nn / 64) * 32;
        for (int j = 0; j < 32; j++) {
            uint8_t l1 = L[nn + j], l2 = L[nn + j + 32];
            if (l1 > 15) {
                l1 = (uint8_t)(l1 - 16);
                qh[j] |= m1;
            }
            if (l2 > 15) {
                l2 = (uint8_t)(l2 - 16);
                qh[j] |= m2;
            }
            qs[off + j] = (uint8_t)(l1 | (l2 << 4));
        }
        m1 = (uint8_t)(m1 << 2);
        m2 = (uint8_t)(m2 << 2);
    }
}

}  // namespace

hipError_t launch_quantize_act(const ALayout& L, const float* x, void* ws, hipStream_t s) {
    uint8_t* b = static_cast<uint8_t*>(ws);
    if (L.m == 0) return hipSuccess;
    if (L.act_dtype == XNQ_Q8K) {
        const size_t nblocks = L.m * (L.k / 256);
        if (L.tiled)
            quantize_q8k_tiled_kernel<8><<<(unsigned)(L.tile.rbs * (L.k / 256) * 8), 512, 0, s>>>(
                x, (uint32_t)L.m, L.img, b, b + L.tile_off, L.tile);
        else
            quantize_q8k_kernel<false><<<(unsigned)((nblocks + 3) / 4), 256, 0, s>>>(x, nblocks, L.img, b);
    } else {
        const size_t nblocks = L.m * (L.k / 32);
        quantize_q80_kernel<false><<<(unsigned)((nblocks * 8 + 255) / 256), 256, 0, s>>>(x, nblocks, L.img, b);
    }
    return hipGetLastError();
}

hipError_t launch_quantize_act_blocks(uint32_t act_dtype, size_t m, size_t k, const float* x,
                                      void* blocks, hipStream_t s) {
    uint8_t* b = static_cast<uint8_t*>(blocks);
    if (m == 0) return hipSuccess;
    const ActImg A = act_img((uint32_t)k, act_dtype == XNQ_Q8K);
    if (act_dtype == XNQ_Q8K) {
        const size_t nblocks = m * (k / 256);
        quantize_q8k_kernel<true><<<(unsigned)((nblocks + 3) / 4), 256, 0, s>>>(x, nblocks, A, b);
    } else {
        const size_t nblocks = m * (k / 32);
        quantize_q80_kernel<true><<<(unsigned)((nblocks * 8 + 255) / 256), 256, 0, s>>>(x, nblocks, A, b);
    }
    return hipGetLastError();
}

hipError_t launch_weight_from_float(uint32_t dtype, size_t nblocks, const float* x, void* gguf,
                                    hipStream_t s) {
    if (nblocks == 0) return hipSuccess;
    uint8_t* out = static_cast<uint8_t*>(gguf);
    const unsigned threads = 64;
    const unsigned grid = (unsigned)((nblocks + threads - 1) / threads);
    switch (dtype) {
    case XNQ_Q8_0: w_q80_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q4_0: w_q40_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q4K: w_q4k_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q6K: w_q6k_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q4_1: w_q41_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q5_0: w_q50_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q5_1: w_q51_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q2K: w_q2k_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q3K: w_q3k_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    case XNQ_Q5K: w_q5k_kernel<<<grid, threads, 0, s>>>(x, nblocks, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace xnq
