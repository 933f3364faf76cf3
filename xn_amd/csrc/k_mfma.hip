// Prefill-path quantized matmul (m > 8) on the CDNA4 int8 matrix cores.
//
// Q4K / Q6K weights, Q8K activations.  For one super-block (256 K) the
// reference's integer block dot is
//   Q4K: I1 = sum_j sc_j * sum_{k in j} q4*q8,   I2 = sum_j m_j * bsum32_j
//   Q6K: I  = sum_j sc_j * sum_{k in j} (q6-32)*q8
// and y += d_a * (d_w * I1 - dmin * I2)  resp.  y += d_a * d_w * I.
//
// The sub-block scale is folded into the weight before the contraction, so
// the MFMA accumulates a whole super-block in int32 with no per-sub-block
// work: w = sc_j * q does not fit int8, so it is split into two int8 digit
// planes and contracted twice,
//   Q4K: sc = 8*sh + sl (sh, sl in 0..7):  w = 8*(sh*q) + (sl*q), digits <= 105
//   Q6K: w = sc*(q-32) in -4096..4096:      w = 128*(w >> 7) + (w & 127)
// giving the exact integer I1 (resp. I) per super-block; the f32 epilogue then
// applies d_a * d_w once per super-block.  The Q4K min term is a GEMM over
// (super-block, sub-block) pairs with f32 operands -d_a*bsum32 and dmin*m_j;
// it runs on the bf16 matrix cores with both operands split hi+lo (three
// products, ~16-bit mantissa) and accumulates straight into the f32 output.
//
// Tiling: 512 threads (8 wavefronts as 4 x 2), 256 x 128 output tile, each
// wavefront 64 x 64 = 2 x 2 v_mfma_i32_32x32x32_i8 tiles.  K advances 64 at a
// time through double-buffered LDS; the activation tile is copied from the
// quantized workspace, the weight tile is expanded into its two digit planes
// by the workgroup on the way into LDS.
#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kWaves = 8, kThreads = kWaves * 64;
constexpr int kTM = 2, kTN = 2;  // 32x32 tiles per wavefront
constexpr int kAPer = 2 * 2 * kBM / kThreads;  // 16-byte activation pieces per thread per stage
constexpr int kBPer = 2 * 2 * kBN / kThreads;  // weight half-chunks per thread per stage
// LDS: per stage A [2 ks][2 h][kBM][16 B] + B [2 ks][2 planes][2 h][kBN][16 B]
constexpr int kAStage = 2 * 2 * kBM * 16;       // 16 KiB
constexpr int kBStage = 2 * 2 * 2 * kBN * 16;   // 16 KiB
constexpr int kStage = kAStage + kBStage;
constexpr int kLds = 2 * kStage + kBM * 4;      // + d_a of the current super-block

// bytes of d (each <= 15) times s (<= 7); no byte overflows, so no carries
__device__ __forceinline__ uint32_t mul_bytes(uint32_t d, uint32_t s) {
    const uint32_t a = d & 0x00FF00FFu, b = (d >> 8) & 0x00FF00FFu;
    return __umul24(a, s) | (__umul24(b, s) << 8);
}

// Q6K digit planes of 4 six-bit values (bytes of q) times a signed scale.
__device__ __forceinline__ void q6_digits(uint32_t q, int sc, uint32_t& lo, uint32_t& hi) {
    v2s x01 = {(short)(q & 0xFF), (short)((q >> 8) & 0xFF)};
    v2s x23 = {(short)((q >> 16) & 0xFF), (short)(q >> 24)};
    const v2s off = {32, 32};
    const v2s s2 = {(short)sc, (short)sc};
    const v2s w01 = (x01 - off) * s2, w23 = (x23 - off) * s2;
    const v2s m7 = {127, 127};
    const v2s l01 = w01 & m7, l23 = w23 & m7;
    const v2s h01 = w01 >> 7, h23 = w23 >> 7;
    lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, l23), __builtin_bit_cast(uint32_t, l01), 0x06040200u);
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h23), __builtin_bit_cast(uint32_t, h01), 0x06040200u);
}

__device__ __forceinline__ void bf16_split(float v, __bf16& h, __bf16& l) {
    h = (__bf16)v;
    l = (__bf16)(v - (float)h);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void qmm_kernel(WView w, AView a, uint32_t m, float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool kQ4K = DT == XNQ_Q4K;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;  // 4 x 2 wavefronts, 64 x 64 each
    const uint32_t m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    const uint32_t K = w.k, nsb = K / 256, nstage = K / kBK;
    const ActImg& A = a.A;
    float* lds_da = reinterpret_cast<float*>(lds + 2 * kStage);

    // ---- global -> register staging for one K stage ----
    // A: 1024 pieces of 16 B (ks, h, row); B: 512 (n, chunk, half) work items
    uint4 ra[kAPer];
    uint4 rq[kBPer];
    uint4 rx[kBPer];  // Q4K: meta of the super-block; Q6K: .x/.y qh, .z scale pair
    auto load_stage = [&](uint32_t s) {
#pragma unroll
        for (int i = 0; i < kAPer; i++) {
            const uint32_t p = tid + i * kThreads;
            const uint32_t row = p & (kBM - 1), h = (p >> 8) & 1, ks = p >> 9;
            const uint32_t c = s * 2 + ks;  // activation chunk
            ra[i] = make_uint4(0u, 0u, 0u, 0u);
            if (m0 + row < m)
                ra[i] = *reinterpret_cast<const uint4*>(a.img + (size_t)(m0 + row) * A.row_bytes + h * (K / 2) + c * 16);
        }
#pragma unroll
        for (int i = 0; i < kBPer; i++) {
            const uint32_t it = tid + i * kThreads;
            const uint32_t bn = it & (kBN - 1), bc = (it >> 7) & 1;
            const uint32_t n = n0 + bn, c = s * 2 + bc;
            rq[i] = make_uint4(0u, 0u, 0u, 0u);
            rx[i] = make_uint4(0u, 0u, 0u, 0u);
            if (n < w.n) {
                rq[i] = *reinterpret_cast<const uint4*>(w.q + (size_t)n * w.q_row + c * 16);
                if (kQ4K) {
                    rx[i] = *reinterpret_cast<const uint4*>(w.s + (size_t)n * w.s_row + (c >> 3) * 16);
                } else {
                    const uint2 hh = *reinterpret_cast<const uint2*>(w.h + (size_t)n * w.h_row + c * 8);
                    rx[i].x = hh.x;
                    rx[i].y = hh.y;
                    rx[i].z = *reinterpret_cast<const uint16_t*>(w.s + (size_t)n * w.s_row + (c >> 3) * 16 + 2 * (c & 7));
                }
            }
        }
    };
    // registers -> LDS buffer `buf` (weights expanded into digit planes)
    auto store_stage = [&](uint32_t s, int buf) {
        uint8_t* base = lds + buf * kStage;
#pragma unroll
        for (int i = 0; i < kAPer; i++) {
            const uint32_t p = tid + i * kThreads;
            const uint32_t row = p & (kBM - 1), h = (p >> 8) & 1, ks = p >> 9;
            *reinterpret_cast<uint4*>(base + ((ks * 2 + h) * kBM + row) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < kBPer; i++) {
            const uint32_t it = tid + i * kThreads;
            const uint32_t bn = it & (kBN - 1), bc = (it >> 7) & 1, bh = it >> 8;
            uint32_t p0[4], p1[4];  // plane 0 (high digit) and plane 1 (low digit), 16 elements
            if (kQ4K) {
                int sc, mn;
                q4k_scale_min(rx[i].y, rx[i].z, rx[i].w, (int)((s * 2 + bc) & 7), sc, mn);
                const uint32_t sh = (uint32_t)sc >> 3, sl = (uint32_t)sc & 7;
                const uint32_t q4[4] = {rq[i].x, rq[i].y, rq[i].z, rq[i].w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t nib = bh ? ((q4[j] >> 4) & 0x0F0F0F0Fu) : (q4[j] & 0x0F0F0F0Fu);
                    p0[j] = mul_bytes(nib, sh);
                    p1[j] = mul_bytes(nib, sl);
                }
            } else {
                int b[8];
                q6k_unpack(rq[i], make_uint2(rx[i].x, rx[i].y), b);
                const int sc = bh ? (int)(int8_t)(rx[i].z >> 8) : (int)(int8_t)(rx[i].z & 0xff);
#pragma unroll
                for (int j = 0; j < 4; j++) q6_digits((uint32_t)b[4 * bh + j], sc, p1[j], p0[j]);
            }
            uint8_t* bb = base + kAStage;
            *reinterpret_cast<uint4*>(bb + (((bc * 2 + 0) * 2 + bh) * kBN + bn) * 16) = make_uint4(p0[0], p0[1], p0[2], p0[3]);
            *reinterpret_cast<uint4*>(bb + (((bc * 2 + 1) * 2 + bh) * kBN + bn) * 16) = make_uint4(p1[0], p1[1], p1[2], p1[3]);
        }
    };

    v16f accf[kTM][kTN];
    v16i hi[kTM][kTN], lo[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            accf[i][j] = v16f{};
            hi[i][j] = v16i{};
            lo[i][j] = v16i{};
        }

    load_stage(0);
    store_stage(0, 0);
    __syncthreads();

    const uint32_t lrow = lane & 31, lgrp = lane >> 5;
    for (uint32_t s = 0; s < nstage; s++) {
        const int buf = s & 1;
        const bool more = s + 1 < nstage;
        if (more) load_stage(s + 1);
        // ---- 2 K-steps x 2 x 2 tiles x 2 digit planes of int8 MFMA ----
        const uint8_t* base = lds + buf * kStage;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i av[kTM], bv[2][kTN];
#pragma unroll
            for (int i = 0; i < kTM; i++)
                av[i] = *reinterpret_cast<const v4i*>(base + ((ks * 2 + lgrp) * kBM + wm * 64 + i * 32 + lrow) * 16);
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    bv[p][j] = *reinterpret_cast<const v4i*>(base + kAStage +
                                                             (((ks * 2 + p) * 2 + lgrp) * kBN + wn * 64 + j * 32 + lrow) * 16);
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int j = 0; j < kTN; j++) {
                    hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[0][j], hi[i][j], 0, 0, 0);
                    lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[1][j], lo[i][j], 0, 0, 0);
                }
        }
        // ---- super-block epilogue ----
        if ((s & 3) == 3) {
            const uint32_t sb = s >> 2;
            // d_a of the tile's rows for this super-block (filled below by the
            // previous iteration's barrier-protected store, see `sb_prep`)
            for (uint32_t r = tid; r < kBM; r += kThreads) {
                const uint32_t row = m0 + r;
                lds_da[r] = row < m ? reinterpret_cast<const float*>(a.img + (size_t)row * A.row_bytes + A.d_off)[sb] : 0.0f;
            }
            __syncthreads();
            float dw[kTN], dmn[kTN];
#pragma unroll
            for (int j = 0; j < kTN; j++) {
                const uint32_t n = n0 + wn * 64 + j * 32 + lrow;
                dw[j] = 0.0f;
                dmn[j] = 0.0f;
                if (n < w.n) {
                    if (kQ4K) {
                        const uint32_t md = *reinterpret_cast<const uint32_t*>(w.s + (size_t)n * w.s_row + sb * 16);
                        dw[j] = f16_bits_to_f32(md);
                        dmn[j] = f16_bits_to_f32(md >> 16);
                    } else {
                        dw[j] = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(w.d + (size_t)n * w.d_row + sb * 2));
                    }
                }
            }
            constexpr int kShift = kQ4K ? 3 : 7;
#pragma unroll
            for (int i = 0; i < kTM; i++) {
                float da[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 d4 = *reinterpret_cast<const float4*>(lds_da + wm * 64 + i * 32 + q * 8 + lgrp * 4);
                    da[4 * q + 0] = d4.x;
                    da[4 * q + 1] = d4.y;
                    da[4 * q + 2] = d4.z;
                    da[4 * q + 3] = d4.w;
                }
#pragma unroll
                for (int j = 0; j < kTN; j++) {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int iv = hi[i][j][e] * (1 << kShift) + lo[i][j][e];
                        accf[i][j][e] = fmaf((float)iv * dw[j], da[e], accf[i][j][e]);
                    }
                    hi[i][j] = v16i{};
                    lo[i][j] = v16i{};
                }
            }
            if (kQ4K && ((sb & 1) == 1 || sb + 1 == nsb)) {
                // min term of the super-block pair (sb-1, sb) (or the lone last
                // one): K'' = 16 = 2 super-blocks x 8 sub-blocks, lane group g
                // covers super-block (pair base + g).
                const uint32_t sbp = (sb & 1) ? sb - 1 : sb;
                const uint32_t my_sb = sbp + lgrp;
                const bool live_sb = my_sb <= sb;
                v8bf bh2[kTN], bl2[kTN];
#pragma unroll
                for (int j2 = 0; j2 < kTN; j2++) {
                    const uint32_t n = n0 + wn * 64 + j2 * 32 + lrow;
                    float dm = 0.0f;
                    uint4 meta = make_uint4(0u, 0u, 0u, 0u);
                    if (n < w.n && live_sb) {
                        meta = *reinterpret_cast<const uint4*>(w.s + (size_t)n * w.s_row + my_sb * 16);
                        dm = f16_bits_to_f32(meta.x >> 16);
                    }
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        int sc, mn;
                        q4k_scale_min(meta.y, meta.z, meta.w, j, sc, mn);
                        __bf16 h, l;
                        bf16_split(dm * (float)mn, h, l);
                        bh2[j2][j] = h;
                        bl2[j2][j] = l;
                    }
                }
#pragma unroll
                for (int i = 0; i < kTM; i++) {
                    v8bf ah, al;
                    const uint32_t row = m0 + wm * 64 + i * 32 + lrow;
                    float dav = 0.0f;
                    int32_t sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    if (row < m && live_sb) {
                        const uint8_t* img = a.img + (size_t)row * A.row_bytes;
                        dav = reinterpret_cast<const float*>(img + A.d_off)[my_sb];
                        const int4 s0 = reinterpret_cast<const int4*>(img + A.s_off)[my_sb * 2];
                        const int4 s1 = reinterpret_cast<const int4*>(img + A.s_off)[my_sb * 2 + 1];
                        const int32_t pr[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                        for (int j = 0; j < 8; j++) sums[j] = (int)(int16_t)(pr[j] & 0xffff) + (int)(int16_t)(pr[j] >> 16);
                    }
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        __bf16 h, l;
                        bf16_split(-dav * (float)sums[j], h, l);
                        ah[j] = h;
                        al[j] = l;
                    }
#pragma unroll
                    for (int j = 0; j < kTN; j++) {
                        accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh2[j], accf[i][j], 0, 0, 0);
                        accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl2[j], accf[i][j], 0, 0, 0);
                        accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh2[j], accf[i][j], 0, 0, 0);
                    }
                }
            }
        }
        if (more) store_stage(s + 1, buf ^ 1);
        __syncthreads();
    }

    // ---- write the tile ----
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            const uint32_t n = n0 + wn * 64 + j * 32 + lrow;
            if (n >= w.n) continue;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = m0 + wm * 64 + i * 32 + 8 * (e / 4) + 4 * lgrp + (e % 4);
                if (row < m) y[(size_t)row * w.n + n] = accf[i][j][e];
            }
        }
}

}  // namespace

bool mfma_supported(uint32_t dtype, size_t m, size_t n, size_t k) {
    (void)m;
    (void)n;
    return (dtype == XNQ_Q4K || dtype == XNQ_Q6K) && k % 256 == 0;
}

hipError_t launch_mfma(const WView& w, const AView& a, size_t m, float* y, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    const dim3 grid((w.n + kBN - 1) / kBN, (unsigned)((m + kBM - 1) / kBM));
    if (w.dtype == XNQ_Q4K) {
        static bool attr = false;
        if (!attr) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(qmm_kernel<XNQ_Q4K>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
            attr = true;
        }
        hipLaunchKernelGGL(qmm_kernel<XNQ_Q4K>, grid, dim3(kThreads), kLds, s, w, a, (uint32_t)m, y);
    } else if (w.dtype == XNQ_Q6K) {
        static bool attr = false;
        if (!attr) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(qmm_kernel<XNQ_Q6K>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
            attr = true;
        }
        hipLaunchKernelGGL(qmm_kernel<XNQ_Q6K>, grid, dim3(kThreads), kLds, s, w, a, (uint32_t)m, y);
    } else {
        return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace xnq
