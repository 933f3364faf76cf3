// Prefill-path quantized matmul (m > 8) on the CDNA4 int8 matrix cores.
//
// Q4K / Q6K weights, Q8K activations.  For one super-block (256 K) the
// reference's integer block dot is
//   Q4K: I1 = sum_j sc_j * sum_{k in j} q4*q8,   I2 = sum_j m_j * bsum32_j
//   Q6K: I  = sum_j sc_j * sum_{k in j} (q6-32)*q8
// and y += d_a * (d_w * I1 - dmin * I2)  resp.  y += d_a * d_w * I
// (k_quants.rs:1406-1474 / 1686-1754 restate this per block on the CPU).
//
// The sub-block scale is folded into the weight before the contraction, so
// the MFMA accumulates a whole super-block in int32 with no per-sub-block
// work: w = sc_j * q does not fit int8, so it is split into two int8 digit
// planes and contracted twice,
//   Q4K: sc = 8*sh + sl (sh, sl in 0..7):  w = 8*(sh*q) + (sl*q), digits <= 105
//   Q6K: w = sc*(q-32) in -4096..4096:      w = 128*(w >> 7) + (w & 127)
// giving the exact integer I1 (resp. I) per super-block; the f32 epilogue then
// applies d_a * d_w once per super-block.  The Q4K min term is a GEMM over
// the 8 sub-blocks of a super-block with f32 operands -d_a*bsum32 and
// dmin*m_j; it runs on the bf16 matrix cores with both operands split hi+lo
// (three products, ~16-bit mantissa) and accumulates into the f32 output.
//
// Tiling: 512 threads (8 wavefronts as 4 x 2), 256 x 128 output tile, each
// wavefront 64 x 64 = 2 x 2 v_mfma_i32_32x32x32_i8 tiles.  K advances 64 per
// stage.  Every byte a stage needs (activation tile, raw weight chunks and
// scales, the per-super-block epilogue operands) is fetched with
// global_load_lds DMA straight into a 4-slot LDS ring, three stages ahead of
// the one being multiplied, so no registers hold data in flight.  Each
// wavefront waits only for its own DMA (s_waitcnt vmcnt with the exact count
// of younger DMA it has issued).  A wavefront expands into the digit planes
// exactly the weight chunks it fetched itself, so the single barrier per
// stage publishes both the next activation tile and the next digit planes.
#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 128;
constexpr int kWaves = 8, kThreads = kWaves * 64;
constexpr int kTM = 2, kTN = 2;  // 32x32 tiles per wavefront
constexpr int kRing = 4;         // LDS ring slots (3 stages in flight + the current one)

// LDS map (bytes)
constexpr int kASlot = 2 * 2 * kBM * 16;  // activations [ks][h][row][16]                 16 KiB
constexpr int kQSlot = 2 * kBN * 16;      // raw weight chunks [bc][n][16]                 4 KiB
constexpr int kMSlot = 2 * kBN * 16;      // Q4K header / Q6K qh pair, [bc][n][16]         4 KiB
constexpr int kSSlot = 2 * kBN * 4;       // Q6K scale dword [bc][n]                       1 KiB
constexpr int kDSlot = 2 * kBN * 4;       // Q6K d dword [bc][n]                           1 KiB
constexpr int kRawSlot = kQSlot + kMSlot + kSSlot + kDSlot;
constexpr int kPlanes = 2 * 2 * 2 * kBN * 16;  // digit planes [ks][plane][h][n][16]     16 KiB
constexpr int kEpiDa = kBM * 4;                // d_a [row]                               1 KiB
constexpr int kEpiSums = kBM * 32;             // Q4K chunk bsum pairs [row][8]           8 KiB
constexpr int kEpi = kEpiDa + kEpiSums;
constexpr int kOffA = 0;
constexpr int kOffRaw = kOffA + kRing * kASlot;
constexpr int kOffPlanes = kOffRaw + kRing * kRawSlot;
constexpr int kOffEpi = kOffPlanes + 2 * kPlanes;
constexpr int kLds = kOffEpi + 2 * kEpi;
static_assert(kLds <= 160 * 1024, "LDS budget");

// DMA instructions one wavefront issues per stage: 2 activation pieces plus
// its weight share (Q4K: chunk + header; Q6K: chunk, qh, scale, d); at a
// super-block's first stage also d_a (wavefronts 0-3) and Q4K bsums (all).
template <int DT>
struct DmaPlan {
    static constexpr int kBase = DT == XNQ_Q4K ? 4 : 6;
    __device__ static int extra(uint32_t wave) { return (wave < 4 ? 1 : 0) + (DT == XNQ_Q4K ? 1 : 0); }
};

// global_load_lds: uniform 64-bit base + 32-bit per-lane byte offset; m0
// holds the LDS address lane 0 writes (lane i writes i * size beyond it).
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr), "v"(off), "s"(base)
                 : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_addr), "v"(off), "s"(base)
                 : "memory");
}
// Wait until at most n of this wavefront's vector memory operations are
// outstanding (n is wavefront-uniform; counts above 15 wait for all).
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
#define XNQ_W(N)                                              \
    case N:                                                   \
        asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); \
        break;
        XNQ_W(1) XNQ_W(2) XNQ_W(3) XNQ_W(4) XNQ_W(5) XNQ_W(6) XNQ_W(7) XNQ_W(8)
        XNQ_W(9) XNQ_W(10) XNQ_W(11) XNQ_W(12) XNQ_W(13) XNQ_W(14) XNQ_W(15)
#undef XNQ_W
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}

// bytes of d (each <= 15) times s (<= 7); no product leaves its byte
__device__ __forceinline__ uint32_t mul_bytes(uint32_t d, uint32_t s) {
    const uint32_t a = d & 0x00FF00FFu, b = (d >> 8) & 0x00FF00FFu;
    return __umul24(a, s) | (__umul24(b, s) << 8);
}

// Q6K digit planes of 4 six-bit values (bytes of q) times a signed scale.
__device__ __forceinline__ void q6_digits(uint32_t q, int sc, uint32_t& lo, uint32_t& hi) {
    const v2s x01 = {(short)(q & 0xFF), (short)((q >> 8) & 0xFF)};
    const v2s x23 = {(short)((q >> 16) & 0xFF), (short)(q >> 24)};
    const v2s off = {32, 32};
    const v2s s2 = {(short)sc, (short)sc};
    const v2s w01 = (x01 - off) * s2, w23 = (x23 - off) * s2;
    const v2s m7 = {127, 127};
    const v2s l01 = w01 & m7, l23 = w23 & m7;
    const v2s h01 = w01 >> 7, h23 = w23 >> 7;
    lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, l23), __builtin_bit_cast(uint32_t, l01), 0x06040200u);
    hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h23), __builtin_bit_cast(uint32_t, h01), 0x06040200u);
}

__device__ __forceinline__ short bf16_hi(float v) { return __builtin_bit_cast(short, (__bf16)v); }
__device__ __forceinline__ short bf16_lo(float v) {
    return __builtin_bit_cast(short, (__bf16)(v - (float)(__bf16)v));
}

template <int DT>
__global__ __launch_bounds__(kThreads) void qmm_kernel(WView w, AView a, uint32_t m, float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool kQ4K = DT == XNQ_Q4K;
    using P = DmaPlan<DT>;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;  // 4 x 2 wavefronts, 64 x 64 each
    const uint32_t m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    const uint32_t K = w.k, nstage = K / 64;
    const ActImg& A = a.A;
    const uint32_t lbase = (uint32_t)(uintptr_t)lds;  // low half of the flat address = LDS offset

    // ---- this wavefront's DMA streams (byte offsets of stage 0) ----
    // activation pieces t = 2*wave + {0,1}: (ks, h, 64-row block)
    uint32_t a_off[2], a_lds[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t t = 2 * wave + i, ks = t >> 3, h = (t >> 2) & 1, rb = t & 3;
        const uint32_t row = min(m0 + rb * 64 + lane, m - 1);
        a_off[i] = row * A.row_bytes + h * (K / 2) + ks * 16;
        a_lds[i] = ((ks * 2 + h) * kBM + rb * 64) * 16;
    }
    // weights: chunk bc = wave & 1 of the stage, columns cb*32 .. +31
    // (cb = wave >> 1); lanes 32-63 mirror lanes 0-31 and issue no DMA
    const uint32_t bc = wave & 1, cb = wave >> 1;
    const uint32_t bn = cb * 32 + (lane & 31);
    const uint32_t ncol = min(n0 + bn, w.n - 1);
    const bool dma_lane = lane < 32;
    const uint32_t q_off = ncol * w.q_row + bc * 16;
    const uint32_t s_off = ncol * w.s_row;
    const uint32_t h_off = ncol * w.h_row;
    const uint32_t d_off = ncol * w.d_row;
    // d_a (wavefronts 0-3: 64 rows each) and Q4K bsums (512 16-byte pieces)
    const uint32_t da_row = min(m0 + (wave & 3) * 64 + lane, m - 1);
    const uint32_t da_off = da_row * A.row_bytes + A.d_off;
    const uint32_t sp = wave * 64 + lane, sums_row = min(m0 + (sp >> 1), m - 1);
    const uint32_t sums_off = sums_row * A.row_bytes + A.s_off + (sp & 1) * 16;
    const uint32_t col_lds = (bc * kBN + cb * 32);

    auto stage_count = [&](uint32_t st) -> int {
        if (st >= nstage) return 0;
        return P::kBase + ((st & 3) == 0 ? P::extra(wave) : 0);
    };
    auto issue = [&](uint32_t st) {
        if (st >= nstage) return;
        const uint32_t slot = st % kRing, sb = st >> 2;
        const uint32_t abase = lbase + kOffA + slot * kASlot;
#pragma unroll
        for (int i = 0; i < 2; i++) dma16(a.img, a_off[i] + st * 32, abase + a_lds[i]);
        const uint32_t raw = lbase + kOffRaw + slot * kRawSlot;
        if (dma_lane) {
            dma16(w.q, q_off + st * 32, raw + col_lds * 16);
            if (kQ4K) {
                dma16(w.s, s_off + sb * 16, raw + kQSlot + col_lds * 16);
            } else {
                // qh of chunks 2st, 2st+1; scales of the same two chunks; d
                dma16(w.h, h_off + st * 16, raw + kQSlot + col_lds * 16);
                dma4(w.s, s_off + sb * 16 + 4 * (st & 3), raw + kQSlot + kMSlot + col_lds * 4);
                dma4(w.d, (d_off + sb * 2) & ~3u, raw + kQSlot + kMSlot + kSSlot + col_lds * 4);
            }
        }
        if ((st & 3) == 0) {
            const uint32_t epi = lbase + kOffEpi + (sb & 1) * kEpi;
            if (wave < 4) dma4(a.img, da_off + sb * 4, epi + wave * 64 * 4);
            if (kQ4K) dma16(a.img, sums_off + sb * 32, epi + kEpiDa + wave * 64 * 16);
        }
    };

    // ---- this wavefront's weight chunks of stage st -> digit planes (st & 1) ----
    const uint32_t bh = lane >> 5;
    auto expand = [&](uint32_t st) {
        const uint8_t* raw = lds + kOffRaw + (st % kRing) * kRawSlot;
        const uint4 rq = *reinterpret_cast<const uint4*>(raw + (bc * kBN + bn) * 16);
        uint32_t p0[4], p1[4];  // high digit, low digit; 16 elements each
        if (kQ4K) {
            const uint4 hd = *reinterpret_cast<const uint4*>(raw + kQSlot + (bc * kBN + bn) * 16);
            int sc, mn;
            q4k_scale_min(hd.y, hd.z, hd.w, (int)((2 * st + bc) & 7), sc, mn);
            const uint32_t sh = (uint32_t)sc >> 3, sl = (uint32_t)sc & 7;
            const uint32_t q4[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t nib = bh ? ((q4[j] >> 4) & 0x0F0F0F0Fu) : (q4[j] & 0x0F0F0F0Fu);
                p0[j] = mul_bytes(nib, sh);
                p1[j] = mul_bytes(nib, sl);
            }
        } else {
            const uint2 qh = *reinterpret_cast<const uint2*>(raw + kQSlot + (bc * kBN + bn) * 16 + bc * 8);
            const uint32_t scw = *reinterpret_cast<const uint32_t*>(raw + kQSlot + kMSlot + (bc * kBN + bn) * 4);
            int b[8];
            q6k_unpack(rq, qh, b);
            const int sc = (int)(int8_t)(scw >> (8 * (2 * bc + bh)));
#pragma unroll
            for (int j = 0; j < 4; j++) q6_digits((uint32_t)b[4 * bh + j], sc, p1[j], p0[j]);
        }
        uint8_t* pl = lds + kOffPlanes + (st & 1) * kPlanes;
        *reinterpret_cast<uint4*>(pl + (((bc * 2 + 0) * 2 + bh) * kBN + bn) * 16) = make_uint4(p0[0], p0[1], p0[2], p0[3]);
        *reinterpret_cast<uint4*>(pl + (((bc * 2 + 1) * 2 + bh) * kBN + bn) * 16) = make_uint4(p1[0], p1[1], p1[2], p1[3]);
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

    // prologue: stages 0-2 in flight, stage 0 expanded and published
    issue(0);
    issue(1);
    issue(2);
    wait_vmcnt(stage_count(1) + stage_count(2));
    expand(0);
    __syncthreads();

    const uint32_t lrow = lane & 31, lgrp = lane >> 5;
    for (uint32_t s = 0; s < nstage; s++) {
        issue(s + 3);
        if (s + 1 < nstage) {
            wait_vmcnt(stage_count(s + 2) + stage_count(s + 3));
            expand(s + 1);
        }
        // ---- 2 chunks x 2 x 2 tiles x 2 digit planes of int8 MFMA ----
        const uint8_t* abase = lds + kOffA + (s % kRing) * kASlot;
        const uint8_t* pbase = lds + kOffPlanes + (s & 1) * kPlanes;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i av[kTM], bv[2][kTN];
#pragma unroll
            for (int i = 0; i < kTM; i++)
                av[i] = *reinterpret_cast<const v4i*>(abase + ((ks * 2 + lgrp) * kBM + wm * 64 + i * 32 + lrow) * 16);
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    bv[p][j] = *reinterpret_cast<const v4i*>(
                        pbase + (((ks * 2 + p) * 2 + lgrp) * kBN + wn * 64 + j * 32 + lrow) * 16);
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
            const uint8_t* raw = lds + kOffRaw + (s % kRing) * kRawSlot;
            const uint8_t* epi = lds + kOffEpi + (sb & 1) * kEpi;
            const float* ep_da = reinterpret_cast<const float*>(epi);
            float dw[kTN];
            v4s bh2[kTN], bl2[kTN];  // Q4K min-term operands, sub-blocks 4*lgrp .. +3
#pragma unroll
            for (int j = 0; j < kTN; j++) {
                const uint32_t nl = wn * 64 + j * 32 + lrow;
                if (kQ4K) {
                    // the super-block header, as fetched for chunk 1
                    const uint4 hd = *reinterpret_cast<const uint4*>(raw + kQSlot + (kBN + nl) * 16);
                    dw[j] = f16_bits_to_f32(hd.x & 0xffffu);
                    const float dm = f16_bits_to_f32(hd.x >> 16);
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        int sc, mn;
                        q4k_scale_min(hd.y, hd.z, hd.w, (int)(4 * lgrp + t), sc, mn);
                        const float v = dm * (float)mn;
                        bh2[j][t] = bf16_hi(v);
                        bl2[j][t] = bf16_lo(v);
                    }
                } else {
                    const uint32_t n = min(n0 + nl, w.n - 1);
                    const uint32_t dd =
                        *reinterpret_cast<const uint32_t*>(raw + kQSlot + kMSlot + kSSlot + (kBN + nl) * 4);
                    dw[j] = f16_bits_to_f32(((n * w.d_row + sb * 2) & 2) ? (dd >> 16) : (dd & 0xffffu));
                }
            }
            constexpr int kShift = kQ4K ? 3 : 7;
#pragma unroll
            for (int i = 0; i < kTM; i++) {
                float da[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 d4 = *reinterpret_cast<const float4*>(ep_da + wm * 64 + i * 32 + q * 8 + lgrp * 4);
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
                if (kQ4K) {
                    const uint32_t rl = wm * 64 + i * 32 + lrow;
                    const float dav = ep_da[rl];
                    const int4 pr = reinterpret_cast<const int4*>(epi + kEpiDa)[rl * 2 + lgrp];
                    const int32_t prs[4] = {pr.x, pr.y, pr.z, pr.w};
                    v4s ah, al;
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const int bs = (int)(int16_t)(prs[t] & 0xffff) + (int)(int16_t)(prs[t] >> 16);
                        const float v = -dav * (float)bs;
                        ah[t] = bf16_hi(v);
                        al[t] = bf16_lo(v);
                    }
#pragma unroll
                    for (int j = 0; j < kTN; j++) {
                        accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(ah, bh2[j], accf[i][j], 0, 0, 0);
                        accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(ah, bl2[j], accf[i][j], 0, 0, 0);
                        accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(al, bh2[j], accf[i][j], 0, 0, 0);
                    }
                }
            }
        }
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

template <int DT>
hipError_t launch_dt(const WView& w, const AView& a, size_t m, float* y, hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(qmm_kernel<DT>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const dim3 grid((w.n + kBN - 1) / kBN, (unsigned)((m + kBM - 1) / kBM));
    hipLaunchKernelGGL(qmm_kernel<DT>, grid, dim3(kThreads), kLds, s, w, a, (uint32_t)m, y);
    return hipGetLastError();
}

}  // namespace

bool mfma_supported(uint32_t dtype, size_t m, size_t n, size_t k) {
    (void)m;
    (void)n;
    return (dtype == XNQ_Q4K || dtype == XNQ_Q6K) && k % 256 == 0;
}

hipError_t launch_mfma(const WView& w, const AView& a, size_t m, float* y, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (w.dtype == XNQ_Q4K) return launch_dt<XNQ_Q4K>(w, a, m, y, s);
    if (w.dtype == XNQ_Q6K) return launch_dt<XNQ_Q6K>(w, a, m, y, s);
    return hipErrorNotSupported;
}

}  // namespace xnq
