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
//   Q6K: w = sc*(q-32) in -3968..4096:      w = 256*hi + lo, hi = (w+128) >> 8, lo signed
// giving the exact integer I1 (resp. I) per super-block; the f32 epilogue then
// applies d_a * d_w once per super-block.  The Q4K min term is a GEMM over
// the 8 sub-blocks of a super-block with f32 operands -d_a*bsum32 and
// dmin*m_j, both split into bf16 hi + lo (~16 significant bits); it runs on
// the bf16 matrix cores (two K=16 products) into the f32 output.
//
// Tiling: 512 threads = 8 wavefronts, two per SIMD, as 4 x 2 over a 256 x
// 128 output tile; each wavefront owns 64 x 64 = 2 x 2 tiles of
// v_mfma_i32_32x32x32_i8 (192 accumulator registers: two int32 digit sums
// and the f32 output).  K advances 64 per stage.  Every byte a stage needs
// (activation tile, raw weight chunks, once per super-block d_a, bsums and
// block headers) is fetched with global_load_lds DMA straight into a 4-slot
// LDS ring three stages ahead, one DMA instruction at a time between MFMAs,
// so a DMA issue that the memory pipeline holds back does not idle the
// matrix core.  The wavefronts come in two groups of four (one of each per
// SIMD): group 0 fetches and expands the weights (weight chunks -> int8
// digit planes, block headers -> the column-side min-term operand), group 1
// fetches the per-super-block activation data (d_a, bsums -> the row-side
// min-term operand); both fetch activation tiles.  Each wavefront waits only
// for its own DMA (s_waitcnt vmcnt with the exact count of younger DMA it has
// issued) and processes only data it fetched itself, so one barrier per stage
// publishes both the next activation tile and the next digit planes.
//
// Activations come from the row-tiled copy of the Q8K image (TileImg), in
// which every activation DMA instruction reads 1 KiB of consecutive bytes:
// reading the row images directly costs one cache line per lane (64 per
// instruction), which measured a quarter of the kernel's time at M = 512.
#include <type_traits>

#include "xnq_device.h"
#include "xnq_internal.h"
#include "xnq_quant_dev.h"

namespace xnq {

namespace {

// y = sum of the split-K partial outputs, in split order (deterministic).
// The loads of up to 8 splits are issued together (addresses clamped to the
// last split, values past it never added), so a call costs one memory round
// trip per 8 splits rather than one per split.
__global__ __launch_bounds__(256) void sum_splits_kernel(const float* __restrict__ part, size_t count,
                                                         uint32_t splits, float* __restrict__ y) {
    constexpr uint32_t kBatch = 8;
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (count % 4 == 0) {
        if (i4 * 4 >= count) return;
        const float4* p4 = reinterpret_cast<const float4*>(part);
        const size_t c4 = count / 4;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t z0 = 0; z0 < splits; z0 += kBatch) {
            float4 v[kBatch];
#pragma unroll
            for (uint32_t j = 0; j < kBatch; j++) v[j] = p4[min(z0 + j, splits - 1) * c4 + i4];
#pragma unroll
            for (uint32_t j = 0; j < kBatch; j++) {
                if (z0 + j >= splits) break;
                if (z0 + j == 0) {
                    acc = v[0];
                } else {
                    acc.x += v[j].x;
                    acc.y += v[j].y;
                    acc.z += v[j].z;
                    acc.w += v[j].w;
                }
            }
        }
        reinterpret_cast<float4*>(y)[i4] = acc;
        return;
    }
    for (size_t i = i4 * 4; i < i4 * 4 + 4 && i < count; i++) {
        float acc = part[i];
        for (uint32_t z = 1; z < splits; z++) acc += part[z * count + i];
        y[i] = acc;
    }
}

// Sum of `splits` consecutive partials of one element, in split order, the
// loads of up to 8 splits issued together.
__device__ __forceinline__ float sum_over_splits(const float* __restrict__ p, size_t stride, uint32_t splits) {
    constexpr uint32_t kBatch = 8;
    float acc = 0.0f;
    for (uint32_t z0 = 0; z0 < splits; z0 += kBatch) {
        float v[kBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBatch; j++) v[j] = p[min(z0 + j, splits - 1) * stride];
#pragma unroll
        for (uint32_t j = 0; j < kBatch; j++) {
            if (z0 + j >= splits) break;
            acc = z0 + j == 0 ? v[0] : acc + v[j];
        }
    }
    return acc;
}

// Element i of the regions laid end to end; silu: y[0] = silu(g) * u over
// region 0's elements (cpu_backend.rs:354-356).
__global__ __launch_bounds__(256) void sum_group_kernel(SumGroup S, uint32_t splits, bool silu) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (silu) {
        if (i >= S.cnt[0]) return;
        const float g = sum_over_splits(S.part[0] + i, S.cnt[0], splits);
        const float u = sum_over_splits(S.part[1] + i, S.cnt[1], splits);
        S.y[0][i] = g / (1.0f + expf(0.0f - g)) * u;
        return;
    }
    uint32_t t = 0;
    while (t < S.count && i >= S.cnt[t]) i -= S.cnt[t++];
    if (t >= S.count) return;
    S.y[t][i] = sum_over_splits(S.part[t] + i, S.cnt[t], splits);
}

// The gate/up split-sum with its SiLU-multiply, fused with the Q8K
// quantization of the result for the next matmul (the down projection):
// one wavefront per 256-element block of a row of h, four consecutive
// elements per lane, the same arithmetic as sum_group_kernel (silu) followed
// by quantize_q8k_kernel, so h and the image are the bits those two write.
__global__ __launch_bounds__(256) void sum_silu_quant_kernel(SumGroup S, uint32_t splits, uint32_t m, uint32_t n,
                                                             ActImg A, uint8_t* __restrict__ img) {
    const uint32_t nbr = n / 256;
    const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= (size_t)m * nbr) return;  // uniform over the wavefront
    const int lane = threadIdx.x & 63;
    const uint32_t row = (uint32_t)(blk / nbr), b = (uint32_t)(blk % nbr);
    const size_t i0 = (size_t)row * n + (size_t)b * 256 + 4 * lane;
    float h[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float g = sum_over_splits(S.part[0] + i0 + e, S.cnt[0], splits);
        const float u = sum_over_splits(S.part[1] + i0 + e, S.cnt[1], splits);
        h[e] = g / (1.0f + expf(0.0f - g)) * u;
    }
    const float4 v = make_float4(h[0], h[1], h[2], h[3]);
    *reinterpret_cast<float4*>(S.y[0] + i0) = v;
    const Q8KLane r = q8k_quant_wave(v, lane);
    q8k_store(img + (size_t)row * A.row_bytes, A, b, lane, r);
}

}  // namespace

hipError_t launch_sum_silu_quant(const SumGroup& S, uint32_t splits, size_t m, size_t n, const ALayout& L,
                                 void* img, hipStream_t s) {
    if (L.act_dtype != XNQ_Q8K || L.tiled || L.k != n || L.m != m || n % 256) return hipErrorInvalidValue;
    const size_t blocks = m * (n / 256);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(sum_silu_quant_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, s, S, splits,
                       (uint32_t)m, (uint32_t)n, L.img, static_cast<uint8_t*>(img));
    return hipGetLastError();
}

hipError_t launch_sum_group(const SumGroup& S, uint32_t splits, bool silu, hipStream_t s) {
    size_t total = 0;
    for (uint32_t t = 0; t < S.count; t++) total += S.cnt[t];
    if (silu) total = S.cnt[0];
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(sum_group_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, S, splits, silu);
    return hipGetLastError();
}

hipError_t launch_sum_splits(const float* partial, size_t count, uint32_t splits, float* y, hipStream_t s) {
    const unsigned blocks = (unsigned)((count / 4 + 255) / 256 + 1);
    hipLaunchKernelGGL(sum_splits_kernel, dim3(blocks), dim3(256), 0, s, partial, count, splits, y);
    return hipGetLastError();
}

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 128;
constexpr int kWaves = 8, kThreads = kWaves * 64;
constexpr int kTM = 2, kTN = 2;  // 32x32 tiles per wavefront (64 x 64)
constexpr int kRing = 4;         // LDS ring slots (3 stages in flight + the current one)

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// LDS map (bytes).  Per stage: activation tile, raw weight chunks (Q6K: and
// their high bits).  Per super-block (two buffers, by parity): d_a; Q4K: the
// bsum pairs, turned in place into the row-side min-term operand; the
// 16-byte block header (Q4K: d, dmin, scales; Q6K: the int8 scales); Q4K:
// the column-side min-term operand, Q6K: the d dword.
template <int DT>
struct Lay {
    static constexpr bool kQ4K = DT == XNQ_Q4K;
    static constexpr int kASlot = 2 * 2 * kBM * 16;  // activations [ks][h][row][16]       16 KiB
    static constexpr int kQSlot = 2 * kBN * 16;      // weight chunks [bc][n][16]           4 KiB
    static constexpr int kHSlot = kQ4K ? 0 : 2 * kBN * 16;  // Q6K qh of the stage [bc][n][16]
    static constexpr int kRawSlot = kQSlot + kHSlot;
    static constexpr int kPlanes = 2 * 2 * 2 * kBN * 16;  // digit planes [ks][plane][h][n][16]
    static constexpr int kEDa = 0;                          // f32 [kBM]
    static constexpr int kESum = kEDa + kBM * 4;            // Q4K [kBM/32][2][32][16]
    static constexpr int kEHdr = kESum + (kQ4K ? kBM * 32 : 0);  // [kBN][16]
    static constexpr int kEB = kEHdr + kBN * 16;            // Q4K [kBN/32][2][32][16]; Q6K d dword [kBN]
    static constexpr int kEpi = kEB + (kQ4K ? kBN * 32 : kBN * 4);
    static constexpr int kOffA = 0;
    static constexpr int kOffRaw = kOffA + kRing * kASlot;
    static constexpr int kOffPlanes = kOffRaw + kRing * kRawSlot;
    static constexpr int kOffEpi = kOffPlanes + 2 * kPlanes;
    static constexpr int kLds = kOffEpi + 2 * kEpi;
    static_assert(kLds <= 160 * 1024, "LDS budget");
    // DMA instructions per stage of a group-0 / group-1 wavefront, and the
    // extra ones at a super-block's first stage
    static constexpr int kBase0 = kQ4K ? 3 : 4;   // 2 activation pieces, chunks, Q6K qh
    static constexpr int kExtra0 = kQ4K ? 1 : 2;  // header (Q6K scales), Q6K d
    static constexpr int kBase1 = 2;              // 2 activation pieces
    static constexpr int kExtra1 = kQ4K ? 3 : 1;  // d_a, Q4K 2 x bsums
};

template <int DT, bool PART>
__global__ __launch_bounds__(kThreads) void qmm_kernel(WView w, AView a, uint32_t m, uint32_t sb_per_split,
                                                       float* __restrict__ y, size_t split_stride) {
    using L = Lay<DT>;
    constexpr bool kQ4K = L::kQ4K;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;  // 4 x 2 wavefronts, 64 x 64 each
    const uint32_t m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    // split-K: this workgroup's super-blocks sb0 .. sb0 + nsb - 1; with more
    // than one split each writes its own partial output, summed afterwards
    const uint32_t sb0 = blockIdx.z * sb_per_split;
    const uint32_t K = w.k, nsb = min(sb_per_split, K / 256 - sb0);
    y += blockIdx.z * split_stride;
    const uint32_t lbase = (uint32_t)(uintptr_t)lds;  // low half of the flat address = LDS offset
    const uint32_t lrow = lane & 31, lgrp = lane >> 5;

    // Every DMA instruction is issued by the whole wavefront (the vmcnt
    // bookkeeping counts instructions): lanes past the last row or column
    // re-read the last one, and those outputs are dropped at the store.
    const uint32_t col_max = w.n - 1 - n0;
    // Activations come from the row-tiled image: every DMA instruction reads
    // 1 KiB (d_a: 256 B) of consecutive bytes, lane i's at i * 16 (i * 4).
    // 64-row blocks past the last one re-read it (those outputs are dropped).
    const TileImg& T = a.T;
    const uint32_t nsb_all = K / 256;
    auto rblk = [&](uint32_t r64) { return min(m0 / 64 + r64, T.rbs - 1); };  // tile-row block r64 -> image block
    const uint8_t* t_q = a.tile + (size_t)sb0 * 4 * 4096;  // stage st of block rb at rb * 64K + st * 4096
    const uint8_t* t_d = a.tile + T.d_off + (size_t)sb0 * 256;
    const uint8_t* t_s = a.tile + T.s_off + (size_t)sb0 * 2048;
    const uint32_t lane16 = lane * 16, lane4 = lane * 4;
    auto epi_base = [&](uint32_t sb) -> uint8_t* { return lds + L::kOffEpi + (sb & 1) * L::kEpi; };

    v16f accf[kTM][kTN];
    v16i hi[kTM][kTN], lo[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) accf[i][j] = v16f{};

    // ---- super-block epilogue of tile (i, j): y += d_a d_w (hi * 2^s + lo) [- d_a dmin I2] ----
    constexpr int kShift = kQ4K ? 3 : 8;
    auto epilogue_tile = [&](uint32_t sb, int i, int j) {
        const uint8_t* epi = epi_base(sb);
        const float* eda = reinterpret_cast<const float*>(epi + L::kEDa);
        const uint32_t nl = wn * 64 + j * 32 + lrow;
        float dw;
        if (kQ4K) {
            dw = f16_bits_to_f32(*reinterpret_cast<const uint32_t*>(epi + L::kEHdr + nl * 16) & 0xffffu);
        } else {
            // d rows are padded to 4 bytes: the dword holds super-blocks 2*(sb/2), +1
            const uint32_t dd = reinterpret_cast<const uint32_t*>(epi + L::kEB)[nl];
            dw = f16_bits_to_f32(((sb0 + sb) & 1) ? (dd >> 16) : (dd & 0xffffu));
        }
        const uint32_t rl = wm * 64 + i * 32;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 d4 = *reinterpret_cast<const float4*>(eda + rl + q * 8 + lgrp * 4);
            const float da[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int iv = hi[i][j][4 * q + e] * (1 << kShift) + lo[i][j][4 * q + e];
                accf[i][j][4 * q + e] = fmaf((float)iv, dw * da[e], accf[i][j][4 * q + e]);
            }
        }
        if (kQ4K) {
            // both min-term operands are laid out [32-block][half][32] (16 B
            // each), so the lane's entry is at lane * 16 past a uniform base
            const uint4 bmin = reinterpret_cast<const uint4*>(epi + L::kEB)[(wn * 2 + j) * 64 + lane];
            const uint4 av = reinterpret_cast<const uint4*>(epi + L::kESum)[(wm * 2 + i) * 64 + lane];
            const v8bf a8 = __builtin_bit_cast(v8bf, av);
            const v8bf bh8 = __builtin_bit_cast(v8bf, make_uint4(bmin.x, bmin.y, bmin.x, bmin.y));
            const v8bf bl8 = __builtin_bit_cast(v8bf, make_uint4(bmin.z, bmin.w, bmin.z, bmin.w));
            accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bh8, accf[i][j], 0, 0, 0);
            accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bl8, accf[i][j], 0, 0, 0);
        }
    };

    // The main loop, specialised per wavefront group (G = 0: weights, 1:
    // activation side data) and by whether the wavefront's 64 rows hold any
    // row below m (MF; without, its MFMAs and epilogues are left out and it
    // only fetches and expands its share for the others).
    auto run = [&](auto gc, auto mfc) {
        constexpr int G = decltype(gc)::value;
        constexpr bool MF = decltype(mfc)::value;
        constexpr int kBase = G == 0 ? L::kBase0 : L::kBase1;
        constexpr int kExtra = G == 0 ? L::kExtra0 : L::kExtra1;
        constexpr int kParts = kBase + kExtra;
        const uint32_t gw = wave & 3;                  // index within the group
        const uint32_t bc = gw >> 1, cw = gw & 1;      // group 0: chunk and 64-column half
        const uint32_t col = cw * 64 + lane;           // group 0: this lane's weight column
        // q and h planes row-major; the tiled header copy (kq_tile_off): the
        // 128-column tile starting at n0, super-block sb0 + sb at sb * 2048,
        // this lane's column at col * 16
        const uint32_t lc = min(col, col_max);
        const uint32_t q_lane = lc * w.q_row;
        const uint8_t* wq = w.q + (size_t)n0 * w.q_row + sb0 * 128;
        const uint8_t* wh = w.h + (size_t)n0 * w.h_row + sb0 * 64;
        const uint8_t* ws = w.st + kq_tile_off(w.nb, n0, sb0, 16);
        const uint8_t* wd = w.dt + kq_tile_off((w.nb + 1) / 2, n0, 0, 4);
        const uint32_t nstage = 4 * nsb;

        // The LDS addresses are wavefront-uniform; readfirstlane states it
        // where the row specialisation (PART) hides it from the compiler.
        auto dma16u = [](const void* base, uint32_t off, uint32_t lds_addr) {
            dma16(base, off, PART ? __builtin_amdgcn_readfirstlane(lds_addr) : lds_addr);
        };
        auto dma4u = [](const void* base, uint32_t off, uint32_t lds_addr) {
            dma4(base, off, PART ? __builtin_amdgcn_readfirstlane(lds_addr) : lds_addr);
        };
        // DMA instruction p of stage st (parts past kBase only at a super-block's first stage)
        auto issue_part = [&](uint32_t st, int p) {
            const uint32_t slot = st % kRing, sb = st >> 2;
            const uint32_t epi = lbase + L::kOffEpi + (sb & 1) * L::kEpi;
            if (p < 2) {
                // activation piece t = 2*wave + p: (ks, h, 64-row block)
                const uint32_t t = 2 * wave + p, ks = t >> 3, h = (t >> 2) & 1, rb = t & 3;
                dma16u(t_q + (size_t)rblk(rb) * 64 * K + st * 4096 + (ks * 2 + h) * 1024, lane16,
                      lbase + L::kOffA + slot * L::kASlot + ((ks * 2 + h) * kBM + rb * 64) * 16);
                return;
            }
            if (G == 0) {
                const uint32_t raw = lbase + L::kOffRaw + slot * L::kRawSlot + (bc * kBN + cw * 64) * 16;
                // chunk 2 * (st & 3) + bc of super-block st >> 2
                if (p == 2) dma16u(wq + bc * 16 + st * 32, q_lane, raw);
                if (!kQ4K && p == 3) dma16u(wh + st * 16, q_lane >> 1, raw + L::kQSlot);  // qh of chunks 2st, 2st+1
                if (p == kBase) dma16u(ws + sb * 2048, lc * 16, epi + L::kEHdr + cw * 64 * 16);
                if (!kQ4K && p == kBase + 1)
                    dma4u(wd + ((sb0 + sb) >> 1) * 512, lc * 4, epi + L::kEB + cw * 64 * 4);
            } else {
                if (p == kBase)
                    dma4u(t_d + ((size_t)rblk(gw) * nsb_all + sb) * 256, lane4, epi + L::kEDa + 64 * gw * 4);
                if (kQ4K && p > kBase) {
                    const uint32_t i = p - kBase - 1;  // row 64*gw + 32*i + lane%32, half lane/32
                    dma16u(t_s + (((size_t)rblk(gw) * nsb_all + sb) * 2 + i) * 1024, lane16,
                          epi + L::kESum + (64 * gw + 32 * i) * 32);
                }
            }
        };

        // Stage st's own-data work after its DMA has landed: group 0 turns its
        // weight chunks into digit planes (st & 1) and, at a super-block's first
        // stage, its columns' block headers into the min-term operand; group 1
        // turns its rows' bsums into the min-term operand at a first stage.
        auto expand = [&](uint32_t st, auto firstc) {
            constexpr bool kFirst = decltype(firstc)::value;
            uint8_t* epi = epi_base(st >> 2);
            if (G == 1) {
                if (kQ4K && kFirst) {
                    const float* eda = reinterpret_cast<const float*>(epi + L::kEDa);
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        uint4* sp = reinterpret_cast<uint4*>(epi + L::kESum + (64 * gw + 32 * i) * 32) + lane;
                        const uint4 pr = *sp;
                        const float da = eda[64 * gw + 32 * i + (lane & 31)];
                        const uint32_t prs[4] = {pr.x, pr.y, pr.z, pr.w};
                        float v[4];
#pragma unroll
                        for (int t = 0; t < 4; t++)
                            v[t] = -da * (float)((int)(int16_t)(prs[t] & 0xffffu) + (int)(int16_t)(prs[t] >> 16));
                        *sp = bf16_hilo4(v);
                    }
                }
                return;
            }
            const uint8_t* raw = lds + L::kOffRaw + (st % kRing) * L::kRawSlot;
            const uint4 rq = *reinterpret_cast<const uint4*>(raw + (bc * kBN + col) * 16);
            const uint4 hd = *reinterpret_cast<const uint4*>(epi + L::kEHdr + col * 16);
            uint8_t* pl = lds + L::kOffPlanes + (st & 1) * L::kPlanes;
            auto put = [&](int plane, int half, uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3) {
                *reinterpret_cast<uint4*>(pl + (((bc * 2 + plane) * 2 + half) * kBN + col) * 16) = make_uint4(x0, x1, x2, x3);
            };
            if (kQ4K) {
                int sc, mn;
                q4k_scale_min(hd.y, hd.z, hd.w, (int)((2 * st + bc) & 7), sc, mn);
                const uint32_t sh = (uint32_t)sc >> 3, sl = (uint32_t)sc & 7;
                const uint32_t q4[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    uint32_t nib[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) nib[j] = (q4[j] >> (4 * half)) & 0x0F0F0F0Fu;
                    put(0, half, mul_bytes(nib[0], sh), mul_bytes(nib[1], sh), mul_bytes(nib[2], sh), mul_bytes(nib[3], sh));
                    put(1, half, mul_bytes(nib[0], sl), mul_bytes(nib[1], sl), mul_bytes(nib[2], sl), mul_bytes(nib[3], sl));
                }
                if (kFirst) {
                    // this column: dmin * m_j of sub-blocks 4*bc .. 4*bc+3 -> bf16 hi|lo
                    const float dm = f16_bits_to_f32(hd.x >> 16);
                    float v[4];
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        int sc2, mn2;
                        q4k_scale_min(hd.y, hd.z, hd.w, (int)(4 * bc + t), sc2, mn2);
                        v[t] = dm * (float)mn2;
                    }
                    *reinterpret_cast<uint4*>(epi + L::kEB + (((cw * 2 + (lane >> 5)) * 2 + bc) * 32 + (lane & 31)) * 16) =
                        bf16_hilo4(v);
                }
            } else {
                const uint2 qh = *reinterpret_cast<const uint2*>(raw + L::kQSlot + (bc * kBN + col) * 16 + bc * 8);
                int b[8];
                q6k_unpack(rq, qh, b);
                const uint32_t q = st & 3;  // scales of chunks 2st, 2st+1
                const uint32_t sw = q == 0 ? hd.x : (q == 1 ? hd.y : (q == 2 ? hd.z : hd.w));
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int sc = (int)(int8_t)(sw >> (8 * (2 * bc + half)));
                    uint32_t lo4[4], hi4[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) q6_digits((uint32_t)b[4 * half + j], sc, lo4[j], hi4[j]);
                    put(0, half, hi4[0], hi4[1], hi4[2], hi4[3]);
                    put(1, half, lo4[0], lo4[1], lo4[2], lo4[3]);
                }
            }
        };

        // ---- one stage s = 4*sb + t: 2 chunks x 2 x 2 tiles x 2 digit planes of
        //      int8 MFMA.  Chunk 0 issues stage s+3's DMA between its MFMAs and,
        //      at a super-block's first stage, starts the sums from zero.  Chunk
        //      1's MFMAs are interleaved with stage s+1's expansion.  A
        //      super-block's last stage ends with its epilogue.  kLast marks the
        //      final super-block, where stages past the end are neither fetched
        //      nor expanded ----
        auto stage = [&](uint32_t sb, auto tc, auto lastc) {
            constexpr int t = decltype(tc)::value;
            constexpr bool kLast = decltype(lastc)::value != 0;
            constexpr bool kMore = !kLast || t == 0;      // stage s+3 exists
            constexpr bool kExpand = !kLast || t < 3;     // stage s+1 exists
            constexpr bool kFirst3 = ((t + 3) & 3) == 0;  // stage s+3 starts a super-block
            constexpr int kNParts = kFirst3 ? kParts : kBase;
            // this wavefront's DMA still in flight once stage s+1's has landed
            constexpr int kC2 = (kLast && t >= 2) ? 0 : kBase + (t == 2 ? kExtra : 0);
            constexpr int kC3 = kMore ? kBase + (kFirst3 ? kExtra : 0) : 0;
            const uint32_t s = 4 * sb + t;
            const uint8_t* abase = lds + L::kOffA + t * L::kASlot;  // slot s % 4 = t
            const uint8_t* pbase = lds + L::kOffPlanes + (t & 1) * L::kPlanes;
            auto a_frag = [&](int ks, int i) {
                return *reinterpret_cast<const v4i*>(abase + ((ks * 2 + lgrp) * kBM + wm * 64 + i * 32 + lrow) * 16);
            };
            auto b_frag = [&](int ks, int p, int j) {
                return *reinterpret_cast<const v4i*>(
                    pbase + (((ks * 2 + p) * 2 + lgrp) * kBN + wn * 64 + j * 32 + lrow) * 16);
            };
            {
                v4i av[kTM], bv[2][kTN];
                if constexpr (MF) {
#pragma unroll
                    for (int i = 0; i < kTM; i++) av[i] = a_frag(0, i);
#pragma unroll
                    for (int p = 0; p < 2; p++)
#pragma unroll
                        for (int j = 0; j < kTN; j++) bv[p][j] = b_frag(0, p, j);
                }
#pragma unroll
                for (int i = 0; i < kTM; i++)
#pragma unroll
                    for (int j = 0; j < kTN; j++) {
                        const int k = (i * kTN + j) * 2;
                        if constexpr (!MF) {
                        } else if (t == 0) {
                            hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[0][j], v16i{}, 0, 0, 0);
                            lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[1][j], v16i{}, 0, 0, 0);
                        } else {
                            hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[0][j], hi[i][j], 0, 0, 0);
                            lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[1][j], lo[i][j], 0, 0, 0);
                        }
                        if (kMore && k < kNParts) issue_part(s + 3, k);
                        if (kMore && k + 1 < kNParts) issue_part(s + 3, k + 1);
                    }
            }
            if (kExpand) wait_vm<kC2 + kC3>();
            {
                v4i av[kTM], bv[2][kTN];
                if constexpr (MF) {
#pragma unroll
                    for (int i = 0; i < kTM; i++) av[i] = a_frag(1, i);
#pragma unroll
                    for (int p = 0; p < 2; p++)
#pragma unroll
                        for (int j = 0; j < kTN; j++) bv[p][j] = b_frag(1, p, j);
                }
                if (kExpand) expand(s + 1, std::integral_constant<bool, ((t + 1) & 3) == 0>{});
                if constexpr (MF) {
#pragma unroll
                    for (int i = 0; i < kTM; i++)
#pragma unroll
                        for (int j = 0; j < kTN; j++) {
                            hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[0][j], hi[i][j], 0, 0, 0);
                            lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[1][j], lo[i][j], 0, 0, 0);
                        }
                }
                // interleave: LDS reads first, then one MFMA per few VALU
                // instructions of the expansion, then its LDS writes
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
                for (int k = 0; k < 2 * kTM * kTN; k++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x200, 8, 0);
            }
            if (MF && t == 3) {
#pragma unroll
                for (int i = 0; i < kTM; i++)
#pragma unroll
                    for (int j = 0; j < kTN; j++) epilogue_tile(sb, i, j);
            }
            __syncthreads();
        };

        // prologue: stages 0-2 in flight, stage 0 expanded and published
#pragma unroll
        for (int p = 0; p < kParts; p++) issue_part(0, p);
        if (nstage > 1)
#pragma unroll
            for (int p = 0; p < kBase; p++) issue_part(1, p);
        if (nstage > 2)
#pragma unroll
            for (int p = 0; p < kBase; p++) issue_part(2, p);
        wait_vm<0>();
        expand(0, std::true_type{});
        __syncthreads();

        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        for (uint32_t sb = 0; sb + 1 < nsb; sb++) {
            stage(sb, I0{}, std::false_type{});
            stage(sb, I1{}, std::false_type{});
            stage(sb, I2{}, std::false_type{});
            stage(sb, I3{}, std::false_type{});
        }
        stage(nsb - 1, I0{}, std::true_type{});
        stage(nsb - 1, I1{}, std::true_type{});
        stage(nsb - 1, I2{}, std::true_type{});
        stage(nsb - 1, I3{}, std::true_type{});
    };
    // wavefront-uniform: does this wavefront's 64-row band hold a row below m
    // (PART: the launch has a last row tile at most half full; the variant
    // without MFMAs costs the full tiles a few spilled registers, so only
    // such launches carry it)
    const bool rows = !PART || __builtin_amdgcn_readfirstlane(m0 + wm * 64 < m ? 1u : 0u) != 0;
    if (!PART) {
        if (wave < 4) run(std::integral_constant<int, 0>{}, std::true_type{});
        else run(std::integral_constant<int, 1>{}, std::true_type{});
    } else if (wave < 4) {
        if (rows) run(std::integral_constant<int, 0>{}, std::true_type{});
        else run(std::integral_constant<int, 0>{}, std::false_type{});
    } else {
        if (rows) run(std::integral_constant<int, 1>{}, std::true_type{});
        else run(std::integral_constant<int, 1>{}, std::false_type{});
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

template <int DT, bool PART>
hipError_t launch_dt(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                     hipStream_t s) {
    {
        const hipError_t e = set_max_lds(reinterpret_cast<const void*>(qmm_kernel<DT, PART>), Lay<DT>::kLds);
        if (e != hipSuccess) return e;
    }
    const uint32_t nsb = w.k / 256;
    const uint32_t per = (nsb + splits - 1) / splits;
    splits = (nsb + per - 1) / per;  // every split non-empty
    const dim3 grid((w.n + kBN - 1) / kBN, (unsigned)((m + kBM - 1) / kBM), splits);
    float* out = splits > 1 ? partial : y;
    hipLaunchKernelGGL((qmm_kernel<DT, PART>), grid, dim3(kThreads), Lay<DT>::kLds, s, w, a, (uint32_t)m, per, out,
                       splits > 1 ? m * (size_t)w.n : (size_t)0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    const size_t count = m * (size_t)w.n;
    return launch_sum_splits(partial, count, splits, y, s);
}

}  // namespace

bool mfma_supported(uint32_t dtype, size_t m, size_t n, size_t k) {
    (void)m;
    (void)n;
    return (dtype == XNQ_Q4K || dtype == XNQ_Q6K) && k % 256 == 0;
}

uint32_t mfma_splits(size_t m, size_t n, size_t k) {
    // Split K while whole splits of the grid still fit on the 256 CUs at
    // once (one workgroup per CU), each split at least two super-blocks long.
    const size_t tiles = ((n + kBN - 1) / kBN) * ((m + kBM - 1) / kBM);
    const size_t nsb = k / 256;
    size_t splits = 256 / tiles;
    if (splits > nsb / 2) splits = nsb / 2;
    return splits < 1 ? 1u : (uint32_t)splits;
}

hipError_t launch_mfma(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                       hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    // the kernel reads the row-tiled activation image, which must cover m rows
    if (!a.tile || (size_t)a.T.rbs * 64 < m || a.k != w.k) return hipErrorInvalidValue;
    if (splits > 1 && !partial) splits = 1;
    if (prefill_supported(w.dtype, m, w.n, w.k)) return launch_prefill(w, a, m, splits, y, partial, s);
    // a last row tile at most half full leaves its wavefronts 4-7 without
    // rows: the PART kernel drops their MFMAs (Q6_K 4096 -> 14336, µs, one
    // box: m = 65 46 -> 43, 128 49 -> 45; Q4_K m = 600 136 -> 121; full tiles
    // keep the kernel without the branch: 256 51 against 53, 512 75-78
    // against 80-81)
    const size_t tail = m % kBM;
    const bool part = tail != 0 && tail <= kBM / 2;
    if (w.dtype == XNQ_Q4K)
        return part ? launch_dt<XNQ_Q4K, true>(w, a, m, splits, y, partial, s)
                    : launch_dt<XNQ_Q4K, false>(w, a, m, splits, y, partial, s);
    if (w.dtype == XNQ_Q6K)
        return part ? launch_dt<XNQ_Q6K, true>(w, a, m, splits, y, partial, s)
                    : launch_dt<XNQ_Q6K, false>(w, a, m, splits, y, partial, s);
    return hipErrorNotSupported;
}

}  // namespace xnq
