// Small-batch quantized matmul (m = 2 .. 64) on the int8 matrix cores.
//
// At a few rows the product is bound by the weight stream, so every weight
// byte is read once, and what limits the rate is how much of the stream is
// in flight.  This kernel therefore fetches everything a super-block (256
// columns of K) needs -- the weight chunks and block headers of its columns,
// the activation tile in MFMA order, d_a and the Q8K block sums -- with
// global_load_lds DMA into a ring of LDS slots, one super-block ahead of the
// one being multiplied, so the stream costs no registers and the wavefronts
// do not wait on a load they issued just before.
//
// A workgroup of NW = 4 or 8 wavefronts owns 32 * NW weight columns (output
// columns) and a range of super-blocks; wavefront w owns columns 32w ..
// 32w+31 and all m activation rows: up to 16 rows one 16-row tile on
// v_mfma_i32_16x16x64_i8 (two 16-column tiles per wavefront, compute16),
// above that one or two 32-row tiles on v_mfma_i32_32x32x32_i8.  Per
// super-block each wavefront expands its columns' chunks from LDS into the
// two int8 digit planes of the prefill kernel (Q4K: sc = 8*sh + sl, digits
// sh*q and sl*q; Q6K: sc*(q-32) = 256*hi + lo), contracts them with the
// activation tile and applies d_a * d_w in an f32 epilogue; the Q4K min term
// is a GEMM of -d_a*bsum32 by dmin*m_j on the bf16 matrix cores.  The integer sums per super-block are exact, as in the reference's
// block dots (k_quants.rs:1337-1416, 1743-1798).  When the column tiles alone
// do not fill the GPU, the super-blocks are split across workgroups and the
// partial outputs are summed in split order afterwards.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// LDS slot of one super-block (byte offsets).  R = 16 activation rows for
// MT == 0 (16-row tiles), else 32 * MT; C = 32 * NW columns.
//   wq   [col C][slot 8][16]  weight chunk (slot ^ (col & 7)) of the column
//   hdr  Q4K: d | dmin, scales[12]; Q6K: int8 scales[16]; 16-row tiles
//        [col C][16], else [wave NW][lane 64][16] (the wavefront's column
//        lane & 31)
//   wh   Q6K [col C][slot 4][16]  high-bit words of chunks 2p, 2p+1, p = slot ^ (col & 3)
//   wd   Q6K dword holding the f16 d of super-blocks 2j, 2j+1: 16-row tiles
//        [col C], else [wave NW][lane 64]
//   act  [chunk 8][half 2][row R][16]  activation quants in MFMA A order
//   bs   Q4K [row R][part 2][16]   chunk bsum pairs of sub-blocks 4*part .. +3
//   da   [64] f32 d_a per row (rows past m repeat the last)
// The XOR slot order makes the 32 columns' reads of one chunk hit distinct
// banks while each column's bytes still arrive as one 128-byte line.
// Two slots: the smaller LDS footprint lets two or three workgroups share a
// CU, and their barriers and expansion interleave, which beats a deeper
// ring in one workgroup (batch-16 decode step 2633 us with four slots, 2581
// with three, 2514 with two).  A larger XNQ_SKINNY_RING_MAX at build time
// deepens it where the LDS allows.
#ifndef XNQ_SKINNY_RING_MAX
#define XNQ_SKINNY_RING_MAX 2
#endif
constexpr int kRingMax = XNQ_SKINNY_RING_MAX;

template <int DT, int MT, int NW>
struct KLay {
    static constexpr bool kQ4K = DT == XNQ_Q4K;
    static constexpr int kWaves = NW, kThreads = 64 * NW, kCols = 32 * NW;
    static constexpr int R = MT == 0 ? 16 : 32 * MT;
    // 16-row tiles: headers and Q6K d once per column ([col][16], [col]
    // dword), fetched by the first kCols / 64 wavefronts, and no padding DMA
    static constexpr bool kNarrow = MT == 0;
    static constexpr int kHdrWaves = kCols / 64;
    static constexpr int kWq = 0;
    static constexpr int kHdr = kWq + kCols * 128;
    static constexpr int kWh = kHdr + (kNarrow ? kCols * 16 : kWaves * 64 * 16);
    static constexpr int kWd = kWh + (kQ4K ? 0 : kCols * 64);
    static constexpr int kAct = kWd + (kQ4K ? 0 : (kNarrow ? kCols * 4 : kWaves * 64 * 4));
    static constexpr int kBs = kAct + 8 * 2 * R * 16;
    static constexpr int kDa = kBs + (kQ4K ? (R < 32 ? 32 : R) * 32 : 0);  // one DMA fills 32 rows
    static constexpr int kDummy = kDa + 64 * 4;  // target of the padding DMA
    static constexpr int kSlot = kDummy + (kNarrow ? 0 : 64 * 4);
    static constexpr int kRing = (kRingMax * kSlot <= 160 * 1024) ? kRingMax
                                 : (4 * kSlot <= 160 * 1024)        ? 4
                                 : (3 * kSlot <= 160 * 1024)        ? 3
                                                                    : 2;
    static constexpr int kLds = kRing * kSlot;
    // DMA instructions per wavefront per super-block, the same in every
    // wavefront so one vmcnt count fits all: weights, activation pieces, and
    // one of {bsums, d_a, padding}
    // 8 * MT KiB of activation over NW wavefronts (MT == 0: 4 KiB, one each)
    static constexpr int kActPer = MT == 0 ? 1 : 8 * MT / NW;
    static constexpr int kWPer = kQ4K ? 4 + 1 : 4 + 1 + 2 + 1;
    static constexpr int kD = kWPer + kActPer + 1;  // the most any wavefront issues
    static_assert(kLds <= 160 * 1024, "LDS budget");
    static_assert((kRing - 2) * kD < 64, "vmcnt range");
    // 16-row tiles: DMA instructions per super-block of wavefront w (the
    // weights, then a header, activation piece and bsum / d_a load only for
    // the wavefronts that have one)
    static constexpr uint32_t kExtra = kQ4K ? 2u : 1u;  // Q4K: bsums (w 0), d_a (w 1); Q6K: d_a (w 0)
    __host__ __device__ static constexpr int dma_count(uint32_t w) {
        return (kQ4K ? 4 : 4 + 2) + (w < (uint32_t)kHdrWaves ? (kQ4K ? 1 : 2) : 0) + (w < 4u ? 1 : 0) +
               (w < kExtra ? 1 : 0);
    }
};

// Wait until at most `younger` super-blocks' DMA (KD instructions each) are
// outstanding, younger <= Y (wavefront-uniform).
template <int KD, int Y>
__device__ __forceinline__ void wait_younger(uint32_t younger) {
    if constexpr (Y == 0) {
        wait_vm<0>();
    } else {
        if (younger >= (uint32_t)Y) wait_vm<Y * KD>();
        else wait_younger<KD, Y - 1>(younger);
    }
}

// wait_younger for a wavefront-uniform per-super-block DMA count kd (one of
// the few values KLay::dma_count takes)
template <int Y>
__device__ __forceinline__ void wait_younger_n(uint32_t kd, uint32_t younger) {
    switch (kd) {
    case 4: wait_younger<4, Y>(younger); break;
    case 5: wait_younger<5, Y>(younger); break;
    case 6: wait_younger<6, Y>(younger); break;
    case 7: wait_younger<7, Y>(younger); break;
    case 8: wait_younger<8, Y>(younger); break;
    case 9: wait_younger<9, Y>(younger); break;
    case 10: wait_younger<10, Y>(younger); break;
    default: wait_vm<0>(); break;
    }
}


// One super-block of a 16-row tile (m <= 16) for wavefront `wave`'s 16 * TC
// columns, as TC 16-column tiles on v_mfma_i32_16x16x64_i8: lane l holds
// row / column l & 15 and the 16-element K slice g = l >> 4 of each
// 64-element step, that is half g & 1 of chunk 2*ks + (g >> 1); the
// accumulator holds rows 4g .. 4g+3 of column l & 15.  Digit planes,
// epilogue and min term as in the 32-row path (skinny_kernel).
template <int DT, class L, int TC = 2>
__device__ __forceinline__ void compute16(const uint8_t* S, uint32_t wave, uint32_t lane, bool odd_sb, v4f* acc) {
    constexpr bool kQ4K = L::kQ4K;
    constexpr int kShift = kQ4K ? 3 : 8;
    const uint32_t g = lane >> 4, li = lane & 15, h = g & 1;
    uint4 hdr[TC];
    Q4KScales qs[TC];
#pragma unroll
    for (int ct = 0; ct < TC; ct++) {
        hdr[ct] = *reinterpret_cast<const uint4*>(S + L::kHdr + (wave * 32 + ct * 16 + li) * 16);
        if (kQ4K) qs[ct] = q4k_scales(hdr[ct].y, hdr[ct].z, hdr[ct].w);
    }
    v4i hi[TC], lo[TC];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const int c = 2 * ks + (int)(g >> 1);
        const v4i av = *reinterpret_cast<const v4i*>(S + L::kAct + ((4 * ks + g) * 16 + li) * 16);
#pragma unroll
        for (int ct = 0; ct < TC; ct++) {
            const uint32_t cl = wave * 32 + ct * 16 + li;
            const uint4 qc = *reinterpret_cast<const uint4*>(S + L::kWq + cl * 128 + ((c ^ (cl & 7)) * 16));
            const uint32_t q4[4] = {qc.x, qc.y, qc.z, qc.w};
            uint32_t p0[4], p1[4];
            if (kQ4K) {
                // scale of sub-block c = 2 ks + (g >> 1): dword by ks, byte by lane
                const uint32_t sc = ((ks < 2 ? qs[ct].sc_lo : qs[ct].sc_hi) >> (8 * ((2 * ks) & 3) + 8 * (g >> 1))) & 0xffu;
                const uint32_t sh = sc >> 3, sl = sc & 7;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t nib = (q4[j] >> (4 * h)) & 0x0F0F0F0Fu;
                    p0[j] = mul_bytes(nib, sh);
                    p1[j] = mul_bytes(nib, sl);
                }
            } else {
                const uint2 qh = *reinterpret_cast<const uint2*>(S + L::kWh + cl * 64 + (((c >> 1) ^ (cl & 3)) * 16) +
                                                                 (c & 1) * 8);
                const uint32_t qhw = h ? qh.y : qh.x;
                const uint32_t hw = hdr[ct].x, hy = hdr[ct].y, hz = hdr[ct].z, hv = hdr[ct].w;
                const uint32_t sw = (c >> 1) == 0 ? hw : (c >> 1) == 1 ? hy : (c >> 1) == 2 ? hz : hv;
                const int sc = (int)(int8_t)(sw >> (8 * (2 * (c & 1) + h)));
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t qs = j < 2 ? qhw << (4 - 2 * j) : qhw >> (2 * j - 4);
                    const uint32_t b = ((q4[j] >> (4 * h)) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
                    q6_digits(b, sc, p1[j], p0[j]);
                }
            }
            const v4i b0 = {(int)p0[0], (int)p0[1], (int)p0[2], (int)p0[3]};
            const v4i b1 = {(int)p1[0], (int)p1[1], (int)p1[2], (int)p1[3]};
            if (ks == 0) {
                hi[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b0, v4i{}, 0, 0, 0);
                lo[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b1, v4i{}, 0, 0, 0);
            } else {
                hi[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b0, hi[ct], 0, 0, 0);
                lo[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b1, lo[ct], 0, 0, 0);
            }
        }
    }
    // epilogue: acc += d_a d_w (hi * 2^s + lo)  [- d_a dmin sum_j m_j bsum32_j]
    const float* eda = reinterpret_cast<const float*>(S + L::kDa);
    const float4 d4 = *reinterpret_cast<const float4*>(eda + 4 * g);
    const float da[4] = {d4.x, d4.y, d4.z, d4.w};
    v8bf a8;
    if (kQ4K) {
        // row side of the min term: -d_a * bsum32 of sub-blocks 2g, 2g+1 of row li,
        // as bf16 hi/lo pairs (ah0, al0, ah1, al1) twice
        const uint2 pr = *reinterpret_cast<const uint2*>(S + L::kBs + (li * 2 + (g >> 1)) * 16 + (g & 1) * 8);
        const float dr = eda[li];
        float v[2];
        v[0] = -dr * (float)((int)(int16_t)(pr.x & 0xffffu) + (int)(int16_t)(pr.x >> 16));
        v[1] = -dr * (float)((int)(int16_t)(pr.y & 0xffffu) + (int)(int16_t)(pr.y >> 16));
        const __bf16 h0 = (__bf16)v[0], h1 = (__bf16)v[1];
        const __bf16 l0 = (__bf16)(v[0] - (float)h0), l1 = (__bf16)(v[1] - (float)h1);
        a8 = v8bf{h0, l0, h1, l1, h0, l0, h1, l1};
    }
#pragma unroll
    for (int ct = 0; ct < TC; ct++) {
        float dw;
        if (kQ4K) {
            dw = f16_bits_to_f32(hdr[ct].x & 0xffffu);
        } else {
            const uint32_t dd = reinterpret_cast<const uint32_t*>(S + L::kWd)[wave * 32 + ct * 16 + li];
            dw = f16_bits_to_f32(odd_sb ? (dd >> 16) : (dd & 0xffffu));
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int iv = hi[ct][e] * (1 << kShift) + lo[ct][e];
            acc[ct][e] = fmaf((float)iv, dw * da[e], acc[ct][e]);
        }
        if (kQ4K) {
            // column side: dmin * m_j of sub-blocks 2g, 2g+1, hi/lo bf16 pairs
            // (mh0, mh0, mh1, mh1, ml0, ml0, ml1, ml1): the 8-term dot with a8
            // is (ah0 + al0)(mh0 + ml0) + (ah1 + al1)(mh1 + ml1)
            const float dm = f16_bits_to_f32(hdr[ct].x >> 16);
            // mins of sub-blocks 2g, 2g + 1: bytes 2 (g & 1), +1 of m_lo (g < 2) or m_hi
            const uint32_t mw = (g < 2 ? qs[ct].m_lo : qs[ct].m_hi) >> (16 * (g & 1));
            const float w0 = dm * (float)(mw & 0xffu), w1 = dm * (float)((mw >> 8) & 0xffu);
            const __bf16 h0 = (__bf16)w0, h1 = (__bf16)w1;
            const __bf16 l0 = (__bf16)(w0 - (float)h0), l1 = (__bf16)(w1 - (float)h1);
            const v8bf b8 = {h0, h0, h1, h1, l0, l0, l1, l1};
            acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a8, b8, acc[ct], 0, 0, 0);
        }
    }
}

// Where each weight of a launch writes: y[t] (the destination, or its
// split-K partial region of `stride[t]` floats per split) for the column
// tiles below tile_end[t] (cumulative over the group).
struct SkOut {
    float* y[kMaxGroup];
    size_t stride[kMaxGroup];
    uint32_t tile_end[kMaxGroup];
};

// One launch covers the column tiles of up to kMaxGroup weights of one dtype
// and K (G.w[0..count)): a workgroup's tile picks its weight, uniformly, so
// the weight view is read with scalar loads.
template <int DT, int MT, int NW>
__global__ __launch_bounds__(64 * NW) void skinny_kernel(WGroup G, SkOut O, AView a, uint32_t m,
                                                          uint32_t sb_per_split) {
    using L = KLay<DT, MT, NW>;
    constexpr int kCols = L::kCols;
    constexpr bool kQ4K = L::kQ4K;
    constexpr int kShift = kQ4K ? 3 : 8;
    constexpr int kD = L::kD;
    constexpr int kRing = L::kRing;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lrow = lane & 31, half = lane >> 5;
    const uint32_t bx = blockIdx.x;
    const uint32_t t = G.count > 1 && bx >= O.tile_end[0] ? (G.count > 2 && bx >= O.tile_end[1] ? 2u : 1u) : 0u;
    const WView w = G.w[t];
    float* __restrict__ y = O.y[t] + blockIdx.y * O.stride[t];
    const uint32_t sb0 = blockIdx.y * sb_per_split;
    const uint32_t nsb = min(sb_per_split, w.k / 256 - sb0);
    const uint32_t col0 = (bx - (t > 0 ? O.tile_end[t - 1] : 0u)) * kCols;
    const uint32_t ncol = col0 + wave * 32 + lrow;  // this lane's output column
    const uint32_t lbase = (uint32_t)(uintptr_t)lds;  // low half of the flat address = LDS offset
    const ActImg& A = a.A;
    // lanes past the last column or row re-read the last one (every DMA
    // instruction is issued by the whole wavefront: vmcnt counts instructions);
    // those outputs are dropped at the store
    const uint32_t cmax = w.n - 1, rmax = m - 1;
    // Q4K: bsums take the first MT wavefronts' extra instruction, d_a the next
    constexpr uint32_t kExtraBs = kQ4K ? (uint32_t)(MT == 0 ? 1 : MT) : 0u;

    // ---- the DMA of super-block i: kD instructions per wavefront ----
    // Per-lane byte offsets are fixed for the whole walk; the super-block
    // moves only the uniform base pointers (one super-block of a 128-row
    // tile is 128 * P bytes in the tiled st and dt copies).
    // weight chunks: instruction j covers columns 32*wave + 8j .. +7,
    // lane = 8 * column + slot, slot s holding chunk s ^ (column & 7)
    uint32_t oq[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t cl = wave * 32 + 8 * j + (lane >> 3);
        oq[j] = min(col0 + cl, cmax) * w.q_row + ((lane & 7) ^ (cl & 7)) * 16;
    }
    // block header (Q4K) / scales (Q6K) of column lane & 31; Q6K d dword
    // (16-row tiles: column 64 * wave + lane, for the first kCols / 64 wavefronts)
    const uint32_t ocol = min(col0 + (L::kNarrow ? wave * 64 + lane : wave * 32 + lrow), cmax);
    // tiled copies of the s and (Q6K) d planes
    const uint32_t os = kq_tile_off(w.nb, ocol, 0, 16), od = kq_tile_off((w.nb + 1) / 2, ocol, 0, 4);
    // Q6K high-bit words: instruction j covers columns 32*wave + 16j .. +15,
    // lane = 4 * column + slot, slot s holding chunk pair s ^ (column & 3)
    uint32_t oh[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t cl = wave * 32 + 16 * j + (lane >> 2);
        oh[j] = kQ4K ? 0u : min(col0 + cl, cmax) * w.h_row + ((lane & 3) ^ (cl & 3)) * 16;
    }
    // activation pieces of 1 KiB.  MT == 1: piece = chunk c, lanes 0-31 rows
    // of half 0, lanes 32-63 rows of half 1.  MT == 2: piece = (chunk, half),
    // lane = row.  MT == 0: four 16-row (chunk, half) pieces p = 4w + lane/16
    // (wavefront w & 3), lane & 15 = row.
    uint32_t oa[L::kActPer];
#pragma unroll
    for (int j = 0; j < L::kActPer; j++) {
        const uint32_t t = MT == 0 ? (wave & 3) * 4 + (lane >> 4) : wave * L::kActPer + j;
        const uint32_t c = MT == 1 ? t : t >> 1;
        const uint32_t hsel = MT == 1 ? half : (t & 1);
        const uint32_t row = MT == 1 ? lrow : MT == 0 ? (lane & 15) : lane;
        oa[j] = min(row, rmax) * A.row_bytes + hsel * (A.k / 2) + c * 16;
    }
    // the extra instruction: Q4K bsums (rows 32*wave .. +31), d_a, or padding
    const uint32_t obs = min(wave * 32 + (lane >> 1), rmax) * A.row_bytes + A.s_off + (lane & 1) * 16;
    const uint32_t oda = min(lane, rmax) * A.row_bytes + A.d_off;

    auto issue = [&](uint32_t i) {
        const uint32_t sb = sb0 + i;
        const uint32_t slot = lbase + (i % kRing) * L::kSlot;
#pragma unroll
        for (int j = 0; j < 4; j++) dma16(w.q + sb * 128, oq[j], slot + L::kWq + (wave * 32 + 8 * j) * 128);
        if (!L::kNarrow || wave < (uint32_t)L::kHdrWaves)
            dma16(w.st + sb * 16 * 128, os, slot + L::kHdr + wave * 64 * 16);
        if (!kQ4K) {
#pragma unroll
            for (int j = 0; j < 2; j++) dma16(w.h + sb * 64, oh[j], slot + L::kWh + (wave * 32 + 16 * j) * 64);
            if (!L::kNarrow || wave < (uint32_t)L::kHdrWaves)
                dma4(w.dt + (sb >> 1) * 512, od, slot + L::kWd + wave * 64 * 4);
        }
        if (MT == 0) {
            if (wave < 4) dma16(a.img + sb * 128, oa[0], slot + L::kAct + wave * 1024);
        } else {
#pragma unroll
            for (int j = 0; j < L::kActPer; j++) {
                const uint32_t t = wave * L::kActPer + j;
                const uint32_t c = MT == 1 ? t : t >> 1;
                const uint32_t hsel = MT == 1 ? 0u : (t & 1);
                dma16(a.img + sb * 128, oa[j], slot + L::kAct + (c * 2 + hsel) * L::R * 16);
            }
        }
        if (wave < kExtraBs) dma16(a.img + sb * 32, obs, slot + L::kBs + wave * 32 * 32);
        else if (wave == kExtraBs) dma4(a.img + sb * 4, oda, slot + L::kDa);
        else if (!L::kNarrow) dma4(a.img + sb * 4, oda, slot + L::kDummy);
    };

    const uint32_t kDw = L::dma_count(wave);  // 16-row tiles: this wavefront's DMA per super-block
    constexpr int kAccT = MT == 0 ? 1 : MT;
    v16f acc[kAccT];
#pragma unroll
    for (int t = 0; t < kAccT; t++) acc[t] = v16f{};
    v4f acc16[2] = {v4f{}, v4f{}};  // MT == 0: the two 16-column tiles

    // prologue: super-blocks 0 .. kRing-2 in flight
#pragma unroll
    for (int i = 0; i < kRing - 1; i++)
        if ((uint32_t)i < nsb) issue(i);

    for (uint32_t i = 0; i < nsb; i++) {
        // wait for super-block i: the younger ones in flight are i+1 .. i+kRing-2
        const uint32_t younger = min((uint32_t)(kRing - 2), nsb - 1 - i);
        if constexpr (L::kNarrow) wait_younger_n<kRing - 2>(kDw, younger);
        else wait_younger<kD, kRing - 2>(younger);
        __syncthreads();  // every wavefront's DMA of i landed; slot (i-1) % kRing is free
        if (i + kRing - 1 < nsb) issue(i + kRing - 1);

        const uint8_t* S = lds + (i % kRing) * L::kSlot;
        if constexpr (MT == 0) {
            compute16<DT, L>(S, wave, lane, ((sb0 + i) & 1) != 0, acc16);
        } else {
        const uint32_t cl = wave * 32 + lrow;
        const uint4 hdr = *reinterpret_cast<const uint4*>(S + L::kHdr + (wave * 64 + lrow) * 16);
        v16i hi[MT], lo[MT];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint4 qc = *reinterpret_cast<const uint4*>(S + L::kWq + cl * 128 + ((c ^ (cl & 7)) * 16));
            uint32_t p0[4], p1[4];  // high and low digit of this lane's 16 elements of chunk c
            if (kQ4K) {
                int sc, mn;
                q4k_scale_min(hdr.y, hdr.z, hdr.w, c, sc, mn);
                const uint32_t sh = (uint32_t)sc >> 3, sl = (uint32_t)sc & 7;
                const uint32_t q4[4] = {qc.x, qc.y, qc.z, qc.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t nib = (q4[j] >> (4 * half)) & 0x0F0F0F0Fu;
                    p0[j] = mul_bytes(nib, sh);
                    p1[j] = mul_bytes(nib, sl);
                }
            } else {
                const uint2 qh = *reinterpret_cast<const uint2*>(S + L::kWh + cl * 64 + (((c >> 1) ^ (cl & 3)) * 16) +
                                                                 (c & 1) * 8);
                // this lane's 16 elements: low (half 0) or high (half 1)
                // nibbles of ql, the two high bits from qh word `half`
                // (the q6k_unpack bit layout, one half of it)
                const uint32_t qhw = half ? qh.y : qh.x;
                const uint32_t q4[4] = {qc.x, qc.y, qc.z, qc.w};
                const uint32_t sw = (c >> 1) == 0 ? hdr.x : (c >> 1) == 1 ? hdr.y : (c >> 1) == 2 ? hdr.z : hdr.w;
                const int sc = (int)(int8_t)(sw >> (8 * (2 * (c & 1) + half)));
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t b = ((q4[j] >> (4 * half)) & 0x0F0F0F0Fu) | (((qhw >> (2 * j)) & 0x03030303u) << 4);
                    q6_digits(b, sc, p1[j], p0[j]);
                }
            }
            const v4i b0 = {(int)p0[0], (int)p0[1], (int)p0[2], (int)p0[3]};
            const v4i b1 = {(int)p1[0], (int)p1[1], (int)p1[2], (int)p1[3]};
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i av = *reinterpret_cast<const v4i*>(S + L::kAct + ((c * 2 + half) * L::R + t * 32 + lrow) * 16);
                if (c == 0) {
                    hi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, v16i{}, 0, 0, 0);
                    lo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, v16i{}, 0, 0, 0);
                } else {
                    hi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, hi[t], 0, 0, 0);
                    lo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, lo[t], 0, 0, 0);
                }
            }
        }
        // epilogue: acc += d_a d_w (hi * 2^s + lo)  [- d_a dmin sum_j m_j bsum32_j]
        const float* eda = reinterpret_cast<const float*>(S + L::kDa);
        float dw;
        if (kQ4K) {
            dw = f16_bits_to_f32(hdr.x & 0xffffu);
        } else {
            const uint32_t dd = reinterpret_cast<const uint32_t*>(S + L::kWd)[wave * 64 + lrow];
            dw = f16_bits_to_f32(((sb0 + i) & 1) ? (dd >> 16) : (dd & 0xffffu));
        }
        v8bf bh8, bl8;
        if (kQ4K) {
            const float dm = f16_bits_to_f32(hdr.x >> 16);
            // mins of sub-blocks 4 half .. 4 half + 3: the bytes of m_lo / m_hi
            const Q4KScales qs = q4k_scales(hdr.y, hdr.z, hdr.w);
            const uint32_t mw = half ? qs.m_hi : qs.m_lo;
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = dm * (float)((mw >> (8 * u)) & 0xffu);
            const uint4 bv = bf16_hilo4(v);
            bh8 = __builtin_bit_cast(v8bf, make_uint4(bv.x, bv.y, bv.x, bv.y));
            bl8 = __builtin_bit_cast(v8bf, make_uint4(bv.z, bv.w, bv.z, bv.w));
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 d4 = *reinterpret_cast<const float4*>(eda + t * 32 + q * 8 + half * 4);
                const float da[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int iv = hi[t][4 * q + e] * (1 << kShift) + lo[t][4 * q + e];
                    acc[t][4 * q + e] = fmaf((float)iv, dw * da[e], acc[t][4 * q + e]);
                }
            }
            if (kQ4K) {
                // row side of the min term: -d_a * bsum32 of sub-blocks 4*half .. +3
                const uint32_t row = t * 32 + lrow;
                const uint4 pr = *reinterpret_cast<const uint4*>(S + L::kBs + (row * 2 + half) * 16);
                const float da = eda[row];
                const uint32_t prs[4] = {pr.x, pr.y, pr.z, pr.w};
                float v[4];
#pragma unroll
                for (int u = 0; u < 4; u++)
                    v[u] = -da * (float)((int)(int16_t)(prs[u] & 0xffffu) + (int)(int16_t)(prs[u] >> 16));
                const v8bf a8 = __builtin_bit_cast(v8bf, bf16_hilo4(v));
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bh8, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bl8, acc[t], 0, 0, 0);
            }
        }
        }  // MT >= 1
    }

    if constexpr (MT == 0) {
        const uint32_t g = lane >> 4;
#pragma unroll
        for (int ct = 0; ct < 2; ct++) {
            const uint32_t col = col0 + wave * 32 + ct * 16 + (lane & 15);
            if (col < w.n) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t row = 4 * g + e;
                    if (row < m) y[(size_t)row * w.n + col] = acc16[ct][e];
                }
            }
        }
        return;
    }
    if (ncol < w.n) {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t row = t * 32 + 8 * (e / 4) + 4 * half + (e % 4);
                if (row < m) y[(size_t)row * w.n + ncol] = acc[t][e];
            }
    }
}

// ---------------------------------------------------------------------------
// 16-row tiles with K split over the wavefronts of one workgroup instead of
// over workgroups: every wavefront of a workgroup owns the same 16 * TC columns
// and super-blocks wave, wave + NW, ...; it streams them through D LDS slots
// of its own (weights, block headers, the activation tile, d_a and bsums, all
// by DMA), so it never waits for another wavefront until the end, where the
// NW partial sums are added in wavefront order in LDS and stored.  No split-K
// partials and no sum launch.

// One wavefront's LDS slot (byte offsets; the compute16 layout for one
// wavefront of C = 16 * TC columns, wave index 0).
template <int DT, int TC>
struct WkLay {
    static constexpr bool kQ4K = DT == XNQ_Q4K;
    static constexpr int kCols = 16 * TC;
    static constexpr int kWq = 0;                            // [col C][slot 8][16]
    static constexpr int kHdr = kWq + kCols * 128;           // [col C][16]
    static constexpr int kWh = kHdr + kCols * 16;            // Q6K [col C][slot 4][16]
    static constexpr int kWd = kWh + (kQ4K ? 0 : kCols * 64);  // Q6K [col C] dword (lanes past C repeat them)
    static constexpr int kAct = kWd + (kQ4K ? 0 : 64 * 4);   // [chunk 8][half 2][row 16][16]
    static constexpr int kBs = kAct + 8 * 2 * 16 * 16;       // Q4K [row 16][part 2][16]
    static constexpr int kDa = kBs + (kQ4K ? 16 * 32 : 0);   // [64] f32
    static constexpr int kSlot = kDa + 64 * 4;
    // DMA instructions per super-block: weights (2 per 16 columns), header
    // (one dword DMA per 16 columns), (Q6K: high bits, one per 16 columns,
    // and d), activation, (Q4K: bsums, two dword DMAs), d_a
    static constexpr int kD = kQ4K ? 3 * TC + 4 + 2 + 1 : 3 * TC + TC + 1 + 4 + 1;
};

template <int DT, int NW, int D, int TC>
__global__ __launch_bounds__(64 * NW) void skinny_wk_kernel(WGroup G, SkOut O, AView a, uint32_t m) {
    using L = WkLay<DT, TC>;
    constexpr bool kQ4K = L::kQ4K;
    static_assert((D - 2) * L::kD < 64, "vmcnt range");
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t bx = blockIdx.x;
    const uint32_t t = G.count > 1 && bx >= O.tile_end[0] ? (G.count > 2 && bx >= O.tile_end[1] ? 2u : 1u) : 0u;
    const WView w = G.w[t];
    float* __restrict__ y = O.y[t];
    const uint32_t col0 = (bx - (t > 0 ? O.tile_end[t - 1] : 0u)) * L::kCols;
    const uint32_t nsb_all = w.k / 256;
    const uint32_t nsb = wave < nsb_all ? (nsb_all - wave + NW - 1) / NW : 0u;  // this wavefront's super-blocks
    const uint32_t lbase = (uint32_t)(uintptr_t)lds + wave * D * L::kSlot;
    const ActImg& A = a.A;
    const uint32_t cmax = w.n - 1, rmax = m - 1;

    // per-lane DMA offsets (lanes past the last column or row re-read the last one)
    uint32_t oq[2 * TC];
#pragma unroll
    for (int j = 0; j < 2 * TC; j++) {
        const uint32_t cl = 8 * j + (lane >> 3);
        oq[j] = min(col0 + cl, cmax) * w.q_row + ((lane & 7) ^ (cl & 7)) * 16;
    }
    // headers: dword lane & 3 of column 16 j + lane / 4 (one dword DMA per 16
    // columns); Q6K d: column lane % C (lanes past C repeat the columns into
    // the rest of the 256-byte region)
    uint32_t os[TC];
#pragma unroll
    for (int j = 0; j < TC; j++) os[j] = kq_tile_off(w.nb, min(col0 + 16 * j + (lane >> 2), cmax), 0, 16) + (lane & 3) * 4;
    const uint32_t od = kq_tile_off((w.nb + 1) / 2, min(col0 + (lane % (uint32_t)L::kCols), cmax), 0, 4);
    uint32_t oh[TC];
#pragma unroll
    for (int j = 0; j < TC; j++) {
        const uint32_t cl = 16 * j + (lane >> 2);
        oh[j] = kQ4K ? 0u : min(col0 + cl, cmax) * w.h_row + ((lane & 3) ^ (cl & 3)) * 16;
    }
    uint32_t oa[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t p = j * 4 + (lane >> 4);  // piece = (chunk p / 2, half p & 1), lane & 15 = row
        oa[j] = min(lane & 15, rmax) * A.row_bytes + (p & 1) * (A.k / 2) + (p >> 1) * 16;
    }
    // bsums of rows 0..15: dword lane & 7 of row 8 j + lane / 8 (two dword DMAs)
    const uint32_t obs0 = min(lane >> 3, rmax) * A.row_bytes + A.s_off + (lane & 7) * 4;
    const uint32_t obs1 = min(8 + (lane >> 3), rmax) * A.row_bytes + A.s_off + (lane & 7) * 4;
    const uint32_t oda = min(lane, rmax) * A.row_bytes + A.d_off;

    auto issue = [&](uint32_t i) {
        const uint32_t sb = wave + i * NW;
        const uint32_t slot = lbase + (i % D) * L::kSlot;
#pragma unroll
        for (int j = 0; j < 2 * TC; j++) dma16(w.q + sb * 128, oq[j], slot + L::kWq + 8 * j * 128);
#pragma unroll
        for (int j = 0; j < TC; j++) dma4(w.st + sb * 16 * 128, os[j], slot + L::kHdr + 256 * j);
        if (!kQ4K) {
#pragma unroll
            for (int j = 0; j < TC; j++) dma16(w.h + sb * 64, oh[j], slot + L::kWh + 16 * j * 64);
            dma4(w.dt + (sb >> 1) * 512, od, slot + L::kWd);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) dma16(a.img + sb * 128, oa[j], slot + L::kAct + j * 1024);
        if (kQ4K) {
            dma4(a.img + sb * 32, obs0, slot + L::kBs);
            dma4(a.img + sb * 32, obs1, slot + L::kBs + 256);
        }
        dma4(a.img + sb * 4, oda, slot + L::kDa);
    };

    v4f acc[TC];
#pragma unroll
    for (int ct = 0; ct < TC; ct++) acc[ct] = v4f{};
#pragma unroll
    for (int i = 0; i < D - 1; i++)
        if ((uint32_t)i < nsb) issue(i);
    for (uint32_t i = 0; i < nsb; i++) {
        wait_younger<L::kD, D - 2>(min((uint32_t)(D - 2), nsb - 1 - i));
        // slot (i - 1) % D was read by this wavefront's last compute, whose
        // LDS reads have all been consumed; the asm barrier of the DMA keeps
        // them ahead of it
        if (i + D - 1 < nsb) issue(i + D - 1);
        compute16<DT, L, TC>(lds + (lbase - (uint32_t)(uintptr_t)lds) + (i % D) * L::kSlot, 0, lane,
                             ((wave + i * NW) & 1) != 0, acc);
    }

    // the wavefronts' sums, added in wavefront order
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);
    if (wave > 0) {
#pragma unroll
        for (int ct = 0; ct < TC; ct++)
            *reinterpret_cast<v4f*>(red + (((wave - 1) * TC + ct) * 64 + lane) * 4) = acc[ct];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (uint32_t v = 1; v < (uint32_t)NW; v++)
#pragma unroll
        for (int ct = 0; ct < TC; ct++)
            acc[ct] += *reinterpret_cast<const v4f*>(red + (((v - 1) * TC + ct) * 64 + lane) * 4);
    const uint32_t g = lane >> 4;
#pragma unroll
    for (int ct = 0; ct < TC; ct++) {
        const uint32_t col = col0 + ct * 16 + (lane & 15);
        if (col < w.n) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t row = 4 * g + e;
                if (row < m) y[(size_t)row * w.n + col] = acc[ct][e];
            }
        }
    }
}

template <int DT, int NW, int D, int TC>
hipError_t launch_skinny_wk(const WGroup& G, const AView& a, size_t m, float* partial, bool silu, hipStream_t s,
                            const ALayout* next, void* next_img) {
    using L = WkLay<DT, TC>;
    constexpr uint32_t kLds = (uint32_t)(NW * D * L::kSlot);
    static_assert(kLds <= 160 * 1024, "LDS budget");
    static_assert(NW * D * L::kSlot >= (NW - 1) * TC * 64 * 16, "reduction area");
    {
        const hipError_t e = set_max_lds(reinterpret_cast<const void*>(skinny_wk_kernel<DT, NW, D, TC>), kLds);
        if (e != hipSuccess) return e;
    }
    SkOut O{};
    SumGroup S{};
    uint32_t tiles = 0;
    size_t off = 0;
    for (uint32_t t = 0; t < G.count; t++) {
        const size_t cnt = m * (size_t)G.w[t].n;
        tiles += (G.w[t].n + L::kCols - 1) / L::kCols;
        O.tile_end[t] = tiles;
        O.y[t] = silu ? partial + off : G.y[t];
        S.part[t] = partial + off;
        S.y[t] = G.y[t];
        S.cnt[t] = cnt;
        off += cnt;
    }
    S.count = G.count;
    hipLaunchKernelGGL((skinny_wk_kernel<DT, NW, D, TC>), dim3(tiles), dim3(64 * NW), kLds, s, G, O, a, (uint32_t)m);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !silu) return e;
    if (next) return launch_sum_silu_quant(S, 1, m, G.w[0].n, *next, next_img, s);
    return launch_sum_group(S, 1, true, s);
}

// One 16-column tile per wavefront (twice the workgroups, a 7-8 KB slot)
// where the 32-column form leaves CUs idle or, for Q6_K, fits only one
// workgroup per CU (graph steps at m = 16, µs, two tiles -> one): Q4_K 4096 x
// 4096 (128 column tiles of 32) 11.2 -> 9.7; Q6_K 1792 -> 4096 10.2 -> 8.3,
// 4096 x 4096 14.2 -> 10.6, 4096 -> 14336 24.9 -> 23.1; the Q4_K q/k/v group
// (192 tiles) 11.7 -> 13.0 and 4096 -> 14336 16.8 -> 19.9 keep two.
static bool wk_one_tile(uint32_t dtype, size_t tiles32) { return dtype == XNQ_Q6K || tiles32 <= 128; }
// Eight wavefronts (half the serial chain each, one workgroup per CU) for
// the one-tile form up to 8 rows when its workgroups fit on the CUs one each
// (graph steps, µs, four -> eight): 14336 -> 4096 Q4_K at m = 5 17.9 -> 14.4,
// m = 8 17.2 -> 15.4; Q6_K 20.6 -> 19.7, 20.1 -> 18.6; 4096 x 4096 Q4_K at
// m = 5 9.4 -> 8.4, Q6_K 10.2 -> 9.8; 4096 -> 1792 8.5 -> 7.6.  More
// workgroups than CUs lose (Q6_K 2048 -> 8192 9.9 -> 11.8, 4096 -> 14336
// 20.5 -> 24.7), and so do more rows (m = 16: 18.0 -> 18.6, 20.1 -> 21.6).
static bool wk_eight_waves(size_t tiles32, size_t m) { return m <= 8 && 2 * tiles32 <= 256; }

// The wavefront-split kernel where it measured faster than the split-K one
// plus its sum launch (graph steps at m = 16, µs): at most 512 column tiles
// of 32, and K <= 4096 unless the one-tile form's workgroups fit one round
// at two per CU.  Q4_K 4096 x 4096 13.4 -> 9.7, the q/k/v group 15.0 ->
// 11.7, 4096 -> 14336 18.3 -> 16.8, 14336 -> 4096 18.9 -> 18.2; Q6_K 1792 ->
// 4096 14.8 -> 8.3, 14336 -> 4096 25.3 -> 21.0.  With two tiles per
// wavefront, K = 14336 was slower (Q4_K 14336 -> 4096 19.4 -> 22.3: half the
// CUs, 14 super-blocks per wavefront), and so are more tiles, which take
// extra rounds (the gate/up pair 25.5 -> 29.9, 8192 -> 28672 40.1 -> 44.2,
// the Q6_K lm_head 125 -> 164).
static bool skinny_wk(uint32_t dtype, size_t tiles32, size_t k) {
    if (tiles32 > 512) return false;
    // the one-tile form at any K while its workgroups fit one round at two
    // per CU (Q6_K 14336 -> 4096, 128 tiles: 25.3 -> 21.0 µs; Q4_K
    // 14336 -> 4096 18.9 -> 18.2), else K <= 4096
    if (wk_one_tile(dtype, tiles32) && 2 * tiles32 <= 512) return true;
    return k <= 4096;
}

template <int DT, int MT, int NW>
hipError_t launch_skinny_dt(const WGroup& G, const AView& a, size_t m, uint32_t splits, float* partial, bool silu,
                            hipStream_t s, const ALayout* next, void* next_img) {
    using L = KLay<DT, MT, NW>;
    constexpr int kCols = L::kCols;
    {
        const hipError_t e = set_max_lds(reinterpret_cast<const void*>(skinny_kernel<DT, MT, NW>), L::kLds);
        if (e != hipSuccess) return e;
    }
    const uint32_t nsb = G.w[0].k / 256;
    const uint32_t per = (nsb + splits - 1) / splits;
    splits = (nsb + per - 1) / per;  // every split non-empty
    // partial regions, weight after weight: [split][m][n_t]
    const bool reduce = splits > 1 || silu;
    SkOut O{};
    SumGroup S{};
    uint32_t tiles = 0;
    size_t off = 0;
    for (uint32_t t = 0; t < G.count; t++) {
        const size_t cnt = m * (size_t)G.w[t].n;
        tiles += (G.w[t].n + kCols - 1) / kCols;
        O.tile_end[t] = tiles;
        O.y[t] = reduce ? partial + off : G.y[t];
        O.stride[t] = reduce ? cnt : 0;
        S.part[t] = partial + off;
        S.y[t] = G.y[t];
        S.cnt[t] = cnt;
        off += splits * cnt;
    }
    S.count = G.count;
    const dim3 grid(tiles, splits);
    hipLaunchKernelGGL((skinny_kernel<DT, MT, NW>), grid, dim3(L::kThreads), L::kLds, s, G, O, a, (uint32_t)m, per);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !reduce) return e;
    if (silu && next) return launch_sum_silu_quant(S, splits, m, G.w[0].n, *next, next_img, s);
    return launch_sum_group(S, splits, silu, s);
}

}  // namespace

// Wavefronts per workgroup (32 columns each): 4 for the 16-row tiles (m <=
// 16), whose 47 KB workgroups fit three to a CU (8192 -> 28672 at m = 16
// 40.2 against 45.6 us with 8 at the same split count, 37.9 with twice the
// splits); above, 8 (two per SIMD, so one wavefront's expansion overlaps the
// other's waits) above 32 rows (two row tiles: 4096 x 4096 at m = 64 13.8
// against 16.2 us) or where the column tiles still cover the CUs with K
// split at most 4 ways, else 4.
static int skinny_waves(size_t m, size_t n, size_t k) {
    if (m <= 16) return 4;
    if (m > 32) return 8;
    const size_t tiles8 = (n + 255) / 256, nsb = k / 256;
    return tiles8 * std::min<size_t>(4, nsb / 2) >= 200 ? 8 : 4;
}

uint32_t skinny_splits(size_t m, size_t n, size_t k) {
    // split K while the grid has about one workgroup per CU (16-row tiles:
    // two, which fit three to a CU), each split at least two super-blocks
    // long.  The 16-row split-K launches that remain (those the
    // wavefront-split kernel does not take: many column tiles) gained from
    // the second workgroup per CU (8192 -> 28672 at m = 16 40.2 -> 37.9 us,
    // the Q6_K lm_head 116 -> 111); the 32-row tiles keep one.
    const size_t tiles = (n + 32 * skinny_waves(m, n, k) - 1) / (32 * skinny_waves(m, n, k));
    const size_t nsb = k / 256;
    const size_t target = m <= 16 ? 512 : 256;
    size_t splits = target / tiles;
    if (splits > nsb / 2) splits = nsb / 2;
    return splits < 1 ? 1u : (uint32_t)splits;
}

bool skinny_supported(uint32_t dtype, size_t m, size_t n, size_t k) {
    (void)n;
    return (dtype == XNQ_Q4K || dtype == XNQ_Q6K) && k % 256 == 0 && m >= 1 && m <= 64;
}

hipError_t launch_skinny_group(const WGroup& G, const AView& a, size_t m, uint32_t splits, float* partial, bool silu,
                               hipStream_t s, const ALayout* next, void* next_img) {
    if (m == 0 || G.count == 0) return hipSuccess;
    if (m > 64 || G.count > (uint32_t)kMaxGroup || (silu && G.count != 2)) return hipErrorInvalidValue;
    if (silu && !partial) return hipErrorInvalidValue;
    if (splits > 1 && !partial) splits = 1;
    size_t n = 0, tiles32 = 0;
    for (uint32_t t = 0; t < G.count; t++) {
        n += G.w[t].n;
        tiles32 += (G.w[t].n + 31) / 32;
    }
    const bool w8 = skinny_waves(m, n, G.w[0].k) == 8;
#define XNQ_SK(DT)                                                                                   \
    if (G.w[0].dtype == DT) {                                                                        \
        if (m <= 16 && skinny_wk(DT, tiles32, G.w[0].k) && (!silu || partial))                     \
            return wk_one_tile(DT, tiles32)                                                          \
                       ? (wk_eight_waves(tiles32, m)                                                  \
                              ? launch_skinny_wk<DT, 8, 2, 1>(G, a, m, partial, silu, s, next, next_img) \
                              : launch_skinny_wk<DT, 4, 2, 1>(G, a, m, partial, silu, s, next, next_img)) \
                       : launch_skinny_wk<DT, 4, 2, 2>(G, a, m, partial, silu, s, next, next_img);     \
        /* 16-row tiles on the 16x16x64 op (four wavefronts) up to 16 rows */                      \
        if (m <= 16) return launch_skinny_dt<DT, 0, 4>(G, a, m, splits, partial, silu, s, next, next_img); \
        if (m <= 32)                                                                                 \
            return w8 ? launch_skinny_dt<DT, 1, 8>(G, a, m, splits, partial, silu, s, next, next_img)               \
                      : launch_skinny_dt<DT, 1, 4>(G, a, m, splits, partial, silu, s, next, next_img);              \
        return launch_skinny_dt<DT, 2, 8>(G, a, m, splits, partial, silu, s, next, next_img);                       \
    }
    XNQ_SK(XNQ_Q4K)
    XNQ_SK(XNQ_Q6K)
#undef XNQ_SK
    return hipErrorNotSupported;
}

hipError_t launch_skinny(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                         hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    WGroup G{};
    G.w[0] = w;
    G.y[0] = y;
    G.row_end[0] = w.n;
    G.count = 1;
    G.rows = w.n;
    return launch_skinny_group(G, a, m, splits, partial, false, s);
}

}  // namespace xnq
