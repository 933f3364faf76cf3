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
#include <type_traits>

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

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));

// LDS map (bytes).  Per stage: activation tile, raw weight chunks (Q6K: and
// their high bits).  Per super-block (two buffers, by parity): d_a; Q4K: the
// bsum pairs, turned in place into the min-term operand; the 16-byte block
// header (Q4K: d, dmin, scales; Q6K: the int8 scales); Q4K: the weight-side
// min-term operand, Q6K: the d dword.
template <int DT>
struct Lay {
    static constexpr bool kQ4K = DT == XNQ_Q4K;
    static constexpr int kASlot = 2 * 2 * kBM * 16;  // activations [ks][h][row][16]       16 KiB
    static constexpr int kQSlot = 2 * kBN * 16;      // weight chunks [bc][n][16]           4 KiB
    static constexpr int kHSlot = kQ4K ? 0 : 2 * kBN * 16;  // Q6K qh of the stage [bc][n][16]
    static constexpr int kRawSlot = kQSlot + kHSlot;
    static constexpr int kPlanes = 2 * 2 * 2 * kBN * 16;  // digit planes [ks][plane][h][n][16]
    static constexpr int kEDa = 0;                          // f32 [kBM]
    static constexpr int kESum = kEDa + kBM * 4;            // Q4K [kBM][2][16]
    static constexpr int kEHdr = kESum + (kQ4K ? kBM * 32 : 0);  // [kBN][16]
    static constexpr int kEB = kEHdr + kBN * 16;            // Q4K [kBN][2][16]; Q6K d dword [kBN]
    static constexpr int kEpi = kEB + (kQ4K ? kBN * 32 : kBN * 4);
    static constexpr int kOffA = 0;
    static constexpr int kOffRaw = kOffA + kRing * kASlot;
    static constexpr int kOffPlanes = kOffRaw + kRing * kRawSlot;
    static constexpr int kOffEpi = kOffPlanes + 2 * kPlanes;
    static constexpr int kLds = kOffEpi + 2 * kEpi;
    static_assert(kLds <= 160 * 1024, "LDS budget");
    // DMA instructions one wavefront issues per stage, and the extra ones at
    // a super-block's first stage (d_a, bsums or scales, header or d)
    static constexpr int kBase = kQ4K ? 3 : 4;
    static constexpr int kExtra = 3;
};

// global_load_lds: uniform 64-bit base + 32-bit per-lane byte offset; m0
// holds the LDS address lane 0 writes (lane i writes i * size beyond it).
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds_addr)),
                 "v"(off), "s"(base)
                 : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds_addr)),
                 "v"(off), "s"(base)
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

// v = hi + lo with hi = bf16(v), lo = bf16(v - hi): ~16 significant bits
__device__ __forceinline__ void bf16_split(float v, __bf16& h, __bf16& l) {
    h = (__bf16)v;
    l = (__bf16)(v - (float)h);
}

template <int N>
using ic = std::integral_constant<int, N>;

template <int DT>
__global__ __launch_bounds__(kThreads) void qmm_kernel(WView w, AView a, uint32_t m, float* __restrict__ y) {
    using L = Lay<DT>;
    constexpr bool kQ4K = L::kQ4K;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave >> 1, wn = wave & 1;  // 4 x 2 wavefronts, 64 x 64 each
    const uint32_t m0 = blockIdx.y * kBM, n0 = blockIdx.x * kBN;
    const uint32_t K = w.k, nsb = K / 256, nstage = 4 * nsb;
    const ActImg& A = a.A;
    const uint32_t lbase = (uint32_t)(uintptr_t)lds;  // low half of the flat address = LDS offset
    const uint32_t lrow = lane & 31, lgrp = lane >> 5;

    // ---- this wavefront's DMA streams (byte offsets of stage / super-block 0) ----
    // activation pieces t = 2*wave + {0,1}: (ks, h, 64-row block)
    uint32_t a_off[2], a_lds[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t t = 2 * wave + i, ks = t >> 3, h = (t >> 2) & 1, rb = t & 3;
        const uint32_t row = min(m0 + rb * 64 + lane, m - 1);
        a_off[i] = row * A.row_bytes + h * (K / 2) + ks * 16;
        a_lds[i] = ((ks * 2 + h) * kBM + rb * 64) * 16;
    }
    // weights: chunk bc = wave & 1 of each stage, columns cb*32 .. +31
    // (cb = wave >> 1); lanes 32-63 mirror lanes 0-31 and issue no DMA
    const uint32_t bc = wave & 1, cb = wave >> 1;
    const uint32_t bn = cb * 32 + lrow;
    const uint32_t ncol = min(n0 + bn, w.n - 1);  // clamped: edge tiles read a valid row
    const bool lo_half = lane < 32;
    const uint32_t q_off = ncol * w.q_row + bc * 16;
    const uint32_t da_off = min(m0 + 32 * wave + lrow, m - 1) * A.row_bytes + A.d_off;
    const uint32_t sum_off = min(m0 + 32 * wave + (lane >> 1), m - 1) * A.row_bytes + A.s_off + (lane & 1) * 16;

    auto count = [&](uint32_t st) -> int {
        if (st >= nstage) return 0;
        return L::kBase + ((st & 3) == 0 ? L::kExtra : 0);
    };
    auto epi_base = [&](uint32_t sb) -> uint8_t* { return lds + L::kOffEpi + (sb & 1) * L::kEpi; };
    auto issue = [&](uint32_t st) {
        if (st >= nstage) return;
        const uint32_t slot = st % kRing, sb = st >> 2;
        const uint32_t abase = lbase + L::kOffA + slot * L::kASlot;
#pragma unroll
        for (int i = 0; i < 2; i++) dma16(a.img, a_off[i] + st * 32, abase + a_lds[i]);
        const uint32_t raw = lbase + L::kOffRaw + slot * L::kRawSlot + (bc * kBN + cb * 32) * 16;
        if (lo_half) {
            dma16(w.q, q_off + st * 32, raw);
            if (!kQ4K) dma16(w.h, ((q_off - bc * 16) >> 1) + st * 16, raw + L::kQSlot);  // qh of chunks 2st, 2st+1
        }
        if ((st & 3) == 0) {
            const uint32_t epi = lbase + L::kOffEpi + (sb & 1) * L::kEpi;
            if (lo_half) {
                dma4(a.img, da_off + sb * 4, epi + L::kEDa + 32 * wave * 4);
                dma16(w.s, ncol * w.s_row + sb * 16, epi + L::kEHdr + cb * 32 * 16);
                if (!kQ4K) dma4(w.d, ncol * w.d_row + (sb & ~1u) * 2, epi + L::kEB + cb * 32 * 4);
            }
            if (kQ4K) dma16(a.img, sum_off + sb * 32, epi + L::kESum + 32 * wave * 32);
        }
    };

    // ---- this wavefront's weight chunks of stage st -> digit planes (st & 1);
    //      at a super-block's first stage also the min-term operands of its rows/columns ----
    auto expand = [&](uint32_t st) {
        const uint8_t* raw = lds + L::kOffRaw + (st % kRing) * L::kRawSlot;
        uint8_t* epi = epi_base(st >> 2);
        const uint4 rq = *reinterpret_cast<const uint4*>(raw + (bc * kBN + bn) * 16);
        const uint4 hd = *reinterpret_cast<const uint4*>(epi + L::kEHdr + bn * 16);
        uint32_t p0[4], p1[4];  // high digit, low digit; 16 elements each
        if (kQ4K) {
            int sc, mn;
            q4k_scale_min(hd.y, hd.z, hd.w, (int)((2 * st + bc) & 7), sc, mn);
            const uint32_t sh = (uint32_t)sc >> 3, sl = (uint32_t)sc & 7;
            const uint32_t q4[4] = {rq.x, rq.y, rq.z, rq.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t nib = lgrp ? ((q4[j] >> 4) & 0x0F0F0F0Fu) : (q4[j] & 0x0F0F0F0Fu);
                p0[j] = mul_bytes(nib, sh);
                p1[j] = mul_bytes(nib, sl);
            }
            if ((st & 3) == 0) {
                // rows: -d_a * bsum32 of 4 sub-blocks, split to bf16 hi|lo, in place
                int4* sp = reinterpret_cast<int4*>(epi + L::kESum + 32 * wave * 32) + lane;
                const int4 pr = *sp;
                const float da = reinterpret_cast<const float*>(epi + L::kEDa)[32 * wave + (lane >> 1)];
                const int32_t prs[4] = {pr.x, pr.y, pr.z, pr.w};
                v4bf h4, l4;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int bs = (int)(int16_t)(prs[t] & 0xffff) + (int)(int16_t)(prs[t] >> 16);
                    __bf16 hh, ll;
                    bf16_split(-da * (float)bs, hh, ll);
                    h4[t] = hh;
                    l4[t] = ll;
                }
                uint4 o;
                o.x = __builtin_bit_cast(uint2, h4).x;
                o.y = __builtin_bit_cast(uint2, h4).y;
                o.z = __builtin_bit_cast(uint2, l4).x;
                o.w = __builtin_bit_cast(uint2, l4).y;
                *reinterpret_cast<uint4*>(sp) = o;
                if (lo_half) {
                    // columns: dmin * m_j of sub-blocks 4*bc .. 4*bc+3, bf16 hi|lo
                    const float dm = f16_bits_to_f32(hd.x >> 16);
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        int sc2, mn2;
                        q4k_scale_min(hd.y, hd.z, hd.w, (int)(4 * bc + t), sc2, mn2);
                        __bf16 hh, ll;
                        bf16_split(dm * (float)mn2, hh, ll);
                        h4[t] = hh;
                        l4[t] = ll;
                    }
                    o.x = __builtin_bit_cast(uint2, h4).x;
                    o.y = __builtin_bit_cast(uint2, h4).y;
                    o.z = __builtin_bit_cast(uint2, l4).x;
                    o.w = __builtin_bit_cast(uint2, l4).y;
                    *reinterpret_cast<uint4*>(epi + L::kEB + (bn * 2 + bc) * 16) = o;
                }
            }
        } else {
            const uint2 qh = *reinterpret_cast<const uint2*>(raw + L::kQSlot + (bc * kBN + bn) * 16 + bc * 8);
            int b[8];
            q6k_unpack(rq, qh, b);
            const uint32_t q = st & 3;  // scales of chunks 2st, 2st+1
            const uint32_t sw = q == 0 ? hd.x : (q == 1 ? hd.y : (q == 2 ? hd.z : hd.w));
            const int sc = (int)(int8_t)(sw >> (8 * (2 * bc + lgrp)));
#pragma unroll
            for (int j = 0; j < 4; j++) q6_digits((uint32_t)b[4 * lgrp + j], sc, p1[j], p0[j]);
        }
        uint8_t* pl = lds + L::kOffPlanes + (st & 1) * L::kPlanes;
        *reinterpret_cast<uint4*>(pl + (((bc * 2 + 0) * 2 + lgrp) * kBN + bn) * 16) = make_uint4(p0[0], p0[1], p0[2], p0[3]);
        *reinterpret_cast<uint4*>(pl + (((bc * 2 + 1) * 2 + lgrp) * kBN + bn) * 16) = make_uint4(p1[0], p1[1], p1[2], p1[3]);
    };

    v16f accf[kTM][kTN];
    v16i hi[kTM][kTN], lo[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; i++)
#pragma unroll
        for (int j = 0; j < kTN; j++) accf[i][j] = v16f{};

    // ---- super-block epilogue of tile (i, j): y += d_a d_w (hi * 2^s + lo) [- d_a dmin I2] ----
    constexpr int kShift = kQ4K ? 3 : 7;
    auto tile_dw = [&](uint32_t sb, int j) -> float {
        const uint8_t* epi = epi_base(sb);
        const uint32_t nl = wn * 64 + j * 32 + lrow;
        if (kQ4K) return f16_bits_to_f32(*reinterpret_cast<const uint32_t*>(epi + L::kEHdr + nl * 16) & 0xffffu);
        // d rows are padded to 4 bytes, so the dword holds super-blocks 2*(sb/2), +1
        const uint32_t dd = reinterpret_cast<const uint32_t*>(epi + L::kEB)[nl];
        return f16_bits_to_f32((sb & 1) ? (dd >> 16) : (dd & 0xffffu));
    };
    auto epilogue_tile = [&](uint32_t sb, int i, int j, float dw, const float* da) {
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int iv = hi[i][j][e] * (1 << kShift) + lo[i][j][e];
            accf[i][j][e] = fmaf((float)iv, dw * da[e], accf[i][j][e]);
        }
        if (kQ4K) {
            const uint8_t* epi = epi_base(sb);
            const uint4 av = reinterpret_cast<const uint4*>(epi + L::kESum)[(wm * 64 + i * 32 + lrow) * 2 + lgrp];
            const uint4 bv = reinterpret_cast<const uint4*>(epi + L::kEB)[(wn * 64 + j * 32 + lrow) * 2 + lgrp];
            const v8bf a8 = __builtin_bit_cast(v8bf, av);
            const v8bf bh8 = __builtin_bit_cast(v8bf, make_uint4(bv.x, bv.y, bv.x, bv.y));
            const v8bf bl8 = __builtin_bit_cast(v8bf, make_uint4(bv.z, bv.w, bv.z, bv.w));
            accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bh8, accf[i][j], 0, 0, 0);
            accf[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bl8, accf[i][j], 0, 0, 0);
        }
    };
    auto load_da = [&](uint32_t sb, int i, float* da) {
        const float* ep = reinterpret_cast<const float*>(epi_base(sb) + L::kEDa);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 d4 = *reinterpret_cast<const float4*>(ep + wm * 64 + i * 32 + q * 8 + lgrp * 4);
            da[4 * q + 0] = d4.x;
            da[4 * q + 1] = d4.y;
            da[4 * q + 2] = d4.z;
            da[4 * q + 3] = d4.w;
        }
    };

    auto epilogue = [&](uint32_t sb) {
#pragma unroll
        for (int j = 0; j < kTN; j++) {
            const float dw = tile_dw(sb, j);
#pragma unroll
            for (int i = 0; i < kTM; i++) {
                float da[16];
                load_da(sb, i, da);
                epilogue_tile(sb, i, j, dw, da);
            }
        }
    };

    // ---- one stage: 2 chunks x 2 x 2 tiles x 2 digit planes of int8 MFMA.  At a
    //      super-block's first stage the sums start from zero; its last stage
    //      ends with the super-block's epilogue ----
    auto stage = [&](uint32_t sb, auto tc) {
        constexpr int t = decltype(tc)::value;
        const uint32_t s = 4 * sb + t;
        issue(s + 3);
        const uint8_t* abase = lds + L::kOffA + (s % kRing) * L::kASlot;
        const uint8_t* pbase = lds + L::kOffPlanes + (s & 1) * L::kPlanes;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            auto a_frag = [&](int i) {
                return *reinterpret_cast<const v4i*>(abase + ((ks * 2 + lgrp) * kBM + wm * 64 + i * 32 + lrow) * 16);
            };
            auto b_frag = [&](int p, int j) {
                return *reinterpret_cast<const v4i*>(
                    pbase + (((ks * 2 + p) * 2 + lgrp) * kBN + wn * 64 + j * 32 + lrow) * 16);
            };
            v4i av[kTM];
#pragma unroll
            for (int i = 0; i < kTM; i++) av[i] = a_frag(i);
            if (t == 0 && ks == 0) {
                // a super-block's first chunk: the sums start from zero
#pragma unroll
                for (int j = 0; j < kTN; j++) {
                    const v4i b0 = b_frag(0, j), b1 = b_frag(1, j);
#pragma unroll
                    for (int i = 0; i < kTM; i++) {
                        hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], b0, v16i{}, 0, 0, 0);
                        lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], b1, v16i{}, 0, 0, 0);
                    }
                }
            } else {
                v4i bv[2][kTN];
#pragma unroll
                for (int p = 0; p < 2; p++)
#pragma unroll
                    for (int j = 0; j < kTN; j++) bv[p][j] = b_frag(p, j);
#pragma unroll
                for (int i = 0; i < kTM; i++)
#pragma unroll
                    for (int j = 0; j < kTN; j++) {
                        hi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[0][j], hi[i][j], 0, 0, 0);
                        lo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[1][j], lo[i][j], 0, 0, 0);
                    }
            }
            // the next stage's digit planes, while this chunk's MFMAs run
            if (ks == 0 && s + 1 < nstage) {
                wait_vmcnt(count(s + 2) + count(s + 3));
                expand(s + 1);
            }
        }
        if (t == 3) epilogue(sb);
        __syncthreads();
    };

    // prologue: stages 0-2 in flight, stage 0 expanded and published
    issue(0);
    issue(1);
    issue(2);
    wait_vmcnt(count(1) + count(2));
    expand(0);
    __syncthreads();

    for (uint32_t sb = 0; sb < nsb; sb++) {
        stage(sb, ic<0>{});
        stage(sb, ic<1>{});
        stage(sb, ic<2>{});
        stage(sb, ic<3>{});
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
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, Lay<DT>::kLds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const dim3 grid((w.n + kBN - 1) / kBN, (unsigned)((m + kBM - 1) / kBM));
    hipLaunchKernelGGL(qmm_kernel<DT>, grid, dim3(kThreads), Lay<DT>::kLds, s, w, a, (uint32_t)m, y);
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
