// Prefill-path Q4K quantized matmul (m > 64) on the CDNA4 int8 matrix cores.
//
// Per super-block (256 K) the reference's integer block dot is
//   I1 = sum_j sc_j * sum_{k in j} q4*q8,   I2 = sum_j m_j * bsum32_j
// and y += d_a * (d_w * I1 - dmin * I2)  (k_quants.rs:1324-1416).
//
// Main term.  The 6-bit sub-block scale is folded into the weight before the
// contraction so the MFMA sums a whole super-block in int32: sc = 8*sh + sl
// (sh, sl in 0..7) and w = 8*(sh*q) + (sl*q), two int8 digit planes (each
// digit <= 105) contracted separately; the epilogue applies d_a * d_w once
// per super-block to 8 * hi + lo.
// Min term.  A rank-8 product per super-block with f32 operands -d_a*bsum32
// (precomputed by the activation quantizer, bf16 high + remainder) and
// dmin*m_j (built per super-block from the block header, same split), on the
// bf16 matrix cores into the f32 output (two K = 16 products).
//
// Tiling: a workgroup of 8 wavefronts (two per SIMD) owns 32*TM activation
// rows (TM = 2 or 4 row tiles) by 256 weight columns; wavefront w owns
// columns 32w..32w+31 and all TM row tiles of v_mfma_i32_32x32x32_i8 (hi and
// lo int32 sums plus the f32 output: 192 accumulator registers at TM = 4).
// Each wavefront expands only its own columns' weights, in registers, right
// before the MFMAs that use them, so no digit plane goes through LDS; the
// activation tile is shared through LDS.
//
// One MFMA K-step is 32 K: lane (column c, half g) contributes the low
// (ks = 0) or high (ks = 1) nibbles of chunk 2p + g of the stage's chunk pair
// p, i.e. elements 16ks..16ks+15 of sub-block 2p + g, times that sub-block's
// sh or sl; the activation lane (row, g) holds the same 16 elements.  The
// sub-block scale therefore varies by lane half, which is fine: the scale is
// already inside the digits.
//
// Data movement: every byte a stage needs is fetched with global_load_lds
// DMA straight into LDS, two time steps ahead: the activation tile into a
// shared 4-slot ring; per super-block the min-term operand rows and d_a
// (shared, 4 buffers); per wavefront its own weight chunks (2 KiB per stage,
// 3-slot ring) and block headers (one 1 KiB fetch per super-block, 3
// buffers).  One s_barrier per time step publishes the shared pieces; each
// wavefront waits only for its own DMA (s_waitcnt vmcnt with the exact count
// of younger DMA it issued).
//
// Lead and lag: wavefronts 4-7 (the second wavefront of every SIMD) run the
// same sequence of steps one time step behind wavefronts 0-3 over the same
// activation ring, so the two wavefronts of a SIMD reach their super-block
// epilogues (about 4 VALU instructions per output element) at different time
// steps and each one's epilogue VALU issues beside the other's MFMAs.
#include <cstdlib>
#include <type_traits>

#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

typedef int pf_v4i __attribute__((ext_vector_type(4)));
typedef int pf_v16i __attribute__((ext_vector_type(16)));
typedef float pf_v16f __attribute__((ext_vector_type(16)));
typedef __bf16 pf_v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short pf_v2u16 __attribute__((ext_vector_type(2)));

constexpr int kPBN = 256, kPWaves = 8, kPThreads = kPWaves * 64;

// Time line.  A stage is 128 K (two chunk pairs, four MFMA K-steps, 32 MFMAs
// per wavefront).  Per super-block every wavefront runs two steps:
//   A(sb): epilogue of sb - 1, setup of sb (its header's digit scales, d_w,
//          the min-term products), stage 2sb
//   B(sb): stage 2sb + 1
// so own step q runs stage q.  Wavefronts 0-3 ("lead") run own step q at
// time q, wavefronts 4-7 ("lag") at time q + 1: at every time step both
// wavefronts of a SIMD have a stage of MFMAs and one of them also the
// super-block's VALU work.  (A time line of three steps per super-block,
// with the epilogue in a step of its own, left one wavefront per SIMD
// without MFMAs in two steps of three: 2-5 % slower at 128-384 rows.)

// LDS map (bytes) for TM 32-row tiles per wavefront (BM = 32 TM rows)
template <int TM>
struct PLay {
    static constexpr int kHdrBufs = 3;  // header buffers (super-block % 3)
    static constexpr int kBM = 32 * TM;
    static constexpr int kASlots = 4, kASlot = TM / 2 * 8192;  // [rb][half stage][ks2][h2][row 64][16]
    static constexpr int kRawSlots = 3, kRawSlot = kPWaves * 2048;  // [wave][pair][lane][16]
    static constexpr int kOffA = 0;
    static constexpr int kOffRaw = kOffA + kASlots * kASlot;
    static constexpr int kOffHdr = kOffRaw + kRawSlots * kRawSlot;  // [sb % kHdrBufs][wave][lane][16]
    static constexpr int kOffX = kOffHdr + kHdrBufs * kPWaves * 1024;  // [sb & 3][row / 32][half][row % 32][16]
    static constexpr int kOffDa = kOffX + 4 * TM * 1024;             // [sb & 3][row] f32
    static constexpr int kOffDw = kOffDa + 4 * 512;  // [wave][column] f32 d_w of the current super-block
    static constexpr int kLds = kOffDw + kPWaves * 128;
    static_assert(kLds <= 160 * 1024, "LDS budget");
};

// (base and LDS address are wavefront-uniform; readfirstlane states it)
__device__ __forceinline__ const void* uni_ptr(const void* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void pdma16(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds_addr)),
                 "v"(off), "s"(uni_ptr(base))
                 : "memory");
}
__device__ __forceinline__ void pdma4(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds_addr)),
                 "v"(off), "s"(uni_ptr(base))
                 : "memory");
}
// wait until at most N of this wavefront's VMEM loads are outstanding, then
// meet the other wavefronts
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// bytes of d (each <= 15) times s2 (a digit <= 7 in both 16-bit halves):
// products <= 105 stay in their byte
__device__ __forceinline__ uint32_t mulb(uint32_t d, uint32_t s2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(pf_v2u16, d) * __builtin_bit_cast(pf_v2u16, s2));
}

template <int TM>
__global__ __launch_bounds__(kPThreads) void prefill_q4k_kernel(WView w, AView a, uint32_t m, uint32_t m_tiles,
                                                                uint32_t n_tiles, uint32_t splits,
                                                                uint32_t sb_per_split, float* __restrict__ y,
                                                                size_t split_stride) {
    using Lay = PLay<TM>;
    constexpr int kHdrBufs = Lay::kHdrBufs;
    constexpr int kPTM = TM, kPBM = Lay::kBM, kASlots = Lay::kASlots, kASlot = Lay::kASlot;
    constexpr int kRawSlots = Lay::kRawSlots, kRawSlot = Lay::kRawSlot;
    constexpr int kOffA = Lay::kOffA, kOffRaw = Lay::kOffRaw, kOffHdr = Lay::kOffHdr, kOffX = Lay::kOffX;
    constexpr int kOffDa = Lay::kOffDa, kOffDw = Lay::kOffDw;
    extern __shared__ __align__(16) uint8_t lds[];
    // XCD-aware order: workgroup b runs on XCD b % 8; the workgroups of one
    // XCD take consecutive work items, which share weight columns
    const uint32_t total = m_tiles * n_tiles * splits;
    const uint32_t per = (total + 7) / 8;
    const uint32_t wi = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (wi >= total) return;
    const uint32_t mt = wi % m_tiles, rest = wi / m_tiles;
    const uint32_t nt = rest % n_tiles, split = rest / n_tiles;

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lrow = lane & 31, g = lane >> 5;
    const uint32_t m0 = mt * kPBM, n0 = nt * kPBN;
    const uint32_t K = w.k, nsb_all = K / 256;
    const uint32_t sb0 = split * sb_per_split;
    const uint32_t nsb = min(sb_per_split, nsb_all - sb0);
    const uint32_t nstage = 2 * nsb;
    y += (size_t)split * split_stride;
    const uint32_t lbase = (uint32_t)(uintptr_t)lds;
    const TileImg& T = a.T;

    // ---- shared pieces (the lead's time line) ----
    auto rblk = [&](uint32_t rb) { return min(m0 / 64 + rb, T.rbs - 1); };
    // stage st (128 K = TileImg stages 2st, 2st+1): 4 TM pieces of 1 KiB,
    // pieces wave + 8h (h < TM / 2) from this wavefront
    auto issue_stage = [&](uint32_t st) {
        const uint32_t s = min(st, nstage - 1);  // past the end: re-read the last stage
#pragma unroll
        for (int h = 0; h < TM / 2; h++) {
            const uint32_t j = wave + 8 * h, rb = j >> 3, half = (j >> 2) & 1, pc = j & 3;
            pdma16(a.tile + (size_t)rblk(rb) * 64 * K + (size_t)(4 * sb0 + 2 * s + half) * 4096 + pc * 1024, lane * 16,
                   lbase + kOffA + (st % kASlots) * kASlot + rb * 8192 + half * 4096 + pc * 1024);
        }
    };
    auto issue_sb_shared = [&](uint32_t sb) {
        const uint32_t sbc = min(sb, nsb - 1);
        const size_t blk = (size_t)sb0 + sbc;
        if (wave < 4) {  // min-term operand of 32-row tile wave % TM (repeats are the same bytes)
            const uint32_t i = wave % TM, rb = i >> 1, r32 = i & 1;
            pdma16(a.tile + T.x_off + (((size_t)rblk(rb) * nsb_all + blk) * 2 + r32) * 1024, lane * 16,
                   lbase + kOffX + (sb & 3) * (TM * 1024) + i * 1024);
        } else {  // d_a of 64-row block wave % (TM / 2) (repeats are the same bytes)
            const uint32_t rb = wave % (TM / 2);
            pdma4(a.tile + T.d_off + ((size_t)rblk(rb) * nsb_all + blk) * 256, lane * 4,
                  lbase + kOffDa + (sb & 3) * 512 + rb * 256);
        }
    };
    // ---- own pieces (this wavefront's time line) ----
    const uint32_t ncol = min(n0 + 32 * wave + lrow, w.n - 1);
    const uint32_t raw_off = ncol * w.q_row + g * 16;
    const uint32_t hdr_off = (ncol >> 7) * w.nb * 2048 + (ncol & 127) * 16;
    // stage st's weight chunks: pair p = 2 (st & 1) + h of super-block st / 2,
    // lane (column c, half g) gets chunk 2p + g of column c
    auto issue_own = [&](uint32_t st) {
        const uint32_t sc = min(st, nstage - 1);
#pragma unroll
        for (int h = 0; h < 2; h++)
            pdma16(w.q + (size_t)(sb0 + sc / 2) * 128 + ((sc & 1) * 2 + h) * 32, raw_off,
                   lbase + kOffRaw + (st % kRawSlots) * kRawSlot + wave * 2048 + h * 1024);
    };
    auto issue_hdr = [&](uint32_t sb) {
        const uint32_t sbc = min(sb, nsb - 1);
        pdma16(w.st + (size_t)(sb0 + sbc) * 2048, hdr_off, lbase + kOffHdr + (sb % kHdrBufs) * 8192 + wave * 1024);
    };

    pf_v16f accf[kPTM];
    pf_v16i hi[kPTM], lo[kPTM];
#pragma unroll
    for (int i = 0; i < kPTM; i++) accf[i] = pf_v16f{};

    // byte selectors that splat byte (2 * parity + g) of a dword into both
    // 16-bit halves (v_perm_b32; 0x0c reads as zero)
    const uint32_t sel0 = 0x0c000c00u | (g * 0x00010001u);
    const uint32_t sel1 = 0x0c020c02u | (g * 0x00010001u);
    const uint32_t M4 = 0x0F0F0F0Fu;

    // Both groups run the same code over their own step index q (lead: time
    // q, lag: time q + 1); the group only decides, uniformly per wavefront,
    // which shared DMA a step issues and how many of its DMA may still be in
    // flight at the step's barrier.
    const uint32_t G = wave >> 2;
    // digit scales of the current super-block: bytes j (resp. j - 4) of
    // sh_lo / sl_lo (resp. sh_hi / sl_hi) are sub-block j's sc >> 3, sc & 7
    uint32_t sh_lo = 0, sh_hi = 0, sl_lo = 0, sl_hi = 0;

    // Setup of super-block sb from its headers: digit scales, d_w for the
    // epilogue, and the min-term products into the output.
    auto setup = [&](uint32_t sb) {
        const uint4 hd =
            *reinterpret_cast<const uint4*>(lds + kOffHdr + (sb % kHdrBufs) * 8192 + wave * 1024 + lane * 16);
        const Q4KScales qs = q4k_scales(hd.y, hd.z, hd.w);
        sh_lo = (qs.sc_lo >> 3) & 0x07070707u;
        sl_lo = qs.sc_lo & 0x07070707u;
        sh_hi = (qs.sc_hi >> 3) & 0x07070707u;
        sl_hi = qs.sc_hi & 0x07070707u;
        // both lane halves hold column lrow's header: the same value, no branch
        reinterpret_cast<float*>(lds + kOffDw + wave * 128)[lrow] = f16_bits_to_f32(hd.x & 0xffffu);
        // min term: column operand dmin * m_j for j = 4g .. 4g+3
        const float dm = f16_bits_to_f32(hd.x >> 16);
        const uint32_t mv = g ? qs.m_hi : qs.m_lo;
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; t++) v[t] = dm * (float)((mv >> (8 * t)) & 0xffu);
        const uint4 yb = bf16_hilo4(v);
        const pf_v8bf bh8 = __builtin_bit_cast(pf_v8bf, make_uint4(yb.x, yb.y, yb.x, yb.y));
        const pf_v8bf bl8 = __builtin_bit_cast(pf_v8bf, make_uint4(yb.z, yb.w, yb.z, yb.w));
        const uint8_t* xb = lds + kOffX + (sb & 3) * (TM * 1024) + lane * 16;
        pf_v8bf a8[kPTM];
#pragma unroll
        for (int i = 0; i < kPTM; i++) a8[i] = __builtin_bit_cast(pf_v8bf, *reinterpret_cast<const uint4*>(xb + i * 1024));
#pragma unroll
        for (int i = 0; i < kPTM; i++) accf[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bh8, a8[i], accf[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < kPTM; i++) accf[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bl8, a8[i], accf[i], 0, 0, 0);
    };

    // Epilogue of super-block sb: y += d_a d_w (8 hi + lo).  Tile i's
    // outputs: activation row 32i + lrow, weight columns 8q + 4g + e'
    // (q = e / 4, e' = e % 4) of this wavefront's 32.
    auto epilogue = [&](uint32_t sb) {
        const float* dap = reinterpret_cast<const float*>(lds + kOffDa + (sb & 3) * 512) + lrow;
        const float* dwp = reinterpret_cast<const float*>(lds + kOffDw + wave * 128) + 4 * g;
        float dv[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 w4 = *reinterpret_cast<const float4*>(dwp + 8 * q);
            dv[4 * q] = w4.x;
            dv[4 * q + 1] = w4.y;
            dv[4 * q + 2] = w4.z;
            dv[4 * q + 3] = w4.w;
        }
#pragma unroll
        for (int i = 0; i < kPTM; i++) {
            const float dai = dap[32 * i];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int iv = hi[i][e] * 8 + lo[i][e];
                accf[i][e] = fmaf((float)iv, dai * dv[e], accf[i][e]);
            }
        }
    };

    // Stage st = 2 sb + P2 (P2 compile-time): chunk pairs 2 P2 and 2 P2 + 1,
    // four K-steps of TM fragment pairs.  The activation fragment of the
    // (K-step, tile) kAhead positions later is read before each MFMA pair,
    // and the second raw chunk two K-steps before its use, so the MFMAs issue
    // back to back instead of each pair waiting on its own LDS read (the
    // scheduler, left alone, sinks every read next to its use).
    auto stage = [&](uint32_t st, auto pc) {
        constexpr int P2 = decltype(pc)::value;
        constexpr int kN = 4 * kPTM, kAhead = 4;
        const uint8_t* raw = lds + kOffRaw + (st % kRawSlots) * kRawSlot + wave * 2048 + lane * 16;
        const uint8_t* abase = lds + kOffA + (st % kASlots) * kASlot + g * 2048 + lrow * 16;
        const uint32_t shw = P2 == 0 ? sh_lo : sh_hi, slw = P2 == 0 ? sl_lo : sl_hi;
        auto frag = [&](int j) {  // fragment j = kk * TM + i
            const int kk = j / kPTM, i = j % kPTM, pp = kk >> 1, ks = kk & 1;
            return *reinterpret_cast<const pf_v4i*>(abase + (i >> 1) * 8192 + pp * 4096 + ks * 1024 + (i & 1) * 512);
        };
        pf_v4i av[kN];
#pragma unroll
        for (int j = 0; j < kAhead; j++) av[j] = frag(j);
        uint4 rq = *reinterpret_cast<const uint4*>(raw);
        const uint4 rqn = *reinterpret_cast<const uint4*>(raw + 1024);
        pf_v4i bh, bl;
#pragma unroll
        for (int j = 0; j < kN; j++) {
            const int kk = j / kPTM, i = j % kPTM;
            if (i == 0) {
                // this lane's chunk 2p + g (p = 2 P2 + pp) and its sub-block's digits
                const int pp = kk >> 1, ks = kk & 1;
                if (kk == 2) rq = rqn;
                const uint32_t sel = pp ? sel1 : sel0;
                const uint32_t sh2 = __builtin_amdgcn_perm(shw, shw, sel), sl2 = __builtin_amdgcn_perm(slw, slw, sel);
                uint32_t d[4];
                if (ks == 0) {
                    d[0] = rq.x & M4; d[1] = rq.y & M4; d[2] = rq.z & M4; d[3] = rq.w & M4;
                } else {
                    d[0] = (rq.x >> 4) & M4; d[1] = (rq.y >> 4) & M4; d[2] = (rq.z >> 4) & M4; d[3] = (rq.w >> 4) & M4;
                }
                bh = pf_v4i{(int)mulb(d[0], sh2), (int)mulb(d[1], sh2), (int)mulb(d[2], sh2), (int)mulb(d[3], sh2)};
                bl = pf_v4i{(int)mulb(d[0], sl2), (int)mulb(d[1], sl2), (int)mulb(d[2], sl2), (int)mulb(d[3], sl2)};
            }
            if (j + kAhead < kN) av[j + kAhead] = frag(j + kAhead);
            __builtin_amdgcn_sched_barrier(0);
            if (P2 == 0 && kk == 0) {
                hi[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bh, av[j], pf_v16i{}, 0, 0, 0);
                lo[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bl, av[j], pf_v16i{}, 0, 0, 0);
            } else {
                hi[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bh, av[j], hi[i], 0, 0, 0);
                lo[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bl, av[j], lo[i], 0, 0, 0);
            }
        }
    };

    {
        // DMA is issued two time steps ahead: at time t the activation pieces
        // of stage t + 2 and, at even t, the min-term / d_a pieces of
        // super-block t / 2 + 1; at own step q the wavefront's weight chunks
        // of stage q + 2 and, at even q, the headers of super-block q / 2 + 1.
        // KIND (compile-time, so each step's work is one basic block the
        // scheduler can interleave): 0 setup(0) + stage 0; 1 epilogue(sb - 1)
        // + setup(sb) + stage 2 sb; 2 the last epilogue; 3 stage q (odd);
        // 4 no work (the lag's time 0, the lead's last time step).
        auto step2 = [&](int q, auto kindc, auto wlc, auto wgc) {
            constexpr int KIND = decltype(kindc)::value;
            constexpr int PS = (KIND == 3 || KIND == 4) ? 1 : 0;
            if (G) wait_and_barrier<decltype(wgc)::value>();
            else wait_and_barrier<decltype(wlc)::value>();
            const uint32_t t = (uint32_t)(q + (int)G);
            issue_stage(t + 2);
            if ((t & 1u) == 0) issue_sb_shared(t / 2 + 1);
            issue_own((uint32_t)(q + 2));
            if (PS == 0) issue_hdr((uint32_t)(q / 2 + 1));
            const uint32_t sb = (uint32_t)q / 2;
            if constexpr (KIND == 0) {
                setup(0);
                stage(0, std::integral_constant<int, 0>{});
            } else if constexpr (KIND == 1) {
                epilogue(sb - 1);
                setup(sb);
                stage((uint32_t)q, std::integral_constant<int, 0>{});
            } else if constexpr (KIND == 2) {
                epilogue(sb - 1);
            } else if constexpr (KIND == 3) {
                stage((uint32_t)q, std::integral_constant<int, 1>{});
            }
        };
        issue_stage(0);
        issue_stage(1);
        issue_sb_shared(0);
        issue_own(0);
        issue_own(1);
        issue_hdr(0);
        wait_and_barrier<0>();
        using K0 = std::integral_constant<int, 0>;
        using K1 = std::integral_constant<int, 1>;
        using K2 = std::integral_constant<int, 2>;
        using K3 = std::integral_constant<int, 3>;
        using K4 = std::integral_constant<int, 4>;
        using WZ = std::integral_constant<int, 0>;
        // wait counts: the DMA this wavefront issued at the previous time step
        using WL0 = std::integral_constant<int, TM / 2 + 2>;  // lead, even step (previous: odd time)
        using WL1 = std::integral_constant<int, TM / 2 + 4>;  // lead, odd step
        using WG = std::integral_constant<int, TM / 2 + 3>;   // lag, every step
        if (G) step2(-1, K4{}, WZ{}, WZ{});  // the lag's time 0
        step2(0, K0{}, WZ{}, WG{});
        step2(1, K3{}, WL1{}, WG{});
        for (uint32_t sb = 1; sb < nsb; sb++) {
            step2((int)(2 * sb), K1{}, WL0{}, WG{});
            step2((int)(2 * sb + 1), K3{}, WL1{}, WG{});
        }
        step2((int)(2 * nsb), K2{}, WL0{}, WG{});  // the last epilogue
        if (!G) step2((int)(2 * nsb + 1), K4{}, WL1{}, WZ{});  // the lead's last time step
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // ---- write the tile: lane (lrow, g) of tile i holds row m0 + 32i + lrow,
    //      columns 8q + 4g .. 8q + 4g + 3 of the wavefront's 32 ----
    const uint32_t nb0 = n0 + 32 * wave + 4 * g;
#pragma unroll
    for (int i = 0; i < kPTM; i++) {
        const uint32_t row = m0 + 32 * i + lrow;
        if (row >= m) continue;
        float* yr = y + (size_t)row * w.n;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t n = nb0 + 8 * q;
            if (n + 3 < w.n && (w.n & 3) == 0) {
                *reinterpret_cast<float4*>(yr + n) =
                    make_float4(accf[i][4 * q], accf[i][4 * q + 1], accf[i][4 * q + 2], accf[i][4 * q + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (n + e < w.n) yr[n + e] = accf[i][4 * q + e];
            }
        }
    }
}

}  // namespace

// Row tiles of the workgroup: 2 (64 rows) up to m = 64 and where 128-row
// tiles would leave most CUs idle, else 4 (128 rows).
static int prefill_tm(size_t m, size_t n) {
    const size_t tiles128 = ((n + kPBN - 1) / kPBN) * ((m + 127) / 128);
    return (m <= 64 || tiles128 < 128) ? 2 : 4;
}

// Where this kernel replaces the tiled kernel of k_mfma.hip: Q4_K up to
// 512 rows.  K = 4096 -> N = 14336, HIP graph steps, µs, tiled kernel
// against this one, on one box: m = 128 50.6 / 33.6, 256 64.5 / 48.5, 384
// 72.0 / 70.9, 512 81.9 / 74.1, 1024 155.0 / 147.6; on others 512 ran
// 82.2 / 76.1 and 83.2 / 83.2, 768 136.2 / 138.8.  Past 512 the tiled
// kernel stays (XNQ_PREFILL_MAX_ROWS moves the limit, tuning).
constexpr size_t kPrefillMaxRows = 512;

static int env_int_pf(const char* name, int dflt) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

bool prefill_supported(uint32_t dtype, size_t m, size_t n, size_t k) {
    (void)n;
    static const size_t max_rows = (size_t)env_int_pf("XNQ_PREFILL_MAX_ROWS", (int)kPrefillMaxRows);
    return dtype == XNQ_Q4K && k % 256 == 0 && k >= 256 && m <= max_rows;
}

uint32_t prefill_splits(size_t m, size_t n, size_t k) {
    // split K while the grid stays within one workgroup per CU (256), each
    // split at least two super-blocks long
    const size_t bm = 32 * (size_t)prefill_tm(m, n);
    const size_t tiles = ((n + kPBN - 1) / kPBN) * ((m + bm - 1) / bm);
    const size_t nsb = k / 256;
    size_t splits = 256 / tiles;
    if (splits > nsb / 2) splits = nsb / 2;
    return splits < 1 ? 1u : (uint32_t)splits;
}

template <int TM>
static hipError_t launch_prefill_tm(const WView& w, const AView& a, size_t m, uint32_t splits, float* y,
                                    float* partial, hipStream_t s) {
    using Lay = PLay<TM>;
    {
        const hipError_t e = set_max_lds(reinterpret_cast<const void*>(prefill_q4k_kernel<TM>), Lay::kLds);
        if (e != hipSuccess) return e;
    }
    const uint32_t nsb = w.k / 256;
    const uint32_t per = (nsb + splits - 1) / splits;
    splits = (nsb + per - 1) / per;  // every split non-empty
    const uint32_t m_tiles = (uint32_t)((m + Lay::kBM - 1) / Lay::kBM), n_tiles = (w.n + kPBN - 1) / kPBN;
    const uint32_t total = m_tiles * n_tiles * splits;
    const uint32_t grid = (total + 7) / 8 * 8;
    float* out = splits > 1 ? partial : y;
    hipLaunchKernelGGL(prefill_q4k_kernel<TM>, dim3(grid), dim3(kPThreads), Lay::kLds, s, w, a, (uint32_t)m, m_tiles,
                       n_tiles, splits, per, out, splits > 1 ? m * (size_t)w.n : (size_t)0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_sum_splits(partial, m * (size_t)w.n, splits, y, s);
}

hipError_t launch_prefill(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                          hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (w.dtype != XNQ_Q4K) return hipErrorNotSupported;
    if (!a.tile || (size_t)a.T.rbs * 64 < m || a.k != w.k || w.k % 256) return hipErrorInvalidValue;
    if (splits > 1 && !partial) splits = 1;
    return prefill_tm(m, w.n) == 2 ? launch_prefill_tm<2>(w, a, m, splits, y, partial, s)
                                   : launch_prefill_tm<4>(w, a, m, splits, y, partial, s);
}

}  // namespace xnq
