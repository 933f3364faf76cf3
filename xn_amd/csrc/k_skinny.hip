// Small-batch quantized matmul (m = 2 .. 64) on the int8 matrix cores.
//
// At a few rows the product is bound by the weight stream, so this kernel
// keeps the weight path of a matvec (every weight byte read once, straight
// from HBM into registers, no LDS) and does the dot products on
// v_mfma_i32_32x32x32_i8: each wavefront owns 32 weight rows (output
// columns) and all m activation rows (one or two 32-row MFMA tiles).  Per
// super-block the wavefront expands its 32 columns' chunks into the two int8
// digit planes of the prefill kernel (Q4K: sc = 8*sh + sl, digits sh*q and
// sl*q; Q6K: sc*(q-32) = 128*hi + lo), contracts them against the activation
// tile in LDS, and applies d_a * d_w in an f32 epilogue; the Q4K min term is
// a K = 8 GEMM of -d_a*bsum32 by dmin*m_j on the bf16 matrix cores.  The
// integer sums per super-block are exact, as in the reference's block dots
// (k_quants.rs:1337-1416, 1743-1798).
//
// A workgroup (4 wavefronts, 128 columns) walks a range of super-blocks:
// the next super-block's weights and activation tile are loaded into
// registers while the current one is multiplied, and the activation tile is
// written to the second LDS buffer after it.  When the column tiles alone do
// not fill the GPU, the super-blocks are split across workgroups and the
// partial outputs are summed in split order afterwards.
#include <type_traits>

#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4, kThreads = kWaves * 64, kCols = 32 * kWaves;

// LDS image of one super-block of the activation rows (R = 32 * MT rows):
//   q    [chunk 8][half 2][row R][16 bytes]   (MFMA A-operand order)
//   min  Q4K: [row R][half 2][16 bytes] = bf16 hi4 | lo4 of -d_a * bsum32
//        of sub-blocks 4*half .. 4*half+3
//   d_a  [row R] f32
template <int DT, int MT>
struct SLay {
    static constexpr int R = 32 * MT;
    static constexpr int kQ = 256 * R;
    static constexpr int kMin = DT == XNQ_Q4K ? 32 * R : 0;
    static constexpr int kBuf = kQ + kMin + 4 * R;
    static constexpr int kLds = 2 * kBuf;
    static constexpr int kPieces = 16 * R / kThreads;  // 16-byte activation pieces per thread
};

// bytes of d (each <= 15) times s (<= 7): one packed 16-bit multiply
__device__ __forceinline__ uint32_t mul_bytes(uint32_t d, uint32_t s) {
    const v2u16 s2 = {(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2u16, d) * s2);
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

// 4 floats -> bf16 hi | bf16 lo (v = hi + lo to ~16 significant bits), packed as 16 bytes
__device__ __forceinline__ uint4 bf16_split4(const float* v) {
    v4bf h, l;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const __bf16 hb = (__bf16)v[t];
        h[t] = hb;
        l[t] = (__bf16)(v[t] - (float)hb);
    }
    const uint2 hu = __builtin_bit_cast(uint2, h), lu = __builtin_bit_cast(uint2, l);
    return make_uint4(hu.x, hu.y, lu.x, lu.y);
}

typedef unsigned int nt_u4 __attribute__((ext_vector_type(4)));

// weight stream: read once per call, non-temporal
__device__ __forceinline__ uint4 ldw(const uint4* p) {
    const nt_u4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// One super-block of this lane's weight column, in registers.  Lanes 0-31
// load chunks 0-3 (Q6K: high-bit words 0-1) of their column and lanes 32-63
// chunks 4-7 (words 2-3) of the same column, so each load instruction
// touches 32 rows once instead of twice; one v_permlane32_swap per dword
// then gives every lane all of them.
template <int DT>
struct WeightSB {
    uint4 q[4];   // raw: this half's four chunks
    uint4 s;      // Q4K: d | dmin, scales[12]; Q6K: int8 scales[16]
    uint4 h[2];   // Q6K: this half's high-bit words
    uint32_t d;   // Q6K: f16 d
};

template <int DT>
__device__ __forceinline__ void load_weight_sb(const WView& w, uint32_t col, uint32_t sb, WeightSB<DT>& x) {
    const uint32_t hsel = (threadIdx.x & 63) >> 5;
    const uint4* q = reinterpret_cast<const uint4*>(w.q + col * w.q_row + sb * 128) + 4 * hsel;
#pragma unroll
    for (int c = 0; c < 4; c++) x.q[c] = ldw(&q[c]);
    x.s = *reinterpret_cast<const uint4*>(w.s + col * w.s_row + sb * 16);
    if (DT == XNQ_Q6K) {
        const uint4* h = reinterpret_cast<const uint4*>(w.h + col * w.h_row + sb * 64) + 2 * hsel;
#pragma unroll
        for (int i = 0; i < 2; i++) x.h[i] = ldw(&h[i]);
        x.d = *reinterpret_cast<const uint16_t*>(w.d + col * w.d_row + sb * 2);
    }
}

// (lanes 0-31 value, lanes 32-63 value) -> lo = the lanes-0-31 value, hi = the lanes-32-63 value, in every lane
__device__ __forceinline__ void join_halves(uint32_t v, uint32_t& lo, uint32_t& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    lo = r[0];
    hi = r[1];
}
__device__ __forceinline__ void join_halves4(uint4 v, uint4& lo, uint4& hi) {
    join_halves(v.x, lo.x, hi.x);
    join_halves(v.y, lo.y, hi.y);
    join_halves(v.z, lo.z, hi.z);
    join_halves(v.w, lo.w, hi.w);
}

// Activation pieces of one super-block, in registers on their way to LDS
// (named members, not an array, so that they stay in registers).
template <int DT, int MT>
struct ActSB {
    uint4 q0, q1, q2, q3;  // pieces t, t + 256, (MT == 2) t + 512, t + 768
    int4 sums;             // Q4K: chunk bsum pairs of sub-blocks 4*half .. (threads < 2R)
    float da;              // d_a of the thread's row (threads < 2R)
};

// Piece p of a super-block's activation tile: chunk fastest, so 8
// consecutive threads read one row's 128 contiguous bytes of a half.
template <int DT, int MT>
__device__ __forceinline__ uint4 load_piece(const AView& a, uint32_t m, uint32_t sb, uint32_t p) {
    const uint32_t c = p & 7, half = (p >> 3) & 1, row = min(p >> 4, m - 1);
    return *reinterpret_cast<const uint4*>(a.img + row * a.A.row_bytes + half * (a.A.k / 2) + (sb * 8 + c) * 16);
}

template <int DT, int MT>
__device__ __forceinline__ void store_piece(uint8_t* buf, uint32_t p, uint4 v) {
    using L = SLay<DT, MT>;
    const uint32_t c = p & 7, half = (p >> 3) & 1, row = p >> 4;
    *reinterpret_cast<uint4*>(buf + ((c * 2 + half) * L::R + row) * 16) = v;
}

template <int DT, int MT>
__device__ __forceinline__ void load_act_sb(const AView& a, uint32_t m, uint32_t sb, ActSB<DT, MT>& x) {
    using L = SLay<DT, MT>;
    static_assert(L::kPieces == 2 || L::kPieces == 4, "pieces per thread");
    const uint32_t t = threadIdx.x;
    const ActImg& A = a.A;
    x.q0 = load_piece<DT, MT>(a, m, sb, t);
    x.q1 = load_piece<DT, MT>(a, m, sb, t + kThreads);
    if (L::kPieces == 4) {
        x.q2 = load_piece<DT, MT>(a, m, sb, t + 2 * kThreads);
        x.q3 = load_piece<DT, MT>(a, m, sb, t + 3 * kThreads);
    }
    x.da = 0.0f;
    x.sums = make_int4(0, 0, 0, 0);
    if (t < 2 * L::R) {
        const uint32_t row = min(t >> 1, m - 1);
        x.da = reinterpret_cast<const float*>(a.img + row * A.row_bytes + A.d_off)[sb];
        if (DT == XNQ_Q4K)
            x.sums = *reinterpret_cast<const int4*>(a.img + row * A.row_bytes + A.s_off + sb * 32 + (t & 1) * 16);
    }
}

template <int DT, int MT>
__device__ __forceinline__ void store_act_sb(const ActSB<DT, MT>& x, uint8_t* buf) {
    using L = SLay<DT, MT>;
    const uint32_t t = threadIdx.x;
    store_piece<DT, MT>(buf, t, x.q0);
    store_piece<DT, MT>(buf, t + kThreads, x.q1);
    if (L::kPieces == 4) {
        store_piece<DT, MT>(buf, t + 2 * kThreads, x.q2);
        store_piece<DT, MT>(buf, t + 3 * kThreads, x.q3);
    }
    if (t < 2 * L::R) {
        const uint32_t row = t >> 1, half = t & 1;
        if (half == 0) reinterpret_cast<float*>(buf + L::kQ + L::kMin)[row] = x.da;
        if (DT == XNQ_Q4K) {
            const int32_t prs[4] = {x.sums.x, x.sums.y, x.sums.z, x.sums.w};
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                v[u] = -x.da * (float)((int)(int16_t)(prs[u] & 0xffff) + (int)(int16_t)(prs[u] >> 16));
            *reinterpret_cast<uint4*>(buf + L::kQ + (row * 2 + half) * 16) = bf16_split4(v);
        }
    }
}

template <int DT, int MT>
__global__ __launch_bounds__(kThreads) void skinny_kernel(WView w, AView a, uint32_t m, uint32_t sb_per_split,
                                                          float* __restrict__ y, size_t split_stride) {
    using L = SLay<DT, MT>;
    constexpr bool kQ4K = DT == XNQ_Q4K;
    constexpr int kShift = kQ4K ? 3 : 7;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t lrow = lane & 31, half = lane >> 5;
    const uint32_t sb0 = blockIdx.y * sb_per_split;
    const uint32_t nsb = min(sb_per_split, w.k / 256 - sb0);
    y += blockIdx.y * split_stride;
    const uint32_t ncol = blockIdx.x * kCols + wave * 32 + lrow;  // this lane's output column
    const uint32_t col = min(ncol, w.n - 1);

    v16f acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = v16f{};

    WeightSB<DT> wa, wb;  // two weight buffers, alternated statically (no register copies)
    load_weight_sb<DT>(w, col, sb0, wa);
    {
        ActSB<DT, MT> a0;
        load_act_sb<DT, MT>(a, m, sb0, a0);
        store_act_sb<DT, MT>(a0, lds);
    }
    __syncthreads();

    // super-block i from `wcur`; super-block i+1 is fetched into `wnext`
    auto step = [&](uint32_t i, WeightSB<DT>& wcur, WeightSB<DT>& wnext) __attribute__((always_inline)) {
        const uint32_t sb = sb0 + i;
        const bool more = i + 1 < nsb;
        ActSB<DT, MT> anext;
        if (more) {
            // activation first: its LDS store below then waits only for these
            // loads, not for the weight loads, which stay in flight until the
            // next super-block
            load_act_sb<DT, MT>(a, m, sb + 1, anext);
            __builtin_amdgcn_sched_barrier(0);  // keep every activation load ahead of the weight loads
            load_weight_sb<DT>(w, col, sb + 1, wnext);
            __builtin_amdgcn_sched_barrier(0);
        }
        const uint8_t* buf = lds + (i & 1) * L::kBuf;
        uint4 qc[8], hq[4];
#pragma unroll
        for (int c = 0; c < 4; c++) join_halves4(wcur.q[c], qc[c], qc[c + 4]);
        if (!kQ4K) {
            join_halves4(wcur.h[0], hq[0], hq[2]);
            join_halves4(wcur.h[1], hq[1], hq[3]);
        }
        v16i hi[MT], lo[MT];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            uint32_t p0[4], p1[4];  // high and low digit of this lane's 16 elements of chunk c
            if (kQ4K) {
                int sc, mn;
                q4k_scale_min(wcur.s.y, wcur.s.z, wcur.s.w, c, sc, mn);
                const uint32_t sh = (uint32_t)sc >> 3, sl = (uint32_t)sc & 7;
                const uint32_t q4[4] = {qc[c].x, qc[c].y, qc[c].z, qc[c].w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t nib = (q4[j] >> (4 * half)) & 0x0F0F0F0Fu;
                    p0[j] = mul_bytes(nib, sh);
                    p1[j] = mul_bytes(nib, sl);
                }
            } else {
                const uint4 hw = hq[c >> 1];
                const uint2 qh = (c & 1) ? make_uint2(hw.z, hw.w) : make_uint2(hw.x, hw.y);
                int b[8];
                q6k_unpack(qc[c], qh, b);
                const uint32_t sw = (c >> 1) == 0 ? wcur.s.x : (c >> 1) == 1 ? wcur.s.y : (c >> 1) == 2 ? wcur.s.z : wcur.s.w;
                const int sc = (int)(int8_t)(sw >> (8 * (2 * (c & 1) + half)));
#pragma unroll
                for (int j = 0; j < 4; j++) q6_digits((uint32_t)b[4 * half + j], sc, p1[j], p0[j]);
            }
            const v4i b0 = {(int)p0[0], (int)p0[1], (int)p0[2], (int)p0[3]};
            const v4i b1 = {(int)p1[0], (int)p1[1], (int)p1[2], (int)p1[3]};
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i av = *reinterpret_cast<const v4i*>(buf + ((c * 2 + half) * L::R + t * 32 + lrow) * 16);
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
        const float* eda = reinterpret_cast<const float*>(buf + L::kQ + L::kMin);
        const float dw = f16_bits_to_f32(kQ4K ? (wcur.s.x & 0xffffu) : wcur.d);
        v8bf bh8, bl8;
        if (kQ4K) {
            const float dm = f16_bits_to_f32(wcur.s.x >> 16);
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                int sc2, mn2;
                q4k_scale_min(wcur.s.y, wcur.s.z, wcur.s.w, (int)(4 * half + u), sc2, mn2);
                v[u] = dm * (float)mn2;
            }
            const uint4 bv = bf16_split4(v);
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
                const uint4 av = *reinterpret_cast<const uint4*>(buf + L::kQ + ((t * 32 + lrow) * 2 + half) * 16);
                const v8bf a8 = __builtin_bit_cast(v8bf, av);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bh8, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8, bl8, acc[t], 0, 0, 0);
            }
        }
        if (more) store_act_sb<DT, MT>(anext, lds + ((i + 1) & 1) * L::kBuf);
        __syncthreads();
    };
    for (uint32_t i = 0; i < nsb; i += 2) {
        step(i, wa, wb);
        if (i + 1 >= nsb) break;
        step(i + 1, wb, wa);
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

template <int DT, int MT>
hipError_t launch_skinny_dt(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                            hipStream_t s) {
    using L = SLay<DT, MT>;
    const uint32_t nsb = w.k / 256;
    const uint32_t per = (nsb + splits - 1) / splits;
    splits = (nsb + per - 1) / per;
    const dim3 grid((w.n + kCols - 1) / kCols, splits);
    float* out = splits > 1 ? partial : y;
    hipLaunchKernelGGL((skinny_kernel<DT, MT>), grid, dim3(kThreads), L::kLds, s, w, a, (uint32_t)m, per, out,
                       splits > 1 ? m * (size_t)w.n : (size_t)0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_sum_splits(partial, m * (size_t)w.n, splits, y, s);
}

}  // namespace

uint32_t skinny_splits(size_t m, size_t n, size_t k) {
    (void)m;
    // about three workgroups per CU, at least one super-block per split
    const size_t tiles = (n + kCols - 1) / kCols;
    const size_t nsb = k / 256;
    size_t splits = (768 + tiles - 1) / tiles;
    if (splits > nsb) splits = nsb;
    return splits < 1 ? 1u : (uint32_t)splits;
}

bool skinny_supported(uint32_t dtype, size_t m, size_t n, size_t k) {
    (void)n;
    return (dtype == XNQ_Q4K || dtype == XNQ_Q6K) && k % 256 == 0 && m >= 1 && m <= 64;
}

hipError_t launch_skinny(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                         hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (m > 64) return hipErrorInvalidValue;
    if (splits > 1 && !partial) splits = 1;
    if (w.dtype == XNQ_Q4K)
        return m <= 32 ? launch_skinny_dt<XNQ_Q4K, 1>(w, a, m, splits, y, partial, s)
                       : launch_skinny_dt<XNQ_Q4K, 2>(w, a, m, splits, y, partial, s);
    if (w.dtype == XNQ_Q6K)
        return m <= 32 ? launch_skinny_dt<XNQ_Q6K, 1>(w, a, m, splits, y, partial, s)
                       : launch_skinny_dt<XNQ_Q6K, 2>(w, a, m, splits, y, partial, s);
    return hipErrorNotSupported;
}

}  // namespace xnq
