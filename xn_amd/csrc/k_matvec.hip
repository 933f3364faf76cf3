// Decode-path matmul for m <= 8 activation rows: a wavefront per weight row.
//
// Every lane owns 32-element chunks of the row (chunk c = lane + 64*i), loads
// them with dwordx4 global loads (a wavefront instruction covers 1 KiB of one
// plane), dequantizes in registers and forms integer dot products with the
// Q8_0/Q8_K activations staged in LDS (v_dot4_i32_i8), applies the block
// scales in f32 and reduces over the wavefront with DPP row operations.
// The integer part of every block dot is exact; only the final f32 combine
// differs in rounding order from xn's vec_dot (k_quants.rs:287-304, 677-691,
// 1337-1416, 1743-1798).
#include "xnq_device.h"
#include "xnq_internal.h"

namespace xnq {

namespace {

constexpr int kWave = 64;
constexpr int kWavesPerWG = 4;
constexpr int kThreads = kWave * kWavesPerWG;

// LDS image of MB activation rows.
//   q8   : [MB][2][K/32][16]  (both 16-byte halves of chunk c stored so that
//          lane-consecutive chunks are byte-consecutive: conflict-free reads)
//   sums : [MB][K/32] int32  Q8K: bsum[2c] | bsum[2c+1] << 16 ; Q8_0: block sum
//   d    : [MB][blocks] f32
struct LdsPlan {
    uint32_t q_bytes, s_off, d_off, total;
};

__host__ __device__ inline LdsPlan lds_plan(int mb, uint32_t k, bool kquant) {
    LdsPlan p;
    p.q_bytes = (uint32_t)mb * k;
    p.s_off = p.q_bytes;
    const uint32_t s_bytes = (uint32_t)mb * (k / 32) * 4;
    p.d_off = p.s_off + s_bytes;
    const uint32_t nblk = kquant ? k / 256 : k / 32;
    p.total = p.d_off + (uint32_t)mb * nblk * 4;
    return p;
}

// Sum over the 64 lanes with DPP row shifts and the cross-row swizzles;
// the result is valid in lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

template <int DT, int MB>
__device__ void stage_activations(const AView& a, uint32_t m0, uint32_t mcount, uint8_t* lds,
                                  const LdsPlan& P) {
    const uint32_t k = a.k;
    const uint32_t pieces_per_row = k / 16;
    const uint32_t cpr = k / 32;
    // q8
    for (uint32_t i = threadIdx.x; i < (uint32_t)MB * pieces_per_row; i += kThreads) {
        const uint32_t mb = i / pieces_per_row, g = i % pieces_per_row;
        const uint32_t c = g >> 1, hh = g & 1;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (mb < mcount) v = *reinterpret_cast<const uint4*>(a.q + (size_t)(m0 + mb) * k + g * 16);
        *reinterpret_cast<uint4*>(lds + mb * k + hh * (k / 2) + c * 16) = v;
    }
    int32_t* ls = reinterpret_cast<int32_t*>(lds + P.s_off);
    float* ld = reinterpret_cast<float*>(lds + P.d_off);
    constexpr bool kq = (DT == XNQ_Q4K || DT == XNQ_Q6K);
    for (uint32_t i = threadIdx.x; i < (uint32_t)MB * cpr; i += kThreads) {
        const uint32_t mb = i / cpr, c = i % cpr;
        int32_t v = 0;
        if (mb < mcount) {
            if (kq) {
                v = reinterpret_cast<const int32_t*>(a.s + (size_t)(m0 + mb) * a.s_per_row)[c];
            } else {
                v = (int32_t)a.s[(size_t)(m0 + mb) * a.s_per_row + c];
            }
        }
        ls[i] = v;
    }
    const uint32_t nblk = a.d_per_row;
    for (uint32_t i = threadIdx.x; i < (uint32_t)MB * nblk; i += kThreads) {
        const uint32_t mb = i / nblk, b = i % nblk;
        float v = 0.0f;
        if (mb < mcount) {
            if (kq) {
                v = reinterpret_cast<const float*>(a.d)[(size_t)(m0 + mb) * nblk + b];
            } else {
                v = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(a.d)[(size_t)(m0 + mb) * nblk + b]);
            }
        }
        ld[i] = v;
    }
}

// Per-chunk weight data held in registers between the load and the compute.
struct Chunk {
    uint4 q;
    uint4 x;  // Q8_0: second 16 bytes; Q4K: {d|dmin, scales}; Q6K: qh in .x/.y, scales pair in .z
    float dw;
};

template <int DT>
__device__ __forceinline__ void load_chunk(const WView& w, uint32_t row, uint32_t c, Chunk& ch) {
    if (DT == XNQ_Q8_0) {
        const uint8_t* p = w.q + (size_t)row * w.q_row + (size_t)c * 32;
        ch.q = *reinterpret_cast<const uint4*>(p);
        ch.x = *reinterpret_cast<const uint4*>(p + 16);
        ch.dw = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(w.d + (size_t)row * w.d_row + c * 2));
    } else if (DT == XNQ_Q4_0) {
        ch.q = *reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16);
        ch.dw = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(w.d + (size_t)row * w.d_row + c * 2));
    } else if (DT == XNQ_Q4K) {
        ch.q = *reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16);
        ch.x = *reinterpret_cast<const uint4*>(w.s + (size_t)row * w.s_row + (size_t)(c >> 3) * 16);
    } else {  // Q6K
        const uint32_t sb = c >> 3, j = c & 7;
        ch.q = *reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16);
        const uint2 h = *reinterpret_cast<const uint2*>(w.h + (size_t)row * w.h_row + (size_t)c * 8);
        ch.x.x = h.x;
        ch.x.y = h.y;
        ch.x.z = *reinterpret_cast<const uint16_t*>(w.s + (size_t)row * w.s_row + sb * 16 + 2 * j);
        ch.dw = f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(w.d + (size_t)row * w.d_row + sb * 2));
    }
}

template <int DT, int MB>
__device__ __forceinline__ void compute_chunk(const Chunk& ch, uint32_t c, uint32_t k,
                                              const uint8_t* lds, const LdsPlan& P, float* acc) {
    const int32_t* ls = reinterpret_cast<const int32_t*>(lds + P.s_off);
    const float* ld = reinterpret_cast<const float*>(lds + P.d_off);
    const uint32_t cpr = k / 32;
    int sc = 0, mn = 0;
    float dw = ch.dw, dmin = 0.0f;
    if (DT == XNQ_Q4K) {
        dw = f16_bits_to_f32(ch.x.x);
        dmin = f16_bits_to_f32(ch.x.x >> 16);
        q4k_scale_min(ch.x.y, ch.x.z, ch.x.w, (int)(c & 7), sc, mn);
    }
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const uint8_t* qrow = lds + mb * k;
        const uint4 a0 = *reinterpret_cast<const uint4*>(qrow + c * 16);
        const uint4 a1 = *reinterpret_cast<const uint4*>(qrow + k / 2 + c * 16);
        const int a[8] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                          (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        const int32_t sv = ls[mb * cpr + c];
        if (DT == XNQ_Q4K) {
            int lo, hi;
            nib_dot2(ch.q, a, lo, hi);
            const int isum = sc * (lo + hi);
            const int msum = mn * ((int)(int16_t)(sv & 0xffff) + (int)(int16_t)(sv >> 16));
            const float da = ld[mb * (k / 256) + (c >> 3)];
            acc[mb] += (dw * da) * (float)isum - (dmin * da) * (float)msum;
        } else if (DT == XNQ_Q6K) {
            const int sc0 = (int)(int8_t)(ch.x.z & 0xff), sc1 = (int)(int8_t)((ch.x.z >> 8) & 0xff);
            const int v = q6k_chunk_int(ch.q, make_uint2(ch.x.x, ch.x.y), a, sc0, sc1,
                                        (int)(int16_t)(sv & 0xffff), (int)(int16_t)(sv >> 16));
            const float da = ld[mb * (k / 256) + (c >> 3)];
            acc[mb] += (dw * da) * (float)v;
        } else if (DT == XNQ_Q4_0) {
            int lo, hi;
            nib_dot2(ch.q, a, lo, hi);
            const int v = lo + hi - 8 * sv;
            const float da = ld[mb * cpr + c];
            acc[mb] += (dw * da) * (float)v;
        } else {
            const int v = i8_dot32(ch.q, ch.x, a);
            const float da = ld[mb * cpr + c];
            acc[mb] += (dw * da) * (float)v;
        }
    }
}

template <int DT, int MB, int U>
__global__ __launch_bounds__(kThreads) void matvec_kernel(WView w, AView a, uint32_t m0,
                                                          uint32_t mcount, float* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr bool kq = (DT == XNQ_Q4K || DT == XNQ_Q6K);
    const LdsPlan P = lds_plan(MB, w.k, kq);
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t nchunks = w.k / 32;
    const uint32_t row_stride = gridDim.x * kWavesPerWG;
    uint32_t row = blockIdx.x * kWavesPerWG + wave;

    // Issue the first row's weight loads before staging the activations so
    // the HBM latency overlaps the LDS fill.
    Chunk ch[U];
    if (row < w.n) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t c = lane + u * kWave;
            if (c < nchunks) load_chunk<DT>(w, row, c, ch[u]);
        }
    }
    stage_activations<DT, MB>(a, m0, mcount, lds, P);
    __syncthreads();

    for (; row < w.n; row += row_stride) {
        float acc[MB];
#pragma unroll
        for (int i = 0; i < MB; i++) acc[i] = 0.0f;
        for (uint32_t c0 = 0; c0 < nchunks; c0 += U * kWave) {
            if (c0 > 0) {
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const uint32_t c = c0 + lane + u * kWave;
                    if (c < nchunks) load_chunk<DT>(w, row, c, ch[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint32_t c = c0 + lane + u * kWave;
                if (c < nchunks) compute_chunk<DT, MB>(ch[u], c, w.k, lds, P, acc);
            }
        }
        // Prefetch the next row's first chunks before the reduction.
        const uint32_t next = row + row_stride;
        if (next < w.n) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint32_t c = lane + u * kWave;
                if (c < nchunks) load_chunk<DT>(w, next, c, ch[u]);
            }
        }
#pragma unroll
        for (int i = 0; i < MB; i++) {
            const float s = wave_sum(acc[i]);
            if (lane == (uint32_t)i && (uint32_t)i < mcount) y[(size_t)(m0 + i) * w.n + row] = s;
        }
    }
}

// Integer parts of every block dot (for exactness tests): one thread per
// (activation row, weight row, block), using the same chunk arithmetic.
__global__ void block_ints_kernel(WView w, AView a, uint32_t m, int32_t* __restrict__ out) {
    const bool kq = w.dtype == XNQ_Q4K || w.dtype == XNQ_Q6K;
    const uint32_t nb = w.nb;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)m * w.n * nb;
    if (t >= total) return;
    const uint32_t b = (uint32_t)(t % nb);
    const uint32_t row = (uint32_t)((t / nb) % w.n);
    const uint32_t mr = (uint32_t)(t / ((size_t)nb * w.n));
    const int8_t* aq = a.q + (size_t)mr * w.k;
    int32_t r0 = 0, r1 = 0;
    const uint32_t c_begin = kq ? b * 8 : b, c_end = kq ? b * 8 + 8 : b + 1;
    for (uint32_t c = c_begin; c < c_end; c++) {
        const int* ap = reinterpret_cast<const int*>(aq + (size_t)c * 32);
        int av[8];
        for (int i = 0; i < 8; i++) av[i] = ap[i];
        if (w.dtype == XNQ_Q8_0) {
            const uint8_t* p = w.q + (size_t)row * w.q_row + (size_t)c * 32;
            r0 += i8_dot32(*reinterpret_cast<const uint4*>(p), *reinterpret_cast<const uint4*>(p + 16), av);
        } else if (w.dtype == XNQ_Q4_0) {
            int lo, hi;
            nib_dot2(*reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16), av, lo, hi);
            r0 += lo + hi - 8 * (int)a.s[(size_t)mr * a.s_per_row + c];
        } else if (w.dtype == XNQ_Q4K) {
            const uint4 meta = *reinterpret_cast<const uint4*>(w.s + (size_t)row * w.s_row + (size_t)b * 16);
            int sc, mn, lo, hi;
            q4k_scale_min(meta.y, meta.z, meta.w, (int)(c & 7), sc, mn);
            nib_dot2(*reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16), av, lo, hi);
            const int16_t* bs = a.s + (size_t)mr * a.s_per_row;
            r0 += sc * (lo + hi);
            r1 += mn * ((int)bs[2 * c] + (int)bs[2 * c + 1]);
        } else {
            const uint4 ql = *reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16);
            const uint2 qh = *reinterpret_cast<const uint2*>(w.h + (size_t)row * w.h_row + (size_t)c * 8);
            const int8_t* sc = reinterpret_cast<const int8_t*>(w.s + (size_t)row * w.s_row + (size_t)b * 16);
            const int16_t* bs = a.s + (size_t)mr * a.s_per_row;
            const uint32_t j = c & 7;
            r0 += q6k_chunk_int(ql, qh, av, sc[2 * j], sc[2 * j + 1], bs[2 * c], bs[2 * c + 1]);
        }
    }
    out[2 * t] = r0;
    out[2 * t + 1] = r1;
}

template <int DT, int MB, int U>
hipError_t launch_mv(const WView& w, const AView& a, uint32_t m0, uint32_t mcount, float* y,
                     hipStream_t s) {
    constexpr bool kq = (DT == XNQ_Q4K || DT == XNQ_Q6K);
    const LdsPlan P = lds_plan(MB, w.k, kq);
    auto fn = matvec_kernel<DT, MB, U>;
    static int max_wg_per_cu = -1;
    static uint32_t cached_lds = 0;
    static int num_cu = 0;
    if (max_wg_per_cu < 0 || cached_lds != P.total) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)P.total);
        if (e != hipSuccess) return e;
        int occ = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kThreads, P.total);
        if (e != hipSuccess) return e;
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, dev);
        max_wg_per_cu = occ > 0 ? occ : 1;
        cached_lds = P.total;
    }
    const uint32_t need = (w.n + kWavesPerWG - 1) / kWavesPerWG;
    const uint32_t cap = (uint32_t)(max_wg_per_cu * num_cu);
    const uint32_t grid = need < cap ? need : cap;
    hipLaunchKernelGGL(fn, dim3(grid), dim3(kThreads), P.total, s, w, a, m0, mcount, y);
    return hipGetLastError();
}

constexpr uint32_t kMaxLds = 160 * 1024;

template <int DT>
hipError_t launch_dt(const WView& w, const AView& a, size_t m, float* y, hipStream_t s) {
    constexpr bool kq = (DT == XNQ_Q4K || DT == XNQ_Q6K);
    // Largest row group whose activations fit in LDS.
    int gmax = 8;
    while (gmax > 1 && lds_plan(gmax, w.k, kq).total > kMaxLds) gmax >>= 1;
    if (lds_plan(gmax, w.k, kq).total > kMaxLds) return hipErrorInvalidConfiguration;
    // U (chunks in flight per lane) covers k up to U*64*32 elements in one pass.
    for (size_t m0 = 0; m0 < m; m0 += gmax) {
        const uint32_t mc = (uint32_t)((m - m0) < (size_t)gmax ? (m - m0) : (size_t)gmax);
        hipError_t e;
        if (mc == 1) e = launch_mv<DT, 1, 8>(w, a, (uint32_t)m0, mc, y, s);
        else if (mc == 2) e = launch_mv<DT, 2, 4>(w, a, (uint32_t)m0, mc, y, s);
        else if (mc <= 4) e = launch_mv<DT, 4, 4>(w, a, (uint32_t)m0, mc, y, s);
        else e = launch_mv<DT, 8, 2>(w, a, (uint32_t)m0, mc, y, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

size_t matvec_lds_bytes(uint32_t dtype, size_t mb, size_t k) {
    const bool kq = dtype == XNQ_Q4K || dtype == XNQ_Q6K;
    return lds_plan((int)mb, (uint32_t)k, kq).total;
}

hipError_t launch_matvec(const WView& w, const AView& a, size_t m, float* y, hipStream_t s) {
    switch (w.dtype) {
    case XNQ_Q8_0: return launch_dt<XNQ_Q8_0>(w, a, m, y, s);
    case XNQ_Q4_0: return launch_dt<XNQ_Q4_0>(w, a, m, y, s);
    case XNQ_Q4K: return launch_dt<XNQ_Q4K>(w, a, m, y, s);
    case XNQ_Q6K: return launch_dt<XNQ_Q6K>(w, a, m, y, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_block_ints(const WView& w, const AView& a, size_t m, int32_t* out, hipStream_t s) {
    const size_t total = m * w.n * w.nb;
    if (total == 0) return hipSuccess;
    block_ints_kernel<<<(unsigned)((total + 127) / 128), 128, 0, s>>>(w, a, (uint32_t)m, out);
    return hipGetLastError();
}

}  // namespace xnq
