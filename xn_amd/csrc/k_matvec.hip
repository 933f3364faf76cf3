// Dispatch of the matvec kernels (k_matvec_impl.h, instantiated per dtype in
// k_matvec_<dtype>.hip) and the block-integer kernels used by exactness tests.
// The integer part of every block dot is exact; only the final f32 combine
// differs in rounding order from xn's vec_dot (k_quants.rs:287-304, 677-691,
// 1337-1416, 1743-1798).
#include "k_matvec_impl.h"

namespace xnq {

namespace {

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
    const uint8_t* img = a.img + (size_t)mr * a.A.row_bytes;
    const int32_t* sums = reinterpret_cast<const int32_t*>(img + a.A.s_off);
    int32_t r0 = 0, r1 = 0;
    const uint32_t c_begin = kq ? b * 8 : b, c_end = kq ? b * 8 + 8 : b + 1;
    for (uint32_t c = c_begin; c < c_end; c++) {
        const uint4 lo4 = *reinterpret_cast<const uint4*>(img + c * 16);
        const uint4 hi4 = *reinterpret_cast<const uint4*>(img + w.k / 2 + c * 16);
        const int av[8] = {(int)lo4.x, (int)lo4.y, (int)lo4.z, (int)lo4.w,
                           (int)hi4.x, (int)hi4.y, (int)hi4.z, (int)hi4.w};
        const int32_t sv = sums[c];
        if (w.dtype == XNQ_Q8_0) {
            const uint8_t* p = w.q + (size_t)row * w.q_row + (size_t)c * 32;
            r0 += i8_dot32(*reinterpret_cast<const uint4*>(p), *reinterpret_cast<const uint4*>(p + 16), av);
        } else if (w.dtype == XNQ_Q4_0) {
            int lo, hi;
            nib_dot2(*reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16), av, lo, hi);
            r0 += lo + hi - 8 * sv;
        } else if (w.dtype == XNQ_Q4K) {
            const uint4 meta = *reinterpret_cast<const uint4*>(w.s + (size_t)row * w.s_row + (size_t)b * 16);
            int sc, mn, lo, hi;
            q4k_scale_min(meta.y, meta.z, meta.w, (int)(c & 7), sc, mn);
            nib_dot2(*reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16), av, lo,
                     hi);
            r0 += sc * (lo + hi);
            r1 += mn * ((int)(int16_t)(sv & 0xffff) + (int)(int16_t)(sv >> 16));
        } else {
            const uint4 ql = *reinterpret_cast<const uint4*>(w.q + (size_t)row * w.q_row + (size_t)c * 16);
            const uint2 qh = *reinterpret_cast<const uint2*>(w.h + (size_t)row * w.h_row + (size_t)c * 8);
            const int8_t* sc = reinterpret_cast<const int8_t*>(w.s + (size_t)row * w.s_row + (size_t)b * 16);
            const uint32_t j = c & 7;
            r0 += q6k_chunk_int(ql, qh, av, sc[2 * j], sc[2 * j + 1], (int)(int16_t)(sv & 0xffff),
                                (int)(int16_t)(sv >> 16));
        }
    }
    out[2 * t] = r0;
    out[2 * t + 1] = r1;
}

// The same for the padded-block types: one thread per (activation row,
// weight row, block), the block's chunks through load_chunk / chunk_ints, so
// the integers are the ones the matvec kernels scale.
template <int DT>
__global__ void block_ints_raw_kernel(WView w, AView a, uint32_t m, int32_t* __restrict__ out) {
    constexpr uint32_t kChunks = is_kquant(DT) ? 8 : 1;
    const uint32_t nb = w.nb;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)m * w.n * nb;
    if (t >= total) return;
    const uint32_t b = (uint32_t)(t % nb);
    const uint32_t row = (uint32_t)((t / nb) % w.n);
    const uint32_t mr = (uint32_t)(t / ((size_t)nb * w.n));
    const uint8_t* img = a.img + (size_t)mr * a.A.row_bytes;
    const int32_t* sums = reinterpret_cast<const int32_t*>(img + a.A.s_off);
    int32_t r0 = 0, r1 = 0;
    for (uint32_t c = b * kChunks; c < b * kChunks + kChunks; c++) {
        const uint4 lo4 = *reinterpret_cast<const uint4*>(img + c * 16);
        const uint4 hi4 = *reinterpret_cast<const uint4*>(img + w.k / 2 + c * 16);
        const int av[8] = {(int)lo4.x, (int)lo4.y, (int)lo4.z, (int)lo4.w,
                           (int)hi4.x, (int)hi4.y, (int)hi4.z, (int)hi4.w};
        mv::Chunk ch;
        mv::load_chunk<DT>(w, row, c, ch);
        int i0, i1;
        mv::chunk_ints<DT>(ch, c, av, sums[c], i0, i1);
        r0 += i0;
        r1 += i1;
    }
    out[2 * t] = r0;
    out[2 * t + 1] = r1;
}

// g = silu(g) * u, silu(s) = s / (1 + exp(0 - s)) (cpu_backend.rs:354-356)
__global__ __launch_bounds__(256) void silu_mul_kernel(float* __restrict__ g, const float* __restrict__ u,
                                                       size_t count) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    const float t = g[i];
    g[i] = t / (1.0f + expf(0.0f - t)) * u[i];
}

}  // namespace

hipError_t launch_silu_mul(float* g, const float* u, size_t count, hipStream_t s) {
    if (count == 0) return hipSuccess;
    silu_mul_kernel<<<(unsigned)((count + 255) / 256), 256, 0, s>>>(g, u, count);
    return hipGetLastError();
}

hipError_t launch_matvec(const WView& w, const AView& a, size_t m, float* y, hipStream_t s) {
    switch (w.dtype) {
    case XNQ_Q8_0: return launch_matvec_q8_0(w, a, nullptr, m, y, s, false);
    case XNQ_Q4_0: return launch_matvec_q4_0(w, a, nullptr, m, y, s, false);
    case XNQ_Q4K: return launch_matvec_q4k(w, a, nullptr, m, y, s, false);
    case XNQ_Q6K: return launch_matvec_q6k(w, a, nullptr, m, y, s, false);
    case XNQ_Q4_1: return launch_matvec_q4_1(w, a, nullptr, m, y, s, false);
    case XNQ_Q5_0: return launch_matvec_q5_0(w, a, nullptr, m, y, s, false);
    case XNQ_Q5_1: return launch_matvec_q5_1(w, a, nullptr, m, y, s, false);
    case XNQ_Q2K: return launch_matvec_q2k(w, a, nullptr, m, y, s, false);
    case XNQ_Q3K: return launch_matvec_q3k(w, a, nullptr, m, y, s, false);
    case XNQ_Q5K: return launch_matvec_q5k(w, a, nullptr, m, y, s, false);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_fused(const WView& w, const float* x, size_t m, float* y, hipStream_t s,
                               bool one_shot) {
    const int fused = one_shot ? kFusedOneShot : kFusedPersistent;
    AView a{};
    a.k = w.k;
    a.m = (uint32_t)m;
    a.A = act_img(w.k, is_kquant(w.dtype));
    switch (w.dtype) {
    case XNQ_Q8_0: return launch_matvec_q8_0(w, a, x, m, y, s, fused);
    case XNQ_Q4_0: return launch_matvec_q4_0(w, a, x, m, y, s, fused);
    case XNQ_Q4K: return launch_matvec_q4k(w, a, x, m, y, s, fused);
    case XNQ_Q6K: return launch_matvec_q6k(w, a, x, m, y, s, fused);
    case XNQ_Q4_1: return launch_matvec_q4_1(w, a, x, m, y, s, fused);
    case XNQ_Q5_0: return launch_matvec_q5_0(w, a, x, m, y, s, fused);
    case XNQ_Q5_1: return launch_matvec_q5_1(w, a, x, m, y, s, fused);
    case XNQ_Q2K: return launch_matvec_q2k(w, a, x, m, y, s, fused);
    case XNQ_Q3K: return launch_matvec_q3k(w, a, x, m, y, s, fused);
    case XNQ_Q5K: return launch_matvec_q5k(w, a, x, m, y, s, fused);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_group(const WGroup& g, const float* x, bool gate, hipStream_t s) {
    switch (g.w[0].dtype) {
    case XNQ_Q8_0: return launch_group_q8_0(g, x, gate, s);
    case XNQ_Q4_0: return launch_group_q4_0(g, x, gate, s);
    case XNQ_Q4K: return launch_group_q4k(g, x, gate, s);
    case XNQ_Q6K: return launch_group_q6k(g, x, gate, s);
    case XNQ_Q4_1: return launch_group_q4_1(g, x, gate, s);
    case XNQ_Q5_0: return launch_group_q5_0(g, x, gate, s);
    case XNQ_Q5_1: return launch_group_q5_1(g, x, gate, s);
    case XNQ_Q2K: return launch_group_q2k(g, x, gate, s);
    case XNQ_Q3K: return launch_group_q3k(g, x, gate, s);
    case XNQ_Q5K: return launch_group_q5k(g, x, gate, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_block_ints(const WView& w, const AView& a, size_t m, int32_t* out, hipStream_t s) {
    const size_t total = m * w.n * w.nb;
    if (total == 0) return hipSuccess;
    const unsigned grid = (unsigned)((total + 127) / 128);
    switch (w.dtype) {
    case XNQ_Q4_1: block_ints_raw_kernel<XNQ_Q4_1><<<grid, 128, 0, s>>>(w, a, (uint32_t)m, out); return hipGetLastError();
    case XNQ_Q5_0: block_ints_raw_kernel<XNQ_Q5_0><<<grid, 128, 0, s>>>(w, a, (uint32_t)m, out); return hipGetLastError();
    case XNQ_Q5_1: block_ints_raw_kernel<XNQ_Q5_1><<<grid, 128, 0, s>>>(w, a, (uint32_t)m, out); return hipGetLastError();
    case XNQ_Q2K: block_ints_raw_kernel<XNQ_Q2K><<<grid, 128, 0, s>>>(w, a, (uint32_t)m, out); return hipGetLastError();
    case XNQ_Q3K: block_ints_raw_kernel<XNQ_Q3K><<<grid, 128, 0, s>>>(w, a, (uint32_t)m, out); return hipGetLastError();
    case XNQ_Q5K: block_ints_raw_kernel<XNQ_Q5K><<<grid, 128, 0, s>>>(w, a, (uint32_t)m, out); return hipGetLastError();
    }
    block_ints_kernel<<<(unsigned)((total + 127) / 128), 128, 0, s>>>(w, a, (uint32_t)m, out);
    return hipGetLastError();
}

}  // namespace xnq
