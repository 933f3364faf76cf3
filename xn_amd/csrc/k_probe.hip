// Measurement kernels behind the xnq_probe_* / xnq_stream_read hooks: the
// hardware ceilings the quantized-matmul kernels are judged against, kept in
// the library so every figure quoted for them can be re-measured.
//   stream_read  bare HBM read (the weight-stream ceiling of the matvec);
//   mfma_valu    int8 MFMA chains with independent VALU work, in the same
//                wavefront or in the other wavefront of the SIMD (whether
//                VALU time hides under the matrix cores);
//   lds_read     conflict-free ds_read_b128 bandwidth per CU.
#include "xnq_internal.h"

namespace xnq {

namespace {

typedef unsigned int pr_u4 __attribute__((ext_vector_type(4)));
typedef int pr_v4i __attribute__((ext_vector_type(4)));
typedef int pr_v16i __attribute__((ext_vector_type(16)));

// 4 non-temporal dwordx4 loads in flight per lane, grid-strided; one atomic
// XOR per wavefront folds the data into *sink so no load is dead.
constexpr int kSrLoads = 4, kSrThreads = 256;
__global__ __launch_bounds__(kSrThreads) void stream_read_kernel(const pr_u4* __restrict__ p, size_t n16,
                                                                 uint32_t* sink) {
    size_t i = (size_t)blockIdx.x * kSrThreads * kSrLoads + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * kSrThreads * kSrLoads;
    uint32_t acc = 0;
    for (; i < n16; i += stride) {
        pr_u4 v[kSrLoads];
#pragma unroll
        for (int j = 0; j < kSrLoads; j++) {
            const size_t t = i + (size_t)j * kSrThreads;
            v[j] = t < n16 ? __builtin_nontemporal_load(p + t) : pr_u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < kSrLoads; j++) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
    if ((threadIdx.x & 63) == 0 && acc) atomicXor(sink, acc);
}

// 8 wavefronts (2 per SIMD).  Per iteration a wavefront that does MFMA work
// issues 4 independent v_mfma_i32_32x32x32_i8, and one that does VALU work
// runs V rounds of 8 dependent-free integer ops (4 chains of shift + xor-add,
// not foldable by the compiler).  SPLIT: waves 0-3 MFMA only, 4-7 VALU only.
template <int V, bool SPLIT>
__global__ __launch_bounds__(512) void mfma_valu_kernel(int iters, uint32_t* sink) {
    pr_v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
    const pr_v4i a = {(int)threadIdx.x, 1, 2, 3}, b = {3, 2, 1, (int)threadIdx.x};
    uint32_t x0 = threadIdx.x, x1 = x0 * 3u, x2 = x0 * 5u, x3 = x0 * 7u;
    const uint32_t wave = threadIdx.x >> 6;
    const bool mf = !SPLIT || wave < 4, va = !SPLIT || wave >= 4;
    for (int it = 0; it < iters; it++) {
        if (mf) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
        }
        if (va) {
#pragma unroll
            for (int v = 0; v < V; v++) {
                x0 = (x0 ^ (x1 >> 3)) + x2;
                x1 = (x1 ^ (x2 << 5)) + x3;
                x2 = (x2 ^ (x3 >> 7)) + x0;
                x3 = (x3 ^ (x0 << 11)) + x1;
            }
        }
    }
    uint32_t s = x0 ^ x1 ^ x2 ^ x3;
    for (int i = 0; i < 16; i++) s += (uint32_t)(c0[i] + c1[i] + c2[i] + c3[i]);
    if (s == 0x9e3779b9u) atomicXor(sink, s);  // keeps the work live; practically never taken
}

// Every wavefront reads 8 conflict-free ds_read_b128 per iteration from a
// 128 KiB LDS array (lane-consecutive 16-byte words).
__global__ __launch_bounds__(512) void lds_read_kernel(int iters, uint32_t* sink) {
    extern __shared__ __align__(16) pr_u4 buf[];
    for (int i = threadIdx.x; i < 8192; i += blockDim.x) buf[i] = pr_u4{(uint32_t)i, 1u, 2u, 3u};
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    pr_u4 acc = {0u, 0u, 0u, 0u};
    const int base = wave * 512;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int r = 0; r < 8; r++) acc ^= buf[(base + r * 64 + lane + it) & 8191];
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) atomicXor(sink, acc.x);
}

}  // namespace

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return hipSuccess;
    // 2048 workgroups (8 per CU) reached the ceiling on MI355X; fewer for small reads
    size_t grid = (n16 + kSrThreads * kSrLoads - 1) / (kSrThreads * kSrLoads);
    if (grid > 2048) grid = 2048;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(kSrThreads), 0, s,
                       static_cast<const pr_u4*>(src), n16, sink);
    return hipGetLastError();
}

hipError_t launch_probe_mfma_valu(int valu_rounds, bool split, int iters, int workgroups, uint32_t* sink,
                                  hipStream_t s) {
#define XNQ_PROBE_MV(V)                                                                                    \
    if (valu_rounds == V) {                                                                                \
        if (split) hipLaunchKernelGGL((mfma_valu_kernel<V, true>), dim3(workgroups), dim3(512), 0, s, iters, sink); \
        else hipLaunchKernelGGL((mfma_valu_kernel<V, false>), dim3(workgroups), dim3(512), 0, s, iters, sink);     \
        return hipGetLastError();                                                                          \
    }
    XNQ_PROBE_MV(0) XNQ_PROBE_MV(2) XNQ_PROBE_MV(4) XNQ_PROBE_MV(8) XNQ_PROBE_MV(16)
#undef XNQ_PROBE_MV
    return hipErrorInvalidValue;
}

hipError_t launch_probe_lds_read(int iters, int workgroups, uint32_t* sink, hipStream_t s) {
    const hipError_t e = set_max_lds(reinterpret_cast<const void*>(lds_read_kernel), 128 * 1024);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(lds_read_kernel, dim3(workgroups), dim3(512), 128 * 1024, s, iters, sink);
    return hipGetLastError();
}

}  // namespace xnq
