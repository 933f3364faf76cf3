// Measurement library (libxnq_measure.so), not part of the product: the bare
// HBM read that the decode matvec's weight stream is judged against.  Only
// bench.py's `--only stream` leg and its GPU test load it.
//
//   int xnqm_stream_read(const void* src_dev, size_t bytes, uint32_t* sink_dev, void* stream)
//     reads `bytes` (a multiple of 16) of device memory with the matvec
//     kernels' access pattern (dwordx4, non-temporal, 4 loads in flight per
//     lane, a grid of 4-wavefront workgroups filling the GPU) and XORs every
//     32-bit word into *sink_dev (which the caller zeroes); returns 0, or 1
//     for bad arguments, 2 for a launch error.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef unsigned int pr_u4 __attribute__((ext_vector_type(4)));

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

}  // namespace

extern "C" int xnqm_stream_read(const void* src_dev, size_t bytes, uint32_t* sink_dev, void* stream) {
    if (bytes % 16 || (bytes && (!src_dev || !sink_dev))) return 1;
    return launch_stream_read(src_dev, bytes, sink_dev, (hipStream_t)stream) == hipSuccess ? 0 : 2;
}
