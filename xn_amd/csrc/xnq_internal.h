// Internal declarations shared by the libxnq translation units: the repacked
// weight layout in HBM, the private activation workspace layout, small device
// helpers and the launchers each .hip file provides.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/xnq.h"

namespace xnq {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr size_t kAlign = 256;

inline size_t align_up(size_t v, size_t a = kAlign) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// Repacked weight storage.  Every plane is row major over the n weight rows,
// so one row of one plane is a contiguous run of bytes; a wavefront working
// on a row reads 1 KiB per dwordx4 instruction.
//
// A "chunk" is 32 consecutive elements of a row: the unit one lane handles.
//   Q8_0: q plane [n][nb][32] int8      d plane [n][nb] f16
//   Q4_0: q plane [n][nb][16] nibbles   d plane [n][nb] f16
//         byte i: low nibble = element i, high nibble = element i+16
//         (the GGUF order, already what the dot4 grouping wants)
//   Q4K:  q plane [n][nb][8 chunks][16] s plane [n][nb][16] = {d, dmin, scales[12]}
//         chunk c = sub-block c; byte i: low = element i, high = element i+16
//   Q6K:  q plane [n][nb][8][16] low 4 bits, nibble order as Q4K
//         h plane [n][nb][8][8]  high 2 bits: dword u, byte p, bits 2g'..2g'+1
//                                hold element 4*(4u+g')+p of the chunk
//         s plane [n][nb][16] int8 scales, d plane [n][nb] f16
//   Q4K and Q6K also keep a second copy of their s plane (st) and Q6K of
//         its d plane (dt) in 128-row tiles, for the matrix-core kernels:
//         super-block sb of rows 128t .. 128t+127 is one contiguous run of
//         128 * P bytes (P = the plane's bytes per row and super-block: s 16,
//         d 4 per super-block pair), row r's P bytes at (r & 127) * P in it
//         (kq_tile_off); rows are padded to a multiple of 128.  Their header
//         fetch covers 64 or 128 consecutive columns, which is one cache line
//         per column row-major and contiguous tiled; the matvec kernels read
//         the row-major planes.
//   Q4_1, Q5_0, Q5_1, Q2K, Q3K, Q5K: one q plane [n][nb][stride] of the GGUF
//         blocks padded to a 4-byte multiple (raw_stride below) so every field
//         is dword aligned: Q5_0 {d, 2 pad, qh[4], qs[16]}, Q3K 2 tail bytes;
//         the others are their GGUF bytes unchanged.
// nb = blocks per row (k/32 for the 32-element types, k/256 for the K types).
// ---------------------------------------------------------------------------

// Byte offset of (row, super-block sb) in a tiled Q4K / Q6K plane of P bytes
// per row and super-block (every plane is < 4 GiB, checked at upload).
__host__ __device__ inline uint32_t kq_tile_off(uint32_t nb, uint32_t row, uint32_t sb, uint32_t P) {
    return ((row >> 7) * nb + sb) * (P * 128u) + (row & 127u) * P;
}
constexpr uint32_t kTileRows = 128;

// Super-block (256-element) types, whose activations are Q8K.
__host__ __device__ constexpr bool is_kquant(uint32_t dt) {
    return dt == XNQ_Q2K || dt == XNQ_Q3K || dt == XNQ_Q4K || dt == XNQ_Q5K || dt == XNQ_Q6K;
}
// Types kept as padded GGUF blocks in one plane, and their stride in bytes.
__host__ __device__ constexpr bool is_raw_layout(uint32_t dt) {
    return dt == XNQ_Q4_1 || dt == XNQ_Q5_0 || dt == XNQ_Q5_1 || dt == XNQ_Q2K || dt == XNQ_Q3K || dt == XNQ_Q5K;
}
__host__ __device__ constexpr uint32_t raw_stride(uint32_t dt) {
    return dt == XNQ_Q4_1 ? 20 : dt == XNQ_Q5_0 ? 24 : dt == XNQ_Q5_1 ? 24 : dt == XNQ_Q2K ? 84
         : dt == XNQ_Q3K ? 112 : dt == XNQ_Q5K ? 176 : 0;
}
struct WLayout {
    uint32_t dtype = 0;
    size_t n = 0, k = 0, nb = 0;
    size_t q_row = 0, h_row = 0, s_row = 0, d_row = 0;  // bytes per row, per plane
    size_t off_q = 0, off_h = 0, off_s = 0, off_d = 0;  // plane offsets in the allocation
    size_t off_st = 0;  // Q4K / Q6K: the s plane again, tiled
    size_t off_dt = 0;  // Q6K: the d plane again, tiled by super-block pairs
    size_t bytes = 0;
};

// Plain-pointer view passed to kernels by value.
struct WView {
    const uint8_t* q;
    const uint8_t* h;
    const uint8_t* s;
    const uint8_t* d;
    const uint8_t* st;  // Q4K / Q6K: tiled copy of the s plane
    const uint8_t* dt;  // Q6K: tiled copy of the d plane (4 bytes = a super-block pair)
    uint32_t q_row, h_row, s_row, d_row;
    uint32_t n, k, nb;
    uint32_t dtype;
};

// ---------------------------------------------------------------------------
// Quantized activation workspace (private layout): one image per activation
// row, row_bytes apart, byte-identical to what the matvec kernels keep in LDS.
//   [0, K)             q8; chunk c's bytes 0-15 at c*16, bytes 16-31 at K/2 + c*16
//                      (lane-consecutive chunks are byte-consecutive in each half)
//   [K, K + K/8)       int32 per chunk: Q8K bsum[2c] | bsum[2c+1] << 16, Q8_0 block sum
//   [K + K/8, ...)     f32 scale per block (K/256 blocks for Q8K, K/32 for Q8_0)
// ---------------------------------------------------------------------------
struct ActImg {
    uint32_t k, s_off, d_off, row_bytes;
};

__host__ __device__ inline ActImg act_img(uint32_t k, bool kquant) {
    ActImg A;
    A.k = k;
    A.s_off = k;
    A.d_off = k + k / 8;
    const uint32_t end = A.d_off + (kquant ? k / 64 : k / 8);
    A.row_bytes = (end + 15u) & ~15u;
    return A;
}

// Byte offset of activation element e (0..K-1) inside the q8 part of an image.
__host__ __device__ inline uint32_t act_q_off(uint32_t k, uint32_t e) {
    const uint32_t c = e >> 5, o = e & 31;
    return (o >> 4) * (k / 2) + c * 16 + (o & 15);
}

// Row-tiled copy of a Q8K image, written beside it when the prefill kernel
// may read it: rows in blocks of 64 (the last block padded), and within a
// block every piece one DMA instruction of the prefill kernel fetches is
// 1 KiB (or 256 B) of consecutive bytes, lane i's 16 (or 4) at i * 16 (i * 4):
//   quants  [rb][stage = 64 K][ks][h][row 64][16]: chunk 2*stage+ks, bytes 16h..16h+15
//   d       [rb][sb][row 64] f32
//   bsums   [rb][sb][row / 32][half][row % 32][16]: int16 bsums 8*half..8*half+7
//   xmin    [rb][sb][row / 32][half][row % 32][16]: the Q4K min-term operand of
//           sub-blocks 4*half..4*half+3, v_j = -d * (bsum[2j] + bsum[2j+1]),
//           as 4 bf16 high parts then 4 bf16 remainders (v - hi)
struct TileImg {
    uint32_t rbs = 0;  // 64-row blocks
    size_t d_off = 0, s_off = 0, x_off = 0, bytes = 0;
};

__host__ __device__ inline TileImg tile_img(size_t m, uint32_t k) {
    TileImg T;
    T.rbs = (uint32_t)((m + 63) / 64);
    const size_t nsb = k / 256;
    T.d_off = (size_t)T.rbs * 64 * k;
    T.s_off = T.d_off + (size_t)T.rbs * nsb * 256;
    T.x_off = T.s_off + (size_t)T.rbs * nsb * 2048;
    T.bytes = T.x_off + (size_t)T.rbs * nsb * 2048;
    return T;
}

struct ALayout {
    uint32_t act_dtype = 0;
    size_t m = 0, k = 0, bytes = 0;
    ActImg img{};
    bool tiled = false;  // a TileImg follows the row images at tile_off
    size_t tile_off = 0;
    TileImg tile{};
};

struct AView {
    const uint8_t* img;
    uint32_t m, k;
    ActImg A;
    const uint8_t* tile;  // null unless the layout is tiled
    TileImg T;
};

// Weights that share one activation row in a decode launch (matvec
// kernels, m == 1): the row spaces of up to kMaxGroup weights of one dtype
// and K laid end to end, each row's output to its own weight's destination;
// or (gate) two weights of one shape combined as silu(x . w0) * (x . w1).
constexpr int kMaxGroup = 3;
struct WGroup {
    WView w[kMaxGroup];
    float* y[kMaxGroup];
    uint32_t row_end[kMaxGroup];  // cumulative row counts
    uint32_t count;
    uint32_t rows;  // rows of the row space (gate: n)
};

bool weight_layout(uint32_t dtype, size_t n, size_t k, WLayout* out, std::string* err);
ALayout act_layout(uint32_t weight_dtype, size_t m, size_t k, int forced_route);
uint32_t vec_dot_type(uint32_t weight_dtype);
size_t type_size(uint32_t dtype);
size_t block_size(uint32_t dtype);

inline WView make_wview(const WLayout& L, const void* base) {
    const uint8_t* b = static_cast<const uint8_t*>(base);
    WView v;
    v.q = b + L.off_q;
    v.h = b + L.off_h;
    v.s = b + L.off_s;
    v.d = b + L.off_d;
    v.st = b + L.off_st;
    v.dt = b + L.off_dt;
    v.q_row = (uint32_t)L.q_row;
    v.h_row = (uint32_t)L.h_row;
    v.s_row = (uint32_t)L.s_row;
    v.d_row = (uint32_t)L.d_row;
    v.n = (uint32_t)L.n;
    v.k = (uint32_t)L.k;
    v.nb = (uint32_t)L.nb;
    v.dtype = L.dtype;
    return v;
}

inline AView make_aview(const ALayout& L, const void* base) {
    AView v;
    v.img = static_cast<const uint8_t*>(base);
    v.m = (uint32_t)L.m;
    v.k = (uint32_t)L.k;
    v.A = L.img;
    v.tile = L.tiled ? v.img + L.tile_off : nullptr;
    v.T = L.tile;
    return v;
}

// Raises a kernel's dynamic LDS limit to `bytes` on the current device, once
// per (kernel, device); safe to call from several host threads.
hipError_t set_max_lds(const void* kernel, int bytes);

// ---------------------------------------------------------------------------
// Launchers (each returns hipSuccess or the first HIP error).
// ---------------------------------------------------------------------------
// k_repack.hip
hipError_t launch_repack(const WLayout& L, const void* gguf_dev, void* dst_dev, hipStream_t s);
hipError_t launch_unrepack(const WLayout& L, const void* src_dev, void* gguf_dev, hipStream_t s);
hipError_t launch_dequant(const WLayout& L, const void* src_dev, float* y, hipStream_t s);
// k_quantize.hip
hipError_t launch_quantize_act(const ALayout& A, const float* x, void* ws, hipStream_t s);
hipError_t launch_quantize_act_blocks(uint32_t act_dtype, size_t m, size_t k, const float* x,
                                      void* blocks, hipStream_t s);
hipError_t launch_weight_from_float(uint32_t dtype, size_t nblocks, const float* x, void* gguf,
                                    hipStream_t s);
// k_matvec.hip
hipError_t launch_matvec(const WView& w, const AView& a, size_t m, float* y, hipStream_t s);
// Quantizes the f32 rows inside the kernel (no workspace).  `one_shot`: at
// m == 1 the one-shot group kernel (one wavefront per weight row; small
// weights), else the persistent matvec kernel.
constexpr int kFusedPersistent = 1, kFusedOneShot = 2;
hipError_t launch_matvec_fused(const WView& w, const float* x, size_t m, float* y, hipStream_t s,
                               bool one_shot);
// m == 1 over a weight group (gate: silu(x . w0) * (x . w1)); hipErrorNotSupported
// for a shape the grouped kernel does not take
hipError_t launch_matvec_group(const WGroup& g, const float* x, bool gate, hipStream_t s);
// g[i] = silu(g[i]) * u[i]
hipError_t launch_silu_mul(float* g, const float* u, size_t count, hipStream_t s);
hipError_t launch_block_ints(const WView& w, const AView& a, size_t m,
                             int32_t* out, hipStream_t s);
// k_mfma.hip
bool mfma_supported(uint32_t dtype, size_t m, size_t n, size_t k);
uint32_t mfma_splits(size_t m, size_t n, size_t k);
bool skinny_supported(uint32_t dtype, size_t m, size_t n, size_t k);
uint32_t skinny_splits(size_t m, size_t n, size_t k);
hipError_t launch_skinny(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                         hipStream_t s);
// y[i] = sum over z < splits of partial[z * count + i], in z order
hipError_t launch_sum_splits(const float* partial, size_t count, uint32_t splits, float* y, hipStream_t s);
// Split-K sums of up to kMaxGroup partial regions (region t: [split][cnt[t]]
// floats at part[t]) into y[t]; `silu` (two regions of one size): y[0] =
// silu(sum 0) * sum 1 with silu(s) = s / (1 + exp(0 - s)).
struct SumGroup {
    const float* part[kMaxGroup];
    float* y[kMaxGroup];
    size_t cnt[kMaxGroup];
    uint32_t count;
};
hipError_t launch_sum_group(const SumGroup& S, uint32_t splits, bool silu, hipStream_t s);
// The skinny kernel over a group of weights of one dtype and K (G.w, G.y,
// G.count; G.row_end unused) in one launch; `silu` (two weights of one
// shape) writes silu(x . w0) * (x . w1) to G.y[0] and needs `partial`.
// `next` (silu only): also quantize the result into the Q8K activation
// image `next_img` of layout *next (the down projection's input) in the
// split-sum launch.
hipError_t launch_skinny_group(const WGroup& G, const AView& a, size_t m, uint32_t splits, float* partial, bool silu,
                               hipStream_t s, const ALayout* next = nullptr, void* next_img = nullptr);
hipError_t launch_sum_silu_quant(const SumGroup& S, uint32_t splits, size_t m, size_t n, const ALayout& L,
                                 void* img, hipStream_t s);
hipError_t launch_mfma(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                       hipStream_t s);
// k_prefill.hip: the Q4K matrix-core kernel with in-register weight expansion
bool prefill_supported(uint32_t dtype, size_t m, size_t n, size_t k);
uint32_t prefill_splits(size_t m, size_t n, size_t k);
hipError_t launch_prefill(const WView& w, const AView& a, size_t m, uint32_t splits, float* y, float* partial,
                          hipStream_t s);

}  // namespace xnq
