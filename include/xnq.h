/*
 * xnq.h -- C ABI of libxnq, the MI355X (gfx950) GGUF quantized-matmul backend.
 *
 * Each entry point replaces one piece of xn's quantized-tensor contract
 * (gradium-ai/xn, xn-core/src/quantized/mod.rs) with a device-resident
 * equivalent.  All pointers named *_dev are device (HBM) pointers, all sizes
 * are element or byte counts, `stream` is a hipStream_t (NULL = the null
 * stream).  No torch or C++ types cross this boundary.
 *
 * Errors: every call returns an xnq_status; on failure a message describing
 * the problem is available from xnq_last_error() on the calling thread
 * (mirrors xn's Result<_, Error> + bail!, xn-core/src/error.rs:9-60).
 *
 * Threading: a qtensor is read-only after upload, so concurrent matmul calls
 * on one qtensor from several threads/streams are safe (xn's
 * `QuantizedType: Send + Sync`, mod.rs:199).
 */
#ifndef XNQ_H
#define XNQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    XNQ_OK = 0,
    XNQ_ERR_INVALID = 1,     /* shape / size / argument error (xn: bail!) */
    XNQ_ERR_UNSUPPORTED = 2, /* dtype has no device implementation */
    XNQ_ERR_HIP = 3,         /* a HIP runtime call failed */
    XNQ_ERR_OOM = 4          /* device allocation failed */
} xnq_status;

/* GGML dtype ids, identical to GgmlDType::to_u32 (mod.rs:119-137). */
enum {
    XNQ_F32 = 0,
    XNQ_F16 = 1,
    XNQ_Q4_0 = 2,
    XNQ_Q4_1 = 3,
    XNQ_Q5_0 = 6,
    XNQ_Q5_1 = 7,
    XNQ_Q8_0 = 8,
    XNQ_Q8_1 = 9,
    XNQ_Q2K = 10,
    XNQ_Q3K = 11,
    XNQ_Q4K = 12,
    XNQ_Q5K = 13,
    XNQ_Q6K = 14,
    XNQ_Q8K = 15
};

typedef struct xnq_qtensor xnq_qtensor;

/* Message of the last failed call on this thread ("" if none). */
const char* xnq_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int xnq_abi_version(void);

/* Bytes per block / elements per block of a GGML dtype, 0 if unknown.
 * Replaces GgmlDType::type_size / block_size (mod.rs:160-195). */
size_t xnq_type_size(uint32_t dtype);
size_t xnq_block_size(uint32_t dtype);

/* Upload a GGUF tensor of n rows x k columns whose canonical block bytes sit
 * in host memory, and repack it on the device.  Replaces the
 * `ggml_file::qtensor_from_ggml` -> `QTensor::new(QStorage::Cpu(..))` load
 * (ggml_file.rs:128-163, mod.rs:32-34) with a device storage; the GGUF bytes
 * themselves are not changed.  Synchronises `stream` before returning so the
 * host buffer may be released. */
xnq_status xnq_qtensor_upload(int device, uint32_t dtype, const void* gguf_blocks_host,
                              size_t n, size_t k, void* stream, xnq_qtensor** out);

/* As xnq_qtensor_upload, for canonical GGUF block bytes already in device
 * memory (stream ordered, no synchronisation). */
xnq_status xnq_qtensor_upload_device(int device, uint32_t dtype, const void* gguf_blocks_dev,
                                     size_t n, size_t k, void* stream, xnq_qtensor** out);

/* Quantize an n x k f32 weight that lives in device memory.  Replaces
 * QTensor::quantize_f32 (mod.rs:283-303), i.e. the per-dtype
 * GgmlType::from_float (k_quants.rs:235-270, 345-377, 442-476, 546-583, 636-661,
 * 951-1011, 1170-1236, 1418-1473, 1608-1679, 1801-1871) for every device dtype;
 * the blocks produced are byte-identical to the CPU quantizer's. */
xnq_status xnq_qtensor_quantize(int device, uint32_t dtype, const float* src_dev, size_t n,
                                size_t k, void* stream, xnq_qtensor** out);

/* Release a qtensor and its device memory (xn: Drop). */
void xnq_qtensor_free(xnq_qtensor* qt);

/* Introspection (QTensor::dtype / shape / storage_size_in_bytes, mod.rs:305-331).
 * storage bytes = canonical GGUF size; device bytes = what the repacked copy
 * occupies in HBM. */
uint32_t xnq_qtensor_dtype(const xnq_qtensor* qt);
size_t xnq_qtensor_rows(const xnq_qtensor* qt);
size_t xnq_qtensor_cols(const xnq_qtensor* qt);
int xnq_qtensor_device(const xnq_qtensor* qt);
size_t xnq_qtensor_storage_size(const xnq_qtensor* qt);
size_t xnq_qtensor_device_bytes(const xnq_qtensor* qt);

/* dst[m x n] = lhs[m x k] . W^T, with lhs quantized to the weight's vec-dot
 * type first.  Replaces QTensor::matmul_t / QuantizedType::matmul_t /
 * k_quants::matmul (mod.rs:334-339, 221-223; k_quants.rs:1996-2011).  The
 * route is chosen from m and the shape: a wavefront-per-row matvec for small
 * m (Q4_K / Q6_K up to 4 rows, up to 2 for K >= 4096 and 2048 < N <= K),
 * the small-batch int8 MFMA kernel up to 64 rows, the
 * tiled int8 MFMA kernel for prefill-sized m.  Validates what xn validates:
 * mkn against the weight shape (repack.rs:203-215) and m*k == lhs length is
 * the caller's contract.  Stream ordered; allocates its activation scratch
 * stream-ordered (hipMallocAsync). */
xnq_status xnq_qtensor_matmul_t(const xnq_qtensor* qt, size_t m, size_t k, size_t n,
                                const float* lhs_dev, float* dst_dev, void* stream);

/* matmul_t with caller-owned scratch (no allocation inside): workspace_dev
 * holds at least xnq_qtensor_matmul_t_workspace_size(qt, m) bytes, which is
 * 0 on the fused decode route (m == 1 with K <= 4096, or on weights of up
 * to 6144 x 4096 elements: the row quantized in LDS by the matvec kernel;
 * workspace_dev may then be NULL).  Same contract as xnq_qtensor_matmul_t
 * (QTensor::matmul_t, mod.rs:334-339; k_quants::matmul, k_quants.rs:1996-2011). */
size_t xnq_qtensor_matmul_t_workspace_size(const xnq_qtensor* qt, size_t m);
xnq_status xnq_qtensor_matmul_t_ws(const xnq_qtensor* qt, size_t m, size_t k, size_t n,
                                   const float* lhs_dev, void* workspace_dev, size_t workspace_bytes,
                                   float* dst_dev, void* stream);

/* matmul_t that allocates nothing: no reference counterpart.  For callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same contract and
 * results as xnq_qtensor_matmul_t / xnq_qtensor_matmul_t_ws (the same
 * kernels), with the workspace taken from a static device array of
 * XNQ_NOALLOC_SCRATCH_BYTES per GPU that the library holds until the
 * process ends.  Fails with XNQ_ERR_INVALID when
 * xnq_qtensor_matmul_t_workspace_size(qt, m) exceeds it (at K = 4096 that
 * is past about 3000 rows).  Every call on one GPU uses that GPU's one
 * array: calls that overlap on one GPU (different streams, or host threads
 * without ordering between them) race and must be serialised by the
 * caller, e.g. by issuing them on one stream. */
#define XNQ_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
xnq_status xnq_qtensor_matmul_t_noalloc(const xnq_qtensor* qt, size_t m, size_t k, size_t n,
                                        const float* lhs_dev, float* dst_dev, void* stream);

/* Decode-step groups (no reference entry point of their own: they compute
 * what two or three QMatMul calls on one activation compute, in one launch
 * for m == 1).
 *
 * silu_gate: dst[m x n] = silu(lhs . gate^T) * (lhs . up^T), the SwiGLU of
 * llama.rs:258-264 (Mlp::forward) with silu(s) = s / (1 + exp(0 - s))
 * (cpu_backend.rs:354-356); gate and up have one shape.  m == 1 with both on
 * the one-launch route (K <= 4096 at any N, or weights of up to 6144 x 4096
 * elements) and K <= 10240 is one kernel and needs no workspace; on the
 * small-batch MFMA route (Q4_K/Q6_K, 3 <= m <= 64 for the 4096 -> 14336
 * pair) one quantize, one launch over both weights and one split-sum that
 * applies the SiLU-multiply;
 * otherwise one activation quantize serves both products (matmul_preq
 * each), then a SiLU-multiply kernel, with workspace for the second product.
 *
 * group: dsts[i][m x n_i] = lhs . qts[i]^T for up to 3 weights of one dtype
 * and K (the q, k, v projections of llama.rs:156-158); m == 1 on the
 * one-launch route is one kernel over the joined rows; on the small-batch
 * MFMA route (from m = 2 for a q/k/v-sized group) one quantize and one
 * launch over the joined column tiles, plus a split-sum where K is split
 * across workgroups; otherwise weights of one dtype and K share one activation
 * quantize (matmul_preq each), and other groups take one matmul_t_ws per
 * weight.  Workspace sizes are 0 when the
 * single-kernel route applies. */
size_t xnq_matmul_t_silu_gate_workspace_size(const xnq_qtensor* gate, const xnq_qtensor* up, size_t m);
xnq_status xnq_matmul_t_silu_gate(const xnq_qtensor* gate, const xnq_qtensor* up, size_t m, size_t k, size_t n,
                                  const float* lhs_dev, void* workspace_dev, size_t workspace_bytes,
                                  float* dst_dev, void* stream);
size_t xnq_matmul_t_group_workspace_size(const xnq_qtensor* const* qts, size_t count, size_t m);
xnq_status xnq_matmul_t_group(const xnq_qtensor* const* qts, size_t count, size_t m, size_t k,
                              const float* lhs_dev, float* const* dsts_dev, void* workspace_dev,
                              size_t workspace_bytes, void* stream);

/* The whole SwiGLU MLP of llama.rs:236-264 (Mlp::forward): h[m x f] =
 * silu(lhs . gate^T) * (lhs . up^T) as silu_gate above, then dst[m x n] =
 * h . down^T with down of shape (n, f).  Both results are written.  With
 * gate/up on the small-batch MFMA route and a K-quant down weight, the
 * gate/up split-sum also quantizes h for the down projection (one launch
 * fewer); otherwise it is silu_gate followed by matmul_t_ws.  The results are
 * the bits those two calls produce. */
size_t xnq_mlp_t_workspace_size(const xnq_qtensor* gate, const xnq_qtensor* up, const xnq_qtensor* down, size_t m);
xnq_status xnq_mlp_t(const xnq_qtensor* gate, const xnq_qtensor* up, const xnq_qtensor* down, size_t m, size_t k,
                     size_t f, const float* lhs_dev, void* workspace_dev, size_t workspace_bytes, float* h_dev,
                     float* dst_dev, void* stream);

/* The two halves of matmul_t, for callers that keep the quantized
 * activation around or manage the scratch memory themselves
 * (k_quants.rs:2014-2026 quantize_lhs, then T::matmul).  The workspace
 * layout is private to the library.  xnq_lhs_workspace_size gives the bytes
 * quantize_lhs writes (the quantized activation image);
 * xnq_qtensor_workspace_size adds the scratch matmul_preq may use on this
 * weight (split-K partial sums of the MFMA route).  matmul_preq is told the
 * workspace's size and uses no scratch it does not fit. */
size_t xnq_lhs_workspace_size(uint32_t weight_dtype, size_t m, size_t k);
size_t xnq_qtensor_workspace_size(const xnq_qtensor* qt, size_t m);
xnq_status xnq_quantize_lhs(uint32_t weight_dtype, size_t m, size_t k, const float* lhs_dev,
                            void* workspace_dev, void* stream);
xnq_status xnq_qtensor_matmul_preq(const xnq_qtensor* qt, size_t m, size_t k, size_t n,
                                   const void* workspace_dev, size_t workspace_bytes, float* dst_dev,
                                   void* stream);

/* Force a route for matmul_t / matmul_preq (testing and benchmarking):
 * 0 = automatic, 1 = matvec kernels, 2 = tiled int8-MFMA (prefill) kernel,
 * 3 = skinny int8-MFMA kernel (m <= 64).  Process wide. */
xnq_status xnq_set_route(int route);

/* Dequantize into elem_count f32 values (QTensor::dequantize /
 * GgmlType::to_float, mod.rs:316-318). */
xnq_status xnq_qtensor_dequantize(const xnq_qtensor* qt, float* dst_dev, size_t elem_count,
                                  void* stream);

/* Canonical GGUF block bytes of the tensor (QuantizedType::raw_data,
 * mod.rs:206-214): undoes the device repack.  Copies into host memory and
 * synchronises. */
xnq_status xnq_qtensor_raw_data(const xnq_qtensor* qt, void* host_dst, size_t cap, void* stream);

/* Quantize m rows of k f32 activations to canonical BlockQ8_0
 * (act_dtype = XNQ_Q8_0, k_quants.rs:636-661) or BlockQ8K
 * (act_dtype = XNQ_Q8K, k_quants.rs:1942-1979) blocks in device memory.
 * Bit-identical to the CPU quantizer. */
xnq_status xnq_quantize_act_blocks(uint32_t act_dtype, size_t m, size_t k, const float* src_dev,
                                   void* blocks_dev, void* stream);

/* Integer parts of every per-block dot product the matvec kernel forms, for
 * bit-exactness checks against the CPU vec_dot (k_quants.rs:287-304,
 * 316-343, 419-440, 513-544, 677-691, 899-948, 1071-1152, 1337-1416,
 * 1524-1605, 1743-1798).  workspace_dev comes from xnq_quantize_lhs.
 * out_dev receives int32 [m][n][k/256 or k/32][2]:
 *   Q4_0, Q8_0, Q4_1, Q5_1: [block integer sum, 0]
 *   Q5_0:       [sum (q5-16)*q8, 0]
 *   Q2K:        [sum_g (sc_g & 15) * sum q2*q8, sum_g (sc_g >> 4) * bsum_g]
 *   Q3K:        [sum_g (sc_g - 32) * sum q3*q8, 0]   (q3 in -4..3)
 *   Q4K, Q5K:   [sum_j sc_j * sum q*q8, sum_j m_j * bsum_j]
 *   Q6K:        [sum_j sc_j * sum (q6-32)*q8, 0] */
xnq_status xnq_qtensor_block_ints(const xnq_qtensor* qt, size_t m, const void* workspace_dev,
                                  int32_t* out_dev, void* stream);

/* Stream capture into a replayable graph (xn's Device::capture_begin /
 * capture_end / CaptureGraph::launch, cuda_backend/mod.rs:251-283): every
 * launch the library makes on `stream` between begin and end is recorded,
 * not run; xnq_graph_launch replays it with the same device pointers.  Inside
 * a capture use the entry points that allocate nothing: matmul_t_ws,
 * quantize_lhs + matmul_preq, silu_gate / group with their workspaces, and
 * matmul_t on the fused decode route; matmul_t fails with XNQ_ERR_INVALID
 * where it would allocate.  A failed capture is discarded with
 * xnq_capture_abort. */
typedef struct xnq_graph xnq_graph;
xnq_status xnq_capture_begin(void* stream);
xnq_status xnq_capture_end(void* stream, xnq_graph** out);
void xnq_capture_abort(void* stream);
xnq_status xnq_graph_launch(const xnq_graph* g, void* stream);
void xnq_graph_free(xnq_graph* g);

#ifdef __cplusplus
}
#endif

#endif /* XNQ_H */
