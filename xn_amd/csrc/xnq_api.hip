// The C ABI of libxnq (include/xnq.h): device qtensors, validation and the
// batch-size routing of matmul_t.  Kernels live in k_*.hip.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "xnq_internal.h"

struct xnq_qtensor {
    int device;
    xnq::WLayout L;
    void* buf;
};

namespace xnq {

namespace {

thread_local std::string g_err;
std::atomic<int> g_route{0};

xnq_status fail(xnq_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return st;
}

xnq_status hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? XNQ_ERR_OOM : XNQ_ERR_HIP, "%s: %s", what,
                hipGetErrorString(e));
}

// Makes `dev` current for the scope and restores the caller's device.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

const char* dtype_name(uint32_t dt) {
    switch (dt) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    case 9: return "Q8_1";
    case 10: return "Q2K";
    case 11: return "Q3K";
    case 12: return "Q4K";
    case 13: return "Q5K";
    case 14: return "Q6K";
    case 15: return "Q8K";
    case 30: return "BF16";
    }
    return nullptr;
}

bool device_dtype(uint32_t dt) {
    return dt == XNQ_Q4_0 || dt == XNQ_Q8_0 || dt == XNQ_Q4K || dt == XNQ_Q6K || is_raw_layout(dt);
}

// Validation shared by the weight constructors (mod.rs:262-274 check_shape,
// mod.rs:114 unknown dtype, lib.rs:284-287 unsupported on the device).
xnq_status check_weight(uint32_t dtype, size_t n, size_t k) {
    const char* name = dtype_name(dtype);
    if (!name) return fail(XNQ_ERR_INVALID, "unknown dtype for tensor %u", dtype);
    if (!device_dtype(dtype))
        return fail(XNQ_ERR_UNSUPPORTED, "%s quantization is not supported on the HIP device", name);
    const size_t bs = block_size(dtype);
    if (k == 0 || k % bs != 0)
        return fail(XNQ_ERR_INVALID,
                    "quantized tensor must have their last dim divisible by block size [%zu, %zu] %zu",
                    n, k, bs);
    // kernels address every plane with 32-bit byte offsets; the largest plane
    // holds at most type_size bytes per block (raw layouts: the padded
    // stride), over the rows (Q4K / Q6K: padded to a multiple of 128 for
    // their tiled header copies)
    const size_t rows = (dtype == XNQ_Q4K || dtype == XNQ_Q6K) ? (n + 127) / 128 * 128 : n;
    const size_t per_block = is_raw_layout(dtype) ? raw_stride(dtype) : type_size(dtype);
    if (n > 0xffffffffull || k > 0x7fffffffull || rows * (k / bs) * per_block >= (1ull << 32))
        return fail(XNQ_ERR_INVALID, "tensor too large for the device layout [%zu, %zu]", n, k);
    return XNQ_OK;
}

xnq_status alloc_qtensor(int device, uint32_t dtype, size_t n, size_t k, xnq_qtensor** out) {
    WLayout L;
    std::string err;
    if (!weight_layout(dtype, n, k, &L, &err)) return fail(XNQ_ERR_INVALID, "%s", err.c_str());
    void* buf = nullptr;
    hipError_t e = hipMalloc(&buf, L.bytes ? L.bytes : kAlign);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(qtensor)");
    xnq_qtensor* qt = new xnq_qtensor;
    qt->device = device;
    qt->L = L;
    qt->buf = buf;
    *out = qt;
    return XNQ_OK;
}

}  // namespace

size_t type_size(uint32_t dt) {
    switch (dt) {
    case XNQ_F32: return 4;
    case XNQ_F16: return 2;
    case XNQ_Q4_0: return 18;
    case XNQ_Q4_1: return 20;
    case XNQ_Q5_0: return 22;
    case XNQ_Q5_1: return 24;
    case XNQ_Q8_0: return 34;
    case XNQ_Q8_1: return 36;
    case XNQ_Q2K: return 84;
    case XNQ_Q3K: return 110;
    case XNQ_Q4K: return 144;
    case XNQ_Q5K: return 176;
    case XNQ_Q6K: return 210;
    case XNQ_Q8K: return 292;
    }
    return 0;
}

size_t block_size(uint32_t dt) {
    switch (dt) {
    case XNQ_F32:
    case XNQ_F16: return 1;
    case XNQ_Q4_0:
    case XNQ_Q4_1:
    case XNQ_Q5_0:
    case XNQ_Q5_1:
    case XNQ_Q8_0:
    case XNQ_Q8_1: return 32;
    case XNQ_Q2K:
    case XNQ_Q3K:
    case XNQ_Q4K:
    case XNQ_Q5K:
    case XNQ_Q6K:
    case XNQ_Q8K: return 256;
    }
    return 0;
}

// k_quants.rs VecDotType of each weight type.  Q8_1 (Q4_1, Q5_1) keeps the
// Q8_0 quants and scale; its f16 s is derived from them in the kernels.
uint32_t vec_dot_type(uint32_t wdt) {
    if (is_kquant(wdt)) return XNQ_Q8K;
    if (wdt == XNQ_Q4_1 || wdt == XNQ_Q5_1) return XNQ_Q8_1;
    return XNQ_Q8_0;
}

bool weight_layout(uint32_t dtype, size_t n, size_t k, WLayout* out, std::string* err) {
    WLayout L;
    L.dtype = dtype;
    L.n = n;
    L.k = k;
    const size_t bs = block_size(dtype);
    if (!bs || k % bs) {
        *err = "bad weight shape";
        return false;
    }
    L.nb = k / bs;
    switch (dtype) {
    case XNQ_Q8_0: L.q_row = L.nb * 32; L.d_row = L.nb * 2; break;
    case XNQ_Q4_0: L.q_row = L.nb * 16; L.d_row = L.nb * 2; break;
    case XNQ_Q4K: L.q_row = L.nb * 128; L.s_row = L.nb * 16; break;
    case XNQ_Q6K:
        // d rows padded to 4 bytes: super-block sb's f16 is half (sb & 1) of dword sb / 2
        L.q_row = L.nb * 128; L.h_row = L.nb * 64; L.s_row = L.nb * 16; L.d_row = ((L.nb + 1) & ~size_t(1)) * 2;
        break;
    default:
        if (!is_raw_layout(dtype)) {
            *err = "unsupported dtype";
            return false;
        }
        L.q_row = L.nb * raw_stride(dtype);
    }
    // Q4K / Q6K: the tiled copies pad their rows to a multiple of 128
    const size_t tiled_rows = (n + kTileRows - 1) / kTileRows * kTileRows;
    size_t off = 0;
    L.off_q = off;
    off = align_up(off + L.q_row * n);
    L.off_h = off;
    off = align_up(off + L.h_row * n);
    L.off_s = off;
    off = align_up(off + L.s_row * n);
    L.off_d = off;
    off = align_up(off + L.d_row * n);
    L.off_st = L.off_s;
    L.off_dt = L.off_d;
    if (dtype == XNQ_Q4K || dtype == XNQ_Q6K) {
        L.off_st = off;
        off = align_up(off + L.s_row * tiled_rows);
    }
    if (dtype == XNQ_Q6K) {
        L.off_dt = off;
        off = align_up(off + L.d_row * tiled_rows);
    }
    L.bytes = off;
    *out = L;
    return true;
}

hipError_t set_max_lds(const void* kernel, int bytes) {
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({kernel, dev})) return hipSuccess;
    e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done.insert({kernel, dev});
    return e;
}

static size_t env_size(const char* name, size_t dflt) {
    const char* e = getenv(name);
    return e ? (size_t)strtoull(e, nullptr, 10) : dflt;
}

size_t skinny_max_rows() {
    static const size_t v = env_size("XNQ_SKINNY_MAX_ROWS", 64);
    return v;
}

// Single Q4_K weights take the prefill kernel (k_prefill.hip, 64-row tiles)
// above this many rows: 4096 -> 14336, graph steps, µs, skinny against
// prefill: m = 32 17.4 / 19.9, 40 24.0 / 20.9, 48 24.6 / 21.7, 56 24.4 /
// 22.0, 64 25.8 / 23.2.  q/k/v groups and gate/up pairs keep the skinny
// kernel's one launch over all their weights.
static size_t skinny_q4k_max_rows() {
    static const size_t v = env_size("XNQ_SKINNY_Q4K_MAX_ROWS", 32);
    return v;
}
static bool q4k_prefill_early(uint32_t dtype, size_t m, size_t k) {
    return dtype == XNQ_Q4K && m > skinny_q4k_max_rows() && m <= skinny_max_rows() &&
           prefill_supported(dtype, m, 0, k);
}

// Whether the prefill (tiled MFMA) route can be taken for m activation rows,
// in which case the activation quantizer also writes the row-tiled image.
// It depends on m and the forced route, not on n, so xnq_quantize_lhs (which
// has no n) and the matmul agree.  `forced` is the route override as read
// once at the public entry point, so sizing and launching within one call
// always agree; between separate quantize_lhs and matmul_preq calls
// xnq_set_route must not change.
static bool tiled_act(uint32_t weight_dtype, size_t m, size_t k, int forced) {
    if (forced == 1 || forced == 3) return false;
    return mfma_supported(weight_dtype, m, 0, k) &&
           (forced == 2 || m > skinny_max_rows() || q4k_prefill_early(weight_dtype, m, k));
}

ALayout act_layout(uint32_t weight_dtype, size_t m, size_t k, int forced) {
    ALayout L;
    L.act_dtype = vec_dot_type(weight_dtype);
    L.m = m;
    L.k = k;
    L.img = act_img((uint32_t)k, L.act_dtype == XNQ_Q8K);  // Q8_1 uses the Q8_0 image
    L.bytes = align_up(m * L.img.row_bytes);
    if (tiled_act(weight_dtype, m, k, forced)) {
        L.tiled = true;
        L.tile_off = L.bytes;
        L.tile = tile_img(m, (uint32_t)k);
        L.bytes = align_up(L.tile_off + L.tile.bytes);
    }
    return L;
}

}  // namespace xnq

using namespace xnq;

extern "C" {

const char* xnq_last_error(void) { return g_err.c_str(); }

int xnq_abi_version(void) { return 5; }

size_t xnq_type_size(uint32_t dtype) { return type_size(dtype); }
size_t xnq_block_size(uint32_t dtype) { return block_size(dtype); }

xnq_status xnq_qtensor_upload_device(int device, uint32_t dtype, const void* gguf_blocks_dev,
                                     size_t n, size_t k, void* stream, xnq_qtensor** out) {
    if (!out) return fail(XNQ_ERR_INVALID, "null output pointer");
    *out = nullptr;
    xnq_status st = check_weight(dtype, n, k);
    if (st) return st;
    if (!gguf_blocks_dev && n) return fail(XNQ_ERR_INVALID, "null block pointer");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    xnq_qtensor* qt = nullptr;
    st = alloc_qtensor(device, dtype, n, k, &qt);
    if (st) return st;
    hipError_t e = launch_repack(qt->L, gguf_blocks_dev, qt->buf, (hipStream_t)stream);
    if (e != hipSuccess) {
        (void)hipFree(qt->buf);
        delete qt;
        return hip_fail(e, "repack");
    }
    *out = qt;
    return XNQ_OK;
}

xnq_status xnq_qtensor_upload(int device, uint32_t dtype, const void* gguf_blocks_host, size_t n,
                              size_t k, void* stream, xnq_qtensor** out) {
    if (!out) return fail(XNQ_ERR_INVALID, "null output pointer");
    *out = nullptr;
    xnq_status st = check_weight(dtype, n, k);
    if (st) return st;
    if (!gguf_blocks_host && n) return fail(XNQ_ERR_INVALID, "null block pointer");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    // Load time, not the hot path: a plain allocation and a blocking copy of
    // the (pageable) host bytes, then the repack on `stream`.
    hipStream_t s = (hipStream_t)stream;
    const size_t bytes = n * (k / block_size(dtype)) * type_size(dtype);
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, bytes ? bytes : kAlign);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(upload)");
    e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipMemcpy(tmp, gguf_blocks_host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(tmp);
        return hip_fail(e, "hipMemcpy(upload)");
    }
    st = xnq_qtensor_upload_device(device, dtype, tmp, n, k, stream, out);
    e = hipStreamSynchronize(s);
    (void)hipFree(tmp);
    if (st) return st;
    if (e != hipSuccess) {
        xnq_qtensor_free(*out);
        *out = nullptr;
        return hip_fail(e, "hipStreamSynchronize(upload)");
    }
    return XNQ_OK;
}

xnq_status xnq_qtensor_quantize(int device, uint32_t dtype, const float* src_dev, size_t n,
                                size_t k, void* stream, xnq_qtensor** out) {
    if (!out) return fail(XNQ_ERR_INVALID, "null output pointer");
    *out = nullptr;
    xnq_status st = check_weight(dtype, n, k);
    if (st) return st;
    if (!src_dev && n) return fail(XNQ_ERR_INVALID, "null source pointer");
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    const size_t nblocks = n * (k / block_size(dtype));
    void* tmp = nullptr;
    hipError_t e = hipMallocAsync(&tmp, nblocks ? nblocks * type_size(dtype) : kAlign, s);
    if (e != hipSuccess) return hip_fail(e, "hipMallocAsync(quantize)");
    e = launch_weight_from_float(dtype, nblocks, src_dev, tmp, s);
    if (e != hipSuccess) {
        (void)hipFreeAsync(tmp, s);
        return hip_fail(e, "quantize kernel");
    }
    st = xnq_qtensor_upload_device(device, dtype, tmp, n, k, stream, out);
    (void)hipFreeAsync(tmp, s);
    return st;
}

void xnq_qtensor_free(xnq_qtensor* qt) {
    if (!qt) return;
    DeviceGuard g(qt->device);
    (void)hipFree(qt->buf);
    delete qt;
}

uint32_t xnq_qtensor_dtype(const xnq_qtensor* qt) { return qt ? qt->L.dtype : 0; }
size_t xnq_qtensor_rows(const xnq_qtensor* qt) { return qt ? qt->L.n : 0; }
size_t xnq_qtensor_cols(const xnq_qtensor* qt) { return qt ? qt->L.k : 0; }
int xnq_qtensor_device(const xnq_qtensor* qt) { return qt ? qt->device : -1; }
size_t xnq_qtensor_storage_size(const xnq_qtensor* qt) {
    return qt ? qt->L.n * qt->L.nb * type_size(qt->L.dtype) : 0;
}
size_t xnq_qtensor_device_bytes(const xnq_qtensor* qt) { return qt ? qt->L.bytes : 0; }

size_t xnq_lhs_workspace_size(uint32_t weight_dtype, size_t m, size_t k) {
    if (!device_dtype(weight_dtype)) return 0;
    return act_layout(weight_dtype, m, k, g_route.load()).bytes;
}

static xnq_status check_lhs(uint32_t weight_dtype, size_t k) {
    const uint32_t vt = vec_dot_type(weight_dtype);
    const size_t bs = block_size(vt);
    if (k % bs != 0)
        return fail(XNQ_ERR_INVALID, "quantize_row_%s: %zu is not divisible by %zu",
                    vt == XNQ_Q8K ? "q8k" : "q8_0", k, bs);
    return XNQ_OK;
}

static xnq_status quantize_lhs_impl(uint32_t weight_dtype, size_t m, size_t k, const float* lhs_dev,
                                    void* workspace_dev, void* stream, int forced) {
    if (!device_dtype(weight_dtype))
        return fail(XNQ_ERR_UNSUPPORTED, "no device activation quantizer for dtype %u", weight_dtype);
    xnq_status st = check_lhs(weight_dtype, k);
    if (st) return st;
    if (m == 0) return XNQ_OK;
    if (!lhs_dev || !workspace_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    const ALayout A = act_layout(weight_dtype, m, k, forced);
    hipError_t e = launch_quantize_act(A, lhs_dev, workspace_dev, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quantize_lhs");
    return XNQ_OK;
}

xnq_status xnq_quantize_lhs(uint32_t weight_dtype, size_t m, size_t k, const float* lhs_dev,
                            void* workspace_dev, void* stream) {
    return quantize_lhs_impl(weight_dtype, m, k, lhs_dev, workspace_dev, stream, g_route.load());
}

xnq_status xnq_set_route(int route) {
    if (route < 0 || route > 3) return fail(XNQ_ERR_INVALID, "route must be 0, 1, 2 or 3");
    g_route.store(route);
    return XNQ_OK;
}

static xnq_status check_mkn(const xnq_qtensor* qt, size_t m, size_t k, size_t n) {
    if (!qt) return fail(XNQ_ERR_INVALID, "null qtensor");
    if (k != qt->L.k || n != qt->L.n)
        return fail(XNQ_ERR_INVALID, "matmul_t: mkn (%zu, %zu, %zu) does not match weight [%zu, %zu]",
                    m, k, n, qt->L.n, qt->L.k);
    if (m > 0x7fffffffull) return fail(XNQ_ERR_INVALID, "m too large: %zu", m);
    // vec_dot_q4_1_q8_1 / q5_0_q8_0 / q5_1_q8_1 take pairs of blocks
    // (k_quants.rs:323-325, 413-415, 519-521)
    const uint32_t dt = qt->L.dtype;
    if ((dt == XNQ_Q4_1 || dt == XNQ_Q5_0 || dt == XNQ_Q5_1) && (k / 32) % 2)
        return fail(XNQ_ERR_INVALID, "vec_dot_%s_%s: %zu, nb is not divisible by 2",
                    dt == XNQ_Q4_1 ? "q4_1" : dt == XNQ_Q5_0 ? "q5_0" : "q5_1", dt == XNQ_Q5_0 ? "q8_0" : "q8_1", k);
    return XNQ_OK;
}

// Automatic routes (measured on MI355X):
//   m <= 4   matvec kernels (up to 8 rows per launch), except a group of
//            weights sharing one activation (q/k/v, gate/up) that joins at
//            least 6144 columns: skinny from m = 3, or from m = 2 when the
//            group joins at most 16384 columns (the wavefront-split kernel)
//   m <= 64  skinny int8-MFMA kernel for Q4K / Q6K
//   larger m tiled int8-MFMA prefill kernel
// Q8_0 / Q4_0 and the other dtypes always take the matvec kernels.
// XNQ_SKINNY_MIN_ROWS and XNQ_SKINNY_MAX_ROWS override the skinny range for
// tuning (read once per process); `forced` is xnq_set_route's override as
// read at the entry point; `group_n` is the joined width of a group (0 for a
// single weight).
enum Route { kMatvec, kSkinny, kMfma };

static Route pick_route(uint32_t dtype, size_t m, size_t n, size_t k, int forced, size_t group_n = 0) {
    static const size_t skinny_min = env_size("XNQ_SKINNY_MIN_ROWS", 0);
    const size_t skinny_max = skinny_max_rows();
    if (forced == 1) return kMatvec;
    if (forced == 2) return kMfma;
    if (forced == 3) return kSkinny;
    // measured crossovers (graph steps, µs, matvec against skinny): the
    // matvec kernels' cost jumps from 4 to 5 rows (the 8-row template) and
    // past 8 rows takes a second launch; the skinny kernel's hardly grows
    // below 32 rows.  At m = 5: 4096 x 4096 10.5 against 9.2, 4096 -> 14336
    // 13.9 against 13.9, 4096 -> 1792 8.7 / 8.5, Q6_K 1792 -> 4096 8.8 / 8.2,
    // Q6_K 4096 x 4096 11.7 / 10.2, 2048 x 2048 7.4 / 6.6; at m = 3 the
    // matvec wins for short or many rows (4096 -> 1792 7.2 / 7.3, Q6_K
    // 1792 -> 4096 6.7 / 7.5, 8192 -> 28672 33.9 / 37.4).  Groups: q/k/v at m = 2 13.4 against 10.6; the gate/up
    // pair at m = 2 22.2 against 24.5, at m = 3 24.0 / 24.1.  Single weights
    // with K >= 4096 and 2048 < N <= K (few, long rows) take the skinny
    // kernel from m = 3: 4096 x 4096 8.7 / 8.2 at m = 3 and 8.7 / 8.2 at
    // m = 4, 14336 -> 4096 17.8 / 14.2 and 17.9 / 14.1, Q6_K 14336 -> 4096
    // 19.4 / 18.0 and 19.8 / 18.0; the matvec keeps short or many rows
    // (m = 4: Q6_K 1792 -> 4096 6.6 / 7.7, 4096 -> 6144 10.2 / 10.3,
    // 4096 -> 14336 13.3 / 13.6, 4096 -> 1792 7.3 / 7.3).
    const bool long_rows = group_n == 0 && k >= 4096 && n > 2048 && n <= k;
    const size_t skinny_lo = skinny_min            ? skinny_min
                             : group_n > 16384     ? 3
                             : group_n >= 6144     ? 2
                             : long_rows           ? 3
                                                   : 5;
    if (group_n == 0 && q4k_prefill_early(dtype, m, k) && mfma_supported(dtype, m, n, k)) return kMfma;
    if (m >= skinny_lo && m <= skinny_max && skinny_supported(dtype, m, n, k)) return kSkinny;
    if (m > skinny_max && mfma_supported(dtype, m, n, k)) return kMfma;
    return kMatvec;
}

// Split-K partial sums sit after the activation image in the workspace.
static size_t partial_offset(uint32_t dtype, size_t m, size_t k, int forced) {
    return (act_layout(dtype, m, k, forced).bytes + kAlign - 1) / kAlign * kAlign;
}

static uint32_t route_splits(Route r, uint32_t dtype, size_t m, size_t n, size_t k) {
    if (r == kMfma) return prefill_supported(dtype, m, n, k) ? prefill_splits(m, n, k) : mfma_splits(m, n, k);
    if (r == kSkinny) return skinny_splits(m, n, k);
    return 1;
}

static size_t workspace_size_impl(const xnq_qtensor* qt, size_t m, int forced) {
    if (!qt) return 0;
    const size_t k = qt->L.k, n = qt->L.n;
    size_t bytes = act_layout(qt->L.dtype, m, k, forced).bytes;
    const uint32_t splits = route_splits(pick_route(qt->L.dtype, m, n, k, forced), qt->L.dtype, m, n, k);
    if (splits > 1) bytes = partial_offset(qt->L.dtype, m, k, forced) + (size_t)splits * m * n * sizeof(float);
    return bytes;
}

size_t xnq_qtensor_workspace_size(const xnq_qtensor* qt, size_t m) {
    return workspace_size_impl(qt, m, g_route.load());
}

static xnq_status matmul_preq_impl(const xnq_qtensor* qt, size_t m, size_t k, size_t n, const void* workspace_dev,
                                   size_t workspace_bytes, float* dst_dev, void* stream, int forced) {
    xnq_status st = check_mkn(qt, m, k, n);
    if (st) return st;
    if (m == 0 || n == 0) return XNQ_OK;
    if (!workspace_dev || !dst_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    DeviceGuard g(qt->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    const WView w = make_wview(qt->L, qt->buf);
    const AView a = make_aview(act_layout(qt->L.dtype, m, k, forced), workspace_dev);
    hipError_t e;
    const Route r = pick_route(qt->L.dtype, m, n, k, forced);
    if (r == kMfma || r == kSkinny) {
        if (r == kMfma ? !mfma_supported(qt->L.dtype, m, n, k) : !skinny_supported(qt->L.dtype, m, n, k))
            return fail(XNQ_ERR_UNSUPPORTED, "no MFMA kernel for this dtype/shape");
        uint32_t splits = route_splits(r, qt->L.dtype, m, n, k);
        const size_t off = partial_offset(qt->L.dtype, m, k, forced);
        if (off + (size_t)splits * m * n * sizeof(float) > workspace_bytes) splits = 1;
        float* partial = splits > 1 ? reinterpret_cast<float*>((uint8_t*)workspace_dev + off) : nullptr;
        e = r == kMfma ? launch_mfma(w, a, m, splits, dst_dev, partial, (hipStream_t)stream)
                       : launch_skinny(w, a, m, splits, dst_dev, partial, (hipStream_t)stream);
    } else {
        e = launch_matvec(w, a, m, dst_dev, (hipStream_t)stream);
    }
    if (e == hipErrorInvalidConfiguration)
        return fail(XNQ_ERR_INVALID, "k = %zu is too large for the matvec kernel's LDS", k);
    if (e != hipSuccess) return hip_fail(e, "matmul kernel");
    return XNQ_OK;
}

xnq_status xnq_qtensor_matmul_preq(const xnq_qtensor* qt, size_t m, size_t k, size_t n,
                                   const void* workspace_dev, size_t workspace_bytes, float* dst_dev,
                                   void* stream) {
    return matmul_preq_impl(qt, m, k, n, workspace_dev, workspace_bytes, dst_dev, stream, g_route.load());
}

// Decode: the fused matvec route quantizes the activation row in LDS inside
// the matvec kernel and needs no workspace, which saves the quantize launch
// (~1.8 us).  Every workgroup quantizes the whole row, so it pays only while
// rows are short: m = 1 on weights of up to XNQ_FUSED_MAX_ELEMS (6144 x 4096)
// elements, or rows of K <= XNQ_FUSED_MAX_K (4096) at any N; the q/k/v group
// and the SiLU-gated gate/up pair take one launch for several weights there
// (decode step 1540 -> 1432 us).  Longer rows and more activation rows take
// quantize + matvec (14336 -> 4096 Q6_K: 19.6 fused against 12.8; m = 2,
// 14336 -> 4096: 23 against 11 + 1.8).
static size_t fused_max_elems() {
    static const size_t v = env_size("XNQ_FUSED_MAX_ELEMS", (size_t)6144 * 4096);
    return v;
}

static size_t fused_max_k() {
    static const size_t v = env_size("XNQ_FUSED_MAX_K", 4096);
    return v;
}

// m == 1 takes one kernel that quantizes the row in LDS: weights of up to
// XNQ_FUSED_MAX_ELEMS elements the one-shot group kernel (one wavefront per
// row), rows of K <= XNQ_FUSED_MAX_K at any N (alone, or one of a q/k/v
// group or a gate/up pair, whose one-launch kernels take them) the
// persistent matvec kernel with 16-wavefront workgroups, each quantizing the
// row once (graph steps against quantize + matvec, µs: Q4_K 4096 -> 14336
// 9.3 against 9.7, Q4_0 4096 -> 14336 7.9 against 9.2, Q6_K 4096 -> 128256
// 68.9 against 72.1; at K = 14336 quantizing 56 blocks per workgroup costs
// more than the separate launch: 14336 -> 4096 Q6_K 19.6 against 12.8).
static bool fused_route(const xnq_qtensor* qt, size_t m, int forced) {
    const Route r = pick_route(qt->L.dtype, m, qt->L.n, qt->L.k, forced);
    if (r != kMatvec) return false;
    if (forced == 1) return true;
    return m == 1 && (qt->L.k <= fused_max_k() || qt->L.n * qt->L.k <= fused_max_elems());
}
static bool fused_one_shot(const xnq_qtensor* qt) { return qt->L.n * qt->L.k <= fused_max_elems(); }

static size_t matmul_t_workspace_size_impl(const xnq_qtensor* qt, size_t m, int forced) {
    if (!qt || fused_route(qt, m, forced)) return 0;
    return workspace_size_impl(qt, m, forced);
}

size_t xnq_qtensor_matmul_t_workspace_size(const xnq_qtensor* qt, size_t m) {
    return matmul_t_workspace_size_impl(qt, m, g_route.load());
}

static xnq_status matmul_t_ws_impl(const xnq_qtensor* qt, size_t m, size_t k, size_t n, const float* lhs_dev,
                                   void* workspace_dev, size_t workspace_bytes, float* dst_dev, void* stream,
                                   int forced) {
    xnq_status st = check_mkn(qt, m, k, n);
    if (st) return st;
    st = check_lhs(qt->L.dtype, k);
    if (st) return st;
    if (m == 0 || n == 0) return XNQ_OK;
    if (!lhs_dev || !dst_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    DeviceGuard g(qt->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    if (fused_route(qt, m, forced)) {
        const WView w = make_wview(qt->L, qt->buf);
        hipError_t e = launch_matvec_fused(w, lhs_dev, m, dst_dev, s, fused_one_shot(qt));
        if (e == hipErrorInvalidConfiguration)
            return fail(XNQ_ERR_INVALID, "k = %zu is too large for the matvec kernel's LDS", k);
        if (e != hipSuccess) return hip_fail(e, "matvec kernel");
        return XNQ_OK;
    }
    const size_t need = act_layout(qt->L.dtype, m, k, forced).bytes;
    if (!workspace_dev || workspace_bytes < need)
        return fail(XNQ_ERR_INVALID, "workspace of %zu bytes is smaller than the %zu the activation needs",
                    workspace_bytes, need);
    st = quantize_lhs_impl(qt->L.dtype, m, k, lhs_dev, workspace_dev, stream, forced);
    if (!st) st = matmul_preq_impl(qt, m, k, n, workspace_dev, workspace_bytes, dst_dev, stream, forced);
    return st;
}

xnq_status xnq_qtensor_matmul_t_ws(const xnq_qtensor* qt, size_t m, size_t k, size_t n, const float* lhs_dev,
                                   void* workspace_dev, size_t workspace_bytes, float* dst_dev, void* stream) {
    return matmul_t_ws_impl(qt, m, k, n, lhs_dev, workspace_dev, workspace_bytes, dst_dev, stream, g_route.load());
}

xnq_status xnq_qtensor_matmul_t(const xnq_qtensor* qt, size_t m, size_t k, size_t n,
                                const float* lhs_dev, float* dst_dev, void* stream) {
    xnq_status st = check_mkn(qt, m, k, n);
    if (st) return st;
    const int forced = g_route.load();
    const size_t ws_bytes = matmul_t_workspace_size_impl(qt, m, forced);
    if (ws_bytes == 0 || n == 0 || m == 0)
        return matmul_t_ws_impl(qt, m, k, n, lhs_dev, nullptr, 0, dst_dev, stream, forced);
    DeviceGuard g(qt->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipStream_t s = (hipStream_t)stream;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
        return fail(XNQ_ERR_INVALID,
                    "matmul_t would allocate its workspace inside a stream capture: use matmul_t_ws with a "
                    "workspace of xnq_qtensor_matmul_t_workspace_size(qt, %zu) = %zu bytes",
                    m, ws_bytes);
    void* ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, ws_bytes, s);
    if (e != hipSuccess) return hip_fail(e, "hipMallocAsync(workspace)");
    st = matmul_t_ws_impl(qt, m, k, n, lhs_dev, ws, ws_bytes, dst_dev, stream, forced);
    (void)hipFreeAsync(ws, s);
    return st;
}

// ---------------------------------------------------------------------------
// matmul_t without any allocation: the workspace is a file-scope device
// array.  In host code `scratch` only names the symbol; its device address
// (one per GPU) comes from hipGetSymbolAddress with that GPU current, and
// only that address is ever handed to kernels.

static __device__ __align__(256) uint8_t scratch[XNQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// Device address of `scratch` on `dev`, which must be the current device.
static xnq_status scratch_ptr(int dev, void** out) {
    if (dev < 0 || dev >= kMaxDevices) return fail(XNQ_ERR_INVALID, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(XNQ_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return XNQ_OK;
}

xnq_status xnq_qtensor_matmul_t_noalloc(const xnq_qtensor* qt, size_t m, size_t k, size_t n, const float* lhs_dev,
                                        float* dst_dev, void* stream) {
    xnq_status st = check_mkn(qt, m, k, n);
    if (st) return st;
    const int forced = g_route.load();
    const size_t need = matmul_t_workspace_size_impl(qt, m, forced);
    if (need > XNQ_NOALLOC_SCRATCH_BYTES)
        return fail(XNQ_ERR_INVALID,
                    "matmul_t_noalloc: m = %zu needs %zu bytes of scratch, more than the library's static %zu; "
                    "split the rows or use matmul_t_ws",
                    m, need, (size_t)XNQ_NOALLOC_SCRATCH_BYTES);
    if (need == 0 || m == 0 || n == 0) return matmul_t_ws_impl(qt, m, k, n, lhs_dev, nullptr, 0, dst_dev, stream, forced);
    DeviceGuard g(qt->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    void* ws = nullptr;
    st = scratch_ptr(qt->device, &ws);
    if (st) return st;
    // every kernel writes the scratch it reads (activation image, split-K
    // partials) before reading it, so nothing needs clearing between calls
    return matmul_t_ws_impl(qt, m, k, n, lhs_dev, ws, XNQ_NOALLOC_SCRATCH_BYTES, dst_dev, stream, forced);
}

// ---------------------------------------------------------------------------
// Decode-step groups: weights that read one activation row.

// The grouped m == 1 kernel takes the group when every weight is on the
// fused decode route with one dtype, one K and one device.
static bool group_route(const xnq_qtensor* const* qts, size_t count, size_t m, int forced) {
    if (m != 1 || count == 0 || count > (size_t)kMaxGroup) return false;
    for (size_t i = 0; i < count; i++) {
        if (!qts[i] || !fused_route(qts[i], m, forced)) return false;
        if (qts[i]->L.dtype != qts[0]->L.dtype || qts[i]->L.k != qts[0]->L.k || qts[i]->device != qts[0]->device)
            return false;
    }
    return true;
}

// Off the one-launch route, weights of one dtype, K and device that all
// take a quantized workspace share one quantize launch: the activation image
// depends only on the dtype, m and K.
static bool shared_quantize(const xnq_qtensor* const* qts, size_t count, size_t m, int forced) {
    if (count < 2) return false;
    for (size_t i = 0; i < count; i++) {
        if (!qts[i] || fused_route(qts[i], m, forced)) return false;
        if (qts[i]->L.dtype != qts[0]->L.dtype || qts[i]->L.k != qts[0]->L.k || qts[i]->device != qts[0]->device)
            return false;
    }
    return true;
}

static size_t joined_n(const xnq_qtensor* const* qts, size_t count) {
    size_t n = 0;
    for (size_t i = 0; i < count; i++) n += qts[i]->L.n;
    return n;
}

// Weights that share one quantize and all take the skinny route run as one
// skinny launch over their joined column tiles, with one split-K sum.
static bool skinny_group(const xnq_qtensor* const* qts, size_t count, size_t m, int forced) {
    if (!shared_quantize(qts, count, m, forced)) return false;
    for (size_t i = 0; i < count; i++) {
        const WLayout& L = qts[i]->L;
        if (pick_route(L.dtype, m, L.n, L.k, forced, joined_n(qts, count)) != kSkinny ||
            !skinny_supported(L.dtype, m, L.n, L.k))
            return false;
    }
    return true;
}


// Activation image, then one partial region per weight ([split][m][n_t]).
static size_t skinny_group_ws(const xnq_qtensor* const* qts, size_t count, size_t m, int forced) {
    const size_t k = qts[0]->L.k, n = joined_n(qts, count);
    return partial_offset(qts[0]->L.dtype, m, k, forced) + (size_t)skinny_splits(m, n, k) * m * n * sizeof(float);
}

// Quantize once, then the skinny kernel over the group (silu: gate, up pair
// into G.y[0]).
static xnq_status run_skinny_group(const xnq_qtensor* const* qts, size_t count, size_t m, size_t k,
                                   const float* lhs_dev, float* const* dsts, void* workspace_dev,
                                   size_t workspace_bytes, bool silu, void* stream, int forced,
                                   const ALayout* next = nullptr, void* next_img = nullptr);

static WGroup make_group(const xnq_qtensor* const* qts, size_t count, float* const* dsts) {
    WGroup g{};
    uint32_t end = 0;
    for (size_t i = 0; i < count; i++) {
        g.w[i] = make_wview(qts[i]->L, qts[i]->buf);
        g.y[i] = dsts[i];
        end += (uint32_t)qts[i]->L.n;
        g.row_end[i] = end;
    }
    g.count = (uint32_t)count;
    g.rows = end;
    return g;
}

static xnq_status run_skinny_group(const xnq_qtensor* const* qts, size_t count, size_t m, size_t k,
                                   const float* lhs_dev, float* const* dsts, void* workspace_dev,
                                   size_t workspace_bytes, bool silu, void* stream, int forced,
                                   const ALayout* next, void* next_img) {
    const uint32_t dt = qts[0]->L.dtype;
    const size_t need = skinny_group_ws(qts, count, m, forced);
    if (!workspace_dev || workspace_bytes < need)
        return fail(XNQ_ERR_INVALID, "workspace of %zu bytes is smaller than the %zu needed", workspace_bytes, need);
    DeviceGuard g(qts[0]->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    xnq_status st = quantize_lhs_impl(dt, m, k, lhs_dev, workspace_dev, stream, forced);
    if (st) return st;
    const WGroup G = make_group(qts, count, dsts);
    const AView a = make_aview(act_layout(dt, m, k, forced), workspace_dev);
    float* partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace_dev) + partial_offset(dt, m, k, forced));
    const hipError_t e = launch_skinny_group(G, a, m, skinny_splits(m, joined_n(qts, count), k), partial, silu,
                                             (hipStream_t)stream, next, next_img);
    if (e != hipSuccess) return hip_fail(e, "grouped skinny kernel");
    return XNQ_OK;
}

static size_t silu_gate_ws_impl(const xnq_qtensor* gate, const xnq_qtensor* up, size_t m, int forced) {
    if (!gate || !up) return 0;
    const xnq_qtensor* pair[2] = {gate, up};
    if (group_route(pair, 2, m, forced) && gate->L.k <= 64 * 5 * 32) return 0;
    const size_t a = matmul_t_workspace_size_impl(gate, m, forced), b = matmul_t_workspace_size_impl(up, m, forced);
    const size_t two = align_up(a > b ? a : b, kAlign) + m * up->L.n * sizeof(float);
    if (gate->L.n != up->L.n || !skinny_group(pair, 2, m, forced)) return two;
    const size_t one = skinny_group_ws(pair, 2, m, forced);
    return one > two ? one : two;
}

size_t xnq_matmul_t_silu_gate_workspace_size(const xnq_qtensor* gate, const xnq_qtensor* up, size_t m) {
    return silu_gate_ws_impl(gate, up, m, g_route.load());
}

// `forced` is the route override as read once at the public entry point
// (xnq_matmul_t_silu_gate or xnq_mlp_t), so sizing and launching agree.
static xnq_status silu_gate_impl(const xnq_qtensor* gate, const xnq_qtensor* up, size_t m, size_t k, size_t n,
                                 const float* lhs_dev, void* workspace_dev, size_t workspace_bytes, float* dst_dev,
                                 void* stream, int forced) {
    xnq_status st = check_mkn(gate, m, k, n);
    if (st) return st;
    st = check_mkn(up, m, k, n);
    if (st) return st;
    if (gate->device != up->device) return fail(XNQ_ERR_INVALID, "gate and up live on different devices");
    if (m == 0 || n == 0) return XNQ_OK;
    if (!lhs_dev || !dst_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    const size_t need = silu_gate_ws_impl(gate, up, m, forced);
    hipStream_t s = (hipStream_t)stream;
    if (need == 0) {
        st = check_lhs(gate->L.dtype, k);
        if (st) return st;
        DeviceGuard g(gate->device);
        if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
        const xnq_qtensor* pair[2] = {gate, up};
        float* dsts[2] = {dst_dev, nullptr};
        const WGroup grp = make_group(pair, 2, dsts);
        WGroup gg = grp;
        gg.rows = (uint32_t)n;
        const hipError_t e = launch_matvec_group(gg, lhs_dev, true, s);
        if (e != hipSuccess) return hip_fail(e, "silu-gated matvec kernel");
        return XNQ_OK;
    }
    if (!workspace_dev || workspace_bytes < need)
        return fail(XNQ_ERR_INVALID, "workspace of %zu bytes is smaller than the %zu needed", workspace_bytes, need);
    const size_t a = matmul_t_workspace_size_impl(gate, m, forced), b = matmul_t_workspace_size_impl(up, m, forced);
    const size_t off = align_up(a > b ? a : b, kAlign);
    float* u = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace_dev) + off);
    const xnq_qtensor* pair[2] = {gate, up};
    if (skinny_group(pair, 2, m, forced)) {
        float* dsts[2] = {dst_dev, nullptr};
        return run_skinny_group(pair, 2, m, k, lhs_dev, dsts, workspace_dev, workspace_bytes, true, stream, forced);
    }
    if (shared_quantize(pair, 2, m, forced)) {
        DeviceGuard g(gate->device);
        if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
        st = quantize_lhs_impl(gate->L.dtype, m, k, lhs_dev, workspace_dev, stream, forced);
        if (!st) st = matmul_preq_impl(gate, m, k, n, workspace_dev, off, dst_dev, stream, forced);
        if (!st) st = matmul_preq_impl(up, m, k, n, workspace_dev, off, u, stream, forced);
    } else {
        st = matmul_t_ws_impl(gate, m, k, n, lhs_dev, workspace_dev, off, dst_dev, stream, forced);
        if (!st) st = matmul_t_ws_impl(up, m, k, n, lhs_dev, workspace_dev, off, u, stream, forced);
    }
    if (st) return st;
    DeviceGuard g(gate->device);
    const hipError_t e = launch_silu_mul(dst_dev, u, m * n, s);
    if (e != hipSuccess) return hip_fail(e, "silu_mul kernel");
    return XNQ_OK;
}

xnq_status xnq_matmul_t_silu_gate(const xnq_qtensor* gate, const xnq_qtensor* up, size_t m, size_t k, size_t n,
                                  const float* lhs_dev, void* workspace_dev, size_t workspace_bytes, float* dst_dev,
                                  void* stream) {
    return silu_gate_impl(gate, up, m, k, n, lhs_dev, workspace_dev, workspace_bytes, dst_dev, stream, g_route.load());
}

// ---------------------------------------------------------------------------
// The SwiGLU MLP of llama.rs:236-264: h = silu(x . gate^T) * (x . up^T),
// y = h . down^T.  With gate/up on the small-batch MFMA route and a K-quant
// down weight, the gate/up split-sum also writes the down projection's
// activation image (one launch fewer than silu_gate + matmul_t); otherwise
// it is exactly those two calls.  The workspace holds both calls' scratch.

static bool mlp_fused(const xnq_qtensor* gate, const xnq_qtensor* up, const xnq_qtensor* down, size_t m,
                      int forced) {
    const xnq_qtensor* pair[2] = {gate, up};
    if (gate->L.n != up->L.n || !skinny_group(pair, 2, m, forced)) return false;
    if (down->device != gate->device || !is_kquant(down->L.dtype) || fused_route(down, m, forced)) return false;
    const ALayout L = act_layout(down->L.dtype, m, down->L.k, forced);
    return L.act_dtype == XNQ_Q8K && !L.tiled && down->L.k % 256 == 0;
}

static size_t mlp_ws_impl(const xnq_qtensor* gate, const xnq_qtensor* up, const xnq_qtensor* down, size_t m,
                          int forced) {
    if (!gate || !up || !down) return 0;
    const size_t a = silu_gate_ws_impl(gate, up, m, forced), b = matmul_t_workspace_size_impl(down, m, forced);
    return b ? align_up(a, kAlign) + b : a;
}

size_t xnq_mlp_t_workspace_size(const xnq_qtensor* gate, const xnq_qtensor* up, const xnq_qtensor* down, size_t m) {
    return mlp_ws_impl(gate, up, down, m, g_route.load());
}

xnq_status xnq_mlp_t(const xnq_qtensor* gate, const xnq_qtensor* up, const xnq_qtensor* down, size_t m, size_t k,
                     size_t f, const float* lhs_dev, void* workspace_dev, size_t workspace_bytes, float* h_dev,
                     float* dst_dev, void* stream) {
    if (!gate || !up || !down) return fail(XNQ_ERR_INVALID, "null qtensor");
    xnq_status st = check_mkn(gate, m, k, f);
    if (!st) st = check_mkn(up, m, k, f);
    if (!st) st = check_mkn(down, m, f, down->L.n);
    if (st) return st;
    if (gate->device != up->device || gate->device != down->device)
        return fail(XNQ_ERR_INVALID, "gate, up and down live on different devices");
    if (m == 0) return XNQ_OK;
    if (!lhs_dev || !h_dev || !dst_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    const int forced = g_route.load();
    const size_t need = mlp_ws_impl(gate, up, down, m, forced);
    if (need && (!workspace_dev || workspace_bytes < need))
        return fail(XNQ_ERR_INVALID, "workspace of %zu bytes is smaller than the %zu needed", workspace_bytes, need);
    const size_t a = silu_gate_ws_impl(gate, up, m, forced);
    const size_t off_b = align_up(a, kAlign);
    uint8_t* wsb = need > a ? static_cast<uint8_t*>(workspace_dev) + off_b : nullptr;
    const size_t bytes_b = need > a ? need - off_b : 0;
    if (mlp_fused(gate, up, down, m, forced)) {
        const xnq_qtensor* pair[2] = {gate, up};
        float* dsts[2] = {h_dev, nullptr};
        const ALayout Ld = act_layout(down->L.dtype, m, f, forced);
        st = check_lhs(gate->L.dtype, k);
        if (!st) st = run_skinny_group(pair, 2, m, k, lhs_dev, dsts, workspace_dev, a, true, stream, forced, &Ld, wsb);
        if (!st) st = matmul_preq_impl(down, m, f, down->L.n, wsb, bytes_b, dst_dev, stream, forced);
        return st;
    }
    st = silu_gate_impl(gate, up, m, k, f, lhs_dev, workspace_dev, a, h_dev, stream, forced);
    if (!st) st = matmul_t_ws_impl(down, m, f, down->L.n, h_dev, wsb, bytes_b, dst_dev, stream, forced);
    return st;
}

static size_t group_ws_impl(const xnq_qtensor* const* qts, size_t count, size_t m, int forced) {
    if (!qts || group_route(qts, count, m, forced)) return 0;
    size_t need = 0;
    for (size_t i = 0; i < count; i++) {
        const size_t b = qts[i] ? matmul_t_workspace_size_impl(qts[i], m, forced) : 0;
        if (b > need) need = b;
    }
    if (count <= (size_t)kMaxGroup && skinny_group(qts, count, m, forced)) {
        const size_t one = skinny_group_ws(qts, count, m, forced);
        if (one > need) need = one;
    }
    return need;
}

size_t xnq_matmul_t_group_workspace_size(const xnq_qtensor* const* qts, size_t count, size_t m) {
    return group_ws_impl(qts, count, m, g_route.load());
}

xnq_status xnq_matmul_t_group(const xnq_qtensor* const* qts, size_t count, size_t m, size_t k,
                              const float* lhs_dev, float* const* dsts_dev, void* workspace_dev,
                              size_t workspace_bytes, void* stream) {
    if (!qts || !dsts_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    for (size_t i = 0; i < count; i++) {
        if (!qts[i]) return fail(XNQ_ERR_INVALID, "null qtensor");
        const xnq_status st = check_mkn(qts[i], m, k, qts[i]->L.n);
        if (st) return st;
    }
    if (count == 0 || m == 0) return XNQ_OK;
    if (!lhs_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    for (size_t i = 0; i < count; i++)
        if (!dsts_dev[i]) return fail(XNQ_ERR_INVALID, "null pointer");
    const int forced = g_route.load();
    if (group_route(qts, count, m, forced)) {
        const xnq_status st = check_lhs(qts[0]->L.dtype, k);
        if (st) return st;
        DeviceGuard g(qts[0]->device);
        if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
        const hipError_t e = launch_matvec_group(make_group(qts, count, dsts_dev), lhs_dev, false, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "grouped matvec kernel");
        return XNQ_OK;
    }
    if (count <= (size_t)kMaxGroup && skinny_group(qts, count, m, forced))
        return run_skinny_group(qts, count, m, k, lhs_dev, dsts_dev, workspace_dev, workspace_bytes, false, stream,
                                forced);
    if (shared_quantize(qts, count, m, forced)) {
        // one activation image for every weight, then one matmul each
        const size_t need = act_layout(qts[0]->L.dtype, m, k, forced).bytes;
        if (!workspace_dev || workspace_bytes < need)
            return fail(XNQ_ERR_INVALID, "workspace of %zu bytes is smaller than the %zu the activation needs",
                        workspace_bytes, need);
        DeviceGuard g(qts[0]->device);
        if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
        xnq_status st = quantize_lhs_impl(qts[0]->L.dtype, m, k, lhs_dev, workspace_dev, stream, forced);
        for (size_t i = 0; i < count && !st; i++)
            st = matmul_preq_impl(qts[i], m, k, qts[i]->L.n, workspace_dev, workspace_bytes, dsts_dev[i], stream,
                                  forced);
        return st;
    }
    for (size_t i = 0; i < count; i++) {
        const xnq_status st = matmul_t_ws_impl(qts[i], m, k, qts[i]->L.n, lhs_dev, workspace_dev, workspace_bytes,
                                               dsts_dev[i], stream, forced);
        if (st) return st;
    }
    return XNQ_OK;
}

xnq_status xnq_qtensor_dequantize(const xnq_qtensor* qt, float* dst_dev, size_t elem_count,
                                  void* stream) {
    if (!qt) return fail(XNQ_ERR_INVALID, "null qtensor");
    if (elem_count != qt->L.n * qt->L.k)
        return fail(XNQ_ERR_INVALID, "dequantize: ys (len = %zu) does not match the expected length of %zu",
                    elem_count, qt->L.n * qt->L.k);
    if (elem_count == 0) return XNQ_OK;
    if (!dst_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    DeviceGuard g(qt->device);
    hipError_t e = launch_dequant(qt->L, qt->buf, dst_dev, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "dequantize");
    return XNQ_OK;
}

xnq_status xnq_qtensor_raw_data(const xnq_qtensor* qt, void* host_dst, size_t cap, void* stream) {
    if (!qt) return fail(XNQ_ERR_INVALID, "null qtensor");
    const size_t bytes = xnq_qtensor_storage_size(qt);
    if (cap < bytes) return fail(XNQ_ERR_INVALID, "raw_data: buffer too small (%zu < %zu)", cap, bytes);
    if (bytes == 0) return XNQ_OK;
    if (!host_dst) return fail(XNQ_ERR_INVALID, "null pointer");
    DeviceGuard g(qt->device);
    // Not the hot path: plain allocation, the unrepack on `stream`, then a
    // blocking copy into the (pageable) host buffer.
    hipStream_t s = (hipStream_t)stream;
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(raw_data)");
    e = launch_unrepack(qt->L, qt->buf, tmp, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipMemcpy(host_dst, tmp, bytes, hipMemcpyDeviceToHost);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "raw_data");
    return XNQ_OK;
}

xnq_status xnq_quantize_act_blocks(uint32_t act_dtype, size_t m, size_t k, const float* src_dev,
                                   void* blocks_dev, void* stream) {
    if (act_dtype != XNQ_Q8_0 && act_dtype != XNQ_Q8K)
        return fail(XNQ_ERR_UNSUPPORTED, "activation dtype must be Q8_0 or Q8K, got %u", act_dtype);
    const size_t bs = block_size(act_dtype);
    if (k % bs != 0)
        return fail(XNQ_ERR_INVALID, "%zu is not divisible by %zu", k, bs);
    if (m == 0) return XNQ_OK;
    if (!src_dev || !blocks_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    hipError_t e = launch_quantize_act_blocks(act_dtype, m, k, src_dev, blocks_dev, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "quantize_act_blocks");
    return XNQ_OK;
}

xnq_status xnq_qtensor_block_ints(const xnq_qtensor* qt, size_t m, const void* workspace_dev,
                                  int32_t* out_dev, void* stream) {
    if (!qt) return fail(XNQ_ERR_INVALID, "null qtensor");
    if (m == 0) return XNQ_OK;
    if (!workspace_dev || !out_dev) return fail(XNQ_ERR_INVALID, "null pointer");
    DeviceGuard g(qt->device);
    const WView w = make_wview(qt->L, qt->buf);
    const AView a = make_aview(act_layout(qt->L.dtype, m, qt->L.k, g_route.load()), workspace_dev);
    hipError_t e = launch_block_ints(w, a, m, out_dev, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "block_ints");
    return XNQ_OK;
}

// ---------------------------------------------------------------------------
// Stream capture into a replayable graph (xn's Device::capture_begin /
// capture_end / CaptureGraph::launch, cuda_backend/mod.rs:251-283).

struct xnq_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

xnq_status xnq_capture_begin(void* stream) {
    if (!stream) return fail(XNQ_ERR_INVALID, "stream capture needs a stream other than the null stream");
    const hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
    return XNQ_OK;
}

xnq_status xnq_capture_end(void* stream, xnq_graph** out) {
    if (!out) return fail(XNQ_ERR_INVALID, "null pointer");
    *out = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    if (!g) return fail(XNQ_ERR_INVALID, "stream capture ended without a graph");
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return hip_fail(e, "hipGraphInstantiate");
    }
    *out = new xnq_graph{g, x};
    return XNQ_OK;
}

void xnq_capture_abort(void* stream) {
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture((hipStream_t)stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
    (void)hipGetLastError();  // errors of the discarded capture are dropped
}

xnq_status xnq_graph_launch(const xnq_graph* g, void* stream) {
    if (!g) return fail(XNQ_ERR_INVALID, "null graph");
    const hipError_t e = hipGraphLaunch(g->exec, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
    return XNQ_OK;
}

void xnq_graph_free(xnq_graph* g) {
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

}  // extern "C"
