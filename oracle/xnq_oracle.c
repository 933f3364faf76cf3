/*
 * xnq_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of xn's CPU quantized-matmul path (gradium-ai/xn,
 * xn-core/src/quantized/k_quants.rs and utils.rs).  It is the checker that the
 * HIP kernels in xn_amd/csrc are compared against.  Only tests/, the smoke()
 * hook and bench.py's cpu_baseline leg may load it; the product library never
 * links or calls it.
 *
 * Semantics kept from Rust (reference behaviour, compiled with
 * -ffp-contract=off so no multiply-add is fused where Rust does not fuse):
 *   f32::round          -> roundf (half away from zero)
 *   f32 `as i8/u8/i32`  -> saturating conversion, NaN -> 0
 *   i32 `as u8/i8`      -> two's-complement truncation
 *   f16::from_f32       -> IEEE binary16 round-to-nearest-even (`half` 2.7.1)
 *   iterator .sum()     -> sequential left fold
 *
 * Block layouts (bytes, little endian) follow k_quants.rs:92-205:
 *   BlockQ4_0 18 B  { f16 d; u8 qs[16]; }
 *   BlockQ8_0 34 B  { f16 d; i8 qs[32]; }
 *   BlockQ4K 144 B  { f16 d; f16 dmin; u8 scales[12]; u8 qs[128]; }
 *   BlockQ6K 210 B  { u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d; }
 *   BlockQ8K 292 B  { f32 d; i8 qs[256]; i16 bsums[16]; }
 *
 * Pinning status of each function is recorded in tests/test_oracle.py: every
 * exported function is checked there against an independent computation
 * (numpy float16, brute-force integer sums, closed forms, the reference's own
 * k_quants.rs:2189-2210 known-answer test, round-trip error bounds).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define QK_K 256
#define QK8_0 32
#define QK4_0 32

/* GGML type ids, mod.rs:97-137 */
enum {
    ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7, ORC_Q8_0 = 8, ORC_Q8_1 = 9,
    ORC_Q2K = 10, ORC_Q3K = 11, ORC_Q4K = 12, ORC_Q5K = 13, ORC_Q6K = 14, ORC_Q8K = 15
};

/* xnq_oracle_more.c: Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K */
void orc_q8_1_from_float(const float* xs, void* out, size_t nblocks);
void orc_q4_1_from_float(const float* xs, void* out, size_t nblocks);
void orc_q4_1_to_float(const void* in, float* ys, size_t nblocks);
float orc_q4_1_vec_dot(size_t n, const void* xv, const void* yv);
void orc_q5_0_from_float(const float* xs, void* out, size_t nblocks);
void orc_q5_0_to_float(const void* in, float* ys, size_t nblocks);
float orc_q5_0_vec_dot(size_t n, const void* xv, const void* yv);
void orc_q5_1_from_float(const float* xs, void* out, size_t nblocks);
void orc_q5_1_to_float(const void* in, float* ys, size_t nblocks);
float orc_q5_1_vec_dot(size_t n, const void* xv, const void* yv);
void orc_q2k_from_float(const float* xs, void* out, size_t nblocks);
void orc_q2k_to_float(const void* in, float* ys, size_t nblocks);
float orc_q2k_vec_dot(size_t n, const void* xv, const void* yv);
void orc_q3k_from_float(const float* xs, void* out, size_t nblocks);
void orc_q3k_to_float(const void* in, float* ys, size_t nblocks);
float orc_q3k_vec_dot(size_t n, const void* xv, const void* yv);
void orc_q5k_from_float(const float* xs, void* out, size_t nblocks);
void orc_q5k_to_float(const void* in, float* ys, size_t nblocks);
float orc_q5k_vec_dot(size_t n, const void* xv, const void* yv);

#pragma pack(push, 1)
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4k;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6k;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } blk_q8k;
#pragma pack(pop)

_Static_assert(sizeof(blk_q4_0) == 18, "q4_0");
_Static_assert(sizeof(blk_q8_0) == 34, "q8_0");
_Static_assert(sizeof(blk_q4k) == 144, "q4k");
_Static_assert(sizeof(blk_q6k) == 210, "q6k");
_Static_assert(sizeof(blk_q8k) == 292, "q8k");

/* ---------------------------------------------------------------- f16 */

/* IEEE binary16 <- binary32, round to nearest even (what `half::f16::from_f32`
 * computes, both in software and through F16C). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ----------------------------------------------- Rust cast semantics */

static int8_t f_as_i8(float v) {
    if (v != v) return 0;
    if (v <= -128.0f) return -128;
    if (v >= 127.0f) return 127;
    return (int8_t)v;
}
static uint8_t f_as_u8(float v) {
    if (v != v) return 0;
    if (v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}
static int32_t f_as_i32(float v) {
    if (v != v) return 0;
    if (v <= -2147483648.0f) return INT32_MIN;
    if (v >= 2147483647.0f) return INT32_MAX;
    return (int32_t)v;
}
/* utils.rs:3-5 nearest_int */
static int32_t nearest_int(float v) { return f_as_i32(roundf(v)); }
static int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* f32::max / f32::min: IEEE maxNum/minNum (NaN yields the other operand) */
static float rmax(float a, float b) { return fmaxf(a, b); }
static float rmin(float a, float b) { return fminf(a, b); }

/* ------------------------------------------------------------ Q8_0 */

/* k_quants.rs:636-661 BlockQ8_0::from_float */
void orc_q8_0_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q8_0* ys = (blk_q8_0*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = rmax(amax, fabsf(x[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        ys[i].d = orc_f32_to_f16(d);
        for (int j = 0; j < QK8_0; j++) ys[i].qs[j] = f_as_i8(roundf(x[j] * id));
    }
}

/* k_quants.rs:618-634 */
void orc_q8_0_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q8_0* xs = (const blk_q8_0*)in;
    for (size_t i = 0; i < nblocks; i++) {
        float d = orc_f16_to_f32(xs[i].d);
        for (int j = 0; j < QK8_0; j++) ys[i * QK8_0 + j] = (float)xs[i].qs[j] * d;
    }
}

/* k_quants.rs:677-691 vec_dot_unopt (Q8_0 x Q8_0) */
float orc_q8_0_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q8_0* xs = (const blk_q8_0*)xv;
    const blk_q8_0* ys = (const blk_q8_0*)yv;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / QK8_0; b++) {
        int32_t sum_i = 0;
        for (int j = 0; j < QK8_0; j++) sum_i += (int32_t)xs[b].qs[j] * (int32_t)ys[b].qs[j];
        sumf += (float)sum_i * orc_f16_to_f32(xs[b].d) * orc_f16_to_f32(ys[b].d);
    }
    return sumf;
}

/* ------------------------------------------------------------ Q4_0 */

/* k_quants.rs:235-270 */
void orc_q4_0_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q4_0* ys = (blk_q4_0*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * QK4_0;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK4_0; j++) {
            if (amax < fabsf(x[j])) { amax = fabsf(x[j]); max = x[j]; }
        }
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        ys[i].d = orc_f32_to_f16(d);
        for (int j = 0; j < 16; j++) {
            float x0 = x[j] * id;
            float x1 = x[16 + j] * id;
            uint8_t xi0 = f_as_u8(x0 + 8.5f); if (xi0 > 15) xi0 = 15;
            uint8_t xi1 = f_as_u8(x1 + 8.5f); if (xi1 > 15) xi1 = 15;
            ys[i].qs[j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

/* k_quants.rs:213-233 */
void orc_q4_0_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q4_0* xs = (const blk_q4_0*)in;
    for (size_t i = 0; i < nblocks; i++) {
        float d = orc_f16_to_f32(xs[i].d);
        for (int j = 0; j < 16; j++) {
            int x0 = (xs[i].qs[j] & 0x0F) - 8;
            int x1 = (xs[i].qs[j] >> 4) - 8;
            ys[i * 32 + j] = (float)x0 * d;
            ys[i * 32 + j + 16] = (float)x1 * d;
        }
    }
}

/* k_quants.rs:287-304 vec_dot_unopt (Q4_0 x Q8_0) */
float orc_q4_0_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q4_0* xs = (const blk_q4_0*)xv;
    const blk_q8_0* ys = (const blk_q8_0*)yv;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        int32_t sum_i = 0;
        for (int j = 0; j < 16; j++) {
            int32_t v0 = (xs[b].qs[j] & 0x0F) - 8;
            int32_t v1 = (xs[b].qs[j] >> 4) - 8;
            sum_i += v0 * ys[b].qs[j] + v1 * ys[b].qs[j + 16];
        }
        sumf += (float)sum_i * orc_f16_to_f32(xs[b].d) * orc_f16_to_f32(ys[b].d);
    }
    return sumf;
}

/* ------------------------------------------------------------ Q8_K */

/* k_quants.rs:1942-1979 BlockQ8K::from_float */
void orc_q8k_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q8k* ys = (blk_q8k*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            if (amax < fabsf(x[j])) { amax = fabsf(x[j]); max = x[j]; }
        }
        if (amax == 0.0f) {
            ys[i].d = 0.0f;
            memset(ys[i].qs, 0, sizeof ys[i].qs);
            /* bsums keep their previous (zeroed) content, as in Rust where the
             * block comes from `zeros()` (k_quants.rs:2020). */
            memset(ys[i].bsums, 0, sizeof ys[i].bsums);
        } else {
            float iscale = -128.0f / max;
            for (int j = 0; j < QK_K; j++) {
                float v = roundf(iscale * x[j]);
                ys[i].qs[j] = f_as_i8(rmin(v, 127.0f));
            }
            for (int j = 0; j < QK_K / 16; j++) {
                int32_t sum = 0;
                for (int ii = 0; ii < 16; ii++) sum += ys[i].qs[j * 16 + ii];
                ys[i].bsums[j] = (int16_t)sum;
            }
            ys[i].d = 1.0f / iscale;
        }
    }
}

/* k_quants.rs:1981-1993 */
void orc_q8k_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q8k* xs = (const blk_q8k*)in;
    for (size_t i = 0; i < nblocks; i++)
        for (int j = 0; j < QK_K; j++) ys[i * QK_K + j] = xs[i].d * (float)xs[i].qs[j];
}

/* ------------------------------------------------------------ Q4_K */

/* utils.rs:53-63 */
static void get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void orc_get_scale_min_k4(int j, const uint8_t* q, uint8_t* out2) {
    get_scale_min_k4(j, q, &out2[0], &out2[1]);
}

/* Rust's f32::total_cmp order as a signed integer key. */
static int32_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

/* utils.rs:205-254 make_qkx1_quants; returns scale, writes -min to *neg_min.
 * The _ex form also reports, for the tests that pin it, the levels of the
 * last pass (lout, n bytes) and info[3] = {passes run, the iscale and the min
 * that pass assigned the levels with}; both may be NULL. */
float orc_make_qkx1_quants_ex(int nmax, int ntry, const float* x, int n, float* neg_min, uint8_t* lout,
                              float* info) {
    uint8_t l[QK_K];
    memset(l, 0, sizeof l);
    int passes = 0;
    float iscale_used = 0.0f, min_used = 0.0f;
    /* min_by keeps the first minimum, max_by keeps the last maximum */
    float mn = x[0], mx = x[0];
    for (int i = 1; i < n; i++) {
        if (total_key(x[i]) < total_key(mn)) mn = x[i];
        if (total_key(x[i]) >= total_key(mx)) mx = x[i];
    }
    if (mx == mn) {
        *neg_min = 0.0f;
        if (lout) memset(lout, 0, (size_t)n);
        if (info) info[0] = info[1] = info[2] = 0.0f;
        return 0.0f;
    }
    float min = rmin(mn, 0.0f);
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int t = 0; t < ntry; t++) {
        float sumlx = 0.0f;
        int32_t suml2 = 0;
        int did_change = 0;
        passes = t + 1;
        iscale_used = iscale;
        min_used = min;
        for (int i = 0; i < n; i++) {
            float value = x[i];
            int32_t li = clampi(nearest_int(iscale * (value - min)), 0, nmax);
            uint8_t cl = (uint8_t)li;
            if (cl != l[i]) { l[i] = cl; did_change = 1; }
            sumlx += (value - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = -0.0f;
        for (int i = 0; i < n; i++) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *neg_min = -min;
    if (lout) memcpy(lout, l, (size_t)n);
    if (info) { info[0] = (float)passes; info[1] = iscale_used; info[2] = min_used; }
    return scale;
}

float orc_make_qkx1_quants(int nmax, int ntry, const float* x, int n, float* neg_min) {
    return orc_make_qkx1_quants_ex(nmax, ntry, x, n, neg_min, NULL, NULL);
}

/* k_quants.rs:1418-1473 BlockQ4K::from_float */
void orc_q4k_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q4k* ys = (blk_q4k*)out;
    for (size_t bi = 0; bi < nblocks; bi++) {
        const float* x = xs + bi * QK_K;
        blk_q4k* block = &ys[bi];
        memset(block, 0, sizeof *block);
        float mins[8], scales[8];
        for (int j = 0; j < 8; j++) scales[j] = orc_make_qkx1_quants(15, 5, x + 32 * j, 32, &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) { max_scale = rmax(scales[j], max_scale); max_min = rmax(mins[j], max_min); }
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        for (int j = 0; j < 8; j++) {
            int32_t a = nearest_int(inv_scale * scales[j]); if (a > 63) a = 63;
            int32_t b = nearest_int(inv_min * mins[j]); if (b > 63) b = 63;
            uint8_t ls = (uint8_t)a, lm = (uint8_t)b;
            if (j < 4) {
                block->scales[j] = ls;
                block->scales[j + 4] = lm;
            } else {
                block->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                block->scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                block->scales[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        block->d = orc_f32_to_f16(max_scale / 63.0f);
        block->dmin = orc_f32_to_f16(max_min / 63.0f);
        uint8_t L[QK_K];
        memset(L, 0, sizeof L);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            get_scale_min_k4(j, block->scales, &sc, &m);
            float d = orc_f16_to_f32(block->d) * (float)sc;
            if (d != 0.0f) {
                float dm = orc_f16_to_f32(block->dmin) * (float)m;
                for (int ii = 0; ii < 32; ii++) {
                    int32_t lv = nearest_int((x[32 * j + ii] + dm) / d);
                    L[32 * j + ii] = (uint8_t)clampi(lv, 0, 15);
                }
            }
        }
        for (int j = 0; j < QK_K; j += 64)
            for (int lv = 0; lv < 32; lv++)
                block->qs[(j / 64) * 32 + lv] = (uint8_t)(L[j + lv] | (L[j + lv + 32] << 4));
    }
}

/* k_quants.rs:1475-1503 */
void orc_q4k_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q4k* xs = (const blk_q4k*)in;
    for (size_t bi = 0; bi < nblocks; bi++) {
        const blk_q4k* b = &xs[bi];
        float* y = ys + bi * QK_K;
        float d = orc_f16_to_f32(b->d), min = orc_f16_to_f32(b->dmin);
        int is = 0, yi = 0;
        for (int j = 0; j < QK_K; j += 64) {
            const uint8_t* q = b->qs + j / 2;
            uint8_t sc, m;
            get_scale_min_k4(is, b->scales, &sc, &m);
            float d1 = d * (float)sc, m1 = min * (float)m;
            get_scale_min_k4(is + 1, b->scales, &sc, &m);
            float d2 = d * (float)sc, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) y[yi++] = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) y[yi++] = d2 * (float)(q[l] >> 4) - m2;
            is += 2;
        }
    }
}

/* The scale/min unpacking of k_quants.rs:1375-1385 (the `utmp`/KMASK form).
 * Exposed so tests can check it against get_scale_min_k4. */
void orc_q4k_unpack_scales_kmask(const uint8_t* sc12, uint8_t* scales8, uint8_t* mins8) {
    const uint32_t KMASK1 = 0x3f3f3f3fu, KMASK2 = 0x0f0f0f0fu, KMASK3 = 0x03030303u;
    uint32_t utmp[4];
    memcpy(utmp, sc12, 12);
    utmp[3] = ((utmp[2] >> 4) & KMASK2) | (((utmp[1] >> 6) & KMASK3) << 4);
    uint32_t uaux = utmp[1] & KMASK1;
    utmp[1] = (utmp[2] & KMASK2) | (((utmp[0] >> 6) & KMASK3) << 4);
    utmp[2] = uaux;
    utmp[0] &= KMASK1;
    memcpy(scales8, &utmp[0], 8);
    memcpy(mins8, &utmp[2], 8);
}

/* Integer parts of one Q4K x Q8K super-block dot (k_quants.rs:1337-1416):
 * out[0] = sum_j sc_j * sum_{32} q4*q8   (the sum of aux32[0..8])
 * out[1] = sum_j mins[j/2] * bsums[j]    (`sumi`) */
void orc_q4k_block_ints(const void* xv, const void* yv, int64_t* out) {
    const blk_q4k* x = (const blk_q4k*)xv;
    const blk_q8k* y = (const blk_q8k*)yv;
    uint8_t scales[8], mins[8];
    orc_q4k_unpack_scales_kmask(x->scales, scales, mins);
    int8_t aux8[QK_K];
    for (int i = 0; i < 4; i++) {
        for (int l = 0; l < 32; l++) aux8[64 * i + l] = (int8_t)(x->qs[32 * i + l] & 0xF);
        for (int l = 0; l < 32; l++) aux8[64 * i + 32 + l] = (int8_t)(x->qs[32 * i + l] >> 4);
    }
    int32_t sumi = 0;
    for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
    int32_t aux32[8] = {0};
    int p = 0;
    for (int s = 0; s < 8; s++) {
        int32_t scale = scales[s];
        for (int r = 0; r < 4; r++) {
            for (int l = 0; l < 8; l++) {
                int16_t a16 = (int16_t)((int16_t)y->qs[p + l] * (int16_t)aux8[p + l]);
                aux32[l] += scale * (int32_t)a16;
            }
            p += 8;
        }
    }
    int64_t t = 0;
    for (int l = 0; l < 8; l++) t += aux32[l];
    out[0] = t;
    out[1] = sumi;
}

/* k_quants.rs:1337-1416 vec_dot_unopt (Q4K x Q8K) */
float orc_q4k_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q4k* xs = (const blk_q4k*)xv;
    const blk_q8k* ys = (const blk_q8k*)yv;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (size_t b = 0; b < n / QK_K; b++) {
        const blk_q4k* x = &xs[b];
        const blk_q8k* y = &ys[b];
        uint8_t scales[8], mins[8];
        orc_q4k_unpack_scales_kmask(x->scales, scales, mins);
        int8_t aux8[QK_K];
        for (int i = 0; i < 4; i++) {
            for (int l = 0; l < 32; l++) aux8[64 * i + l] = (int8_t)(x->qs[32 * i + l] & 0xF);
            for (int l = 0; l < 32; l++) aux8[64 * i + 32 + l] = (int8_t)(x->qs[32 * i + l] >> 4);
        }
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * (int32_t)mins[j / 2];
        int32_t aux32[8] = {0};
        int p = 0;
        for (int s = 0; s < 8; s++) {
            int32_t scale = scales[s];
            for (int r = 0; r < 4; r++) {
                for (int l = 0; l < 8; l++) {
                    int16_t a16 = (int16_t)((int16_t)y->qs[p + l] * (int16_t)aux8[p + l]);
                    aux32[l] += scale * (int32_t)a16;
                }
                p += 8;
            }
        }
        float d = orc_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = orc_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

/* ------------------------------------------------------------ Q6_K */

/* utils.rs:65-202 make_qx_quants.  The _ex form also reports, for the tests
 * that pin it, info[4] = {passes of the first (whole-block) refinement loop,
 * passes of the per-element loop, elements the last per-element pass
 * changed, whole-block passes whose levels were kept}, and the stored levels
 * as the whole-block loop left them (ls_mid, n bytes); both may be NULL. */
float orc_make_qx_quants_ex(int n, int nmax, const float* x, int8_t* ls, int rmse_type, int32_t* info,
                            int8_t* ls_mid) {
    if (info) info[0] = info[1] = info[2] = info[3] = 0;
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) ls[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; i++) {
            int32_t l = nearest_int(iscale * x[i]);
            ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        return 1.0f / iscale;
    }
    int weight_type = rmse_type % 2;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        float xi = x[i];
        int32_t l = clampi(nearest_int(iscale * xi), -nmax, nmax - 1);
        ls[i] = (int8_t)(l + nmax);
        float w = weight_type == 1 ? xi * xi : 1.0f;
        float lf = (float)l;
        sumlx += w * xi * lf;
        suml2 += w * lf * lf;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int itry = 0; itry < 3; itry++) {
        if (info) info[0] = itry + 1;
        float is2 = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        int changed = 0;
        for (int i = 0; i < n; i++) {
            float xi = x[i];
            int32_t l = clampi(nearest_int(is2 * xi), -nmax, nmax - 1);
            if (l + nmax != (int32_t)ls[i]) changed = 1;
            float w = weight_type == 1 ? xi * xi : 1.0f;
            float lf = (float)l;
            slx += w * xi * lf;
            sl2 += w * lf * lf;
        }
        if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
        for (int i = 0; i < n; i++) {
            int32_t l = nearest_int(is2 * x[i]);
            ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
        }
        sumlx = slx;
        suml2 = sl2;
        scale = sumlx / suml2;
        best = scale * sumlx;
        if (info) info[3] = itry + 1;
    }
    if (ls_mid) memcpy(ls_mid, ls, (size_t)n);
    for (int itry = 0; itry < 5; itry++) {
        int n_changed = 0;
        if (info) info[1] = itry + 1;
        for (int i = 0; i < n; i++) {
            float xi = x[i];
            float w = weight_type == 1 ? xi * xi : 1.0f;
            int32_t l = (int32_t)ls[i] - nmax;
            float slx = sumlx - w * xi * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int32_t new_l = clampi(nearest_int(xi * sl2 / slx), -nmax, nmax - 1);
                if (new_l != l) {
                    slx += w * xi * (float)new_l;
                    sl2 += w * (float)new_l * (float)new_l;
                    if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                        ls[i] = (int8_t)(nmax + new_l);
                        sumlx = slx;
                        suml2 = sl2;
                        scale = sumlx / suml2;
                        best = scale * sumlx;
                        n_changed++;
                    }
                }
            }
        }
        if (info) info[2] = n_changed;
        if (n_changed == 0) break;
    }
    if (rmse_type < 3) return scale;
    for (int is = -4; is < 4; is++) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        float slx = 0.0f, sl2 = 0.0f;
        for (int i = 0; i < n; i++) {
            float xi = x[i];
            int32_t l = clampi(nearest_int(iscale * xi), -nmax, nmax - 1);
            float w = weight_type == 1 ? xi * xi : 1.0f;
            float lf = (float)l;
            slx += w * xi * lf;
            sl2 += w * lf * lf;
        }
        if (sl2 > 0.0f && slx * slx > best * sl2) {
            for (int i = 0; i < n; i++) {
                int32_t l = nearest_int(iscale * x[i]);
                ls[i] = (int8_t)(nmax + clampi(l, -nmax, nmax - 1));
            }
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    return scale;
}

float orc_make_qx_quants(int n, int nmax, const float* x, int8_t* ls, int rmse_type) {
    return orc_make_qx_quants_ex(n, nmax, x, ls, rmse_type, NULL, NULL);
}

/* k_quants.rs:1801-1871 BlockQ6K::from_float */
void orc_q6k_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q6k* ys = (blk_q6k*)out;
    int8_t L[QK_K];
    memset(L, 0, sizeof L);
    float scales[16];
    for (size_t bi = 0; bi < nblocks; bi++) {
        const float* x = xs + bi * QK_K;
        blk_q6k* y = &ys[bi];
        memset(y, 0, sizeof *y);
        float max_scale = 0.0f, max_abs_scale = 0.0f;
        for (int ib = 0; ib < 16; ib++) {
            float scale = orc_make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, 1);
            scales[ib] = scale;
            float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) { max_abs_scale = abs_scale; max_scale = scale; }
        }
        float iscale = -128.0f / max_scale;
        y->d = orc_f32_to_f16(1.0f / iscale);
        for (int j = 0; j < 16; j++) {
            int32_t v = nearest_int(iscale * scales[j]);
            if (v > 127) v = 127;
            y->scales[j] = (int8_t)v;
        }
        for (int j = 0; j < 16; j++) {
            float d = orc_f16_to_f32(y->d) * (float)y->scales[j];
            if (d == 0.0f) continue;
            for (int ii = 0; ii < 16; ii++) {
                int32_t ll = clampi(nearest_int(x[16 * j + ii] / d), -32, 31);
                L[16 * j + ii] = (int8_t)(ll + 32);
            }
        }
        uint8_t* ql = y->ql;
        uint8_t* qh = y->qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; l++) {
                uint8_t q1 = (uint8_t)(L[j + l] & 0xF);
                uint8_t q2 = (uint8_t)(L[j + l + 32] & 0xF);
                uint8_t q3 = (uint8_t)(L[j + l + 64] & 0xF);
                uint8_t q4 = (uint8_t)(L[j + l + 96] & 0xF);
                ql[l] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                  ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
    }
}

/* k_quants.rs:1874-1904 */
void orc_q6k_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q6k* xs = (const blk_q6k*)in;
    for (size_t bi = 0; bi < nblocks; bi++) {
        const blk_q6k* x = &xs[bi];
        float d = orc_f16_to_f32(x->d);
        for (int n = 0; n < QK_K; n += 128) {
            int idx = n / 128;
            float* y = ys + bi * QK_K + n;
            const int8_t* sc = x->scales + 8 * idx;
            const uint8_t* ql = x->ql + 64 * idx;
            const uint8_t* qh = x->qh + 32 * idx;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int8_t q1 = (int8_t)(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
                int8_t q2 = (int8_t)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                int8_t q3 = (int8_t)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                int8_t q4 = (int8_t)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                y[l] = d * (float)sc[is] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

static void q6k_unpack(const blk_q6k* x, int8_t* aux8) {
    for (int j = 0; j < QK_K; j += 128) {
        const uint8_t* q4 = x->ql + j / 2;
        const uint8_t* qh = x->qh + j / 4;
        int8_t* a = aux8 + j;
        for (int l = 0; l < 32; l++) {
            a[l] = (int8_t)(((q4[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
            a[l + 32] = (int8_t)(((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
            a[l + 64] = (int8_t)(((q4[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            a[l + 96] = (int8_t)(((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
        }
    }
}

/* Integer part of one Q6K x Q8K super-block dot:
 * sum_{j<16} scales[j] * sum_{16} (q6-32)*q8  (exact; the reference holds it
 * in f32 lanes, k_quants.rs:1743-1798, which is exact at these magnitudes). */
void orc_q6k_block_ints(const void* xv, const void* yv, int64_t* out) {
    const blk_q6k* x = (const blk_q6k*)xv;
    const blk_q8k* y = (const blk_q8k*)yv;
    int8_t aux8[QK_K];
    q6k_unpack(x, aux8);
    int64_t t = 0;
    for (int j = 0; j < 16; j++) {
        int32_t s = 0;
        for (int l = 0; l < 16; l++) s += (int32_t)y->qs[16 * j + l] * (int32_t)aux8[16 * j + l];
        t += (int64_t)x->scales[j] * s;
    }
    out[0] = t;
}

/* k_quants.rs:1743-1798 vec_dot_unopt (Q6K x Q8K) */
float orc_q6k_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q6k* xs = (const blk_q6k*)xv;
    const blk_q8k* ys = (const blk_q8k*)yv;
    int8_t aux8[QK_K];
    float sums[8] = {0};
    for (size_t b = 0; b < n / QK_K; b++) {
        const blk_q6k* x = &xs[b];
        const blk_q8k* y = &ys[b];
        float aux32[8] = {0};
        q6k_unpack(x, aux8);
        for (int j = 0; j < 16; j++) {
            float scale = (float)x->scales[j];
            const int8_t* q8 = y->qs + 16 * j;
            const int8_t* a8 = aux8 + 16 * j;
            for (int l = 0; l < 8; l++) aux32[l] += scale * (float)(int16_t)((int16_t)q8[l] * (int16_t)a8[l]);
            for (int l = 0; l < 8; l++) aux32[l] += scale * (float)(int16_t)((int16_t)q8[8 + l] * (int16_t)a8[8 + l]);
        }
        float d = orc_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += aux32[l] * d;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

/* ----------------------------------------------------- matmul driver */

static size_t type_size(int dt) {
    switch (dt) {
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q8_0: return 34;
    case ORC_Q8_1: return 36;
    case ORC_Q2K: return 84;
    case ORC_Q3K: return 110;
    case ORC_Q4K: return 144;
    case ORC_Q5K: return 176;
    case ORC_Q6K: return 210;
    case ORC_Q8K: return 292;
    }
    return 0;
}
static size_t block_size(int dt) { return dt <= ORC_Q8_1 ? 32 : 256; }

size_t orc_type_size(int dt) { return type_size(dt); }
size_t orc_block_size(int dt) { return block_size(dt); }

/* The activation ("vec dot") type of each weight type, k_quants.rs:210, 310,
 * 405, 507, 615, 883, 1059, 1321, 1510, 1727. */
int orc_vec_dot_type(int dt) {
    switch (dt) {
    case ORC_Q4_0: case ORC_Q5_0: case ORC_Q8_0: return ORC_Q8_0;
    case ORC_Q4_1: case ORC_Q5_1: return ORC_Q8_1;
    }
    return ORC_Q8K;
}

int orc_from_float(int dt, const float* xs, void* out, size_t nblocks) {
    switch (dt) {
    case ORC_Q4_0: orc_q4_0_from_float(xs, out, nblocks); return 0;
    case ORC_Q4_1: orc_q4_1_from_float(xs, out, nblocks); return 0;
    case ORC_Q5_0: orc_q5_0_from_float(xs, out, nblocks); return 0;
    case ORC_Q5_1: orc_q5_1_from_float(xs, out, nblocks); return 0;
    case ORC_Q8_0: orc_q8_0_from_float(xs, out, nblocks); return 0;
    case ORC_Q8_1: orc_q8_1_from_float(xs, out, nblocks); return 0;
    case ORC_Q2K: orc_q2k_from_float(xs, out, nblocks); return 0;
    case ORC_Q3K: orc_q3k_from_float(xs, out, nblocks); return 0;
    case ORC_Q4K: orc_q4k_from_float(xs, out, nblocks); return 0;
    case ORC_Q5K: orc_q5k_from_float(xs, out, nblocks); return 0;
    case ORC_Q6K: orc_q6k_from_float(xs, out, nblocks); return 0;
    case ORC_Q8K: orc_q8k_from_float(xs, out, nblocks); return 0;
    }
    return -1;
}

int orc_to_float(int dt, const void* in, float* ys, size_t nblocks) {
    switch (dt) {
    case ORC_Q4_0: orc_q4_0_to_float(in, ys, nblocks); return 0;
    case ORC_Q4_1: orc_q4_1_to_float(in, ys, nblocks); return 0;
    case ORC_Q5_0: orc_q5_0_to_float(in, ys, nblocks); return 0;
    case ORC_Q5_1: orc_q5_1_to_float(in, ys, nblocks); return 0;
    case ORC_Q8_0: orc_q8_0_to_float(in, ys, nblocks); return 0;
    case ORC_Q2K: orc_q2k_to_float(in, ys, nblocks); return 0;
    case ORC_Q3K: orc_q3k_to_float(in, ys, nblocks); return 0;
    case ORC_Q4K: orc_q4k_to_float(in, ys, nblocks); return 0;
    case ORC_Q5K: orc_q5k_to_float(in, ys, nblocks); return 0;
    case ORC_Q6K: orc_q6k_to_float(in, ys, nblocks); return 0;
    case ORC_Q8K: orc_q8k_to_float(in, ys, nblocks); return 0;
    }
    return -1;
}

float orc_vec_dot(int dt, size_t k, const void* w_row, const void* a_row) {
    switch (dt) {
    case ORC_Q4_0: return orc_q4_0_vec_dot(k, w_row, a_row);
    case ORC_Q4_1: return orc_q4_1_vec_dot(k, w_row, a_row);
    case ORC_Q5_0: return orc_q5_0_vec_dot(k, w_row, a_row);
    case ORC_Q5_1: return orc_q5_1_vec_dot(k, w_row, a_row);
    case ORC_Q8_0: return orc_q8_0_vec_dot(k, w_row, a_row);
    case ORC_Q2K: return orc_q2k_vec_dot(k, w_row, a_row);
    case ORC_Q3K: return orc_q3k_vec_dot(k, w_row, a_row);
    case ORC_Q4K: return orc_q4k_vec_dot(k, w_row, a_row);
    case ORC_Q5K: return orc_q5k_vec_dot(k, w_row, a_row);
    case ORC_Q6K: return orc_q6k_vec_dot(k, w_row, a_row);
    }
    return NAN;
}

/* k_quants.rs:2014-2026 quantize_lhs: m rows of k floats -> m*(k/bs) blocks */
int orc_quantize_lhs(int dt, size_t m, size_t k, const float* lhs, void* out) {
    int vt = orc_vec_dot_type(dt);
    size_t bs = block_size(vt);
    if (k % bs) return -1;
    size_t kb = k / bs;
    for (size_t r = 0; r < m; r++)
        orc_from_float(vt, lhs + r * k, (char*)out + r * kb * type_size(vt), kb);
    return 0;
}

/* k_quants.rs:52-90 matmul_by_row over pre-quantized lhs blocks. */
int orc_matmul_preq(int dt, size_t m, size_t k, size_t n, const void* lhs_b, const void* rhs,
                    float* dst) {
    int vt = orc_vec_dot_type(dt);
    size_t bs = block_size(dt);
    if (k % bs) return -1;
    /* vec_dot_q4_1_q8_1 / q5_0_q8_0 / q5_1_q8_1: "nb is not divisible by 2"
     * (k_quants.rs:323-325, 413-415, 519-521) */
    if ((dt == ORC_Q4_1 || dt == ORC_Q5_0 || dt == ORC_Q5_1) && (k / bs) % 2) return -3;
    size_t kb_w = k / bs, kb_a = k / block_size(vt);
    size_t ws = type_size(dt), as = type_size(vt);
    for (size_t r = 0; r < m; r++) {
        const char* a = (const char*)lhs_b + r * kb_a * as;
        for (size_t c = 0; c < n; c++)
            dst[r * n + c] = orc_vec_dot(dt, k, (const char*)rhs + c * kb_w * ws, a);
    }
    return 0;
}

/* k_quants.rs:1996-2011 matmul: quantize_lhs then matmul_by_row. */
int orc_matmul(int dt, size_t m, size_t k, size_t n, const float* lhs, const void* rhs, float* dst) {
    int vt = orc_vec_dot_type(dt);
    size_t bs = block_size(dt);
    if (k % bs || k % block_size(vt)) return -1;
    size_t kb_a = k / block_size(vt);
    void* lb = malloc(m * kb_a * type_size(vt) + 1);
    if (!lb) return -2;
    memset(lb, 0, m * kb_a * type_size(vt));
    orc_quantize_lhs(dt, m, k, lhs, lb);
    int r = orc_matmul_preq(dt, m, k, n, lb, rhs, dst);
    free(lb);
    return r;
}
