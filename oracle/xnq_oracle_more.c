/*
 * xnq_oracle_more.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Scalar C restatement of the remaining GGUF block types of xn's CPU
 * quantized path (gradium-ai/xn, xn-core/src/quantized/k_quants.rs and
 * utils.rs): Q4_1, Q5_0, Q5_1 (with their activation type Q8_1), Q2_K,
 * Q3_K and Q5_K.  Same conventions as xnq_oracle.c (Rust float->int casts
 * saturate, f16 is IEEE binary16 with round-to-nearest-even, no contracted
 * multiply-add).  Only tests/ and the smoke() hook load it.
 *
 * Block layouts (bytes, little endian), k_quants.rs:100-188:
 *   BlockQ4_1  20 B { f16 d; f16 m; u8 qs[16]; }
 *   BlockQ5_0  22 B { f16 d; u8 qh[4]; u8 qs[16]; }
 *   BlockQ5_1  24 B { f16 d; f16 m; u8 qh[4]; u8 qs[16]; }
 *   BlockQ8_1  36 B { f16 d; f16 s; i8 qs[32]; }
 *   BlockQ2K   84 B { u8 scales[16]; u8 qs[64]; f16 d; f16 dmin; }
 *   BlockQ3K  110 B { u8 hmask[32]; u8 qs[64]; u8 scales[12]; f16 d; }
 *   BlockQ5K  176 B { f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]; }
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
float orc_make_qkx1_quants(int nmax, int ntry, const float* x, int n, float* neg_min);

#define QK_K 256

#pragma pack(push, 1)
typedef struct { uint16_t d; uint16_t m; uint8_t qs[16]; } blk_q4_1;
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_0;
typedef struct { uint16_t d; uint16_t m; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_1;
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0m;
typedef struct { uint16_t d; uint16_t s; int8_t qs[32]; } blk_q8_1;
typedef struct { uint8_t scales[16]; uint8_t qs[64]; uint16_t d; uint16_t dmin; } blk_q2k;
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } blk_q3k;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } blk_q5k;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } blk_q8km;
#pragma pack(pop)

_Static_assert(sizeof(blk_q4_1) == 20, "q4_1");
_Static_assert(sizeof(blk_q5_0) == 22, "q5_0");
_Static_assert(sizeof(blk_q5_1) == 24, "q5_1");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1");
_Static_assert(sizeof(blk_q2k) == 84, "q2k");
_Static_assert(sizeof(blk_q3k) == 110, "q3k");
_Static_assert(sizeof(blk_q5k) == 176, "q5k");

/* Rust `f32 as u8 / i8 / i32`: saturating, NaN -> 0 */
static uint8_t as_u8(float v) {
    if (v != v || v <= 0.0f) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)(int)v;
}
static int8_t as_i8(float v) {
    if (v != v) return 0;
    if (v <= -128.0f) return -128;
    if (v >= 127.0f) return 127;
    return (int8_t)(int)v;
}
static int32_t as_i32(float v) {
    if (v != v) return 0;
    if (v <= -2147483648.0f) return INT32_MIN;
    if (v >= 2147483647.0f) return INT32_MAX;
    return (int32_t)v;
}
/* utils.rs:3-5 */
static int32_t nearest(float v) { return as_i32(roundf(v)); }
static int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
static uint32_t rd32(const uint8_t* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}
static void wr32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }

/* half 2.7.1: f16 * f16 computes in f32 and rounds back to f16 */
static uint16_t f16_mul(uint16_t a, uint16_t b) {
    return orc_f32_to_f16(orc_f16_to_f32(a) * orc_f16_to_f32(b));
}

/* ------------------------------------------------------------ Q8_1 */

/* k_quants.rs:847-873 BlockQ8_1::from_float */
void orc_q8_1_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q8_1* ys = (blk_q8_1*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        ys[i].d = orc_f32_to_f16(d);
        int32_t sum = 0;
        for (int j = 0; j < 16; j++) {
            ys[i].qs[j] = as_i8(roundf(x[j] * id));
            ys[i].qs[j + 16] = as_i8(roundf(x[j + 16] * id));
            sum += (int32_t)ys[i].qs[j] + (int32_t)ys[i].qs[j + 16];
        }
        ys[i].s = f16_mul(orc_f32_to_f16((float)sum), ys[i].d);
    }
}

/* ------------------------------------------------------------ Q4_1 */

/* k_quants.rs:345-377 BlockQ4_1::from_float */
void orc_q4_1_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q4_1* ys = (blk_q4_1*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * 32;
        float min = INFINITY, max = -INFINITY;
        for (int j = 0; j < 32; j++) {
            min = fminf(x[j], min);
            max = fmaxf(x[j], max);
        }
        float d = (max - min) / 15.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        ys[i].d = orc_f32_to_f16(d);
        ys[i].m = orc_f32_to_f16(min);
        for (int j = 0; j < 16; j++) {
            float x0 = (x[j] - min) * id;
            float x1 = (x[16 + j] - min) * id;
            uint8_t xi0 = as_u8(x0 + 0.5f), xi1 = as_u8(x1 + 0.5f);
            if (xi0 > 15) xi0 = 15;
            if (xi1 > 15) xi1 = 15;
            ys[i].qs[j] = (uint8_t)(xi0 | (xi1 << 4));
        }
    }
}

/* k_quants.rs:379-399 */
void orc_q4_1_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q4_1* xs = (const blk_q4_1*)in;
    for (size_t i = 0; i < nblocks; i++) {
        float d = orc_f16_to_f32(xs[i].d), m = orc_f16_to_f32(xs[i].m);
        for (int j = 0; j < 16; j++) {
            ys[i * 32 + j] = (float)(xs[i].qs[j] & 0x0F) * d + m;
            ys[i * 32 + j + 16] = (float)(xs[i].qs[j] >> 4) * d + m;
        }
    }
}

/* k_quants.rs:316-343 vec_dot_unopt (Q4_1 x Q8_1) */
float orc_q4_1_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q4_1* xs = (const blk_q4_1*)xv;
    const blk_q8_1* ys = (const blk_q8_1*)yv;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) {
            int32_t v0 = xs[b].qs[j] & 0x0F, v1 = xs[b].qs[j] >> 4;
            sumi += v0 * ys[b].qs[j] + v1 * ys[b].qs[j + 16];
        }
        sumf += (float)sumi * orc_f16_to_f32(xs[b].d) * orc_f16_to_f32(ys[b].d) +
                orc_f16_to_f32(xs[b].m) * orc_f16_to_f32(ys[b].s);
    }
    return sumf;
}

/* ------------------------------------------------------------ Q5_0 */

/* k_quants.rs:442-476 BlockQ5_0::from_float */
void orc_q5_0_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q5_0* ys = (blk_q5_0*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * 32;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++)
            if (amax < fabsf(x[j])) { amax = fabsf(x[j]); max = x[j]; }
        float d = max / -16.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        ys[i].d = orc_f32_to_f16(d);
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            float x0 = x[j] * id, x1 = x[j + 16] * id;
            int8_t a0 = as_i8(x0 + 16.5f), a1 = as_i8(x1 + 16.5f);
            uint8_t xi0 = (uint8_t)(a0 < 31 ? a0 : 31), xi1 = (uint8_t)(a1 < 31 ? a1 : 31);
            ys[i].qs[j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
            qh |= (((uint32_t)xi0 & 0x10) >> 4) << j;
            qh |= (((uint32_t)xi1 & 0x10) >> 4) << (j + 16);
        }
        wr32(ys[i].qh, qh);
    }
}

/* k_quants.rs:478-502 */
void orc_q5_0_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q5_0* xs = (const blk_q5_0*)in;
    for (size_t i = 0; i < nblocks; i++) {
        float d = orc_f16_to_f32(xs[i].d);
        uint32_t qh = rd32(xs[i].qh);
        for (int j = 0; j < 16; j++) {
            uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10), xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
            int32_t x0 = (int32_t)((xs[i].qs[j] & 0x0F) | xh0) - 16;
            int32_t x1 = (int32_t)((xs[i].qs[j] >> 4) | xh1) - 16;
            ys[i * 32 + j] = (float)x0 * d;
            ys[i * 32 + j + 16] = (float)x1 * d;
        }
    }
}

/* k_quants.rs:419-440 vec_dot_unopt (Q5_0 x Q8_0) */
float orc_q5_0_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q5_0* xs = (const blk_q5_0*)xv;
    const blk_q8_0m* ys = (const blk_q8_0m*)yv;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        uint32_t qh = rd32(xs[b].qh);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) {
            uint8_t xh0 = (uint8_t)(((qh & (1u << j)) >> j) << 4);
            uint8_t xh1 = (uint8_t)((qh & (1u << (j + 16))) >> (j + 12));
            int32_t x0 = (int32_t)((xs[b].qs[j] & 0x0F) | xh0) - 16;
            int32_t x1 = (int32_t)((xs[b].qs[j] >> 4) | xh1) - 16;
            sumi += x0 * ys[b].qs[j] + x1 * ys[b].qs[j + 16];
        }
        sumf += (float)sumi * orc_f16_to_f32(xs[b].d) * orc_f16_to_f32(ys[b].d);
    }
    return sumf;
}

/* ------------------------------------------------------------ Q5_1 */

/* k_quants.rs:546-583 BlockQ5_1::from_float */
void orc_q5_1_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q5_1* ys = (blk_q5_1*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * 32;
        float min = INFINITY, max = -INFINITY;
        for (int j = 0; j < 32; j++) {
            min = fminf(x[j], min);
            max = fmaxf(x[j], max);
        }
        float d = (max - min) / 31.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        ys[i].d = orc_f32_to_f16(d);
        ys[i].m = orc_f32_to_f16(min);
        uint32_t qh = 0;
        for (int j = 0; j < 16; j++) {
            float x0 = (x[j] - min) * id, x1 = (x[16 + j] - min) * id;
            uint8_t xi0 = as_u8(x0 + 0.5f), xi1 = as_u8(x1 + 0.5f);
            ys[i].qs[j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
            qh |= (((uint32_t)xi0 & 0x10) >> 4) << j;
            qh |= (((uint32_t)xi1 & 0x10) >> 4) << (j + 16);
        }
        wr32(ys[i].qh, qh);
    }
}

/* k_quants.rs:585-609 */
void orc_q5_1_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q5_1* xs = (const blk_q5_1*)in;
    for (size_t i = 0; i < nblocks; i++) {
        float d = orc_f16_to_f32(xs[i].d), m = orc_f16_to_f32(xs[i].m);
        uint32_t qh = rd32(xs[i].qh);
        for (int j = 0; j < 16; j++) {
            uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10), xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
            uint8_t x0 = (uint8_t)((xs[i].qs[j] & 0x0F) | xh0), x1 = (uint8_t)((xs[i].qs[j] >> 4) | xh1);
            ys[i * 32 + j] = (float)x0 * d + m;
            ys[i * 32 + j + 16] = (float)x1 * d + m;
        }
    }
}

/* k_quants.rs:513-544 vec_dot_unopt (Q5_1 x Q8_1) */
float orc_q5_1_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q5_1* xs = (const blk_q5_1*)xv;
    const blk_q8_1* ys = (const blk_q8_1*)yv;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / 32; b++) {
        uint32_t qh = rd32(xs[b].qh);
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) {
            uint32_t xh0 = ((qh >> j) << 4) & 0x10, xh1 = (qh >> (j + 12)) & 0x10;
            int32_t x0 = (int32_t)((xs[b].qs[j] & 0xF) | xh0), x1 = (int32_t)((xs[b].qs[j] >> 4) | xh1);
            sumi += x0 * ys[b].qs[j] + x1 * ys[b].qs[j + 16];
        }
        sumf += (float)sumi * orc_f16_to_f32(xs[b].d) * orc_f16_to_f32(ys[b].d) +
                orc_f16_to_f32(xs[b].m) * orc_f16_to_f32(ys[b].s);
    }
    return sumf;
}

/* ------------------------------------------------------------ Q2_K */

/* k_quants.rs:951-1011 BlockQ2K::from_float (make_qkx1_quants(3, 5, .) per 16) */
void orc_q2k_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q2k* ys = (blk_q2k*)out;
    const float q4scale = 15.0f;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * QK_K;
        blk_q2k* b = &ys[i];
        float mins[16], scales[16];
        for (int j = 0; j < 16; j++) scales[j] = orc_make_qkx1_quants(3, 5, x + 16 * j, 16, &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 16; j++) max_scale = fmaxf(scales[j], max_scale);
        for (int j = 0; j < 16; j++) max_min = fmaxf(mins[j], max_min);
        if (max_scale > 0.0f) {
            float iscale = q4scale / max_scale;
            for (int j = 0; j < 16; j++) b->scales[j] = (uint8_t)nearest(iscale * scales[j]);
            b->d = orc_f32_to_f16(max_scale / q4scale);
        } else {
            memset(b->scales, 0, 16);
            b->d = orc_f32_to_f16(0.0f);
        }
        if (max_min > 0.0f) {
            float iscale = q4scale / max_min;
            for (int j = 0; j < 16; j++) {
                uint8_t l = (uint8_t)nearest(iscale * mins[j]);
                b->scales[j] = (uint8_t)(b->scales[j] | (uint8_t)(l << 4));
            }
            b->dmin = orc_f32_to_f16(max_min / q4scale);
        } else {
            b->dmin = orc_f32_to_f16(0.0f);
        }
        uint8_t L[QK_K];
        memset(L, 0, sizeof L);
        for (int j = 0; j < 16; j++) {
            float d = orc_f16_to_f32(b->d) * (float)(b->scales[j] & 0xF);
            if (d == 0.0f) continue;
            float dm = orc_f16_to_f32(b->dmin) * (float)(b->scales[j] >> 4);
            for (int ii = 0; ii < 16; ii++) L[16 * j + ii] = (uint8_t)clampi(nearest((x[16 * j + ii] + dm) / d), 0, 3);
        }
        for (int j = 0; j < QK_K; j += 128)
            for (int l = 0; l < 32; l++)
                b->qs[j / 4 + l] =
                    (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
    }
}

/* k_quants.rs:1014-1053 */
void orc_q2k_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q2k* xs = (const blk_q2k*)in;
    for (size_t i = 0; i < nblocks; i++) {
        const blk_q2k* b = &xs[i];
        float d = orc_f16_to_f32(b->d), min = orc_f16_to_f32(b->dmin);
        float* y = ys + i * QK_K;
        int is = 0, yi = 0;
        for (int h = 0; h < 2; h++) {
            const uint8_t* q = b->qs + 32 * h;
            for (int shift = 0; shift < 8; shift += 2) {
                for (int g = 0; g < 2; g++) {
                    uint8_t sc = b->scales[is++];
                    float dl = d * (float)(sc & 0xF), ml = min * (float)(sc >> 4);
                    for (int l = 0; l < 16; l++) y[yi++] = dl * (float)((q[16 * g + l] >> shift) & 3) - ml;
                }
            }
        }
    }
}

/* Integer parts of one Q2K x Q8K super-block dot (k_quants.rs:899-948):
 * out[0] = isum = sum_g (sc_g & 15) * sum_{16} q8 * q2,  out[1] = summs */
void orc_q2k_block_ints(const void* xv, const void* yv, int64_t* out) {
    const blk_q2k* x = (const blk_q2k*)xv;
    const blk_q8km* y = (const blk_q8km*)yv;
    int32_t summs = 0;
    for (int g = 0; g < 16; g++) summs += (int32_t)y->bsums[g] * (int32_t)(x->scales[g] >> 4);
    int32_t isum = 0;
    int is = 0, p = 0;
    for (int h = 0; h < 2; h++) {
        const uint8_t* q2 = x->qs + 32 * h;
        for (int shift = 0; shift < 8; shift += 2) {
            for (int g = 0; g < 2; g++) {
                int32_t d = x->scales[is++] & 0xF;
                int32_t isuml = 0;
                for (int l = 16 * g; l < 16 * g + 16; l++) isuml += (int32_t)y->qs[p + l] * ((q2[l] >> shift) & 3);
                isum += d * isuml;
            }
            p += 32;
        }
    }
    out[0] = isum;
    out[1] = summs;
}

/* k_quants.rs:899-948 vec_dot_unopt (Q2K x Q8K) */
float orc_q2k_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q2k* xs = (const blk_q2k*)xv;
    const blk_q8km* ys = (const blk_q8km*)yv;
    float sumf = 0.0f;
    for (size_t b = 0; b < n / QK_K; b++) {
        int64_t ints[2];
        orc_q2k_block_ints(&xs[b], &ys[b], ints);
        float dall = ys[b].d * orc_f16_to_f32(xs[b].d);
        float dmin = ys[b].d * orc_f16_to_f32(xs[b].dmin);
        sumf += dall * (float)(int32_t)ints[0] - dmin * (float)(int32_t)ints[1];
    }
    return sumf;
}

/* ------------------------------------------------------------ Q3_K */

/* utils.rs:257-320 make_q3_quants.  The _ex form also reports, for the tests
 * that pin it, info[2] = {passes of the per-element loop, elements its last
 * pass changed}; info may be NULL. */
float orc_make_q3_quants_ex(const float* x, int n, int nmax, int do_rmse, int8_t* lout, int32_t* info) {
    if (info) info[0] = info[1] = 0;
    int8_t l[QK_K];
    memset(l, 0, sizeof l);
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax == 0.0f) {
        if (lout) memcpy(lout, l, (size_t)n);
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    if (do_rmse) {
        float sumlx = 0.0f, suml2 = 0.0f;
        for (int i = 0; i < n; i++) {
            int32_t li = clampi(as_i32(roundf(iscale * x[i])), -nmax, nmax - 1);
            l[i] = (int8_t)li;
            float w = x[i] * x[i];
            sumlx += w * x[i] * (float)li;
            suml2 += w * (float)(li * li);
        }
        for (int it = 0; it < 5; it++) {
            int n_changed = 0;
            if (info) info[0] = it + 1;
            for (int i = 0; i < n; i++) {
                float w = x[i] * x[i];
                float slx = sumlx - w * x[i] * (float)l[i];
                if (slx > 0.0f) {
                    float sl2 = suml2 - w * (float)((int32_t)l[i] * (int32_t)l[i]);
                    int32_t new_l = clampi(as_i32(roundf(x[i] * sl2 / slx)), -nmax, nmax - 1);
                    if (new_l != (int32_t)l[i]) {
                        slx += w * x[i] * (float)new_l;
                        sl2 += w * (float)(new_l * new_l);
                        if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
                            l[i] = (int8_t)new_l;
                            sumlx = slx;
                            suml2 = sl2;
                            n_changed++;
                        }
                    }
                }
            }
            if (info) info[1] = n_changed;
            if (n_changed == 0) break;
        }
        for (int i = 0; i < n; i++) l[i] = (int8_t)(l[i] + nmax);
        if (lout) memcpy(lout, l, (size_t)n);
        return sumlx / suml2;
    }
    for (int i = 0; i < n; i++) {
        int32_t li = as_i32(roundf(iscale * x[i]));
        l[i] = (int8_t)(clampi(li, -nmax, nmax - 1) + nmax);
    }
    if (lout) memcpy(lout, l, (size_t)n);
    return 1.0f / iscale;
}

float orc_make_q3_quants(const float* x, int n, int nmax, int do_rmse, int8_t* lout) {
    return orc_make_q3_quants_ex(x, n, nmax, do_rmse, lout, NULL);
}

/* The 16 six-bit scales of a Q3K block (the aux/KMASK shuffle of
 * k_quants.rs:1159-1166 and 1252-1258), as unsigned 0..63. */
void orc_q3k_scales(const uint8_t* sc12, uint8_t* out16) {
    const uint32_t KMASK1 = 0x03030303u, KMASK2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    memcpy(aux, sc12, 12);
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & KMASK2) | (((tmp >> 4) & KMASK1) << 4);
    aux[3] = ((aux[1] >> 4) & KMASK2) | (((tmp >> 6) & KMASK1) << 4);
    aux[0] = (aux[0] & KMASK2) | (((tmp)&KMASK1) << 4);
    aux[1] = (aux[1] & KMASK2) | (((tmp >> 2) & KMASK1) << 4);
    memcpy(out16, aux, 16);
}

/* k_quants.rs:1170-1236 BlockQ3K::from_float */
void orc_q3k_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q3k* ys = (blk_q3k*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * QK_K;
        blk_q3k* b = &ys[i];
        float scales[16];
        for (int j = 0; j < 16; j++) scales[j] = orc_make_q3_quants(x + 16 * j, 16, 4, 1, NULL);
        float max_scale = 0.0f;
        for (int j = 0; j < 16; j++)
            if (fabsf(scales[j]) > fabsf(max_scale)) max_scale = scales[j];
        memset(b->scales, 0, 12);
        if (max_scale != 0.0f) {
            float iscale = -32.0f / max_scale;
            for (int j = 0; j < 16; j++) {
                int32_t l = clampi(nearest(iscale * scales[j]), -32, 31) + 32;
                if (j < 8) b->scales[j] = (uint8_t)(l & 0xF);
                else b->scales[j - 8] = (uint8_t)(b->scales[j - 8] | (uint8_t)((l & 0xF) << 4));
                l >>= 4;
                b->scales[j % 4 + 8] = (uint8_t)(b->scales[j % 4 + 8] | (uint8_t)(l << (2 * (j / 4))));
            }
            b->d = orc_f32_to_f16(1.0f / iscale);
        } else {
            b->d = orc_f32_to_f16(0.0f);
        }
        int8_t L[QK_K];
        memset(L, 0, sizeof L);
        for (int j = 0; j < 16; j++) {
            uint8_t sc = j < 8 ? (uint8_t)(b->scales[j] & 0xF) : (uint8_t)(b->scales[j - 8] >> 4);
            int8_t sci = (int8_t)(uint8_t)(sc | (((b->scales[8 + j % 4] >> (2 * (j / 4))) & 3) << 4));
            sci = (int8_t)(sci - 32);
            float d = orc_f16_to_f32(b->d) * (float)sci;
            if (d != 0.0f)
                for (int ii = 0; ii < 16; ii++)
                    L[16 * j + ii] = (int8_t)(clampi(nearest(x[16 * j + ii] / d), -4, 3) + 4);
        }
        memset(b->hmask, 0, 32);
        int m = 0;
        uint8_t hm = 1;
        for (int e = 0; e < QK_K; e++) {
            if (L[e] > 3) {
                b->hmask[m] |= hm;
                L[e] = (int8_t)(L[e] - 4);
            }
            m++;
            if (m == QK_K / 8) {
                m = 0;
                hm = (uint8_t)(hm << 1);
            }
        }
        for (int j = 0; j < QK_K; j += 128)
            for (int l = 0; l < 32; l++)
                b->qs[j / 4 + l] =
                    (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
    }
}

/* k_quants.rs:1240-1315 */
void orc_q3k_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q3k* xs = (const blk_q3k*)in;
    for (size_t i = 0; i < nblocks; i++) {
        const blk_q3k* b = &xs[i];
        uint8_t sc[16];
        orc_q3k_scales(b->scales, sc);
        float d_all = orc_f16_to_f32(b->d);
        float* y = ys + i * QK_K;
        int is = 0, yi = 0;
        uint8_t m = 1;
        for (int h = 0; h < 2; h++) {
            const uint8_t* q = b->qs + 32 * h;
            for (int shift = 0; shift < 8; shift += 2) {
                for (int g = 0; g < 2; g++) {
                    float dl = d_all * ((float)(int8_t)sc[is] - 32.0f);
                    for (int l = 0; l < 16; l++) {
                        int8_t v = (int8_t)(((q[16 * g + l] >> shift) & 3) - ((b->hmask[16 * g + l] & m) == 0 ? 4 : 0));
                        y[yi++] = dl * (float)v;
                    }
                    is++;
                }
                m = (uint8_t)(m << 1);
            }
        }
    }
}

/* Integer part of one Q3K x Q8K super-block dot (k_quants.rs:1071-1152):
 * out[0] = sum_l aux32[l] = sum_g (sc_g - 32) * sum_{16} q8 * q3, out[1] = 0 */
void orc_q3k_block_ints(const void* xv, const void* yv, int64_t* out, int32_t* aux32_out) {
    const blk_q3k* x = (const blk_q3k*)xv;
    const blk_q8km* y = (const blk_q8km*)yv;
    int8_t aux8[QK_K];
    int p = 0;
    uint8_t m = 1;
    for (int h = 0; h < 2; h++) {
        const uint8_t* q3 = x->qs + 32 * h;
        for (int shift = 0; shift < 8; shift += 2) {
            for (int l = 0; l < 32; l++) {
                int8_t a = (int8_t)((q3[l] >> shift) & 3);
                a = (int8_t)(a - ((x->hmask[l] & m) != 0 ? 0 : 4));
                aux8[p + l] = a;
            }
            p += 32;
            m = (uint8_t)(m << 1);
        }
    }
    uint8_t sc[16];
    orc_q3k_scales(x->scales, sc);
    int32_t aux32[8] = {0};
    p = 0;
    for (int g = 0; g < 16; g++) {
        int32_t scale = (int32_t)(int8_t)sc[g] - 32;
        for (int half = 0; half < 2; half++) {
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
    out[1] = 0;
    if (aux32_out) memcpy(aux32_out, aux32, sizeof aux32);
}

/* k_quants.rs:1071-1152 vec_dot_unopt (Q3K x Q8K) */
float orc_q3k_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q3k* xs = (const blk_q3k*)xv;
    const blk_q8km* ys = (const blk_q8km*)yv;
    float sums[8] = {0};
    for (size_t b = 0; b < n / QK_K; b++) {
        int64_t ints[2];
        int32_t aux32[8];
        orc_q3k_block_ints(&xs[b], &ys[b], ints, aux32);
        float d = orc_f16_to_f32(xs[b].d) * ys[b].d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

/* ------------------------------------------------------------ Q5_K */

static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    /* utils.rs:53-63 get_scale_min_k4 */
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* k_quants.rs:1608-1679 BlockQ5K::from_float (make_qkx1_quants(31, 5, .) per 32) */
void orc_q5k_from_float(const float* xs, void* out, size_t nblocks) {
    blk_q5k* ys = (blk_q5k*)out;
    for (size_t i = 0; i < nblocks; i++) {
        const float* x = xs + i * QK_K;
        blk_q5k* b = &ys[i];
        float mins[8], scales[8];
        for (int j = 0; j < 8; j++) scales[j] = orc_make_qkx1_quants(31, 5, x + 32 * j, 32, &mins[j]);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) max_scale = fmaxf(scales[j], max_scale);
        for (int j = 0; j < 8; j++) max_min = fmaxf(mins[j], max_min);
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        memset(b->scales, 0, 12);
        for (int j = 0; j < 8; j++) {
            int32_t ls0 = nearest(inv_scale * scales[j]), lm0 = nearest(inv_min * mins[j]);
            uint8_t ls = (uint8_t)(ls0 < 63 ? ls0 : 63), lm = (uint8_t)(lm0 < 63 ? lm0 : 63);
            if (j < 4) {
                b->scales[j] = ls;
                b->scales[j + 4] = lm;
            } else {
                b->scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                b->scales[j - 4] = (uint8_t)(b->scales[j - 4] | ((ls >> 4) << 6));
                b->scales[j] = (uint8_t)(b->scales[j] | ((lm >> 4) << 6));
            }
        }
        b->d = orc_f32_to_f16(max_scale / 63.0f);
        b->dmin = orc_f32_to_f16(max_min / 63.0f);
        uint8_t L[QK_K];
        memset(L, 0, sizeof L);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            scale_min_k4(j, b->scales, &sc, &m);
            float d = orc_f16_to_f32(b->d) * (float)sc;
            if (d == 0.0f) continue;
            float dm = orc_f16_to_f32(b->dmin) * (float)m;
            for (int ii = 0; ii < 32; ii++) L[32 * j + ii] = (uint8_t)clampi(nearest((x[32 * j + ii] + dm) / d), 0, 31);
        }
        memset(b->qh, 0, 32);
        uint8_t m1 = 1, m2 = 2;
        for (int nn = 0; nn < QK_K; nn += 64) {
            int off = (nn / 64) * 32;
            for (int j = 0; j < 32; j++) {
                uint8_t l1 = L[nn + j], l2 = L[nn + j + 32];
                if (l1 > 15) { l1 = (uint8_t)(l1 - 16); b->qh[j] |= m1; }
                if (l2 > 15) { l2 = (uint8_t)(l2 - 16); b->qh[j] |= m2; }
                b->qs[off + j] = (uint8_t)(l1 | (l2 << 4));
            }
            m1 = (uint8_t)(m1 << 2);
            m2 = (uint8_t)(m2 << 2);
        }
    }
}

/* k_quants.rs:1682-1721 */
void orc_q5k_to_float(const void* in, float* ys, size_t nblocks) {
    const blk_q5k* xs = (const blk_q5k*)in;
    for (size_t i = 0; i < nblocks; i++) {
        const blk_q5k* b = &xs[i];
        float d = orc_f16_to_f32(b->d), min = orc_f16_to_f32(b->dmin);
        float* y = ys + i * QK_K;
        int is = 0, yi = 0;
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < QK_K; j += 64) {
            const uint8_t* ql = b->qs + j / 2;
            uint8_t sc, m;
            scale_min_k4(is, b->scales, &sc, &m);
            float d1 = d * (float)sc, m1 = min * (float)m;
            scale_min_k4(is + 1, b->scales, &sc, &m);
            float d2 = d * (float)sc, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) y[yi++] = d1 * ((float)(ql[l] & 0xF) + ((b->qh[l] & u1) ? 16.0f : 0.0f)) - m1;
            for (int l = 0; l < 32; l++) y[yi++] = d2 * ((float)(ql[l] >> 4) + ((b->qh[l] & u2) ? 16.0f : 0.0f)) - m2;
            is += 2;
            u1 = (uint8_t)(u1 << 2);
            u2 = (uint8_t)(u2 << 2);
        }
    }
}

/* Integer parts of one Q5K x Q8K super-block dot (k_quants.rs:1524-1605):
 * out[0] = sum_l aux32[l] = sum_j sc_j * sum_{32} q8 * q5, out[1] = sumi */
void orc_q5k_block_ints(const void* xv, const void* yv, int64_t* out, int32_t* aux32_out) {
    const blk_q5k* x = (const blk_q5k*)xv;
    const blk_q8km* y = (const blk_q8km*)yv;
    int8_t aux8[QK_K];
    uint8_t m = 1;
    for (int i = 0; i < 4; i++) {
        const uint8_t* q5 = x->qs + 32 * i;
        for (int l = 0; l < 32; l++) aux8[64 * i + l] = (int8_t)((q5[l] & 0xF) + ((x->qh[l] & m) ? 16 : 0));
        m = (uint8_t)(m << 1);
        for (int l = 0; l < 32; l++) aux8[64 * i + 32 + l] = (int8_t)((q5[l] >> 4) + ((x->qh[l] & m) ? 16 : 0));
        m = (uint8_t)(m << 1);
    }
    /* the utmp/KMASK unpacking of k_quants.rs:1569-1578 gives get_scale_min_k4 */
    uint8_t scales[8], mins[8];
    for (int j = 0; j < 8; j++) scale_min_k4(j, x->scales, &scales[j], &mins[j]);
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
    if (aux32_out) memcpy(aux32_out, aux32, sizeof aux32);
}

/* k_quants.rs:1524-1605 vec_dot_unopt (Q5K x Q8K) */
float orc_q5k_vec_dot(size_t n, const void* xv, const void* yv) {
    const blk_q5k* xs = (const blk_q5k*)xv;
    const blk_q8km* ys = (const blk_q8km*)yv;
    float sums[8] = {0};
    float sumf = 0.0f;
    for (size_t b = 0; b < n / QK_K; b++) {
        int64_t ints[2];
        int32_t aux32[8];
        orc_q5k_block_ints(&xs[b], &ys[b], ints, aux32);
        float d = orc_f16_to_f32(xs[b].d) * ys[b].d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        float dmin = orc_f16_to_f32(xs[b].dmin) * ys[b].d;
        sumf -= dmin * (float)(int32_t)ints[1];
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}
