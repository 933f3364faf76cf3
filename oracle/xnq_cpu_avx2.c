/*
 * xnq_cpu_avx2.c -- TEST / BASELINE INFRASTRUCTURE ONLY.
 *
 * The timed CPU baseline: a C restatement of what xn runs on an x86 host built
 * with `target-cpu=native` (xn .cargo/config.toml:2):
 *   - the AVX2/FMA vec_dots of xn-core/src/quantized/avx.rs
 *       vec_dot_q4_0_q8_0 (61-80), vec_dot_q8_0_q8_0 (82-99),
 *       vec_dot_q6k_q8k (357-443), vec_dot_q4k_q8k (661-743);
 *   - the TinyBLAS Q8_0 x Q8_0 tiling used for Q8_0 weights (avx.rs:187-314,
 *     k_quants.rs:694-760);
 *   - matmul_by_row's 128-column tasks handed out from a shared counter in
 *     runs of ceil(chunks / (8*threads)) (k_quants.rs:52-90,
 *     threadpool.rs:441-466), on a persistent pthread pool.
 * Only bench.py's cpu_baseline leg and tests/ load this library.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4K = 12, ORC_Q6K = 14, ORC_Q8K = 15 };

#pragma pack(push, 1)
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;
typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4k;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6k;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } blk_q8k;
#pragma pack(pop)

/* exported by xnq_oracle.c (same shared object) */
float orc_f16_to_f32(uint16_t h);
int orc_quantize_lhs(int dt, size_t m, size_t k, const float* lhs, void* out);

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

/* avx.rs:13-59 helpers */
static inline __m256 sum_i16_pairs_float(__m256i x) {
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_set1_epi16(1), x));
}
static inline __m256 mul_sum_us8_pairs_float(__m256i ax, __m256i sy) {
    return sum_i16_pairs_float(_mm256_maddubs_epi16(ax, sy));
}
static inline float hsum_float_8(__m256 x) {
    __m128 r = _mm256_extractf128_ps(x, 1);
    r = _mm_add_ps(r, _mm256_castps256_ps128(x));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}
static inline __m256i bytes_from_nibbles_32(const uint8_t* p) {
    __m128i t = _mm_loadu_si128((const __m128i*)p);
    __m256i b = _mm256_insertf128_si256(_mm256_castsi128_si256(t), _mm_srli_epi16(t, 4), 1);
    return _mm256_and_si256(_mm256_set1_epi8(0xF), b);
}
static inline __m256 mul_sum_i8_pairs_float(__m256i x, __m256i y) {
    return mul_sum_us8_pairs_float(_mm256_sign_epi8(x, x), _mm256_sign_epi8(y, x));
}

float cpu_vec_dot_q4_0(size_t n, const void* xv, const void* yv) {
    const blk_q4_0* xs = xv;
    const blk_q8_0* ys = yv;
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < n / 32; b++) {
        __m256 d = _mm256_set1_ps(h2f(xs[b].d) * h2f(ys[b].d));
        __m256i bx = _mm256_sub_epi8(bytes_from_nibbles_32(xs[b].qs), _mm256_set1_epi8(8));
        __m256i by = _mm256_loadu_si256((const __m256i*)ys[b].qs);
        acc = _mm256_fmadd_ps(d, mul_sum_i8_pairs_float(bx, by), acc);
    }
    return hsum_float_8(acc);
}

float cpu_vec_dot_q8_0(size_t n, const void* xv, const void* yv) {
    const blk_q8_0* xs = xv;
    const blk_q8_0* ys = yv;
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < n / 32; b++) {
        __m256 d = _mm256_set1_ps(h2f(xs[b].d) * h2f(ys[b].d));
        __m256i bx = _mm256_loadu_si256((const __m256i*)xs[b].qs);
        __m256i by = _mm256_loadu_si256((const __m256i*)ys[b].qs);
        acc = _mm256_fmadd_ps(d, mul_sum_i8_pairs_float(bx, by), acc);
    }
    return hsum_float_8(acc);
}

/* avx.rs:320-337 shuffle tables, built arithmetically */
static inline __m128i scale_shuffle(int i) {
    uint8_t t[16];
    for (int j = 0; j < 16; j++) t[j] = (uint8_t)(2 * i + j / 8);
    return _mm_loadu_si128((const __m128i*)t);
}
static inline __m256i scale_shuffle_k4(int i) {
    uint8_t t[32];
    for (int j = 0; j < 32; j++) t[j] = (uint8_t)(2 * i + (j & 1));
    return _mm256_loadu_si256((const __m256i*)t);
}

float cpu_vec_dot_q6k(size_t n, const void* xv, const void* yv) {
    const blk_q6k* xs = xv;
    const blk_q8k* ys = yv;
    const __m256i m4 = _mm256_set1_epi8(0xF), m2 = _mm256_set1_epi8(3), m32s = _mm256_set1_epi8(32);
    __m128i shuf[8];
    for (int i = 0; i < 8; i++) shuf[i] = scale_shuffle(i);
    __m256 acc = _mm256_setzero_ps();
    for (size_t b = 0; b < n / 256; b++) {
        const blk_q6k* x = &xs[b];
        const blk_q8k* y = &ys[b];
        float d = y->d * h2f(x->d);
        const uint8_t* q4 = x->ql;
        const uint8_t* qh = x->qh;
        const int8_t* q8 = y->qs;
        __m128i scales = _mm_loadu_si128((const __m128i*)x->scales);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 2; j++) {
            int is = j * 4;
            __m128i s0 = _mm_shuffle_epi8(scales, shuf[is]);
            __m128i s1 = _mm_shuffle_epi8(scales, shuf[is + 1]);
            __m128i s2 = _mm_shuffle_epi8(scales, shuf[is + 2]);
            __m128i s3 = _mm_shuffle_epi8(scales, shuf[is + 3]);
            __m256i b1 = _mm256_loadu_si256((const __m256i*)q4); q4 += 32;
            __m256i b2 = _mm256_loadu_si256((const __m256i*)q4); q4 += 32;
            __m256i bh = _mm256_loadu_si256((const __m256i*)qh); qh += 32;
            __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(bh, m2), 4);
            __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 2), m2), 4);
            __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 4), m2), 4);
            __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(bh, 6), m2), 4);
            __m256i v0 = _mm256_or_si256(_mm256_and_si256(b1, m4), h0);
            __m256i v1 = _mm256_or_si256(_mm256_and_si256(b2, m4), h1);
            __m256i v2 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b1, 4), m4), h2);
            __m256i v3 = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(b2, 4), m4), h3);
            __m256i a0 = _mm256_loadu_si256((const __m256i*)q8); q8 += 32;
            __m256i a1 = _mm256_loadu_si256((const __m256i*)q8); q8 += 32;
            __m256i a2 = _mm256_loadu_si256((const __m256i*)q8); q8 += 32;
            __m256i a3 = _mm256_loadu_si256((const __m256i*)q8); q8 += 32;
            __m256i p0 = _mm256_sub_epi16(_mm256_maddubs_epi16(v0, a0), _mm256_maddubs_epi16(m32s, a0));
            __m256i p1 = _mm256_sub_epi16(_mm256_maddubs_epi16(v1, a1), _mm256_maddubs_epi16(m32s, a1));
            __m256i p2 = _mm256_sub_epi16(_mm256_maddubs_epi16(v2, a2), _mm256_maddubs_epi16(m32s, a2));
            __m256i p3 = _mm256_sub_epi16(_mm256_maddubs_epi16(v3, a3), _mm256_maddubs_epi16(m32s, a3));
            p0 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(s0), p0);
            p1 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(s1), p1);
            p2 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(s2), p2);
            p3 = _mm256_madd_epi16(_mm256_cvtepi8_epi16(s3), p3);
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p2, p3));
        }
        acc = _mm256_fmadd_ps(_mm256_broadcast_ss(&d), _mm256_cvtepi32_ps(sumi), acc);
    }
    return hsum_float_8(acc);
}

float cpu_vec_dot_q4k(size_t n, const void* xv, const void* yv) {
    const blk_q4k* xs = xv;
    const blk_q8k* ys = yv;
    const uint32_t KMASK1 = 0x3f3f3f3fu, KMASK2 = 0x0f0f0f0fu, KMASK3 = 0x03030303u;
    const __m256i m4 = _mm256_set1_epi8(0xF);
    __m256i shuf[8];
    for (int i = 0; i < 8; i++) shuf[i] = scale_shuffle_k4(i);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (size_t b = 0; b < n / 256; b++) {
        const blk_q4k* x = &xs[b];
        const blk_q8k* y = &ys[b];
        float d = y->d * h2f(x->d);
        float dmin = -y->d * h2f(x->dmin);
        uint32_t utmp[4];
        memcpy(utmp, x->scales, 12);
        utmp[3] = ((utmp[2] >> 4) & KMASK2) | (((utmp[1] >> 6) & KMASK3) << 4);
        uint32_t uaux = utmp[1] & KMASK1;
        utmp[1] = (utmp[2] & KMASK2) | (((utmp[0] >> 6) & KMASK3) << 4);
        utmp[2] = uaux;
        utmp[0] &= KMASK1;
        const uint8_t* q4 = x->qs;
        const int8_t* q8 = y->qs;
        __m256i ms = _mm256_cvtepu8_epi16(_mm_set_epi32((int)utmp[3], (int)utmp[2], (int)utmp[1], (int)utmp[0]));
        __m256i q8sums = _mm256_loadu_si256((const __m256i*)y->bsums);
        __m128i q8s = _mm_hadd_epi16(_mm256_extracti128_si256(q8sums, 0), _mm256_extracti128_si256(q8sums, 1));
        __m128i prod = _mm_madd_epi16(_mm256_extracti128_si256(ms, 1), q8s);
        acc_m = _mm_fmadd_ps(_mm_set1_ps(dmin), _mm_cvtepi32_ps(prod), acc_m);
        __m128i sc128 = _mm256_extracti128_si256(ms, 0);
        __m256i scales = _mm256_insertf128_si256(_mm256_castsi128_si256(sc128), sc128, 1);
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i sl = _mm256_shuffle_epi8(scales, shuf[2 * j]);
            __m256i sh = _mm256_shuffle_epi8(scales, shuf[2 * j + 1]);
            __m256i bits = _mm256_loadu_si256((const __m256i*)q4); q4 += 32;
            __m256i ql = _mm256_and_si256(bits, m4);
            __m256i qh = _mm256_and_si256(_mm256_srli_epi16(bits, 4), m4);
            __m256i a = _mm256_loadu_si256((const __m256i*)q8); q8 += 32;
            sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(sl, _mm256_maddubs_epi16(ql, a)));
            a = _mm256_loadu_si256((const __m256i*)q8); q8 += 32;
            sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(sh, _mm256_maddubs_epi16(qh, a)));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    acc_m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    acc_m = _mm_add_ss(acc_m, _mm_movehdup_ps(acc_m));
    return hsum_float_8(acc) + _mm_cvtss_f32(acc_m);
}

/* ---------------- TinyBLAS Q8_0 (avx.rs:187-314) ---------------- */

typedef struct {
    size_t k;
    const blk_q8_0* a; size_t lda;
    const blk_q8_0* b; size_t ldb;
    float* c; size_t ldc;
    size_t ith, nth;
} tinyblas;

static void tb_gemm(const tinyblas* t, int RM, int RN, size_t m0, size_t m, size_t n0, size_t n) {
    size_t ytiles = (m - m0) / RM, xtiles = (n - n0) / RN, tiles = xtiles * ytiles;
    if (tiles == 0) return;
    size_t duty = (tiles + t->nth - 1) / t->nth;
    size_t start = duty * t->ith, end = start + duty < tiles ? start + duty : tiles;
    for (size_t job = start; job < end; job++) {
        size_t ii = m0 + job / xtiles * RM, jj = n0 + job % xtiles * RN;
        __m256 cv[4][4];
        for (int j = 0; j < RN; j++)
            for (int i = 0; i < RM; i++) cv[j][i] = _mm256_setzero_ps();
        for (size_t l = 0; l < t->k; l++)
            for (int j = 0; j < RN; j++)
                for (int i = 0; i < RM; i++) {
                    const blk_q8_0* a = t->a + t->lda * (ii + i) + l;
                    const blk_q8_0* b = t->b + t->ldb * (jj + j) + l;
                    __m256i av = _mm256_loadu_si256((const __m256i*)a->qs);
                    __m256i bv = _mm256_loadu_si256((const __m256i*)b->qs);
                    __m256 dot = mul_sum_i8_pairs_float(av, bv);
                    __m256 sc = _mm256_set1_ps(h2f(a->d) * h2f(b->d));
                    cv[j][i] = _mm256_fmadd_ps(sc, dot, cv[j][i]);
                }
        for (int j = 0; j < RN; j++)
            for (int i = 0; i < RM; i++) t->c[t->ldc * (jj + j) + (ii + i)] = hsum_float_8(cv[j][i]);
    }
}

static void tb_mnpack(const tinyblas* t, size_t m0, size_t m, size_t n0, size_t n) {
    size_t mr = (m - m0) < 4 ? (m - m0) : 4, nr = (n - n0) < 4 ? (n - n0) : 4;
    int mc, nc;
    switch ((mr << 4) | nr) {
    case 0x42: case 0x43: case 0x44: mc = 4; nc = 2; break;
    case 0x34: case 0x24: mc = 2; nc = 4; break;
    case 0x33: case 0x32: mc = 3; nc = 2; break;
    case 0x23: mc = 2; nc = 3; break;
    case 0x41: mc = 4; nc = 1; break;
    case 0x22: mc = 2; nc = 2; break;
    case 0x14: mc = 1; nc = 4; break;
    case 0x31: mc = 3; nc = 1; break;
    case 0x13: mc = 1; nc = 3; break;
    case 0x21: mc = 2; nc = 1; break;
    case 0x12: mc = 1; nc = 2; break;
    case 0x11: mc = 1; nc = 1; break;
    default: return;
    }
    tb_gemm(t, mc, nc, m0, m, n0, n);
    size_t mp = m0 + (m - m0) / mc * mc, np = n0 + (n - n0) / nc * nc;
    tb_mnpack(t, mp, m, n0, np);
    tb_mnpack(t, m0, m, np, n);
}

/* ---------------- persistent pool (threadpool.rs:441-466) ---------------- */

typedef void (*job_fn)(void* ctx, size_t ith, size_t nth);

static struct {
    pthread_t th[256];
    size_t nth;
    pthread_mutex_t mu;
    pthread_cond_t cv_go, cv_done;
    unsigned long gen;
    size_t pending;
    job_fn fn;
    void* ctx;
    int quit;
} P = {.mu = PTHREAD_MUTEX_INITIALIZER, .cv_go = PTHREAD_COND_INITIALIZER, .cv_done = PTHREAD_COND_INITIALIZER};

static void* worker(void* arg) {
    size_t ith = (size_t)arg;
    unsigned long seen = 0;
    for (;;) {
        pthread_mutex_lock(&P.mu);
        while (P.gen == seen && !P.quit) pthread_cond_wait(&P.cv_go, &P.mu);
        if (P.quit) { pthread_mutex_unlock(&P.mu); return NULL; }
        seen = P.gen;
        job_fn fn = P.fn;
        void* ctx = P.ctx;
        size_t nth = P.nth;
        pthread_mutex_unlock(&P.mu);
        fn(ctx, ith, nth);
        pthread_mutex_lock(&P.mu);
        if (--P.pending == 0) pthread_cond_signal(&P.cv_done);
        pthread_mutex_unlock(&P.mu);
    }
}

int cpu_pool_init(size_t nth) {
    if (P.nth) return (int)P.nth;
    if (nth < 1) nth = 1;
    if (nth > 256) nth = 256;
    P.nth = nth;
    for (size_t i = 1; i < nth; i++) pthread_create(&P.th[i], NULL, worker, (void*)i);
    return (int)nth;
}

static void dispatch(job_fn fn, void* ctx) {
    if (P.nth <= 1) { fn(ctx, 0, 1); return; }
    pthread_mutex_lock(&P.mu);
    P.fn = fn;
    P.ctx = ctx;
    P.pending = P.nth - 1;
    P.gen++;
    pthread_cond_broadcast(&P.cv_go);
    pthread_mutex_unlock(&P.mu);
    fn(ctx, 0, P.nth);
    pthread_mutex_lock(&P.mu);
    while (P.pending) pthread_cond_wait(&P.cv_done, &P.mu);
    pthread_mutex_unlock(&P.mu);
}

typedef struct {
    float (*dot)(size_t, const void*, const void*);
    size_t k, n, wrow, nchunks, batch;
    const char* rhs;
    const void* lhs_row;
    float* dst_row;
    atomic_size_t next;
} row_job;

static void row_worker(void* v, size_t ith, size_t nth) {
    (void)ith; (void)nth;
    row_job* j = v;
    for (;;) {
        size_t start = atomic_fetch_add_explicit(&j->next, j->batch, memory_order_relaxed);
        if (start >= j->nchunks) break;
        size_t end = start + j->batch < j->nchunks ? start + j->batch : j->nchunks;
        for (size_t c = start * 128; c < end * 128 && c < j->n; c++)
            j->dst_row[c] = j->dot(j->k, j->rhs + c * j->wrow, j->lhs_row);
    }
}

typedef struct { tinyblas t; size_t m, n; } sgemm_job;
static void sgemm_worker(void* v, size_t ith, size_t nth) {
    sgemm_job* s = v;
    tinyblas t = s->t;
    t.ith = ith;
    t.nth = nth;
    tb_mnpack(&t, 0, s->m, 0, s->n);
}

static size_t tsize(int dt) {
    switch (dt) { case ORC_Q4_0: return 18; case ORC_Q8_0: return 34; case ORC_Q4K: return 144; case ORC_Q6K: return 210; }
    return 0;
}

/* T::matmul over pre-quantized lhs blocks (k_quants.rs:694-707 for Q8_0,
 * matmul_by_row otherwise). */
int cpu_matmul_preq(int dt, size_t m, size_t k, size_t n, const void* lhs_b, const void* rhs, float* dst) {
    if (!P.nth) cpu_pool_init(1);
    if (m == 0 || n == 0) return 0;
    if (dt == ORC_Q8_0) {
        size_t kb = k / 32;
        sgemm_job s = {.t = {.k = kb, .a = rhs, .lda = kb, .b = lhs_b, .ldb = kb, .c = dst, .ldc = n}, .m = n, .n = m};
        dispatch(sgemm_worker, &s);
        return 0;
    }
    float (*dot)(size_t, const void*, const void*) = NULL;
    size_t abytes;
    if (dt == ORC_Q4_0) { dot = cpu_vec_dot_q4_0; abytes = (k / 32) * 34; }
    else if (dt == ORC_Q4K) { dot = cpu_vec_dot_q4k; abytes = (k / 256) * 292; }
    else if (dt == ORC_Q6K) { dot = cpu_vec_dot_q6k; abytes = (k / 256) * 292; }
    else return -1;
    size_t wrow = (k / (dt == ORC_Q4_0 ? 32 : 256)) * tsize(dt);
    size_t nchunks = (n + 127) / 128;
    size_t runs = P.nth * 8 < nchunks ? P.nth * 8 : nchunks;
    for (size_t r = 0; r < m; r++) {
        row_job j = {.dot = dot, .k = k, .n = n, .wrow = wrow, .nchunks = nchunks,
                     .batch = (nchunks + runs - 1) / runs, .rhs = rhs,
                     .lhs_row = (const char*)lhs_b + r * abytes, .dst_row = dst + r * n};
        atomic_init(&j.next, 0);
        dispatch(row_worker, &j);
    }
    return 0;
}

/* k_quants::matmul: serial quantize_lhs, then the threaded kernel. */
int cpu_matmul(int dt, size_t m, size_t k, size_t n, const float* lhs, const void* rhs, float* dst,
               void* lhs_scratch) {
    if (orc_quantize_lhs(dt, m, k, lhs, lhs_scratch)) return -1;
    return cpu_matmul_preq(dt, m, k, n, lhs_scratch, rhs, dst);
}
