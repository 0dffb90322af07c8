/*
 * C restatement of the reference's Zig CPU forward for PairwiseLinear.
 * TEST INFRASTRUCTURE ONLY: the "Zig-equivalent CPU" baseline timed beside
 * the GPU by bench.py's cpu_baseline leg, and a second forward oracle in
 * tests/. The product never links or loads it.
 *
 * The reference (kernels/src/{lut,simd,parallel}.zig) cannot be built here:
 * there is no zig toolchain in this image. This file restates its algorithm:
 *   - comparator code per table, margin = (x[a] - x[b]) - offset, bit c set
 *     iff margin > 0                                 lut.zig:5-66
 *   - row-major loop (threads > 1) and table-major loop (threads <= 1),
 *     4 tables at a time, out += ((L0 + L1) + L2) + L3, remaining tables
 *     added one at a time                            lut.zig:81-156, 171-246
 *   - f16 LUT rows converted to f32, f32 accumulation simd.zig:160-176
 *   - outputs zeroed by the kernel                   lut.zig:85-86, 117-120
 *   - thread count: process-global, 0 = CPU count, capped at 64; work split
 *     in contiguous row ranges of >= 64 rows, threads spawned per call, the
 *     last range run on the calling thread           parallel.zig:3-63
 * Exported names and argument order are those of the Zig C ABI
 * (lut.zig:255-318, parallel.zig:8-16).
 */
#include <immintrin.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <unistd.h>

#define MAX_THREADS 64
#define MIN_ROWS_PER_THREAD 64

static volatile size_t g_num_threads = 0;

void tropnn_set_num_threads(size_t n) { g_num_threads = n < MAX_THREADS ? n : MAX_THREADS; }

size_t tropnn_get_num_threads(void) {
    size_t n = g_num_threads;
    if (n != 0) return n;
    long cpus = sysconf(_SC_NPROCESSORS_ONLN);
    if (cpus < 1) cpus = 1;
    return (size_t)cpus < MAX_THREADS ? (size_t)cpus : MAX_THREADS;
}

/* parallel.zig:18-25 */
size_t lut_cpu_worker_count(size_t items, size_t min_items) {
    size_t lo = min_items > 0 ? min_items : 1;
    if (items <= lo) return 1;
    size_t req = tropnn_get_num_threads();
    if (req <= 1) return 1;
    size_t useful = (items + lo - 1) / lo;
    size_t n = req < useful ? req : useful;
    if (n > items) n = items;
    return n > 0 ? n : 1;
}

/* IEEE binary16 -> binary32, exact for every input (normals, subnormals,
 * infinities, NaN payloads). */
static inline float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        /* subnormal: normalise */
        int e = -1;
        do {
            man <<= 1;
            e++;
        } while ((man & 0x400u) == 0);
        bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* lut.zig:5-66; the compiler unrolls the fixed-count loop for C = 1..8 */
static inline size_t code_of(const float *x, const size_t *anchors, const float *offsets, size_t table, size_t comps) {
    const size_t *a = anchors + table * comps * 2;
    const float *off = offsets + table * comps;
    size_t idx = 0;
    for (size_t c = 0; c < comps; ++c) {
        float m = x[a[2 * c]] - x[a[2 * c + 1]] - off[c];
        idx |= (size_t)(m > 0.0f) << c;
    }
    return idx;
}

typedef struct {
    size_t tables, comps, in_dim, out_dim, rows_per_table;
    const float *w32;
    const uint16_t *w16;
    const size_t *anchors;
    const float *offsets;
    const float *inputs;
    float *outputs;
} ctx_t;

static inline void add4_f32(float *dst, const float *s0, const float *s1, const float *s2, const float *s3, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] += ((s0[i] + s1[i]) + s2[i]) + s3[i];
}

static inline void add1_f32(float *dst, const float *s, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] += s[i];
}

#if defined(__F16C__) && defined(__AVX__)
/* 8 lanes at a time with the F16C converter (exact, like half_to_float) */
static inline __m256 ld8h(const uint16_t *p) { return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)p)); }
#define HAVE_F16C_PATH 1
#endif

static inline void add4_f16(float *dst, const uint16_t *s0, const uint16_t *s1, const uint16_t *s2, const uint16_t *s3,
                            size_t n) {
    size_t i = 0;
#ifdef HAVE_F16C_PATH
    for (; i + 8 <= n; i += 8) {
        __m256 sum = _mm256_add_ps(_mm256_add_ps(_mm256_add_ps(ld8h(s0 + i), ld8h(s1 + i)), ld8h(s2 + i)), ld8h(s3 + i));
        _mm256_storeu_ps(dst + i, _mm256_add_ps(_mm256_loadu_ps(dst + i), sum));
    }
#endif
    for (; i < n; ++i)
        dst[i] += ((half_to_float(s0[i]) + half_to_float(s1[i])) + half_to_float(s2[i])) + half_to_float(s3[i]);
}

static inline void add1_f16(float *dst, const uint16_t *s, size_t n) {
    size_t i = 0;
#ifdef HAVE_F16C_PATH
    for (; i + 8 <= n; i += 8) _mm256_storeu_ps(dst + i, _mm256_add_ps(_mm256_loadu_ps(dst + i), ld8h(s + i)));
#endif
    for (; i < n; ++i) dst[i] += half_to_float(s[i]);
}

/* one group of 4 tables (or a single table when `one`) for one row */
static inline void row_step(const ctx_t *c, const float *x, float *y, size_t t, int one) {
    const size_t stride = c->rows_per_table * c->out_dim, n = c->out_dim;
    if (one) {
        size_t b0 = t * stride + code_of(x, c->anchors, c->offsets, t, c->comps) * n;
        if (c->w16) add1_f16(y, c->w16 + b0, n);
        else add1_f32(y, c->w32 + b0, n);
        return;
    }
    size_t i0 = code_of(x, c->anchors, c->offsets, t, c->comps);
    size_t i1 = code_of(x, c->anchors, c->offsets, t + 1, c->comps);
    size_t i2 = code_of(x, c->anchors, c->offsets, t + 2, c->comps);
    size_t i3 = code_of(x, c->anchors, c->offsets, t + 3, c->comps);
    size_t b0 = t * stride + i0 * n, b1 = (t + 1) * stride + i1 * n;
    size_t b2 = (t + 2) * stride + i2 * n, b3 = (t + 3) * stride + i3 * n;
    if (c->w16) add4_f16(y, c->w16 + b0, c->w16 + b1, c->w16 + b2, c->w16 + b3, n);
    else add4_f32(y, c->w32 + b0, c->w32 + b1, c->w32 + b2, c->w32 + b3, n);
}

/* lut.zig:81-113 / 171-203 */
static void row_major(const ctx_t *c, size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r) {
        const float *x = c->inputs + r * c->in_dim;
        float *y = c->outputs + r * c->out_dim;
        memset(y, 0, c->out_dim * sizeof(float));
        size_t t = 0;
        for (; t + 4 <= c->tables; t += 4) row_step(c, x, y, t, 0);
        for (; t < c->tables; ++t) row_step(c, x, y, t, 1);
    }
}

/* lut.zig:115-156 / 205-246 */
static void table_major(const ctx_t *c, size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; ++r) memset(c->outputs + r * c->out_dim, 0, c->out_dim * sizeof(float));
    size_t t = 0;
    for (; t + 4 <= c->tables; t += 4)
        for (size_t r = r0; r < r1; ++r) row_step(c, c->inputs + r * c->in_dim, c->outputs + r * c->out_dim, t, 0);
    for (; t < c->tables; ++t)
        for (size_t r = r0; r < r1; ++r) row_step(c, c->inputs + r * c->in_dim, c->outputs + r * c->out_dim, t, 1);
}

typedef struct {
    const ctx_t *ctx;
    size_t r0, r1;
    int table_major;
} job_t;

static void *run_job(void *p) {
    job_t *j = (job_t *)p;
    if (j->table_major) table_major(j->ctx, j->r0, j->r1);
    else row_major(j->ctx, j->r0, j->r1);
    return NULL;
}

/* parallel.zig:27-63 */
static void parallel_rows(const ctx_t *c, size_t rows) {
    int tm = tropnn_get_num_threads() <= 1;
    size_t n = lut_cpu_worker_count(rows, MIN_ROWS_PER_THREAD);
    if (n <= 1) {
        job_t j = {c, 0, rows, tm};
        run_job(&j);
        return;
    }
    pthread_t th[MAX_THREADS];
    job_t jobs[MAX_THREADS];
    int spawned[MAX_THREADS] = {0};
    size_t start = 0;
    for (size_t w = 0; w < n; ++w) {
        size_t end = rows * (w + 1) / n;
        jobs[w] = (job_t){c, start, end, tm};
        if (w + 1 == n || pthread_create(&th[w], NULL, run_job, &jobs[w]) != 0) run_job(&jobs[w]);
        else spawned[w] = 1;
        start = end;
    }
    for (size_t w = 0; w < n; ++w)
        if (spawned[w]) pthread_join(th[w], NULL);
}

void lut_forward_batch_with_offsets_no_cache(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                             size_t output_dim, const float *weights, const size_t *anchors,
                                             const float *offsets, const float *inputs, float *outputs) {
    ctx_t c = {tables, comparisons, input_dim, output_dim, (size_t)1 << comparisons,
               weights, NULL, anchors, offsets, inputs, outputs};
    parallel_rows(&c, batch);
}

void lut_forward_batch_f16_no_cache(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                    size_t output_dim, const uint16_t *weights_f16, const size_t *anchors,
                                    const float *offsets, const float *inputs, float *outputs) {
    ctx_t c = {tables, comparisons, input_dim, output_dim, (size_t)1 << comparisons,
               NULL, weights_f16, anchors, offsets, inputs, outputs};
    parallel_rows(&c, batch);
}

/* test hooks for the simd.zig tail KATs (simd.zig:178-218) */
void lut_cpu_test_add4_f32(float *dst, const float *a, const float *b, const float *c, const float *d, size_t n) {
    add4_f32(dst, a, b, c, d, n);
}
void lut_cpu_test_add4_f16(float *dst, const uint16_t *a, const uint16_t *b, const uint16_t *c, const uint16_t *d,
                           size_t n) {
    add4_f16(dst, a, b, c, d, n);
}
size_t lut_cpu_test_code(const float *x, const size_t *anchors, const float *offsets, size_t table, size_t comps) {
    return code_of(x, anchors, offsets, table, comps);
}
float lut_cpu_test_half_to_float(uint16_t h) { return half_to_float(h); }
