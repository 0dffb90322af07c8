/*
 * Sanitizer driver for the C restatement of the Zig CPU forward (lut_cpu.c).
 * TEST INFRASTRUCTURE ONLY: built with AddressSanitizer and
 * UndefinedBehaviorSanitizer by `make -C oracle sanitize` (tests/test_lut_cpu.py
 * runs it); never part of the product.
 *
 * It drives both exported forwards over shapes that reach every loop of the
 * restatement: the row-major (threads > 1) and table-major (threads = 1)
 * loops, table counts with and without a remainder after the groups of four,
 * output widths with and without a remainder after the 8-wide vector steps,
 * batches below and above the 64-row minimum per worker, one comparison and
 * the maximum of eight, plus the known-answer helpers. Any out-of-bounds
 * access, use after free, data race on the heap or undefined operation makes
 * the sanitizers abort with a report; a clean run exits 0.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void tropnn_set_num_threads(size_t n);
void lut_forward_batch_with_offsets_no_cache(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                             size_t output_dim, const float *weights, const size_t *anchors,
                                             const float *offsets, const float *inputs, float *outputs);
void lut_forward_batch_f16_no_cache(size_t batch, size_t tables, size_t comparisons, size_t input_dim,
                                    size_t output_dim, const uint16_t *weights, const size_t *anchors,
                                    const float *offsets, const float *inputs, float *outputs);
void lut_cpu_test_add4_f32(float *dst, const float *a, const float *b, const float *c, const float *d, size_t n);
void lut_cpu_test_add4_f16(float *dst, const uint16_t *a, const uint16_t *b, const uint16_t *c, const uint16_t *d,
                           size_t n);
size_t lut_cpu_test_code(const float *x, const size_t *anchors, const float *offsets, size_t table, size_t comps);

static uint32_t g_state = 12345u;
static uint32_t next_u32(void) {
    g_state = g_state * 1664525u + 1013904223u;
    return g_state;
}
static float next_f(void) { return (float)((int32_t)(next_u32() >> 8) - (1 << 23)) / (float)(1 << 23); }

/* Allocations of exactly the size each argument needs, so an access one
 * element past the end is caught. */
static int run(size_t batch, size_t tables, size_t comps, size_t in_dim, size_t out_dim, size_t threads) {
    const size_t rows = (size_t)1 << comps;
    float *w = malloc(tables * rows * out_dim * sizeof(float));
    uint16_t *wh = malloc(tables * rows * out_dim * sizeof(uint16_t));
    size_t *anchors = malloc(tables * comps * 2 * sizeof(size_t));
    float *offsets = malloc(tables * comps * sizeof(float));
    float *x = malloc(batch * in_dim * sizeof(float));
    float *y = malloc(batch * out_dim * sizeof(float));
    float *yh = malloc(batch * out_dim * sizeof(float));
    if (!w || !wh || !anchors || !offsets || !x || !y || !yh) return 1;
    for (size_t k = 0; k < tables * rows * out_dim; ++k) {
        w[k] = next_f();
        wh[k] = (uint16_t)(0x3c00u | (next_u32() & 0x3ffu)); /* finite halves in [1, 2) */
    }
    for (size_t k = 0; k < tables * comps * 2; ++k) anchors[k] = next_u32() % in_dim;
    for (size_t k = 0; k < tables * comps; ++k) offsets[k] = 0.25f * next_f();
    for (size_t k = 0; k < batch * in_dim; ++k) x[k] = next_f();
    tropnn_set_num_threads(threads);
    lut_forward_batch_with_offsets_no_cache(batch, tables, comps, in_dim, out_dim, w, anchors, offsets, x, y);
    lut_forward_batch_f16_no_cache(batch, tables, comps, in_dim, out_dim, wh, anchors, offsets, x, yh);
    double s = 0.0;
    for (size_t k = 0; k < batch * out_dim; ++k) s += (double)y[k] + (double)yh[k];
    free(w);
    free(wh);
    free(anchors);
    free(offsets);
    free(x);
    free(y);
    free(yh);
    return s != s; /* NaN would mean uninitialised output */
}

int main(void) {
    static const size_t shapes[][5] = {
        /* batch, tables, comparisons, input_dim, output_dim */
        {1, 1, 1, 2, 1},     {3, 4, 2, 5, 8},       {7, 5, 3, 9, 17},     {64, 9, 4, 16, 33},
        {65, 16, 6, 256, 512}, {200, 7, 8, 40, 19}, {130, 13, 5, 30, 24},
    };
    static const size_t threads[] = {1, 2, 4, 8};
    for (size_t s = 0; s < sizeof shapes / sizeof shapes[0]; ++s)
        for (size_t t = 0; t < sizeof threads / sizeof threads[0]; ++t)
            if (run(shapes[s][0], shapes[s][1], shapes[s][2], shapes[s][3], shapes[s][4], threads[t])) {
                fprintf(stderr, "shape %zu threads %zu: bad output\n", s, threads[t]);
                return 1;
            }
    /* known-answer helpers on exact-size buffers (tails of 19 and 1) */
    for (size_t n = 1; n <= 19; n += 18) {
        float *d = calloc(n, sizeof(float)), *a = calloc(n, sizeof(float));
        uint16_t *h = calloc(n, sizeof(uint16_t));
        lut_cpu_test_add4_f32(d, a, a, a, a, n);
        lut_cpu_test_add4_f16(d, h, h, h, h, n);
        free(d);
        free(a);
        free(h);
    }
    const float xk[3] = {3.f, 1.f, -1.f};
    const size_t ak[4] = {0, 1, 1, 2};
    const float ok[2] = {1.5f, 3.0f};
    if (lut_cpu_test_code(xk, ak, ok, 0, 2) != 1) return 1; /* lut.zig:320-325 */
    puts("sanitize_check ok");
    return 0;
}
