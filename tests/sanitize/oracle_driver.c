/* Sanitizer driver for the CPU oracle (oracle/ggml_oracle.c), built with
 * AddressSanitizer + UndefinedBehaviorSanitizer.  Runs every entry point on
 * seeded inputs: the reference quantizers on random, constant, all-zero,
 * one-signed, tiny and large finite rows; dequantize on arbitrary block bytes
 * (Inf/NaN/subnormal halves); the activation quantizers and vec_dot; the
 * threaded candle-algorithm matmul and the f64 matmul; the LoRA merge.  Any
 * out-of-bounds access or undefined behaviour aborts the run.  Prints
 * "oracle_driver: ok". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ggml_oracle.h"

static uint64_t g_s = 0x243F6A8885A308D3ull;
static uint64_t rnd(void) {
    g_s ^= g_s << 13;
    g_s ^= g_s >> 7;
    g_s ^= g_s << 17;
    return g_s;
}
static float urand(void) { return (float)((rnd() >> 11) * (1.0 / 9007199254740992.0)); }
static float nrand(void) {
    const float u1 = urand() + 1e-7f, u2 = urand();
    return sqrtf(-2.f * logf(u1)) * cosf(6.2831853f * u2);
}

static const int TYPES[] = {ORC_Q4_0, ORC_Q4_1, ORC_Q5_0, ORC_Q5_1, ORC_Q8_0,
                            ORC_Q2_K, ORC_Q3_K, ORC_Q4_K, ORC_Q5_K, ORC_Q6_K};

/* One row of `k` finite values of the given kind. */
static void fill_row(float *x, int64_t k, int kind) {
    for (int64_t i = 0; i < k; i++) {
        switch (kind) {
        case 0: x[i] = nrand() * 0.02f; break;
        case 1: x[i] = 0.f; break;
        case 2: x[i] = 1.25f; break;
        case 3: x[i] = fabsf(nrand()); break;
        case 4: x[i] = -fabsf(nrand()) * 3.f; break;
        case 5: x[i] = nrand() * 1e-30f; break;
        case 6: x[i] = nrand() * 1e4f; break;
        default: x[i] = (i % 17 == 0) ? nrand() : 0.f; break;
        }
    }
}

int main(void) {
    const int64_t n = 12, k = 512, m = 5;
    float *x = malloc(sizeof(float) * n * k);
    float *y = malloc(sizeof(float) * n * k);
    float *xa = malloc(sizeof(float) * m * k);
    float *ym = malloc(sizeof(float) * m * n);
    double *yd = malloc(sizeof(double) * m * n);
    uint8_t *blocks = malloc((size_t)n * k * 4);
    uint8_t *act = malloc((size_t)k * 4);
    for (int64_t i = 0; i < m * k; i++) xa[i] = nrand();
    for (size_t ti = 0; ti < sizeof(TYPES) / sizeof(TYPES[0]); ti++) {
        const int t = TYPES[ti];
        const int bs = orc_block_size(t), ts = orc_type_size(t);
        const int64_t rowb = k / bs * ts;
        for (int64_t r = 0; r < n; r++) fill_row(x + r * k, k, (int)(r % 8));
        if (orc_quantize_row(t, x, blocks, n * k) != 0) return 1;
        if (orc_dequantize_row(t, blocks, y, n * k) != 0) return 1;
        for (int64_t i = 0; i < n * k; i++)
            if (!isfinite(y[i])) { fprintf(stderr, "type %d: non-finite dequant of a quantized row\n", t); return 1; }
        /* arbitrary block bytes: every pattern is a valid block */
        uint8_t *rb = malloc((size_t)rowb * n);
        for (int64_t i = 0; i < rowb * n; i++) rb[i] = (uint8_t)rnd();
        if (orc_dequantize_row(t, rb, y, n * k) != 0) return 1;
        free(rb);
        /* activations and dots */
        const int vdt = orc_vec_dot_type(t);
        if (vdt == ORC_Q8_0) orc_quantize_row_q8_0(xa, act, k);
        else if (vdt == ORC_Q8_1) orc_quantize_row_q8_1(xa, act, k);
        else orc_quantize_row_q8_K(xa, act, k);
        for (int64_t r = 0; r < n; r++) (void)orc_vec_dot(t, k, blocks + r * rowb, act);
        if (orc_matmul_candle(t, m, n, k, xa, blocks, ym, 3) != 0) return 1;
        if (orc_matmul_f64(t, m, n, k, xa, blocks, yd) != 0) return 1;
        /* bad arguments are refused, not read */
        if (orc_quantize_row(t, x, blocks, k - 1) == 0) return 1;
    }
    /* LoRA merge on a strided slice */
    {
        const int rank = 4;
        float *w = calloc((size_t)8 * 40, sizeof(float));
        float *b = malloc(sizeof(float) * 8 * rank), *a = malloc(sizeof(float) * rank * 40);
        for (int i = 0; i < 8 * rank; i++) b[i] = nrand();
        for (int i = 0; i < rank * 40; i++) a[i] = nrand();
        orc_lora_apply(w, 40, 8, 32, b, rank, a, 40, rank, 0.5f);
        free(w);
        free(b);
        free(a);
    }
    /* halves */
    for (uint32_t h = 0; h < 65536; h++) (void)orc_fp16_to_fp32((uint16_t)h);
    const float specials[] = {0.f, -0.f, 65504.f, 65520.f, 1e-8f, INFINITY, -INFINITY, NAN, 3.4e38f};
    for (size_t i = 0; i < sizeof(specials) / sizeof(specials[0]); i++) {
        (void)orc_fp32_to_fp16(specials[i]);
        (void)orc_fp32_to_bf16(specials[i]);
    }
    free(x);
    free(y);
    free(xa);
    free(ym);
    free(yd);
    free(blocks);
    free(act);
    printf("oracle_driver: ok\n");
    return 0;
}
