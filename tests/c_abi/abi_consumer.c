/* abi_consumer.c — a plain C caller of libmoldq's C ABI (include/moldq.h),
 * as the Rust FFI arm of candle's quantized module would call it: no Python,
 * no torch.  Device buffers for activations and outputs come from the HIP
 * runtime (the candle ROCm device would own them); the five runtime entry
 * points used are declared here rather than through the HIP headers.
 *
 * Checks, on GPU 0:
 *   1. upload of a Q8_0 weight built here, dequantize to f32: bit-exact with
 *      d * q computed on the host (every product is exact in f32);
 *   2. QMatMul::forward at m = 3 (GEMV path: exact f32 weights times f32 x)
 *      within 1e-5 relative L2 of a double-precision product, and at m = 40
 *      (bf16 MFMA GEMM path) within 1e-2, with a bias;
 *   3. an invalid call (x_dtype F16) returns MQ_E_INVALID with a message.
 * Exit status 0 and a final "abi consumer: ok" line on success. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "moldq.h"

/* HIP runtime (libamdhip64): the entry points this program needs. */
extern int hipMalloc(void **ptr, size_t size);
extern int hipFree(void *ptr);
extern int hipMemcpy(void *dst, const void *src, size_t size, int kind);
extern int hipDeviceSynchronize(void);
enum { HIP_H2D = 1, HIP_D2H = 2 };

#define N 192
#define K 512
#define BLK 32
#define BLOCK_BYTES 34 /* Q8_0: f16 d, 32 x int8 */

static int fail(const char *what, int rc) {
    fprintf(stderr, "abi consumer: %s failed (rc %d): %s\n", what, rc, mq_last_error());
    return 1;
}

static double rel_l2(const float *y, const double *ref, int count) {
    double num = 0.0, den = 0.0;
    for (int i = 0; i < count; ++i) {
        const double d = (double)y[i] - ref[i];
        num += d * d;
        den += ref[i] * ref[i];
    }
    return sqrt(num / (den > 0 ? den : 1.0));
}

int main(void) {
    /* Q8_0 blocks: d = 2^-6 * (1 + (b % 7) / 8) as f16 bits 0x2400 | (b % 7) << 7 */
    static uint8_t blocks[N * (K / BLK) * BLOCK_BYTES];
    static float w[N * K];
    for (int r = 0; r < N; ++r)
        for (int b = 0; b < K / BLK; ++b) {
            uint8_t *blk = blocks + ((size_t)r * (K / BLK) + b) * BLOCK_BYTES;
            const int e = (r + b) % 7;
            const uint16_t dbits = (uint16_t)(0x2400 | (e << 7));
            memcpy(blk, &dbits, 2);
            const float d = ldexpf(1.0f + e / 8.0f, -6);
            for (int j = 0; j < BLK; ++j) {
                const int8_t q = (int8_t)((r * 31 + b * 7 + j * 13) % 255 - 127);
                blk[2 + j] = (uint8_t)q;
                w[(size_t)r * K + b * BLK + j] = d * (float)q;
            }
        }

    mq_ctx *ctx = NULL;
    int rc = mq_ctx_create(0, &ctx);
    if (rc) return fail("mq_ctx_create", rc);
    mq_qtensor *qt = NULL;
    rc = mq_qtensor_upload(ctx, MQ_Q8_0, N, K, blocks, sizeof(blocks), &qt);
    if (rc) return fail("mq_qtensor_upload", rc);

    /* 1. dequantize */
    float *dw = NULL;
    if (hipMalloc((void **)&dw, sizeof(w))) return fail("hipMalloc", -1);
    rc = mq_dequantize(ctx, qt, dw, MQ_F32, NULL);
    if (rc) return fail("mq_dequantize", rc);
    static float wd[N * K];
    hipMemcpy(wd, dw, sizeof(wd), HIP_D2H);
    if (memcmp(wd, w, sizeof(w)) != 0) {
        fprintf(stderr, "abi consumer: dequantized weights differ from d * q\n");
        return 1;
    }
    printf("abi consumer: dequantize Q8_0 [%d, %d] bit-exact\n", N, K);

    /* 2. QMatMul::forward with bias at m = 3 (GEMV) and m = 40 (GEMM) */
    const int ms[2] = {3, 40};
    const double tol[2] = {1e-5, 1e-2};
    static float bias[N];
    for (int c = 0; c < N; ++c) bias[c] = (float)((c % 9) - 4) / 16.0f;
    float *dbias = NULL;
    hipMalloc((void **)&dbias, sizeof(bias));
    hipMemcpy(dbias, bias, sizeof(bias), HIP_H2D);
    for (int t = 0; t < 2; ++t) {
        const int m = ms[t];
        float *x = malloc(sizeof(float) * m * K), *y = malloc(sizeof(float) * m * N);
        double *ref = malloc(sizeof(double) * m * N);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < K; ++j) x[i * K + j] = (float)((i * 17 + j * 5) % 101 - 50) / 25.0f;
        for (int i = 0; i < m; ++i)
            for (int c = 0; c < N; ++c) {
                double s = bias[c];
                for (int j = 0; j < K; ++j) s += (double)x[i * K + j] * (double)w[(size_t)c * K + j];
                ref[i * N + c] = s;
            }
        float *dx = NULL, *dy = NULL;
        hipMalloc((void **)&dx, sizeof(float) * m * K);
        hipMalloc((void **)&dy, sizeof(float) * m * N);
        hipMemcpy(dx, x, sizeof(float) * m * K, HIP_H2D);
        rc = mq_qmatmul(ctx, qt, dx, MQ_F32, m, K, dy, MQ_F32, N, dbias, MQ_ACT_NONE, NULL);
        if (rc) return fail("mq_qmatmul", rc);
        hipDeviceSynchronize();
        hipMemcpy(y, dy, sizeof(float) * m * N, HIP_D2H);
        const double err = rel_l2(y, ref, m * N);
        printf("abi consumer: qmatmul Q8_0 m=%d n=%d k=%d rel-L2 %.3e (bar %.0e)\n", m, N, K, err, tol[t]);
        if (!(err <= tol[t])) return 1;
        hipFree(dx);
        hipFree(dy);
        free(x);
        free(y);
        free(ref);
    }

    /* 3. an invalid activation dtype is refused with a message */
    rc = mq_qmatmul(ctx, qt, dw, MQ_F16, 1, K, dw, MQ_F32, N, NULL, MQ_ACT_NONE, NULL);
    if (rc != MQ_E_INVALID || mq_last_error() == NULL || mq_last_error()[0] == '\0') {
        fprintf(stderr, "abi consumer: F16 activations gave rc %d, expected MQ_E_INVALID\n", rc);
        return 1;
    }
    printf("abi consumer: invalid call refused: %s\n", mq_last_error());

    hipFree(dw);
    hipFree(dbias);
    mq_qtensor_free(qt);
    mq_ctx_destroy(ctx);
    printf("abi consumer: ok\n");
    return 0;
}
