/*
 * ggml_oracle.c — CPU oracle for the GGUF quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see ggml_oracle.h).  Only tests/, smoke() and the
 * cpu_baseline leg of bench.py may load this library.
 *
 * The quantizer and dot-product routines restate ggml's (ggml-quants.c,
 * MIT License, Copyright (c) 2023-2024 The ggml authors) step by step, since
 * byte-identical blocks need the same IEEE operations in the same order.
 *
 * Source of each algorithm.  candle-core-mold 0.9.10 (pinned at
 * /root/reference/Cargo.lock:507-535; not vendored, crate source absent from
 * this container) ports ggml's k_quants/ggml-quants C code.  Everything here is
 * restated from ggml's published block spec and reference routines:
 *   block layouts ............ ggml-common.h  (block_q4_0 ... block_q8_K)
 *   dequantize_row_* ......... ggml-quants.c  (candle: k_quants.rs `to_float`)
 *   quantize_row_*_ref ....... ggml-quants.c  (llama-quantize without imatrix)
 *   vec_dot_*_q8_* ........... ggml-quants.c generic paths (candle: `vec_dot_unopt`)
 *   Q8_1 / Q8_K activations .. candle k_quants.rs `from_float` as recalled
 *                              (round-half-away, Q8_K scale -128/max; ggml's
 *                              quantize_row_q8_K_ref uses -127/max and ties to
 *                              even).  The code is pinned to that stated
 *                              convention (known-answer rows that separate the
 *                              two, a second numpy restatement); whether candle
 *                              rounds this way is PARITY UNPINNED: no candle
 *                              source or vectors exist here, so GPU tests report
 *                              agreement with it but assert only bounds that
 *                              hold for either convention.
 *   matmul ................... candle quantized/mod.rs `matmul_t`: quantize each
 *                              activation row, then vec_dot per output column.
 * How each part is pinned (tests/test_oracle.py): dequantize by known-answer
 * blocks, a numpy restatement and the once-rounded exact value; the reference
 * quantizers by known-answer rows (legacy types), a numpy restatement
 * (oracle/np_quant.py, byte for byte) and exact round trips on each format's
 * grid; vec_dot by the exact product to f32 rounding; matmul_candle as
 * quantized rows times vec_dot; matmul_f64 by numpy BLAS.
 * Call sites in the reference that reach these: QTensor::dequantize at
 * crates/mold-inference/src/qwen_image/quantized_transformer.rs:62-66 and
 * crates/mold-inference/src/flux/lora.rs:765; QMatMul::forward through
 * quantized_nn::Linear at crates/mold-inference/src/flux2/quantized_transformer.rs:40-45;
 * QTensor::quantize(.., Q8_0) at crates/mold-inference/src/flux/pipeline.rs:219-229.
 */
#include "ggml_oracle.h"

#include <math.h>
#include <pthread.h>
#include <float.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define QK4_0 32
#define QK4_1 32
#define QK5_0 32
#define QK5_1 32
#define QK8_0 32
#define QK8_1 32
#define QK_K 256
#define K_SCALE_SIZE 12
#define GROUP_MAX_EPS 1e-15f
#define MAX(a, b) ((a) > (b) ? (a) : (b))
#define MIN(a, b) ((a) < (b) ? (a) : (b))

typedef uint16_t half_t;

/* ggml-common.h layouts (packed, little-endian; every member is byte-aligned
 * to its natural size inside the struct so no padding is inserted). */
typedef struct { half_t d; uint8_t qs[QK4_0 / 2]; } block_q4_0;             /* 18 B */
typedef struct { half_t d; half_t m; uint8_t qs[QK4_1 / 2]; } block_q4_1;   /* 20 B */
typedef struct { half_t d; uint8_t qh[4]; uint8_t qs[QK5_0 / 2]; } block_q5_0;            /* 22 B */
typedef struct { half_t d; half_t m; uint8_t qh[4]; uint8_t qs[QK5_1 / 2]; } block_q5_1;  /* 24 B */
typedef struct { half_t d; int8_t qs[QK8_0]; } block_q8_0;                  /* 34 B */
typedef struct { half_t d; half_t s; int8_t qs[QK8_1]; } block_q8_1;        /* 36 B */
typedef struct { uint8_t scales[QK_K / 16]; uint8_t qs[QK_K / 4]; half_t d; half_t dmin; } block_q2_K;  /* 84 B */
typedef struct { uint8_t hmask[QK_K / 8]; uint8_t qs[QK_K / 4]; uint8_t scales[12]; half_t d; } block_q3_K; /* 110 B */
typedef struct { half_t d; half_t dmin; uint8_t scales[K_SCALE_SIZE]; uint8_t qs[QK_K / 2]; } block_q4_K; /* 144 B */
typedef struct { half_t d; half_t dmin; uint8_t scales[K_SCALE_SIZE]; uint8_t qh[QK_K / 8]; uint8_t qs[QK_K / 2]; } block_q5_K; /* 176 B */
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; half_t d; } block_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } block_q8_K; /* 292 B */

_Static_assert(sizeof(block_q4_0) == 18, "q4_0");
_Static_assert(sizeof(block_q4_1) == 20, "q4_1");
_Static_assert(sizeof(block_q5_0) == 22, "q5_0");
_Static_assert(sizeof(block_q5_1) == 24, "q5_1");
_Static_assert(sizeof(block_q8_0) == 34, "q8_0");
_Static_assert(sizeof(block_q8_1) == 36, "q8_1");
_Static_assert(sizeof(block_q2_K) == 84, "q2_K");
_Static_assert(sizeof(block_q3_K) == 110, "q3_K");
_Static_assert(sizeof(block_q4_K) == 144, "q4_K");
_Static_assert(sizeof(block_q5_K) == 176, "q5_K");
_Static_assert(sizeof(block_q6_K) == 210, "q6_K");
_Static_assert(sizeof(block_q8_K) == 292, "q8_K");

/* ------------------------------------------------------------------ halves */

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) {                       /* inf / nan */
        if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    if (a < 0x38800000u) {                        /* below 2^-14: f16 subnormal or zero */
        if (a <= 0x33000000u) return (uint16_t)sign;  /* <= 2^-25 rounds to +-0 (tie to even) */
        const int e = (int)(a >> 23);
        const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;                /* value = mant * 2^(e-150); unit 2^-24 */
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (a - 0x38000000u) >> 13;         /* rebias 127 -> 15 */
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t out;
    if (e == 0) {
        float v = ldexpf((float)m, -24);          /* exact */
        memcpy(&out, &v, 4);
        out |= sign;
    } else if (e == 31) {
        out = sign | 0x7f800000u | (m << 13);
    } else {
        out = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

uint16_t orc_fp32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

#define H2F(h) orc_fp16_to_fp32(h)
#define F2H(f) orc_fp32_to_fp16(f)

/* ------------------------------------------------------------------ geometry */

int orc_block_size(int type) {
    switch (type) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q5_0: case ORC_Q5_1: case ORC_Q8_0: case ORC_Q8_1: return 32;
    case ORC_Q2_K: case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_Q8_K: return QK_K;
    default: return 0;
    }
}

int orc_type_size(int type) {
    switch (type) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q4_0: return sizeof(block_q4_0);
    case ORC_Q4_1: return sizeof(block_q4_1);
    case ORC_Q5_0: return sizeof(block_q5_0);
    case ORC_Q5_1: return sizeof(block_q5_1);
    case ORC_Q8_0: return sizeof(block_q8_0);
    case ORC_Q8_1: return sizeof(block_q8_1);
    case ORC_Q2_K: return sizeof(block_q2_K);
    case ORC_Q3_K: return sizeof(block_q3_K);
    case ORC_Q4_K: return sizeof(block_q4_K);
    case ORC_Q5_K: return sizeof(block_q5_K);
    case ORC_Q6_K: return sizeof(block_q6_K);
    case ORC_Q8_K: return sizeof(block_q8_K);
    default: return 0;
    }
}

/* ggml nearest_int: round half to even through the 1.5*2^23 magic add. */
static inline int nearest_int(float fval) {
    volatile float val = fval + 12582912.f;
    float v = val;
    int i;
    memcpy(&i, &v, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

/* ggml get_scale_min_k4: 6-bit scale/min j of a Q4_K/Q5_K super-block. */
static inline void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

/* ---------------------------------------------------------------- dequantize */

static void deq_q4_0(const block_q4_0 *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK4_0; i++) {
        const float d = H2F(x[i].d);
        for (int j = 0; j < QK4_0 / 2; ++j) {
            const int x0 = (x[i].qs[j] & 0x0F) - 8;
            const int x1 = (x[i].qs[j] >> 4) - 8;
            y[i * QK4_0 + j] = x0 * d;
            y[i * QK4_0 + j + QK4_0 / 2] = x1 * d;
        }
    }
}

static void deq_q4_1(const block_q4_1 *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK4_1; i++) {
        const float d = H2F(x[i].d), m = H2F(x[i].m);
        for (int j = 0; j < QK4_1 / 2; ++j) {
            const int x0 = x[i].qs[j] & 0x0F;
            const int x1 = x[i].qs[j] >> 4;
            y[i * QK4_1 + j] = x0 * d + m;
            y[i * QK4_1 + j + QK4_1 / 2] = x1 * d + m;
        }
    }
}

static void deq_q5_0(const block_q5_0 *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK5_0; i++) {
        const float d = H2F(x[i].d);
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        for (int j = 0; j < QK5_0 / 2; ++j) {
            const uint8_t xh_0 = ((qh >> (j + 0)) << 4) & 0x10;
            const uint8_t xh_1 = ((qh >> (j + 12))) & 0x10;
            const int x0 = ((x[i].qs[j] & 0x0F) | xh_0) - 16;
            const int x1 = ((x[i].qs[j] >> 4) | xh_1) - 16;
            y[i * QK5_0 + j] = x0 * d;
            y[i * QK5_0 + j + QK5_0 / 2] = x1 * d;
        }
    }
}

static void deq_q5_1(const block_q5_1 *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK5_1; i++) {
        const float d = H2F(x[i].d), m = H2F(x[i].m);
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        for (int j = 0; j < QK5_1 / 2; ++j) {
            const uint8_t xh_0 = ((qh >> (j + 0)) << 4) & 0x10;
            const uint8_t xh_1 = ((qh >> (j + 12))) & 0x10;
            const int x0 = (x[i].qs[j] & 0x0F) | xh_0;
            const int x1 = (x[i].qs[j] >> 4) | xh_1;
            y[i * QK5_1 + j] = x0 * d + m;
            y[i * QK5_1 + j + QK5_1 / 2] = x1 * d + m;
        }
    }
}

static void deq_q8_0(const block_q8_0 *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK8_0; i++) {
        const float d = H2F(x[i].d);
        for (int j = 0; j < QK8_0; ++j) y[i * QK8_0 + j] = x[i].qs[j] * d;
    }
}

static void deq_q2_K(const block_q2_K *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d = H2F(x[i].d);
        const float min = H2F(x[i].dmin);
        const uint8_t *q = x[i].qs;
        int is = 0;
        for (int n = 0; n < QK_K; n += 128) {
            int shift = 0;
            for (int j = 0; j < 4; ++j) {
                uint8_t sc = x[i].scales[is++];
                float dl = d * (sc & 0xF), ml = min * (sc >> 4);
                for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l] >> shift) & 3)) - ml;
                sc = x[i].scales[is++];
                dl = d * (sc & 0xF);
                ml = min * (sc >> 4);
                for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l + 16] >> shift) & 3)) - ml;
                shift += 2;
            }
            q += 32;
        }
    }
}

/* Unpack the 16 six-bit Q3_K scales (stored offset by 32) into signed bytes. */
static void q3k_unpack_scales(const uint8_t *packed, int8_t *scales) {
    const uint32_t kmask1 = 0x03030303, kmask2 = 0x0f0f0f0f;
    uint32_t aux[4];
    memcpy(aux, packed, 12);
    const uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    memcpy(scales, aux, 16);
}

static void deq_q3_K(const block_q3_K *x, float *y, int64_t k) {
    int8_t scales[16];
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d_all = H2F(x[i].d);
        const uint8_t *q = x[i].qs;
        const uint8_t *hm = x[i].hmask;
        uint8_t m = 1;
        q3k_unpack_scales(x[i].scales, scales);
        int is = 0;
        for (int n = 0; n < QK_K; n += 128) {
            int shift = 0;
            for (int j = 0; j < 4; ++j) {
                float dl = d_all * (scales[is++] - 32);
                for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l + 0] >> shift) & 3) - ((hm[l + 0] & m) ? 0 : 4));
                dl = d_all * (scales[is++] - 32);
                for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l + 16] >> shift) & 3) - ((hm[l + 16] & m) ? 0 : 4));
                shift += 2;
                m <<= 1;
            }
            q += 32;
        }
    }
}

static void deq_q4_K(const block_q4_K *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++) {
        const uint8_t *q = x[i].qs;
        const float d = H2F(x[i].d), min = H2F(x[i].dmin);
        int is = 0;
        uint8_t sc, m;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = min * m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

static void deq_q5_K(const block_q5_K *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++) {
        const uint8_t *ql = x[i].qs, *qh = x[i].qh;
        const float d = H2F(x[i].d), min = H2F(x[i].dmin);
        int is = 0;
        uint8_t sc, m, u1 = 1, u2 = 2;
        for (int j = 0; j < QK_K; j += 64) {
            get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = min * m;
            get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = min * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
            ql += 32;
            is += 2;
            u1 <<= 2;
            u2 <<= 2;
        }
    }
}

static void deq_q6_K(const block_q6_K *x, float *y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d = H2F(x[i].d);
        const uint8_t *ql = x[i].ql, *qh = x[i].qh;
        const int8_t *sc = x[i].scales;
        for (int n = 0; n < QK_K; n += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * sc[is + 0] * q1;
                y[l + 32] = d * sc[is + 2] * q2;
                y[l + 64] = d * sc[is + 4] * q3;
                y[l + 96] = d * sc[is + 6] * q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

int orc_dequantize_row(int type, const void *b, float *y, int64_t k) {
    const int bs = orc_block_size(type);
    if (bs == 0 || k % bs != 0) return -1;
    switch (type) {
    case ORC_F32: memcpy(y, b, (size_t)k * 4); return 0;
    case ORC_F16: for (int64_t i = 0; i < k; i++) y[i] = H2F(((const uint16_t *)b)[i]); return 0;
    case ORC_BF16:
        for (int64_t i = 0; i < k; i++) {
            uint32_t u = (uint32_t)((const uint16_t *)b)[i] << 16;
            memcpy(&y[i], &u, 4);
        }
        return 0;
    case ORC_Q4_0: deq_q4_0(b, y, k); return 0;
    case ORC_Q4_1: deq_q4_1(b, y, k); return 0;
    case ORC_Q5_0: deq_q5_0(b, y, k); return 0;
    case ORC_Q5_1: deq_q5_1(b, y, k); return 0;
    case ORC_Q8_0: deq_q8_0(b, y, k); return 0;
    case ORC_Q2_K: deq_q2_K(b, y, k); return 0;
    case ORC_Q3_K: deq_q3_K(b, y, k); return 0;
    case ORC_Q4_K: deq_q4_K(b, y, k); return 0;
    case ORC_Q5_K: deq_q5_K(b, y, k); return 0;
    case ORC_Q6_K: deq_q6_K(b, y, k); return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------- quantize */

static void quant_q4_0(const float *x, block_q4_0 *y, int64_t k) {
    const int qk = QK4_0;
    for (int64_t i = 0; i < k / qk; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < qk; j++) {
            const float v = x[i * qk + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        for (int j = 0; j < qk / 2; ++j) {
            const float x0 = x[i * qk + 0 + j] * id;
            const float x1 = x[i * qk + qk / 2 + j] * id;
            const uint8_t xi0 = MIN(15, (int8_t)(x0 + 8.5f));
            const uint8_t xi1 = MIN(15, (int8_t)(x1 + 8.5f));
            y[i].qs[j] = xi0 | (uint8_t)(xi1 << 4);
        }
    }
}

static void quant_q4_1(const float *x, block_q4_1 *y, int64_t k) {
    const int qk = QK4_1;
    for (int64_t i = 0; i < k / qk; i++) {
        float min = FLT_MAX, max = -FLT_MAX;
        for (int j = 0; j < qk; j++) {
            const float v = x[i * qk + j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / ((1 << 4) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        y[i].m = F2H(min);
        for (int j = 0; j < qk / 2; ++j) {
            const float x0 = (x[i * qk + 0 + j] - min) * id;
            const float x1 = (x[i * qk + qk / 2 + j] - min) * id;
            const uint8_t xi0 = MIN(15, (int8_t)(x0 + 0.5f));
            const uint8_t xi1 = MIN(15, (int8_t)(x1 + 0.5f));
            y[i].qs[j] = xi0 | (uint8_t)(xi1 << 4);
        }
    }
}

static void quant_q5_0(const float *x, block_q5_0 *y, int64_t k) {
    const int qk = QK5_0;
    for (int64_t i = 0; i < k / qk; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < qk; j++) {
            const float v = x[i * qk + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -16;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        uint32_t qh = 0;
        for (int j = 0; j < qk / 2; ++j) {
            const float x0 = x[i * qk + 0 + j] * id;
            const float x1 = x[i * qk + qk / 2 + j] * id;
            const uint8_t xi0 = MIN(31, (int8_t)(x0 + 16.5f));
            const uint8_t xi1 = MIN(31, (int8_t)(x1 + 16.5f));
            y[i].qs[j] = (xi0 & 0x0F) | (uint8_t)((xi1 & 0x0F) << 4);
            qh |= ((xi0 & 0x10u) >> 4) << (j + 0);
            qh |= ((xi1 & 0x10u) >> 4) << (j + qk / 2);
        }
        memcpy(y[i].qh, &qh, 4);
    }
}

static void quant_q5_1(const float *x, block_q5_1 *y, int64_t k) {
    const int qk = QK5_1;
    for (int64_t i = 0; i < k / qk; i++) {
        float min = x[i * qk], max = x[i * qk];
        for (int j = 1; j < qk; j++) {
            const float v = x[i * qk + j];
            if (v < min) min = v;
            if (v > max) max = v;
        }
        const float d = (max - min) / ((1 << 5) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        y[i].m = F2H(min);
        uint32_t qh = 0;
        for (int j = 0; j < qk / 2; ++j) {
            const float x0 = (x[i * qk + 0 + j] - min) * id;
            const float x1 = (x[i * qk + qk / 2 + j] - min) * id;
            const uint8_t xi0 = (uint8_t)(x0 + 0.5f);
            const uint8_t xi1 = (uint8_t)(x1 + 0.5f);
            y[i].qs[j] = (xi0 & 0x0F) | (uint8_t)((xi1 & 0x0F) << 4);
            qh |= ((xi0 & 0x10u) >> 4) << (j + 0);
            qh |= ((xi1 & 0x10u) >> 4) << (j + qk / 2);
        }
        memcpy(y[i].qh, &qh, 4);
    }
}

static void quant_q8_0(const float *x, block_q8_0 *y, int64_t k) {
    for (int64_t i = 0; i < k / QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = MAX(amax, fabsf(x[i * QK8_0 + j]));
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        for (int j = 0; j < QK8_0; ++j) y[i].qs[j] = (int8_t)roundf(x[i * QK8_0 + j] * id);
    }
}

/* ggml make_qx_quants (Q6_K uses rmse_type 1, no importance weights). */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *L, int rmse_type, const float *qw) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    if (rmse_type == 0) {
        for (int i = 0; i < n; ++i) {
            const int l = nearest_int(iscale * x[i]);
            L[i] = (int8_t)(nmax + MAX(-nmax, MIN(nmax - 1, l)));
        }
        return 1 / iscale;
    }
    int return_early = 0;
    if (rmse_type < 0) { rmse_type = -rmse_type; return_early = 1; }
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = MAX(-nmax, MIN(nmax - 1, l));
        L[i] = (int8_t)(l + nmax);
        const float w = qw ? qw[i] : rmse_type == 1 ? x[i] * x[i] : rmse_type == 2 ? 1 : rmse_type == 3 ? fabsf(x[i]) : sqrtf(fabsf(x[i]));
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    if (return_early) return suml2 > 0 ? 0.5f * (scale + 1 / iscale) : 1 / iscale;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = MAX(-nmax, MIN(nmax - 1, l));
            const float w = qw ? qw[i] : rmse_type == 1 ? x[i] * x[i] : rmse_type == 2 ? 1 : rmse_type == 3 ? fabsf(x[i]) : sqrtf(fabsf(x[i]));
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                const int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t)(nmax + MAX(-nmax, MIN(nmax - 1, l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* ggml make_q3_quants (Q3_K). */
static float make_q3_quants(int n, int nmax, const float *x, int8_t *L, int do_rmse) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    const float iscale = -nmax / max;
    if (do_rmse) {
        float sumlx = 0, suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = MAX(-nmax, MIN(nmax - 1, l));
            L[i] = (int8_t)l;
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        for (int itry = 0; itry < 5; ++itry) {
            int n_changed = 0;
            for (int i = 0; i < n; ++i) {
                const float w = x[i] * x[i];
                float slx = sumlx - w * x[i] * L[i];
                if (slx > 0) {
                    float sl2 = suml2 - w * L[i] * L[i];
                    int new_l = nearest_int(x[i] * sl2 / slx);
                    new_l = MAX(-nmax, MIN(nmax - 1, new_l));
                    if (new_l != L[i]) {
                        slx += w * x[i] * new_l;
                        sl2 += w * new_l * new_l;
                        if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
                            L[i] = (int8_t)new_l;
                            sumlx = slx;
                            suml2 = sl2;
                            ++n_changed;
                        }
                    }
                }
            }
            if (!n_changed) break;
        }
        for (int i = 0; i < n; ++i) L[i] = (int8_t)(L[i] + nmax);
        return sumlx / suml2;
    }
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = MAX(-nmax, MIN(nmax - 1, l));
        L[i] = (int8_t)(l + nmax);
    }
    return 1 / iscale;
}

/* ggml make_qkx2_quants (Q2_K, Q4_K, Q5_K): scale + min search. */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L,
                              float *the_min, uint8_t *Laux, float rmin, float rdelta, int nstep, int use_mad) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)MAX(0, MIN(nmax, l));
        float diff = scale * L[i] + min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best_mad += weights[i] * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = MAX(0, MIN(nmax, l));
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = use_mad ? fabsf(diff) : diff * diff;
                mad += weights[i] * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

static void quant_q2_K(const float *x, block_q2_K *y, int64_t k) {
    uint8_t L[QK_K], Laux[16];
    float weights[16], mins[QK_K / 16], scales[QK_K / 16];
    const float q4scale = 15.f;
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 16; ++j) {
            for (int l = 0; l < 16; ++l) weights[l] = fabsf(x[16 * j + l]);
            scales[j] = make_qkx2_quants(16, 3, x + 16 * j, weights, L + 16 * j, &mins[j], Laux, -0.5f, 0.1f, 15, 1);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        if (max_scale > 0) {
            const float iscale = q4scale / max_scale;
            for (int j = 0; j < QK_K / 16; ++j) y[i].scales[j] = (uint8_t)nearest_int(iscale * scales[j]);
            y[i].d = F2H(max_scale / q4scale);
        } else {
            for (int j = 0; j < QK_K / 16; ++j) y[i].scales[j] = 0;
            y[i].d = F2H(0.f);
        }
        if (max_min > 0) {
            const float iscale = q4scale / max_min;
            for (int j = 0; j < QK_K / 16; ++j) y[i].scales[j] |= (uint8_t)(nearest_int(iscale * mins[j]) << 4);
            y[i].dmin = F2H(max_min / q4scale);
        } else {
            y[i].dmin = F2H(0.f);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            const float d = H2F(y[i].d) * (y[i].scales[j] & 0xF);
            if (!d) continue;
            const float dm = H2F(y[i].dmin) * (y[i].scales[j] >> 4);
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int((x[16 * j + ii] + dm) / d);
                L[16 * j + ii] = (uint8_t)MAX(0, MIN(3, l));
            }
        }
        for (int j = 0; j < QK_K; j += 128)
            for (int l = 0; l < 32; ++l)
                y[i].qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
        x += QK_K;
    }
}

static void quant_q3_K(const float *x, block_q3_K *y, int64_t k) {
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, amax = 0;
        for (int j = 0; j < QK_K / 16; ++j) {
            scales[j] = make_q3_quants(16, 4, x + 16 * j, L + 16 * j, 1);
            const float scale = fabsf(scales[j]);
            if (scale > amax) { amax = scale; max_scale = scales[j]; }
        }
        memset(y[i].scales, 0, 12);
        if (max_scale) {
            const float iscale = -32.f / max_scale;
            for (int j = 0; j < QK_K / 16; ++j) {
                int8_t l = (int8_t)nearest_int(iscale * scales[j]);
                l = (int8_t)(MAX(-32, MIN(31, l)) + 32);
                if (j < 8) y[i].scales[j] = l & 0xF;
                else y[i].scales[j - 8] |= (uint8_t)((l & 0xF) << 4);
                l >>= 4;
                y[i].scales[j % 4 + 8] |= (uint8_t)(l << (2 * (j / 4)));
            }
            y[i].d = F2H(1 / iscale);
        } else {
            y[i].d = F2H(0.f);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int8_t sc = j < 8 ? (int8_t)(y[i].scales[j] & 0xF) : (int8_t)(y[i].scales[j - 8] >> 4);
            sc = (int8_t)((sc | (((y[i].scales[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32);
            const float d = H2F(y[i].d) * sc;
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = MAX(-4, MIN(3, l));
                L[16 * j + ii] = (int8_t)(l + 4);
            }
        }
        memset(y[i].hmask, 0, QK_K / 8);
        int m = 0;
        uint8_t hm = 1;
        for (int j = 0; j < QK_K; ++j) {
            if (L[j] > 3) {
                y[i].hmask[m] |= hm;
                L[j] -= 4;
            }
            if (++m == QK_K / 8) { m = 0; hm <<= 1; }
        }
        for (int j = 0; j < QK_K; j += 128)
            for (int l = 0; l < 32; ++l)
                y[i].qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
        x += QK_K;
    }
}

/* Pack 6-bit scale ls and min lm of sub-block j (Q4_K / Q5_K scales[12]). */
static void pack_scale_min_k4(uint8_t *s, int j, uint8_t ls, uint8_t lm) {
    if (j < 4) {
        s[j] = ls;
        s[j + 4] = lm;
    } else {
        s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        s[j - 4] |= (uint8_t)((ls >> 4) << 6);
        s[j - 0] |= (uint8_t)((lm >> 4) << 6);
    }
}

static void quant_q4_K(const float *x, block_q4_K *y, int64_t k) {
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20, 0);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
            pack_scale_min_k4(y[i].scales, j, MIN(63, ls), MIN(63, lm));
        }
        y[i].d = F2H(max_scale / 63.f);
        y[i].dmin = F2H(max_min / 63.f);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = H2F(y[i].d) * sc;
            if (!d) continue;
            const float dm = H2F(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                L[32 * j + ii] = (uint8_t)MAX(0, MIN(15, l));
            }
        }
        uint8_t *q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += QK_K;
    }
}

static void quant_q5_K(const float *x, block_q5_K *y, int64_t k) {
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 31, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15, 0);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
            pack_scale_min_k4(y[i].scales, j, MIN(63, ls), MIN(63, lm));
        }
        y[i].d = F2H(max_scale / 63.f);
        y[i].dmin = F2H(max_min / 63.f);
        uint8_t sc, m;
        for (int j = 0; j < QK_K / 32; ++j) {
            get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = H2F(y[i].d) * sc;
            if (!d) continue;
            const float dm = H2F(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((x[32 * j + ii] + dm) / d);
                L[32 * j + ii] = (uint8_t)MAX(0, MIN(31, l));
            }
        }
        uint8_t *qh = y[i].qh, *ql = y[i].qs;
        memset(qh, 0, QK_K / 8);
        uint8_t m1 = 1, m2 = 2;
        for (int n = 0; n < QK_K; n += 64) {
            for (int j = 0; j < 32; ++j) {
                int l1 = L[n + j];
                if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
                int l2 = L[n + j + 32];
                if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
                ql[j] = (uint8_t)(l1 | (l2 << 4));
            }
            m1 <<= 2;
            m2 <<= 2;
            ql += 32;
        }
        x += QK_K;
    }
}

static void quant_q6_K(const float *x, block_q6_K *y, int64_t k) {
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < k / QK_K; i++) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < QK_K / 16; ++ib) {
            const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, 1, NULL);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) { max_abs_scale = abs_scale; max_scale = scale; }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            memset(&y[i], 0, sizeof(block_q6_K));
            y[i].d = F2H(0.f);
            x += QK_K;
            continue;
        }
        const float iscale = -128.f / max_scale;
        y[i].d = F2H(1 / iscale);
        for (int ib = 0; ib < QK_K / 16; ++ib) y[i].scales[ib] = (int8_t)MIN(127, nearest_int(iscale * scales[ib]));
        for (int j = 0; j < QK_K / 16; ++j) {
            const float d = H2F(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[16 * j + ii] / d);
                l = MAX(-32, MIN(31, l));
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = y[i].ql, *qh = y[i].qh;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += QK_K;
    }
}

int orc_quantize_row(int type, const float *x, void *b, int64_t k) {
    const int bs = orc_block_size(type);
    if (bs == 0 || k % bs != 0) return -1;
    switch (type) {
    case ORC_F32: memcpy(b, x, (size_t)k * 4); return 0;
    case ORC_F16: for (int64_t i = 0; i < k; i++) ((uint16_t *)b)[i] = F2H(x[i]); return 0;
    case ORC_BF16: for (int64_t i = 0; i < k; i++) ((uint16_t *)b)[i] = orc_fp32_to_bf16(x[i]); return 0;
    case ORC_Q4_0: quant_q4_0(x, b, k); return 0;
    case ORC_Q4_1: quant_q4_1(x, b, k); return 0;
    case ORC_Q5_0: quant_q5_0(x, b, k); return 0;
    case ORC_Q5_1: quant_q5_1(x, b, k); return 0;
    case ORC_Q8_0: quant_q8_0(x, b, k); return 0;
    case ORC_Q2_K: quant_q2_K(x, b, k); return 0;
    case ORC_Q3_K: quant_q3_K(x, b, k); return 0;
    case ORC_Q4_K: quant_q4_K(x, b, k); return 0;
    case ORC_Q5_K: quant_q5_K(x, b, k); return 0;
    case ORC_Q6_K: quant_q6_K(x, b, k); return 0;
    default: return -1;
    }
}

/* ------------------------------------------------ activation quantizers */

void orc_quantize_row_q8_0(const float *x, void *b, int64_t k) { quant_q8_0(x, (block_q8_0 *)b, k); }

/* candle BlockQ8_1::from_float: s = f16(sum) * d evaluated in half. */
void orc_quantize_row_q8_1(const float *x, void *vb, int64_t k) {
    block_q8_1 *y = (block_q8_1 *)vb;
    for (int64_t i = 0; i < k / QK8_1; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_1; j++) amax = MAX(amax, fabsf(x[i * QK8_1 + j]));
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = F2H(d);
        int sum = 0;
        for (int j = 0; j < QK8_1 / 2; ++j) {
            y[i].qs[j] = (int8_t)roundf(x[i * QK8_1 + j] * id);
            y[i].qs[j + QK8_1 / 2] = (int8_t)roundf(x[i * QK8_1 + j + QK8_1 / 2] * id);
            sum += y[i].qs[j] + y[i].qs[j + QK8_1 / 2];
        }
        y[i].s = F2H(H2F(F2H((float)sum)) * H2F(y[i].d));
    }
}

/* candle BlockQ8K::from_float: iscale = -128/max, round half away from zero. */
void orc_quantize_row_q8_K(const float *x, void *vb, int64_t k) {
    block_q8_K *y = (block_q8_K *)vb;
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float *xs = x + i * QK_K;
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; ++j) {
            if (amax < fabsf(xs[j])) { amax = fabsf(xs[j]); max = xs[j]; }
        }
        if (amax == 0.f) {
            y[i].d = 0.f;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            continue;
        }
        const float iscale = -128.f / max;
        for (int j = 0; j < QK_K; ++j) {
            const float v = roundf(iscale * xs[j]);
            y[i].qs[j] = (int8_t)MIN(v, 127.f);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1.0f / iscale;
    }
}

int orc_vec_dot_type(int type) {
    switch (type) {
    case ORC_Q4_0: case ORC_Q5_0: case ORC_Q8_0: return ORC_Q8_0;
    case ORC_Q4_1: case ORC_Q5_1: return ORC_Q8_1;
    case ORC_Q2_K: case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return ORC_Q8_K;
    default: return -1;
    }
}

/* ----------------------------------------------------------------- vec_dot */

static float vd_q4_0(int64_t k, const block_q4_0 *x, const block_q8_0 *y) {
    float sumf = 0;
    for (int64_t i = 0; i < k / QK8_0; i++) {
        int sumi = 0;
        for (int j = 0; j < QK8_0 / 2; ++j) {
            const int v0 = (x[i].qs[j] & 0x0F) - 8;
            const int v1 = (x[i].qs[j] >> 4) - 8;
            sumi += v0 * y[i].qs[j] + v1 * y[i].qs[j + QK8_0 / 2];
        }
        sumf += (float)sumi * H2F(x[i].d) * H2F(y[i].d);
    }
    return sumf;
}

static float vd_q4_1(int64_t k, const block_q4_1 *x, const block_q8_1 *y) {
    float sumf = 0;
    for (int64_t i = 0; i < k / QK8_1; i++) {
        int sumi = 0;
        for (int j = 0; j < QK8_1 / 2; ++j) {
            const int v0 = x[i].qs[j] & 0x0F;
            const int v1 = x[i].qs[j] >> 4;
            sumi += v0 * y[i].qs[j] + v1 * y[i].qs[j + QK8_1 / 2];
        }
        sumf += (float)sumi * H2F(x[i].d) * H2F(y[i].d) + H2F(x[i].m) * H2F(y[i].s);
    }
    return sumf;
}

static float vd_q5_0(int64_t k, const block_q5_0 *x, const block_q8_0 *y) {
    float sumf = 0;
    for (int64_t i = 0; i < k / QK8_0; i++) {
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < QK8_0 / 2; ++j) {
            const uint8_t xh_0 = (uint8_t)(((qh & (1u << (j + 0))) >> (j + 0)) << 4);
            const uint8_t xh_1 = (uint8_t)((qh & (1u << (j + 16))) >> (j + 12));
            const int x0 = (int8_t)(((x[i].qs[j] & 0x0F) | xh_0) - 16);
            const int x1 = (int8_t)(((x[i].qs[j] >> 4) | xh_1) - 16);
            sumi0 += x0 * y[i].qs[j];
            sumi1 += x1 * y[i].qs[j + QK8_0 / 2];
        }
        sumf += (H2F(x[i].d) * H2F(y[i].d)) * (float)(sumi0 + sumi1);
    }
    return sumf;
}

static float vd_q5_1(int64_t k, const block_q5_1 *x, const block_q8_1 *y) {
    float sumf = 0;
    for (int64_t i = 0; i < k / QK8_1; i++) {
        uint32_t qh;
        memcpy(&qh, x[i].qh, 4);
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < QK8_1 / 2; ++j) {
            const uint8_t xh_0 = (uint8_t)(((qh >> (j + 0)) << 4) & 0x10);
            const uint8_t xh_1 = (uint8_t)((qh >> (j + 12)) & 0x10);
            const int x0 = (x[i].qs[j] & 0xF) | xh_0;
            const int x1 = (x[i].qs[j] >> 4) | xh_1;
            sumi0 += x0 * y[i].qs[j];
            sumi1 += x1 * y[i].qs[j + QK8_1 / 2];
        }
        sumf += (H2F(x[i].d) * H2F(y[i].d)) * (float)(sumi0 + sumi1) + H2F(x[i].m) * H2F(y[i].s);
    }
    return sumf;
}

static float vd_q8_0(int64_t k, const block_q8_0 *x, const block_q8_0 *y) {
    float sumf = 0;
    for (int64_t i = 0; i < k / QK8_0; i++) {
        int sumi = 0;
        for (int j = 0; j < QK8_0; ++j) sumi += x[i].qs[j] * y[i].qs[j];
        sumf += (float)sumi * H2F(x[i].d) * H2F(y[i].d);
    }
    return sumf;
}

static float vd_q2_K(int64_t k, const block_q2_K *x, const block_q8_K *y) {
    float sumf = 0;
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const uint8_t *q2 = x[i].qs;
        const int8_t *q8 = y[i].qs;
        const uint8_t *sc = x[i].scales;
        int summs = 0;
        for (int j = 0; j < 16; ++j) summs += y[i].bsums[j] * (sc[j] >> 4);
        const float dall = y[i].d * H2F(x[i].d);
        const float dmin = y[i].d * H2F(x[i].dmin);
        int isum = 0, is = 0;
        for (int kk = 0; kk < QK_K / 128; ++kk) {
            int shift = 0;
            for (int j = 0; j < 4; ++j) {
                int d = sc[is++] & 0xF;
                int isuml = 0;
                for (int l = 0; l < 16; ++l) isuml += q8[l] * ((q2[l] >> shift) & 3);
                isum += d * isuml;
                d = sc[is++] & 0xF;
                isuml = 0;
                for (int l = 16; l < 32; ++l) isuml += q8[l] * ((q2[l] >> shift) & 3);
                isum += d * isuml;
                shift += 2;
                q8 += 32;
            }
            q2 += 32;
        }
        sumf += dall * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

static float vd_q3_K(int64_t k, const block_q3_K *x, const block_q8_K *y) {
    int8_t scales[16], aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const uint8_t *q3 = x[i].qs, *hm = x[i].hmask;
        const int8_t *q8 = y[i].qs;
        memset(aux32, 0, sizeof(aux32));
        int8_t *a = aux8;
        uint8_t m = 1;
        for (int j = 0; j < QK_K; j += 128) {
            for (int sh = 0; sh < 8; sh += 2) {
                for (int l = 0; l < 32; ++l) a[l] = (int8_t)((q3[l] >> sh) & 3);
                for (int l = 0; l < 32; ++l) a[l] = (int8_t)(a[l] - (hm[l] & m ? 0 : 4));
                a += 32;
                m <<= 1;
            }
            q3 += 32;
        }
        a = aux8;
        q3k_unpack_scales(x[i].scales, scales);
        for (int j = 0; j < QK_K / 16; ++j) {
            for (int half = 0; half < 2; ++half) {
                for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; ++l) aux32[l] += (scales[j] - 32) * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = H2F(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* Unpack Q4_K/Q5_K scales[12] into 8 six-bit scales and 8 six-bit mins. */
static void k4_unpack(const uint8_t *packed, uint8_t *scales, uint8_t *mins) {
    const uint32_t kmask1 = 0x3f3f3f3f, kmask2 = 0x0f0f0f0f, kmask3 = 0x03030303;
    uint32_t utmp[4];
    memcpy(utmp, packed, 12);
    utmp[3] = ((utmp[2] >> 4) & kmask2) | (((utmp[1] >> 6) & kmask3) << 4);
    const uint32_t uaux = utmp[1] & kmask1;
    utmp[1] = (utmp[2] & kmask2) | (((utmp[0] >> 6) & kmask3) << 4);
    utmp[2] = uaux;
    utmp[0] &= kmask1;
    memcpy(scales, &utmp[0], 8);
    memcpy(mins, &utmp[2], 8);
}

static float vd_q45_K(int64_t k, const void *vx, const block_q8_K *y, int five) {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    uint8_t scales[8], mins[8];
    float sumf = 0;
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const uint8_t *q4, *hm = NULL, *packed;
        float xd, xdmin;
        if (five) {
            const block_q5_K *x = (const block_q5_K *)vx + i;
            q4 = x->qs; hm = x->qh; packed = x->scales; xd = H2F(x->d); xdmin = H2F(x->dmin);
        } else {
            const block_q4_K *x = (const block_q4_K *)vx + i;
            q4 = x->qs; packed = x->scales; xd = H2F(x->d); xdmin = H2F(x->dmin);
        }
        const int8_t *q8 = y[i].qs;
        memset(aux32, 0, sizeof(aux32));
        int8_t *a = aux8;
        uint8_t m = 1;
        for (int j = 0; j < QK_K / 64; ++j) {
            for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] & 0xF);
            if (five) for (int l = 0; l < 32; ++l) a[l] = (int8_t)(a[l] + (hm[l] & m ? 16 : 0));
            a += 32;
            m <<= 1;
            for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] >> 4);
            if (five) for (int l = 0; l < 32; ++l) a[l] = (int8_t)(a[l] + (hm[l] & m ? 16 : 0));
            a += 32;
            m <<= 1;
            q4 += 32;
        }
        k4_unpack(packed, scales, mins);
        int sumi = 0;
        for (int j = 0; j < QK_K / 16; ++j) sumi += y[i].bsums[j] * mins[j / 2];
        a = aux8;
        for (int j = 0; j < QK_K / 32; ++j) {
            const int32_t scale = scales[j];
            for (int part = 0; part < 4; ++part) {
                for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = xd * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        const float dmin = xdmin * y[i].d;
        sumf -= dmin * (float)sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static float vd_q6_K(int64_t k, const block_q6_K *x, const block_q8_K *y) {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    for (int64_t i = 0; i < k / QK_K; ++i) {
        const uint8_t *q4 = x[i].ql, *qh = x[i].qh;
        const int8_t *q8 = y[i].qs;
        memset(aux32, 0, sizeof(aux32));
        int8_t *a = aux8;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                a[l + 0] = (int8_t)((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                a[l + 32] = (int8_t)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                a[l + 64] = (int8_t)((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                a[l + 96] = (int8_t)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            }
            a += 128;
            q4 += 64;
            qh += 32;
        }
        a = aux8;
        int is = 0;
        for (int j = 0; j < QK_K / 16; ++j) {
            const int scale = x[i].scales[is++];
            for (int half = 0; half < 2; ++half) {
                for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = H2F(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

float orc_vec_dot(int type, int64_t k, const void *w, const void *a) {
    switch (type) {
    case ORC_Q4_0: return vd_q4_0(k, w, a);
    case ORC_Q4_1: return vd_q4_1(k, w, a);
    case ORC_Q5_0: return vd_q5_0(k, w, a);
    case ORC_Q5_1: return vd_q5_1(k, w, a);
    case ORC_Q8_0: return vd_q8_0(k, w, a);
    case ORC_Q2_K: return vd_q2_K(k, w, a);
    case ORC_Q3_K: return vd_q3_K(k, w, a);
    case ORC_Q4_K: return vd_q45_K(k, w, a, 0);
    case ORC_Q5_K: return vd_q45_K(k, w, a, 1);
    case ORC_Q6_K: return vd_q6_K(k, w, a);
    default: return NAN;
    }
}

/* ------------------------------------------------------------------ matmul */

typedef struct {
    int type, vdt;
    int64_t m, n, k, n0, n1;
    const float *x;
    const uint8_t *w;
    const uint8_t *act;
    float *y;
    double *yd;
    size_t w_row_bytes, a_row_bytes;
} mm_job;

static void *mm_candle_worker(void *p) {
    mm_job *j = (mm_job *)p;
    for (int64_t r = 0; r < j->m; r++) {
        const uint8_t *arow = j->act + (size_t)r * j->a_row_bytes;
        for (int64_t c = j->n0; c < j->n1; c++)
            j->y[r * j->n + c] = orc_vec_dot(j->type, j->k, j->w + (size_t)c * j->w_row_bytes, arow);
    }
    return NULL;
}

static void *mm_f64_worker(void *p) {
    mm_job *j = (mm_job *)p;
    float *wrow = (float *)malloc((size_t)j->k * sizeof(float));
    for (int64_t c = j->n0; c < j->n1; c++) {
        orc_dequantize_row(j->type, j->w + (size_t)c * j->w_row_bytes, wrow, j->k);
        for (int64_t r = 0; r < j->m; r++) {
            const float *xr = j->x + r * j->k;
            double acc = 0.0;
            for (int64_t t = 0; t < j->k; t++) acc += (double)xr[t] * (double)wrow[t];
            j->yd[r * j->n + c] = acc;
        }
    }
    free(wrow);
    return NULL;
}

static int resolve_threads(int nthreads, int64_t n) {
    if (nthreads <= 0) {
        long c = sysconf(_SC_NPROCESSORS_ONLN);
        nthreads = c > 0 ? (int)c : 1;
    }
    if (nthreads > n) nthreads = (int)(n > 0 ? n : 1);
    if (nthreads > 256) nthreads = 256;
    return nthreads;
}

/* Split output columns [0, n) into nthreads contiguous ranges; thread 0's
 * range runs on the calling thread.  A failed pthread_create runs inline. */
static void run_split(mm_job *proto, int nthreads, void *(*fn)(void *)) {
    pthread_t th[256];
    int created[256];
    mm_job jobs[256];
    const int64_t per = (proto->n + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = *proto;
        jobs[t].n0 = t * per;
        jobs[t].n1 = MIN(proto->n, (t + 1) * per);
        created[t] = 0;
        if (t == 0 || jobs[t].n0 >= jobs[t].n1) continue;
        if (pthread_create(&th[t], NULL, fn, &jobs[t]) == 0) created[t] = 1;
        else fn(&jobs[t]);
    }
    if (jobs[0].n0 < jobs[0].n1) fn(&jobs[0]);
    for (int t = 1; t < nthreads; t++)
        if (created[t]) pthread_join(th[t], NULL);
}

int orc_matmul_candle(int type, int64_t m, int64_t n, int64_t k, const float *x, const void *w, float *y, int nthreads) {
    const int vdt = orc_vec_dot_type(type);
    const int bs = orc_block_size(type);
    if (vdt < 0 || bs == 0 || k % bs != 0 || m < 0 || n < 0) return -1;
    if (m == 0 || n == 0) return 0;
    const size_t a_row = (size_t)(k / orc_block_size(vdt)) * orc_type_size(vdt);
    uint8_t *act = (uint8_t *)malloc(a_row * (size_t)m);
    if (!act) return -2;
    for (int64_t r = 0; r < m; r++) {
        uint8_t *dst = act + (size_t)r * a_row;
        if (vdt == ORC_Q8_0) orc_quantize_row_q8_0(x + r * k, dst, k);
        else if (vdt == ORC_Q8_1) orc_quantize_row_q8_1(x + r * k, dst, k);
        else orc_quantize_row_q8_K(x + r * k, dst, k);
    }
    mm_job proto = {0};
    proto.type = type; proto.vdt = vdt; proto.m = m; proto.n = n; proto.k = k;
    proto.x = x; proto.w = (const uint8_t *)w; proto.act = act; proto.y = y;
    proto.w_row_bytes = (size_t)(k / bs) * orc_type_size(type);
    proto.a_row_bytes = a_row;
    run_split(&proto, resolve_threads(nthreads, n), mm_candle_worker);
    free(act);
    return 0;
}

int orc_matmul_f64(int type, int64_t m, int64_t n, int64_t k, const float *x, const void *w, double *y) {
    const int bs = orc_block_size(type);
    if (bs == 0 || k % bs != 0 || m < 0 || n < 0) return -1;
    if (m == 0 || n == 0) return 0;
    mm_job proto = {0};
    proto.type = type; proto.m = m; proto.n = n; proto.k = k;
    proto.x = x; proto.w = (const uint8_t *)w; proto.yd = y;
    proto.w_row_bytes = (size_t)(k / bs) * orc_type_size(type);
    run_split(&proto, resolve_threads(0, n), mm_f64_worker);
    return 0;
}

void orc_lora_apply(float *w, int64_t ldw, int64_t rows, int64_t k, const float *b, int64_t ldb,
                    const float *a, int64_t lda, int rank, float scale) {
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < k; ++j) {
      float d = 0.f;
      for (int r = 0; r < rank; ++r) d = fmaf(b[i * ldb + r], a[(int64_t)r * lda + j], d);
      const float t = d * scale;
      w[i * ldw + j] = w[i * ldw + j] + t;
    }
}
