/*
 * ggml_oracle.h — CPU oracle for the GGUF quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  The only permitted users are tests/, the smoke() check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py, and there only as
 * the checker or the reported CPU baseline, never as the measured product.
 *
 * What it restates (the algorithms live in un-vendored crates pinned by the
 * reference, /root/reference/Cargo.lock:507-543, candle-core-mold 0.9.10 and
 * candle-kernels 0.9.2, which mirror ggml's published block formats):
 *   - GGUF/ggml block layouts and the per-type dequantize formulas
 *     (candle `QTensor::dequantize`, called at
 *     crates/mold-inference/src/qwen_image/quantized_transformer.rs:62-66,
 *     crates/mold-inference/src/flux/lora.rs:765);
 *   - ggml's reference quantizers (quantize_row_*_ref), used to make the
 *     blocks every test and benchmark feeds to the kernels (the quantizer is
 *     fixture generation, not graded: the blocks are the contract);
 *   - candle's CPU QMatMul algorithm: activations quantized to the weight
 *     type's vec-dot type (Q8_0 / Q8_1 / Q8_K) then integer block dots,
 *     parallel over output columns (candle `QTensor::matmul_t`, reached from
 *     `QMatMul::forward`, crates/mold-inference/src/flux2/quantized_transformer.rs:40-45);
 *   - an f64-accumulated dequantize-then-matmul reference (the parity bar).
 *
 * Type ids are ggml's (GGML_TYPE_*), the same ids GGUF files store.
 */
#ifndef MOLD_GGML_ORACLE_H
#define MOLD_GGML_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7,
    ORC_Q8_0 = 8, ORC_Q8_1 = 9, ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12,
    ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_Q8_K = 15, ORC_BF16 = 30
};

/* half <-> float, IEEE binary16, round-to-nearest-even (candle uses half::f16). */
uint16_t orc_fp32_to_fp16(float f);
float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_bf16(float f);  /* RNE, NaN kept quiet */

/* Block geometry: elements per block and bytes per block; 0 for unknown ids. */
int orc_block_size(int type);
int orc_type_size(int type);

/* Dequantize k elements (k multiple of the block size) to f32. */
int orc_dequantize_row(int type, const void *blocks, float *y, int64_t k);
/* ggml reference quantizer for the weight types; returns 0 on success. */
int orc_quantize_row(int type, const float *x, void *blocks, int64_t k);

/* Activation quantizers used by candle's CPU vec_dot. */
void orc_quantize_row_q8_0(const float *x, void *blocks, int64_t k);
void orc_quantize_row_q8_1(const float *x, void *blocks, int64_t k);
void orc_quantize_row_q8_K(const float *x, void *blocks, int64_t k);
/* Which activation type the CPU vec_dot for weight `type` consumes. */
int orc_vec_dot_type(int type);
/* One weight row (k elements) against one quantized activation row. */
float orc_vec_dot(int type, int64_t k, const void *w_blocks, const void *act_blocks);

/* candle CPU QMatMul: y[m,n] = x[m,k] . W[n,k]^T, W rows are GGUF blocks.
 * nthreads <= 0 means one thread per online CPU.  Returns 0 on success. */
int orc_matmul_candle(int type, int64_t m, int64_t n, int64_t k, const float *x,
                      const void *w, float *y, int nthreads);

/* Reference: y[m,n] = sum_k x[m,k] * deq(W)[n,k] with f64 accumulation. */
int orc_matmul_f64(int type, int64_t m, int64_t n, int64_t k, const float *x,
                   const void *w, double *y);

/* LoRA merge of mold's GGUF LoRA path (crates/mold-inference/src/flux/
 * lora.rs:771-833: delta = (B . A) * scale, t = t + delta on a row slice), in
 * the order the device kernel defines: per element d = 0, then
 * d = fmaf(b[i][r], a[r][j], d) for r = 0 .. rank-1, then
 * w[i][j] = w[i][j] + d * scale (a rounded multiply, then a rounded add).
 * w is [rows][ldw], b is [rows][ldb], a is [rank][lda]. */
void orc_lora_apply(float *w, int64_t ldw, int64_t rows, int64_t k, const float *b, int64_t ldb,
                    const float *a, int64_t lda, int rank, float scale);

#ifdef __cplusplus
}
#endif
#endif
