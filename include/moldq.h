/*
 * moldq.h — C ABI of the MI355X (gfx950) GGUF quantized-linear library.
 *
 * This is the drop-in boundary for candle's quantized device arm
 * (candle-core-mold 0.9.10, pinned at /root/reference/Cargo.lock:507-535):
 * a Rust `QStorage::Rocm(QRocmStorage)` arm calls these functions the way
 * `QCudaStorage` calls candle's CUDA kernels.  Plain pointers and sizes only.
 *
 * Conventions
 *   - A weight is a GGUF tensor of `n` rows (output features) by `k` columns
 *     (input features, GGUF ne[0]); each row is k/block_size consecutive
 *     blocks.  The layer computes y[m, n] = x[m, k] . W[n, k]^T (+ bias[n]).
 *   - Dense GGUF tensors (MQ_F32 / MQ_F16 / MQ_BF16: biases, norm scales,
 *     embeddings) are mq_qtensors too, as candle's QTensor holds them: n rows
 *     of k elements (a 1-D tensor is n = 1), stored row-major as in the file.
 *     They upload, download, load from GGUF files and dequantize (convert)
 *     like the block types; a quantized matmul refuses them
 *     (MQ_E_UNSUPPORTED), since candle's QMatMul::from_arc dequantizes a
 *     dense weight once and runs a dense matmul instead.
 *   - Return value 0 is success; a negative MQ_E_* code is failure and
 *     mq_last_error() returns a thread-local message.  Nothing aborts or
 *     throws across the ABI.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL is the null stream)
 *     and is asynchronous unless stated otherwise.
 *   - A context is bound to one device; call it from one thread at a time.
 *     Scratch memory (activation staging, split-K partial sums) is kept per
 *     stream, so quantized matmuls on different streams of one context may
 *     run concurrently.  A stream's workspace only grows, and an outgrown
 *     one is released with the context, so no mq_qmatmul call synchronizes
 *     or frees device memory; it allocates only when its stream's workspace
 *     is too small (mq_ctx_reserve_stream_scratch pre-sizes it).
 */
#ifndef MOLDQ_H
#define MOLDQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOLDQ_VERSION 1

/* ggml / GGUF tensor type ids (candle `GgmlDType`). */
typedef enum mq_dtype {
    MQ_F32 = 0, MQ_F16 = 1, MQ_Q4_0 = 2, MQ_Q4_1 = 3, MQ_Q5_0 = 6, MQ_Q5_1 = 7,
    MQ_Q8_0 = 8, MQ_Q2_K = 10, MQ_Q3_K = 11, MQ_Q4_K = 12, MQ_Q5_K = 13,
    MQ_Q6_K = 14, MQ_BF16 = 30
} mq_dtype;

enum {
    MQ_OK = 0,
    MQ_E_INVALID = -1,      /* bad argument: dtype, shape, k % block, null pointer */
    MQ_E_HIP = -2,          /* HIP runtime error */
    MQ_E_OOM = -3,          /* device or host allocation failed */
    MQ_E_UNSUPPORTED = -4,  /* valid request this build does not implement */
    MQ_E_IO = -5            /* file read / format error (GGUF) */
};

/* Activation format of mq_quantize_x_q8k (not a GGUF type): per row of x,
 * k / 256 blocks of 304 bytes: 256 int8 quants, 8 int32 sums of 32 quants,
 * the f32 scale d, 12 zero bytes; rows contiguous. */
#define MQ_X_Q8K 100
#define MQ_X_Q8K_BLOCK_BYTES 304

/* Epilogue applied to x.W^T + bias before the store. */
typedef enum mq_act { MQ_ACT_NONE = 0, MQ_ACT_GELU_TANH = 1 } mq_act;

typedef struct mq_ctx mq_ctx;
typedef struct mq_qtensor mq_qtensor;
typedef struct mq_gguf mq_gguf;

/* Thread-local description of the last failure on this thread. */
const char *mq_last_error(void);
int mq_version(void);

/* GgmlDType::block_size() / type_size(): elements and bytes per block.
 * Replaces candle's GgmlDType methods used at
 * crates/mold-inference/src/flux/pipeline.rs:198.  Return 0 for unknown ids. */
int mq_block_size(int dtype);
int mq_type_size(int dtype);

/* Device context (candle Device::new_cuda(ordinal), device.rs:165). */
int mq_ctx_create(int device_ordinal, mq_ctx **out);
void mq_ctx_destroy(mq_ctx *ctx);
/* Pre-allocate one HBM arena that later uploads are carved from (bump
 * allocation, released with the context).  Optional. */
int mq_ctx_reserve_arena(mq_ctx *ctx, size_t bytes);
/* Minimum size of every stream workspace (activation staging and split-K
 * partials): grows the workspaces of the streams seen so far and of the null
 * stream to `bytes` now, and later streams' on their first call.  Optional. */
int mq_ctx_reserve_scratch(mq_ctx *ctx, size_t bytes);
/* Grow the workspace of one stream (a hipStream_t) to at least `bytes` now,
 * e.g. before capturing that stream into a HIP graph: a call that would
 * have to grow the workspace of a stream under capture fails with
 * MQ_E_INVALID instead.  Optional. */
int mq_ctx_reserve_stream_scratch(mq_ctx *ctx, void *stream, size_t bytes);
/* Whether GEMMs on `stream` may split K when their last round of tiles over
 * the CUs is partial (default: enabled, for every stream).  The split fills
 * the CUs a lone GEMM's partial round leaves idle, at the cost of f32 partial
 * sums and a reduce launch; on a stream whose GEMMs run beside another
 * stream's (mold's DiT blocks: the text-token linears beside the image-token
 * ones), those CUs are not idle and the split only adds traffic, so such a
 * stream turns it off.  No counterpart in candle, whose device runs one
 * stream; its callers are multi-stream callers such as the DiT block
 * drivers. */
int mq_ctx_set_stream_tail_split(mq_ctx *ctx, void *stream, int enabled);
/* Workspace bytes a quantized matmul of `m` rows against w needs (gated != 0
 * for mq_qmatmul_gated_add), the maximum over every x placement and stride:
 * the size to reserve before capturing such calls into a graph.  No
 * counterpart in candle, whose CUDA matmuls allocate per call. */
int mq_qmatmul_workspace_size(mq_ctx *ctx, const mq_qtensor *w, int x_dtype, int64_t m, int gated,
                              size_t *bytes);

/* Upload a GGUF tensor (blocks, or dense elements, exactly as stored in the
 * file) to the device.
 * Replaces QCudaStorage load_quantized / `content.tensor(reader, name, device)`
 * (crates/mold-inference/src/flux/lora.rs:722) and VarBuilder::from_gguf
 * (crates/mold-inference/src/flux/pipeline.rs:976).  Synchronous: the host
 * buffer may be reused on return.  nbytes must equal n*k/bs*type_size.
 * The raw blocks pass through a context-owned device staging buffer that
 * grows to the largest tensor uploaded and is kept. */
int mq_qtensor_upload(mq_ctx *ctx, int dtype, int64_t n, int64_t k,
                      const void *host_blocks, size_t nbytes, mq_qtensor **out);
/* Same from GGUF blocks already in device memory (copied; caller keeps its
 * buffer).  Ordered on `stream`. */
int mq_qtensor_from_device(mq_ctx *ctx, int dtype, int64_t n, int64_t k,
                           const void *dev_blocks, size_t nbytes, void *stream,
                           mq_qtensor **out);
/* Quantize a dense f32 matrix already on the device, src[n, k] with row
 * stride ld (elements), into a new device-resident GGUF weight of `dtype`.
 * The blocks are byte-identical to ggml's reference quantizers
 * (quantize_row_*_ref).  Byte parity with candle's own k-quant quantizers
 * (Q2_K..Q6_K) is unpinned: candle may use make_qkx1_quants where ggml's
 * reference uses make_qkx2_quants.  Replaces
 * QTensor::quantize / quantize_onto (crates/mold-inference/src/flux/
 * pipeline.rs:219-229, crates/mold-inference/src/flux/lora.rs:849).
 * Runs on `stream` after work already queued there and returns when the
 * blocks are in place (through the context's upload staging buffer).
 * dtype F32 / F16 / BF16 stores the values themselves (rounded to nearest
 * even when narrowing): QTensor::quantize(.., F32), which mold uses for the
 * tensors a block type cannot hold (flux/pipeline.rs:223-228). */
int mq_quantize(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const float *src, int64_t ld,
                void *stream, mq_qtensor **out);
/* Same from FP8 E4M3 weights already on the device: src[n, ld] bytes in the
 * OCP "E4M3FN" encoding (safetensors F8_E4M3, torch.float8_e4m3fn), each
 * decoded exactly to f32 and multiplied by `scale` (1 for mold's cache)
 * before quantization.  The device side of mold's FP8 checkpoint -> Q8_0
 * GGUF cache (ensure_fp8_gguf_cache, crates/mold-inference/src/flux/
 * pipeline.rs:120-252, which loads the FP8 tensor and calls
 * QTensor::quantize(.., Q8_0) at :212-216).  Synchronous like mq_quantize. */
int mq_quantize_fp8(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *src, int64_t ld,
                    float scale, void *stream, mq_qtensor **out);  /* block types only */
/* Read the weight back as GGUF blocks (byte-identical to what was uploaded).
 * Synchronous. */
int mq_qtensor_download(mq_ctx *ctx, const mq_qtensor *w, void *host_blocks, size_t nbytes);
/* Stack `count` tensors of one type and k by rows into a new tensor: row r of
 * parts[i] becomes row n_0 + .. + n_(i-1) + r.  No candle counterpart: the
 * stacked adaLN modulation weight of a DiT step (every block's modulation
 * linear reads the same conditioning vector, crates/mold-inference/src/flux/
 * offload.rs:143-156, qwen_image/quantized_transformer.rs:869-881), built on
 * the device without a host round trip.  The parts stay valid.  Synchronous. */
int mq_qtensor_concat_rows(mq_ctx *ctx, const mq_qtensor *const *parts, int64_t count, mq_qtensor **out);
void mq_qtensor_free(mq_qtensor *w);
/* QTensor::dtype() / shape / storage_size_in_bytes(). */
int mq_qtensor_info(const mq_qtensor *w, int *dtype, int64_t *n, int64_t *k,
                    size_t *gguf_bytes, size_t *device_bytes);

/* QTensor::dequantize(&device) -> dense [n, k] in dst_dtype (F32, F16 or
 * BF16) at dst (row-major, k contiguous).  F32 output is bit-exact with the
 * GGUF formulas; F16/BF16 are that value rounded to nearest even.  A dense
 * tensor converts: the same type is a copy, widening is exact, narrowing
 * rounds to nearest even (candle's dequantize of F32 / F16 tensors,
 * crates/mold-inference/src/qwen_image/quantized_transformer.rs:83-86,
 * crates/mold-inference/src/flux2/quantized_transformer.rs:49-54).
 * Replaces candle's dequantize / dequantize_f16 (called at
 * crates/mold-inference/src/qwen_image/quantized_transformer.rs:62-66). */
int mq_dequantize(mq_ctx *ctx, const mq_qtensor *w, void *dst, int dst_dtype, void *stream);

/* QMatMul::forward (+ quantized_nn::Linear bias, optional GELU-tanh):
 * y[m, :n] = act(x[m, :k] . W^T + bias).  x_dtype F32 or BF16 with row
 * stride ldx (elements); y_dtype F32 or BF16 with row stride ldy.  bias is
 * f32 [n] or NULL.  Picks the skinny GEMV for small m and the fused
 * dequant-MFMA GEMM otherwise.  Replaces QCudaStorage::fwd, reached from
 * crates/mold-inference/src/flux2/quantized_transformer.rs:40-45 and the FLUX
 * quantized model's linears.  For a Q4_K weight at m <= 8, x may also be
 * given as mq_quantize_x_q8k's blocks (x_dtype MQ_X_Q8K, ldx = k, 16-byte
 * aligned): the same result bit for bit as the F32 / BF16 x they came from,
 * without re-quantizing x in every call (MQ_E_UNSUPPORTED for other weights
 * or m, and for the gated call). */
int mq_qmatmul(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype,
               int64_t m, int64_t ldx, void *y, int y_dtype, int64_t ldy,
               const float *bias, int act, void *stream);

/* mq_qmatmul with the activation applied to output columns act_col0 .. n-1
 * only (0 <= act_col0 <= n; 0 is mq_qmatmul, n applies none): columns before
 * act_col0 are x . W^T + bias as computed by mq_qmatmul without act, columns
 * from act_col0 on as computed with it, bit for bit.  No counterpart in
 * candle: for the FLUX single block, whose linear1 output is split into the
 * attention's q, k, v and the MLP half that goes through gelu() before
 * linear2 (crates/mold-inference/src/flux/offload.rs:380-394); with the GELU
 * in linear1's epilogue the MLP half is linear2's input as it stands. */
int mq_qmatmul_act_from(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx, void *y,
                        int y_dtype, int64_t ldy, const float *bias, int act, int64_t act_col0, void *stream);

/* mq_qmatmul that allocates nothing, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments,
 * kernels and results as mq_qmatmul; its scratch (activation staging and
 * split-K partials) is one fixed 64 MiB device array per GPU, held until the
 * process ends.  A call whose scratch would exceed it fails with
 * MQ_E_INVALID (mq_qmatmul_workspace_size gives the need; bf16 x with 16-byte
 * aligned rows needs only the partials).  Every call on one GPU shares that
 * array: calls that overlap in time on one GPU (other streams, other
 * contexts, other threads) race and must be ordered by the caller. */
int mq_qmatmul_noalloc(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype,
                       int64_t m, int64_t ldx, void *y, int y_dtype, int64_t ldy,
                       const float *bias, int act, void *stream);

/* --- Block glue between the quantized linears (fused row passes).  Both are
 *     asynchronous on `stream` and allocate nothing. -------------------------- */

/* out[r, :cols] = bf16(LayerNorm_eps(x[r, :cols]) * (1 + scale) + shift), the
 * LayerNorm without affine weights; shift and scale are f32 [cols].  cols a
 * multiple of 4, at most 8192; x 16-byte aligned, ldx and ldo multiples of 4.
 * Replaces the modulate sequence of candle ops at
 * crates/mold-inference/src/flux/offload.rs:283-286 (norm :75-78) and
 * crates/mold-inference/src/qwen_image/quantized_transformer.rs:913-922. */
int mq_adaln_modulate(const float *x, int64_t rows, int64_t cols, int64_t ldx, const float *shift,
                      const float *scale, float eps, void *out, int64_t ldo, void *stream);

/* dst[r, :cols] = bf16(gelu_tanh(src[r, :cols])) (the tanh approximation in
 * f32, rounded once); src F32 (16-byte aligned) or BF16 (8-byte aligned), dst
 * bf16 8-byte aligned, cols and both row strides (elements) multiples of 4.
 * Replaces the single block's `mlp.gelu()` and the concatenation copy at
 * crates/mold-inference/src/flux/offload.rs:390, 394. */
int mq_gelu_tanh_bf16(const void *src, int src_dtype, int64_t rows, int64_t cols, int64_t lds, void *dst,
                      int64_t ldd, void *stream);

/* For each of `rows` tokens and `heads` heads of the projection output
 * qkv[r, 0:3*heads*128] (qkv_dtype F32 or BF16, row stride ld; q, k, v blocks
 * of heads*128), computed in f32: RmsNorm
 * of q and k (eps, bf16 weights [128]), RoPE rotating pair (2i, 2i+1) by the
 * angle whose cos / sin are cos_table / sin_table[r, i] (f32 [rows, 64]), and
 * q, k, v written as bf16 [heads, l_total, 128] at rows row_off .. row_off +
 * rows - 1.  head_dim must be 128.  Replaces QkNorm + apply_rope + the head
 * split at crates/mold-inference/src/flux/offload.rs:188-201, 56-66 and
 * crates/mold-inference/src/qwen_image/quantized_transformer.rs:739-757. */
int mq_qk_norm_rope(const void *qkv, int qkv_dtype, int64_t ld, int64_t rows, int heads, int head_dim,
                    const void *q_weight, const void *k_weight, float eps, const float *cos_table,
                    const float *sin_table, void *q_out, void *k_out, void *v_out, int64_t row_off, int64_t l_total,
                    void *stream);

/* Correction of an attention computed over zero-padded keys.  o is the bf16
 * attention output [batch, heads, >= rows, 128] (element strides
 * o_batch_stride / o_head_stride / o_row_stride, unit stride along the head
 * dim), lse its f32 log-sum-exp [batch, heads, >= rows] (unit stride along
 * rows), npad f32 [batch] the zero keys (padding plus masked keys, whose k and
 * v rows are zero) each element's rows saw.  For every row r < rows and head h:
 * share = npad[b] * exp(-lse), out[b, r, h * 128 + j] = bf16(o[b, h, r, j] /
 * (1 - share)) (f32, each step correctly rounded, round to nearest even),
 * out bf16 with row stride ldo >= heads * 128; and *guard (f32, >= 0) is
 * raised to the largest share (the caller recomputes rows whose share is near
 * 1, where the division loses precision).  o / out strides multiples of 8,
 * o / out 16-byte aligned.  No counterpart in the reference, whose attention
 * runs over the real keys only: for the DiT step drivers, which pad the joint
 * sequence to a length the fused attention kernels run fastest at.
 * Asynchronous on stream. */
int mq_attn_pad_correct(const void *o, int64_t batch, int heads, int64_t rows, int64_t o_batch_stride,
                        int64_t o_head_stride, int64_t o_row_stride, const float *lse, int64_t lse_batch_stride,
                        int64_t lse_head_stride, const float *npad, void *out, int64_t out_batch_stride, int64_t ldo,
                        float *guard, void *stream);

/* Quantize activations once for several Q4_K GEMVs: x [m, k] (F32 or BF16,
 * row stride ldx, 16-byte aligned rows) -> m * k / 256 blocks of
 * MQ_X_Q8K_BLOCK_BYTES at dst (16-byte aligned), by the Q8_K quantization
 * mq_qmatmul's Q4_K GEMV applies to x (candle's BlockQ8K::from_float
 * convention: iscale = -128 / the first value of largest magnitude, round
 * half away from zero, clamp at 127).  No candle counterpart: candle's CUDA
 * path re-quantizes x (to Q8_1) in every QMatMul::forward; mold's
 * modulation linears of one step all read the same silu(vec)
 * (crates/mold-inference/src/flux/offload.rs:143-156).  Asynchronous on
 * stream. */
int mq_quantize_x_q8k(mq_ctx *ctx, const void *x, int x_dtype, int64_t m, int64_t k, int64_t ldx, void *dst,
                      void *stream);

/* The DiT blocks' gated residual update through one quantized linear:
 * y[m, :n] += gate[:n] * (x[m, :k] . W^T + bias), y f32 (row stride ldy),
 * updated in place; gate f32 [n]; bias f32 [n] or NULL; x F32 or BF16.  Fuses
 * `x + gate * linear(h)` of crates/mold-inference/src/flux/offload.rs:301-305,
 * 314-321, 389-391 and crates/mold-inference/src/qwen_image/
 * quantized_transformer.rs:937-938, 954-958 into the GEMM's epilogue (every m
 * takes the GEMM kernel). */
int mq_qmatmul_gated_add(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx,
                         float *y, int64_t ldy, const float *bias, const float *gate, void *stream);

/* --- GGUF v2/v3 reader (candle gguf_file::Content::read, used at
 *     crates/mold-inference/src/flux/pipeline.rs:286-287). ------------------- */
int mq_gguf_open(const char *path, mq_gguf **out);
void mq_gguf_close(mq_gguf *g);
int64_t mq_gguf_tensor_count(const mq_gguf *g);
/* Index of a tensor by name, or -1. */
int64_t mq_gguf_find(const mq_gguf *g, const char *name);
/* dims[0] is GGUF ne[0] (the contiguous axis). *name stays valid until close. */
int mq_gguf_tensor_info(const mq_gguf *g, int64_t index, const char **name, int *dtype,
                        int *n_dims, int64_t dims[4], uint64_t *file_offset, size_t *nbytes);
/* Read a tensor from the file and upload it (content.tensor(reader, name,
 * device), crates/mold-inference/src/flux/lora.rs:721-723): rows = the
 * product of ne[1..], k = ne[0]; block types and dense F32 / F16 / BF16.
 * Several host threads read the file in chunks into pinned buffers of their
 * own, each chunk copied to the device asynchronously while the thread reads
 * its next one; block types are then repacked on the device.  Synchronous. */
int mq_gguf_load_tensor(mq_ctx *ctx, const mq_gguf *g, int64_t index, mq_qtensor **out);
/* Upload `count` tensors of the file (indices into its tensor table, any
 * order) into out[0..count): what candle's quantized VarBuilder::from_gguf
 * (path, device) does for a whole model (crates/mold-inference/src/flux/
 * pipeline.rs:976, qwen_image/pipeline.rs:936), each tensor as
 * mq_gguf_load_tensor makes it.  One tensor's repack overlaps the next one's
 * file read and copy (two device staging buffers of the largest tensor's
 * size).  Synchronous; on failure every out[i] is NULL and nothing stays
 * allocated. */
int mq_gguf_load_tensors(mq_ctx *ctx, const mq_gguf *g, const int64_t *indices, int64_t count,
                         mq_qtensor **out);
/* The tensor's raw bytes as stored (any type, dense F32/F16/BF16 included)
 * into host memory; nbytes must equal the tensor's size.  What mold reads
 * with content.tensor(&mut file, name, &Device::Cpu) when it copies tensors
 * between GGUF files (flux/pipeline.rs:507-530). */
int mq_gguf_read_tensor(const mq_gguf *g, int64_t index, void *dst, size_t nbytes);
int mq_gguf_version(const mq_gguf *g);

/* LoRA merge step on a dense f32 matrix on the device (the dequantized
 * weight or a row slice of it): w[rows, k] += (b[rows, rank] . a[rank, k]) *
 * scale, in place.  Order per element: d = 0; d = fma(b[i][r], a[r][j], d)
 * for r = 0 .. rank-1; w = w + d * scale (rounded multiply, rounded add).
 * Between mq_dequantize and mq_quantize it replaces the CPU round trip of
 * mold's gguf_lora_var_builder (crates/mold-inference/src/flux/lora.rs:
 * 759-850: dequantize to CPU f32, b.matmul(a) * effective_scale, add on the
 * target rows, QTensor::quantize_onto).  Leading dimensions in elements.
 * Asynchronous on `stream`; allocates nothing. */
int mq_lora_apply(float *w, int64_t ldw, int64_t rows, int64_t k, const float *b, int64_t ldb,
                  const float *a, int64_t lda, int rank, float scale, void *stream);

/* --- GGUF metadata (candle gguf_file::Content::metadata).  Value types are
 *     GGUF's: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
 *     8 string, 9 array, 10 u64, 11 i64, 12 f64.  An array reports type 9,
 *     its element type and its length; elements are read by index (arrays
 *     of arrays report their length only).  Strings are not NUL-free:
 *     use the returned length. ------------------------------------------- */
int64_t mq_gguf_kv_count(const mq_gguf *g);
int64_t mq_gguf_find_kv(const mq_gguf *g, const char *key);  /* -1 if absent */
int mq_gguf_kv_info(const mq_gguf *g, int64_t index, const char **key, int *type, int *elem_type,
                    uint64_t *count);
/* Integer or bool element `elem` (0 for a scalar). */
int mq_gguf_kv_int(const mq_gguf *g, int64_t index, uint64_t elem, int64_t *out);
/* f32 or f64 element. */
int mq_gguf_kv_float(const mq_gguf *g, int64_t index, uint64_t elem, double *out);
int mq_gguf_kv_str(const mq_gguf *g, int64_t index, uint64_t elem, const char **s, uint64_t *len);

/* --- GGUF writer (candle gguf_file::write, used by mold for its FP8 -> Q8_0
 *     cache at flux/pipeline.rs:240 and the embedding-patched cache at
 *     :541).  Writes version 3, metadata in the order added, tensors in the
 *     order added at offsets aligned to `alignment` (0 = 32; another value is
 *     recorded as general.alignment).  finish() writes <path>.tmp.<pid> and
 *     renames it over <path>, so a failed write leaves no partial file.
 *     Device tensors added with add_qtensor are read back (as their GGUF
 *     blocks) during finish and must stay alive until then. ------------- */
typedef struct mq_gguf_writer mq_gguf_writer;
int mq_gguf_writer_create(const char *path, uint32_t alignment, mq_gguf_writer **out);
void mq_gguf_writer_free(mq_gguf_writer *w);
int mq_gguf_writer_kv_scalar(mq_gguf_writer *w, const char *key, int type, const void *value);
int mq_gguf_writer_kv_str(mq_gguf_writer *w, const char *key, const char *value);
int mq_gguf_writer_kv_array(mq_gguf_writer *w, const char *key, int elem_type, const void *values,
                            uint64_t count);
int mq_gguf_writer_kv_str_array(mq_gguf_writer *w, const char *key, const char *const *values,
                                uint64_t count);
/* Raw tensor bytes from host memory (copied); dims in GGUF order (ne[0] is
 * the contiguous dimension). */
int mq_gguf_writer_add_tensor(mq_gguf_writer *w, const char *name, int dtype, int n_dims,
                              const int64_t *dims, const void *data, size_t nbytes);
/* A device-resident weight; n_dims = 0 writes it as [n, k] (ne = {k, n}),
 * otherwise dims (ne[0] = k, same element count) give its stored shape. */
int mq_gguf_writer_add_qtensor(mq_gguf_writer *w, mq_ctx *ctx, const char *name, const mq_qtensor *qt,
                               int n_dims, const int64_t *dims);
int mq_gguf_writer_finish(mq_gguf_writer *w);

#ifdef __cplusplus
}
#endif
#endif /* MOLDQ_H */
