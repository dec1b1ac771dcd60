// mq_kernels.h — launchers shared between the kernel files and the C ABI.
#pragma once

#include "../../include/moldq.h"
#include "mq_common.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

namespace mq {

hipError_t launch_repack(int type, const void *src, void *dst, const Geo &g, bool inverse,
                         hipStream_t stream);
// f32 [n, k] (row stride ld) -> raw GGUF blocks (n rows of k/bs blocks).
hipError_t launch_quantize(int type, const float *src, int64_t ld, int64_t n, int64_t k, void *dst_raw,
                           hipStream_t stream);
// Same from FP8 E4M3 bytes src[n, ld] (decoded exactly, times scale).
hipError_t launch_quantize_fp8(int type, const uint8_t *src, int64_t ld, int64_t n, int64_t k, float scale,
                               void *dst_raw, hipStream_t stream);
// The 32-element block types (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0) quantized straight
// into a tensor's device layout (geometry g), f32 or FP8 E4M3 source.
bool quantize_tiled_ok(int type);
hipError_t launch_quantize_tiled(int type, const void *src, bool fp8, int64_t ld, float scale, void *tiled,
                                 const Geo &g, hipStream_t stream);
hipError_t launch_dequant(int type, const WView &w, int64_t n, int64_t k, void *dst, int dst_type,
                          hipStream_t stream);
// Dense GGUF tensors (F32 / F16 / BF16): src[n, lds] of src_type -> dst[n,
// ldd] of dst_type, element by element: widening is exact, narrowing rounds
// to nearest even (NaN stays NaN).  Same type: a plain copy is cheaper.
hipError_t launch_convert(const void *src, int src_type, int64_t lds, int64_t n, int64_t k, void *dst,
                          int dst_type, int64_t ldd, hipStream_t stream);
// bf16 [m, k] (row stride ldx) -> f32 [m, k] contiguous, for the GEMV.
hipError_t launch_widen_bf16(const __bf16 *x, int64_t m, int64_t k, int64_t ldx, float *out,
                             hipStream_t stream);
hipError_t launch_stage_bf16(const void *x, int x_type, int64_t m, int64_t k, int64_t ldx, __bf16 *out,
                             int64_t kp, hipStream_t stream);

// Skinny-M GEMV (m <= kGemvMaxM).  Q4_K weights (the modulation linears)
// take a kernel that reads f32 or bf16 x with 16-byte aligned rows in place
// and needs no scratch (gemv_reads_x_in_place); everything else reads f32 x
// (contiguous f32 x of the Q4_K shapes also takes the Q4_K kernel) and the
// generic kernel, when it splits K across workgroups, uses `partial` scratch
// of gemv_scratch_bytes.
constexpr int kGemvMaxM = 8;
bool gemv_reads_x_in_place(int type, int64_t m, int64_t n, int64_t k, const void *x, int x_type, int64_t ldx,
                           int cus);
size_t gemv_scratch_bytes(int type, int64_t m, int64_t n, int64_t k, int cus);
// x pre-quantized for the Q4_K GEMV (MQ_X_Q8K): per row, k / 256 blocks of
// kQ8kXBytes (256 int8 quants, 8 int32 sums of 32 quants, f32 d, 12 zero bytes).
constexpr int kQ8kXBytes = MQ_X_Q8K_BLOCK_BYTES;
struct Q8kX {
  uint8_t b[kQ8kXBytes];
};
// x [m, k] (f32 or bf16, row stride ldx) -> m * k / 256 blocks at dst, by the
// same Q8_K quantization the Q4_K GEMV applies to x when it stages it.
// Whether mq_qmatmul's GEMV takes x in MQ_X_Q8K form for this weight and m.
bool gemv_takes_x_q8k(int type, int64_t m, int64_t n, int64_t k, int cus);
hipError_t launch_quantize_x_q8k(const void *x, int x_type, int64_t m, int64_t k, int64_t ldx, void *dst,
                                 hipStream_t stream);
hipError_t launch_gemv(int type, const WView &w, int64_t n, int64_t k, const void *x, int x_type, int64_t m,
                       int64_t ldx, void *y, int y_type, int64_t ldy, const float *bias, int act,
                       float *partial, int cus, hipStream_t stream);

// Fused dequant -> bf16 MFMA GEMM.  a is bf16 [m, lda] with lda a multiple
// of 64 covering ceil(k/64)*64 zero-padded columns.  With `gate` (f32 [n],
// f32 y only) the output is the gated residual update
// y = y + gate * act(a . W^T + bias); without it y = act(a . W^T + bias).
// The fast kernel (k a whole number of the type's 128- or 256-weight units)
// runs 256 (m) x 128 (n) block tiles, two workgroups per CU.  When the last
// round of tiles over the CUs' slots is partial, those tail tiles may split K
// into `kparts` workgroups that write raw sums to `partial`
// (gemm_tail_bytes of it), added in part order by a second kernel that
// applies the epilogue: the plan comes from gemm_tail_plan; partial == NULL
// runs every tile whole.  Other k take a generic 256 x 256 kernel.
constexpr int kGemmTileM = 256;      // fast kernel block tile (rows of x) for large m
// Output features of a block tile: 32 per wave; 256-row tiles run 8 waves
// (256 x 256, one workgroup per CU), 128- and 64-row tiles 4 (x 128).
inline int gemm_tile_n(int fm) { return fm == 256 ? 256 : 128; }
// Workgroups of the fast kernel resident per CU for a row tile of fm: its
// registers (about 225 / 145 / 110 VGPRs at 256 / 128 / 64 rows) allow 2 / 3
// / 4 waves per SIMD, and the LDS (32 / 16 / 8 KiB per slot, two slots) holds
// them: one 8-wave workgroup, or 3 / 4 of 4 waves.
inline int gemm_wgs_per_cu(int fm) { return fm == 64 ? 4 : fm == 128 ? 3 : 1; }
constexpr int kGemmMaxKParts = 8;
struct GemmTail {
  int full_tiles;  // tiles run whole (all of them when kparts == 1)
  int kparts;      // K parts per tail tile
  int fm;          // rows per block tile: 256, or 128 / 64 for small m
};
// K unit of the fast kernel per weight type (the decoder's unit in mq_bfrag.h).
inline int gemm_unit_k(int type) { return type == Q8_0 ? 128 : 256; }
// Rows per block tile of the fast kernel for a call of m rows.
int gemm_tile_m(int type, int64_t m, int64_t n, int64_t k, int cus);
// The call's tile plan: its fm, and with `split` the K split of a partial last round.
GemmTail gemm_tail_plan(int type, int64_t m, int64_t n, int64_t k, int cus, bool split);
size_t gemm_tail_bytes(const GemmTail &t, int64_t m, int64_t n);
// The fast kernel (and tail splitting) applies: whole K units, 16-byte aligned
// rows, and byte offsets of x that fit the 31-bit buffer range.
inline bool gemm_fast_ok(int type, int64_t m, int64_t k, int64_t lda) {
  return (k % gemm_unit_k(type)) == 0 && lda % 8 == 0 && (m + kGemmTileM) * lda * 2 < (int64_t(1) << 31);
}
hipError_t launch_gemm(int type, const WView &w, int64_t n, int64_t k, int64_t ntiles_w,
                       const __bf16 *a, int64_t m, int64_t lda, void *y, int y_type, int64_t ldy,
                       const float *bias, const float *gate, int act, const GemmTail &tail, float *partial,
                       hipStream_t stream);
// One weight type's launcher (instantiated in its own translation unit).
template <int T>
hipError_t launch_gemm_type(const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a, int64_t m,
                            int64_t lda, void *y, int y_type, int64_t ldy, const float *bias, const float *gate,
                            int act, const GemmTail &tail, float *partial, hipStream_t stream);

// The launchers' `act` argument: bit 0 the activation (MQ_ACT_NONE or
// MQ_ACT_GELU_TANH), bits 1 and up the first output column it applies to (0
// for the whole output; mq_qmatmul_act_from sets it).  act_at gives output
// column col's activation.
inline int act_code(int act, int64_t first_col) { return act | (int)(first_col << 1); }
__host__ __device__ __forceinline__ int act_at(int code, int64_t col) { return col >= (code >> 1) ? (code & 1) : 0; }

// Epilogue activation (GELU with the tanh approximation, as candle's gelu()).
__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == 1) {
    const float c = 0.7978845608028654f;  // sqrt(2/pi)
    return 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
  }
  return v;
}

// The same GELU-tanh for the GEMM's epilogues: 0.5 v (1 + tanh u) =
// v / (1 + e^(-2u)), u = sqrt(2/pi) (v + 0.044715 v^3), written as
// v / (1 + 2^(v (K0 + K1 v^2))) with K0 = -2 sqrt(2/pi) / ln 2 and K1 = 0.044715
// K0 folded, and evaluated with the hardware base-2 exponential and
// reciprocal: five ALU operations and two transcendentals, relative error
// about 1e-6, far below bf16's 2^-8 rounding step and below the bf16-input
// GEMM's own error for f32 outputs (apply_act's tanhf made the f32 GELU
// epilogue 12-19 % of the launch).  Large |v| saturate correctly (2^z -> 0
// gives v, -> inf gives 0).  The GEMVs, exact to 1e-5, keep apply_act.
__device__ __forceinline__ float gelu_fast(float v) {
  constexpr float K0 = -2.302208198144325f, K1 = -0.1029432395800235f;
  const float z = v * __builtin_fmaf(v * v, K1, K0);
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}
template <typename OUT>
__device__ __forceinline__ float act_out(float v, int act) {
  return act == 1 ? gelu_fast(v) : v;
}

}  // namespace mq
