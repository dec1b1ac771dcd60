// mq_lora.hip — the device step of mold's GGUF LoRA path: w[rows, k] +=
// (b[rows, rank] . a[rank, k]) * scale on a dense f32 matrix (the dequantized
// weight, or a row slice of it), between mq_dequantize and mq_quantize.
// Replaces the CPU round trip of gguf_lora_var_builder
// (crates/mold-inference/src/flux/lora.rs:759-850: dequantize to CPU f32,
// delta = b.matmul(a) * effective_scale, t + delta on the target rows,
// QTensor::quantize_onto).
//
// The arithmetic order is part of the contract (so that re-quantized blocks
// are reproducible): per element, d = 0; d = fma(b[i][r], a[r][j], d) for
// r = 0 .. rank-1 in order; w = w + d * scale as a rounded multiply then a
// rounded add (contraction is off in this file).
#include "../../include/moldq.h"
#include "mq_internal.h"
#include "mq_kernels.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr int kLT = 64;   // output tile: 64 rows x 64 columns per workgroup
constexpr int kLR = 32;   // rank chunk staged in LDS

// 256 threads: thread (ty, tx) owns rows 4*ty .. +3 and columns 4*tx .. +3 of
// the tile; b[64][32] and a[32][64] chunks are staged in LDS.
__global__ __launch_bounds__(256) void lora_apply_kernel(float *__restrict__ w, int64_t ldw, int64_t rows, int64_t k,
                                                         const float *__restrict__ b, int64_t ldb,
                                                         const float *__restrict__ a, int64_t lda, int rank,
                                                         float scale) {
  __shared__ float bs[kLT][kLR + 1];
  __shared__ float as[kLR][kLT];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t i0 = (int64_t)blockIdx.y * kLT, j0 = (int64_t)blockIdx.x * kLT;
  float d[4][4] = {};
  for (int r0 = 0; r0 < rank; r0 += kLR) {
    for (int e = tid; e < kLT * kLR; e += 256) {
      const int ii = e / kLR, rr = e - ii * kLR;
      const int64_t gi = i0 + ii;
      bs[ii][rr] = (gi < rows && r0 + rr < rank) ? b[gi * ldb + r0 + rr] : 0.f;
    }
    for (int e = tid; e < kLR * kLT; e += 256) {
      const int rr = e / kLT, jj = e - rr * kLT;
      const int64_t gj = j0 + jj;
      as[rr][jj] = (gj < k && r0 + rr < rank) ? a[(int64_t)(r0 + rr) * lda + gj] : 0.f;
    }
    __syncthreads();
    const int rn = rank - r0 < kLR ? rank - r0 : kLR;  // padded ranks are not accumulated
    for (int rr = 0; rr < rn; ++rr) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float bv = bs[4 * ty + u][rr];
#pragma unroll
        for (int v = 0; v < 4; ++v) d[u][v] = __builtin_fmaf(bv, as[rr][4 * tx + v], d[u][v]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t gi = i0 + 4 * ty + u;
    if (gi >= rows) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t gj = j0 + 4 * tx + v;
      if (gj < k) {
        const float t = d[u][v] * scale;
        w[gi * ldw + gj] = w[gi * ldw + gj] + t;
      }
    }
  }
}

}  // namespace
}  // namespace mq

extern "C" int mq_lora_apply(float *w, int64_t ldw, int64_t rows, int64_t k, const float *b, int64_t ldb,
                             const float *a, int64_t lda, int rank, float scale, void *stream) {
  if (!w || !b || !a) return mq::set_error(MQ_E_INVALID, "mq_lora_apply: NULL pointer");
  if (rows < 0 || k < 0 || rank < 1 || ldw < k || ldb < rank || lda < k)
    return mq::set_error(MQ_E_INVALID, "mq_lora_apply: bad shape or leading dimension");
  if (rows == 0 || k == 0) return MQ_OK;
  if ((rows + 63) / 64 > 65535) return mq::set_error(MQ_E_INVALID, "mq_lora_apply: too many rows");
  const dim3 grid((unsigned)((k + 63) / 64), (unsigned)((rows + 63) / 64));
  hipLaunchKernelGGL(mq::lora_apply_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), w, ldw, rows, k, b,
                     ldb, a, lda, rank, scale);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return mq::set_error(MQ_E_HIP, hipGetErrorString(e));
  return MQ_OK;
}
