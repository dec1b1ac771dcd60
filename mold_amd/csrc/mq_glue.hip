// mq_glue.hip — the row-wise passes that sit between the quantized
// linears of a DiT block, each fused into one HBM pass:
//
//   * mq_adaln_modulate: LayerNorm without affine (eps) of each row, times
//     (1 + scale) plus shift, rounded once to bf16: the input of every
//     attention / MLP linear (FLUX crates/mold-inference/src/flux/
//     offload.rs:75-78 and :283-286, :374-377; Qwen-Image qwen_image/
//     quantized_transformer.rs:913-922, :942-951).
//   * mq_gelu_tanh_bf16: GELU-tanh of an f32 block into a bf16 block (FLUX
//     single block's MLP half, offload.rs:390, 394, written straight into the
//     concatenated linear2 input).
//   * mq_qk_norm_rope: per token and head, RmsNorm (eps, bf16 weight) of q and
//     k, RoPE on interleaved pairs, and the head split of q, k and v into bf16
//     [heads, L, 128] at a row offset of a joint sequence: what the qkv
//     projection output goes through before attention (FLUX offload.rs:
//     188-201 and :56-66; Qwen-Image quantized_transformer.rs:739-751).
//   * mq_attn_pad_correct: the output of an attention run over zero-padded
//     keys, rescaled per (row, head) to the softmax over the real keys from
//     the log-sum-exp the attention kernel returns, and written in the
//     [rows, heads * 128] layout the out-projection reads.
//
// All are HBM-bound (f32 or bf16 in, bf16 out, a few flops per byte).
#include "../../include/moldq.h"
#include "mq_kernels.h"

namespace mq {
int set_error(int code, const char *msg);
}

using namespace mq;

namespace {

constexpr int kHead = 128;  // head dim: one wave holds a head as 64 (even, odd) pairs

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const __bf16 x = (__bf16)a, y = (__bf16)b;
  uint16_t ux, uy;
  __builtin_memcpy(&ux, &x, 2);
  __builtin_memcpy(&uy, &y, 2);
  return (uint32_t)ux | ((uint32_t)uy << 16);
}

// One wave per (token, head); lane i owns the pair (2i, 2i+1), which is also
// RoPE's rotation pair i.  Four waves per workgroup.
__device__ __forceinline__ float2 load2(const float *p) { return *reinterpret_cast<const float2 *>(p); }
__device__ __forceinline__ float2 load2(const __bf16 *p) {
  uint32_t u = *reinterpret_cast<const uint32_t *>(p);
  return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xFFFF0000u));
}
__device__ __forceinline__ float4 load4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 load4(const __bf16 *p) {
  const uint2 u = *reinterpret_cast<const uint2 *>(p);
  return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u), __uint_as_float(u.y << 16),
                     __uint_as_float(u.y & 0xFFFF0000u));
}

template <typename IN>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const IN *__restrict__ qkv, int64_t ld, int64_t rows, int heads, const __bf16 *__restrict__ qw,
    const __bf16 *__restrict__ kw, float eps, const float *__restrict__ cosv, const float *__restrict__ sinv,
    uint32_t *__restrict__ qo, uint32_t *__restrict__ ko, uint32_t *__restrict__ vo, int64_t row_off,
    int64_t l_total) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= rows * heads) return;  // whole waves
  const int64_t l = item / heads;
  const int h = (int)(item - l * heads);
  const IN *src = qkv + l * ld + (int64_t)h * kHead + 2 * lane;
  const float2 q = load2(src);
  const float2 k = load2(src + (int64_t)heads * kHead);
  const float2 v = load2(src + 2 * (int64_t)heads * kHead);
  const float c = cosv[l * (kHead / 2) + lane], s = sinv[l * (kHead / 2) + lane];
  const float rq = rsqrtf(wave_sum(q.x * q.x + q.y * q.y) / kHead + eps);
  const float rk = rsqrtf(wave_sum(k.x * k.x + k.y * k.y) / kHead + eps);
  const float q0 = q.x * rq * (float)qw[2 * lane], q1 = q.y * rq * (float)qw[2 * lane + 1];
  const float k0 = k.x * rk * (float)kw[2 * lane], k1 = k.y * rk * (float)kw[2 * lane + 1];
  const int64_t o = ((int64_t)h * l_total + row_off + l) * (kHead / 2) + lane;
  qo[o] = pack_bf16x2(c * q0 - s * q1, s * q0 + c * q1);
  ko[o] = pack_bf16x2(c * k0 - s * k1, s * k0 + c * k1);
  vo[o] = pack_bf16x2(v.x, v.y);
}

// One workgroup of 256 threads per row; thread t owns float4 columns
// t, t + 256, ... (at most kMaxVec of them).
constexpr int kMaxVec = 8;  // cols <= 8192

__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is reused between the two reductions
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void adaln_modulate_kernel(const float *__restrict__ x, int64_t ldx,
                                                             int64_t cols, const float *__restrict__ shift,
                                                             const float *__restrict__ scale, float eps,
                                                             uint2 *__restrict__ out, int64_t ldo) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int nv = (int)(cols / 4);
  const float4 *xr = reinterpret_cast<const float4 *>(x + row * ldx);
  float4 v[kMaxVec];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int c = threadIdx.x + 256 * j;
    v[j] = c < nv ? xr[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  const float mean = block_sum(s, red) / (float)cols;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    if (threadIdx.x + 256 * j < nv) {
      const float a = v[j].x - mean, b = v[j].y - mean, c = v[j].z - mean, d = v[j].w - mean;
      q += (a * a + b * b) + (c * c + d * d);
    }
  }
  const float rstd = rsqrtf(block_sum(q, red) / (float)cols + eps);
  uint2 *orow = out + row * (ldo / 4);
#pragma unroll
  for (int j = 0; j < kMaxVec; ++j) {
    const int c = threadIdx.x + 256 * j;
    if (c < nv) {
      const float4 sc = reinterpret_cast<const float4 *>(scale)[c];
      const float4 sh = reinterpret_cast<const float4 *>(shift)[c];
      const float a = (v[j].x - mean) * rstd * (1.f + sc.x) + sh.x;
      const float b = (v[j].y - mean) * rstd * (1.f + sc.y) + sh.y;
      const float e = (v[j].z - mean) * rstd * (1.f + sc.z) + sh.z;
      const float f = (v[j].w - mean) * rstd * (1.f + sc.w) + sh.w;
      orow[c] = make_uint2(pack_bf16x2(a, b), pack_bf16x2(e, f));
    }
  }
}

// dst[r, c] = bf16(gelu_tanh(src[r, c])), four columns per thread (16-byte
// loads, 8-byte stores), rows strided by gridDim.y.
template <typename IN>
__global__ __launch_bounds__(256) void gelu_bf16_kernel(const IN *__restrict__ src, int64_t rows, int64_t cols4,
                                                        int64_t lds, uint2 *__restrict__ dst, int64_t ldd4) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols4) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float4 v = load4(src + r * lds + 4 * c);
    dst[r * ldd4 + c] = make_uint2(pack_bf16x2(act_out<__bf16>(v.x, 1), act_out<__bf16>(v.y, 1)),
                                   pack_bf16x2(act_out<__bf16>(v.z, 1), act_out<__bf16>(v.w, 1)));
  }
}

// Zero-padded attention: the n zero keys a row of batch element b saw add
// exp(0) = 1 each to its softmax denominator and nothing to the numerator, so
// the output over the real keys is o / s with s = 1 - n exp(-lse), lse the
// row's log-sum-exp over all keys.  Thread t takes the 8 bf16 (16 bytes) of
// chunk c = t % 16 of head h of row r of element b (t = ((b * rows + r) *
// heads + h) * 16 + c, grid-stride): its loads and stores are whole 256-byte
// head rows.  Arithmetic in f32 in the order share = n * exp(-lse), inv =
// 1 / (1 - share), bf16(o * inv) (round to nearest even), each step one
// correctly rounded f32 operation.  guard (f32 bits, never negative) is
// raised to the largest share seen: a block's maximum, one atomic max on the
// bits per block whose maximum exceeds the value it read (a NaN share sticks,
// as a NaN would through a max that propagates it).
__global__ __launch_bounds__(256) void attn_pad_correct_kernel(
    const __bf16 *__restrict__ o, int64_t sob, int64_t soh, int64_t sor, const float *__restrict__ lse, int64_t slb,
    int64_t slh, const float *__restrict__ npad, int heads, int64_t rows, int64_t items, __bf16 *__restrict__ out,
    int64_t sb_out, int64_t ldo, unsigned int *__restrict__ guard) {
#pragma clang fp contract(off)  // share, 1 - share and the product each rounded, as written
  __shared__ float red[4];
  float smax = 0.f;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < items; t += (int64_t)gridDim.x * 256) {
    const int c = (int)(t & 15);
    const uint32_t rh = (uint32_t)(t >> 4);  // (b * rows + r) * heads + h < 2^31 (checked by the host)
    const uint32_t br = rh / (uint32_t)heads;
    const int h = (int)(rh - br * (uint32_t)heads);
    const uint32_t b = br / (uint32_t)rows, r = br - b * (uint32_t)rows;
    const float share = npad[b] * expf(-lse[(int64_t)b * slb + h * slh + r]);
    const float inv = 1.0f / (1.0f - share);
    smax = (share > smax || share != share) ? share : smax;
    const uint4 v = *reinterpret_cast<const uint4 *>(o + (int64_t)b * sob + h * soh + (int64_t)r * sor + 8 * c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      p[i] = pack_bf16x2(__uint_as_float(w[i] << 16) * inv, __uint_as_float(w[i] & 0xFFFF0000u) * inv);
    *reinterpret_cast<uint4 *>(out + (int64_t)b * sb_out + (int64_t)r * ldo + (int64_t)h * kHead + 8 * c) =
        make_uint4(p[0], p[1], p[2], p[3]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float u = __shfl_xor(smax, off);
    smax = (u > smax || u != u) ? u : smax;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = smax;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) m = (red[i] > m || red[i] != red[i]) ? red[i] : m;
    const unsigned int bits = __float_as_uint(m);
    if (bits > __hip_atomic_load(guard, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(guard, bits);
  }
}

int invalid(const char *msg) { return set_error(MQ_E_INVALID, msg); }

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace

extern "C" {

int mq_qk_norm_rope(const void *qkv, int qkv_dtype, int64_t ld, int64_t rows, int heads, int head_dim,
                    const void *q_weight, const void *k_weight, float eps, const float *cos_table,
                    const float *sin_table, void *q_out, void *k_out, void *v_out, int64_t row_off, int64_t l_total,
                    void *stream) {
  if (head_dim != kHead) return invalid("mq_qk_norm_rope: head_dim must be 128");
  if (qkv_dtype != MQ_F32 && qkv_dtype != MQ_BF16) return invalid("mq_qk_norm_rope: qkv dtype must be F32 or BF16");
  if (rows < 0 || heads <= 0 || row_off < 0 || row_off + rows > l_total)
    return invalid("mq_qk_norm_rope: rows, heads or row range out of bounds");
  if (ld < 3 * (int64_t)heads * kHead || ld % 2) return invalid("mq_qk_norm_rope: ld must be even and >= 3*heads*128");
  if (!qkv || !q_weight || !k_weight || !cos_table || !sin_table || !q_out || !k_out || !v_out)
    return invalid("mq_qk_norm_rope: NULL pointer");
  if (!aligned(qkv, qkv_dtype == MQ_F32 ? 8 : 4) || !aligned(q_out, 4) || !aligned(k_out, 4) || !aligned(v_out, 4))
    return invalid("mq_qk_norm_rope: misaligned buffer");
  if (rows == 0) return MQ_OK;
  const int64_t items = rows * heads;
  const dim3 grid((unsigned)((items + 3) / 4));
  const __bf16 *qw = static_cast<const __bf16 *>(q_weight), *kw = static_cast<const __bf16 *>(k_weight);
  uint32_t *qo = static_cast<uint32_t *>(q_out), *ko = static_cast<uint32_t *>(k_out), *vo = static_cast<uint32_t *>(v_out);
  if (qkv_dtype == MQ_F32)
    hipLaunchKernelGGL(qk_norm_rope_kernel<float>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const float *>(qkv), ld, rows, heads, qw, kw, eps, cos_table, sin_table, qo, ko, vo,
                       row_off, l_total);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<__bf16>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const __bf16 *>(qkv), ld, rows, heads, qw, kw, eps, cos_table, sin_table, qo, ko,
                       vo, row_off, l_total);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MQ_OK : set_error(MQ_E_HIP, hipGetErrorString(e));
}

int mq_adaln_modulate(const float *x, int64_t rows, int64_t cols, int64_t ldx, const float *shift,
                      const float *scale, float eps, void *out, int64_t ldo, void *stream) {
  if (rows < 0 || cols <= 0 || cols % 4 || cols > 4 * 256 * kMaxVec)
    return invalid("mq_adaln_modulate: cols must be a positive multiple of 4, at most 8192");
  if (ldx < cols || ldo < cols || ldx % 4 || ldo % 4) return invalid("mq_adaln_modulate: bad row strides");
  if (!x || !shift || !scale || !out) return invalid("mq_adaln_modulate: NULL pointer");
  if (!aligned(x, 16) || !aligned(shift, 16) || !aligned(scale, 16) || !aligned(out, 8))
    return invalid("mq_adaln_modulate: misaligned buffer");
  if (rows == 0) return MQ_OK;
  hipLaunchKernelGGL(adaln_modulate_kernel, dim3((unsigned)rows), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                     ldx, cols, shift, scale, eps, static_cast<uint2 *>(out), ldo);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MQ_OK : set_error(MQ_E_HIP, hipGetErrorString(e));
}

int mq_gelu_tanh_bf16(const void *src, int src_dtype, int64_t rows, int64_t cols, int64_t lds, void *dst,
                      int64_t ldd, void *stream) {
  if (src_dtype != MQ_F32 && src_dtype != MQ_BF16) return invalid("mq_gelu_tanh_bf16: src dtype must be F32 or BF16");
  if (rows < 0 || cols <= 0 || cols % 4 || lds < cols || ldd < cols || lds % 4 || ldd % 4)
    return invalid("mq_gelu_tanh_bf16: cols and row strides must be multiples of 4 with strides >= cols");
  if (!src || !dst) return invalid("mq_gelu_tanh_bf16: NULL pointer");
  if (!aligned(src, src_dtype == MQ_F32 ? 16 : 8) || !aligned(dst, 8))
    return invalid("mq_gelu_tanh_bf16: misaligned buffer");
  if (rows == 0) return MQ_OK;
  const int64_t cols4 = cols / 4;
  const dim3 grid((unsigned)((cols4 + 255) / 256), (unsigned)(rows < 65535 ? rows : 65535));
  if (src_dtype == MQ_F32)
    hipLaunchKernelGGL(gelu_bf16_kernel<float>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const float *>(src), rows, cols4, lds, static_cast<uint2 *>(dst), ldd / 4);
  else
    hipLaunchKernelGGL(gelu_bf16_kernel<__bf16>, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const __bf16 *>(src), rows, cols4, lds, static_cast<uint2 *>(dst), ldd / 4);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MQ_OK : set_error(MQ_E_HIP, hipGetErrorString(e));
}

int mq_attn_pad_correct(const void *o, int64_t batch, int heads, int64_t rows, int64_t o_batch_stride,
                        int64_t o_head_stride, int64_t o_row_stride, const float *lse, int64_t lse_batch_stride,
                        int64_t lse_head_stride, const float *npad, void *out, int64_t out_batch_stride, int64_t ldo,
                        float *guard, void *stream) {
  if (batch < 0 || rows < 0 || heads <= 0) return invalid("mq_attn_pad_correct: negative batch or rows, or heads < 1");
  if (!o || !lse || !npad || !out || !guard) return invalid("mq_attn_pad_correct: NULL pointer");
  if (o_batch_stride < 0 || o_head_stride < 0 || o_row_stride < 0 || lse_batch_stride < 0 || lse_head_stride < 0 ||
      out_batch_stride < 0 || ldo < (int64_t)heads * kHead)
    return invalid("mq_attn_pad_correct: negative stride, or ldo < heads * 128");
  if (o_batch_stride % 8 || o_head_stride % 8 || o_row_stride % 8 || out_batch_stride % 8 || ldo % 8)
    return invalid("mq_attn_pad_correct: o and out strides must be multiples of 8 elements");
  if (!aligned(o, 16) || !aligned(out, 16) || !aligned(lse, 4) || !aligned(npad, 4) || !aligned(guard, 4))
    return invalid("mq_attn_pad_correct: misaligned buffer");
  if (batch * rows * (int64_t)heads >= (int64_t(1) << 31))
    return invalid("mq_attn_pad_correct: batch * rows * heads must be below 2^31");
  const int64_t items = batch * rows * heads * (kHead / 8);
  if (items == 0) return MQ_OK;
  const int64_t blocks = (items + 255) / 256;
  const dim3 grid((unsigned)(blocks < 4096 ? blocks : 4096));
  hipLaunchKernelGGL(attn_pad_correct_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const __bf16 *>(o), o_batch_stride, o_head_stride, o_row_stride, lse,
                     lse_batch_stride, lse_head_stride, npad, heads, rows, items, static_cast<__bf16 *>(out),
                     out_batch_stride, ldo, reinterpret_cast<unsigned int *>(guard));
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MQ_OK : set_error(MQ_E_HIP, hipGetErrorString(e));
}

}  // extern "C"
