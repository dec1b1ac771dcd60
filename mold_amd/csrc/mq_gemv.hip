// mq_gemv.hip — skinny-M quantized GEMV, y[m, n] = x[m, :] . W[n, :] for
// m <= 8 (FLUX/Qwen adaLN modulation, final-layer modulation: m = batch).
//
// HBM-bound: every weight byte is read exactly once.  Mapping: a workgroup
// owns one 64-row weight tile and a slice of K; lane r of every wave decodes
// row r, so each wave load of a 16-byte chunk plane reads one contiguous
// 1 KiB (see the tiled layout in mq_common.h).  The eight waves split the
// workgroup's K slice in 32-element units and combine through LDS in a fixed
// order (deterministic).  When there are too few row tiles to fill the chip
// the K range is also split across workgroups; partial sums then go to
// scratch and a second kernel adds them in a fixed order.  x is uniform
// across the wave, so its loads are scalar.
#include "mq_kernels.h"

namespace mq {

constexpr int kGemvWaves = 8;

template <typename OUT>
__device__ __forceinline__ void store1(OUT *p, float v);
template <>
__device__ __forceinline__ void store1<float>(float *p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store1<__bf16>(__bf16 *p, float v) { *p = (__bf16)v; }

template <int TYPE, int M, typename OUT>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_kernel(
    WView w, int64_t n, int64_t k, const float *__restrict__ x, int64_t ldx, OUT *__restrict__ y,
    int64_t ldy, const float *__restrict__ bias, int act, float *__restrict__ partial, int ksplit,
    int64_t npad) {
  constexpr TypeInfo ti = type_info(TYPE);
  __shared__ float red[kGemvWaves][M][64];
  const int64_t tile = blockIdx.x;
  const int ks = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t units = k >> 5;
  const int64_t per_wg = (units + ksplit - 1) / ksplit;
  const int64_t u_beg = (int64_t)ks * per_wg;
  const int64_t u_end = u_beg + per_wg < units ? u_beg + per_wg : units;
  const int64_t span = u_end > u_beg ? u_end - u_beg : 0;
  const int64_t per_wave = (span + kGemvWaves - 1) / kGemvWaves;
  const int64_t wu0 = u_beg + wave * per_wave;
  const int64_t wu1 = wu0 + per_wave < u_end ? wu0 + per_wave : u_end;

  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;

  for (int64_t u = wu0; u < wu1; ++u) {
    const int64_t kk = u << 5;
    const int64_t b = kk / ti.bs;
    const int e = (int)(kk - b * ti.bs);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float v[8];
      decode8<TYPE>(w, tile, lane, b, e + 8 * s, v);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float *xr = x + m * ldx + kk + 8 * s;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[m] = __builtin_fmaf(v[i], xr[i], acc[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m) red[wave][m][lane] = acc[m];
  __syncthreads();
  if (threadIdx.x < M * 64) {
    const int m = threadIdx.x >> 6, r = threadIdx.x & 63;
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < kGemvWaves; ++wv) s += red[wv][m][r];
    const int64_t row = tile * kRowTile + r;
    if (row < n) {
      if (ksplit == 1) {
        if (bias) s += bias[row];
        store1<OUT>(y + m * ldy + row, apply_act(s, act));
      } else {
        partial[((int64_t)ks * M + m) * npad + row] = s;
      }
    }
  }
}

template <typename OUT>
__global__ void gemv_reduce_kernel(const float *__restrict__ partial, int ksplit, int64_t m, int64_t n,
                                   int64_t npad, OUT *__restrict__ y, int64_t ldy,
                                   const float *__restrict__ bias, int act) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m * n) return;
  const int64_t mm = i / n, row = i - mm * n;
  float s = 0.f;
  for (int ks = 0; ks < ksplit; ++ks) s += partial[((int64_t)ks * m + mm) * npad + row];
  if (bias) s += bias[row];
  store1<OUT>(y + mm * ldy + row, apply_act(s, act));
}

static int pick_ksplit(int64_t ntiles, int64_t k) {
  const int64_t units = k >> 5;
  int64_t ks = 1;
  // aim for >= 2 workgroups per CU on 256 CUs, with >= 2 units per wave
  while (ntiles * ks < 512 && units / (ks * 2) >= 2 * kGemvWaves) ks *= 2;
  return (int)ks;
}

size_t gemv_scratch_bytes(int type, int64_t m, int64_t n, int64_t k) {
  const int64_t ntiles = (n + kRowTile - 1) / kRowTile;
  const int ks = pick_ksplit(ntiles, k);
  if (ks == 1) return 0;
  return (size_t)ks * m * ntiles * kRowTile * sizeof(float);
}

template <int TYPE, int M, typename OUT>
static void launch_gemv_t(const WView &w, int64_t n, int64_t k, const float *x, int64_t ldx, OUT *y,
                          int64_t ldy, const float *bias, int act, float *partial, hipStream_t stream) {
  const int64_t ntiles = (n + kRowTile - 1) / kRowTile;
  const int ks = pick_ksplit(ntiles, k);
  const int64_t npad = ntiles * kRowTile;
  hipLaunchKernelGGL((gemv_kernel<TYPE, M, OUT>), dim3((unsigned)ntiles, ks), dim3(kGemvWaves * 64), 0,
                     stream, w, n, k, x, ldx, y, ldy, bias, act, partial, ks, npad);
  if (ks > 1) {
    const int64_t total = (int64_t)M * n;
    hipLaunchKernelGGL(gemv_reduce_kernel<OUT>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, partial, ks, (int64_t)M, n, npad, y, ldy, bias, act);
  }
}

template <int TYPE, typename OUT>
static void launch_gemv_m(const WView &w, int64_t n, int64_t k, const float *x, int64_t m, int64_t ldx,
                          OUT *y, int64_t ldy, const float *bias, int act, float *partial,
                          hipStream_t stream) {
  switch (m) {
    case 1: launch_gemv_t<TYPE, 1, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    case 2: launch_gemv_t<TYPE, 2, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    case 3: launch_gemv_t<TYPE, 3, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    case 4: launch_gemv_t<TYPE, 4, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    case 5: launch_gemv_t<TYPE, 5, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    case 6: launch_gemv_t<TYPE, 6, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    case 7: launch_gemv_t<TYPE, 7, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
    default: launch_gemv_t<TYPE, 8, OUT>(w, n, k, x, ldx, y, ldy, bias, act, partial, stream); break;
  }
}

hipError_t launch_gemv(int type, const WView &w, int64_t n, int64_t k, const float *x, int64_t m,
                       int64_t ldx, void *y, int y_type, int64_t ldy, const float *bias, int act,
                       float *partial, hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  bool ok = dispatch_type(type, [&]<int T>() {
    if (y_type == F32)
      launch_gemv_m<T, float>(w, n, k, x, m, ldx, static_cast<float *>(y), ldy, bias, act, partial, stream);
    else
      launch_gemv_m<T, __bf16>(w, n, k, x, m, ldx, static_cast<__bf16 *>(y), ldy, bias, act, partial,
                               stream);
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mq
