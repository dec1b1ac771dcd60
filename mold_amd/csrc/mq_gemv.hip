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
#include <utility>

#include "mq_bfrag.h"
#include "mq_kernels.h"

namespace mq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f.template operator()<I>(), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

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

// ---------------------------------------------------------------------------
// Q4_K fast path (every skinny modulation linear of the FLUX / Qwen graphs).
//
// Workgroup = R = 64/SL rows of one 64-row weight tile x all of K; wave w
// takes super-blocks [w*SB, (w+1)*SB) (SB = 1 or 2 dividing K/256, at most
// 16 waves, so K <= 8192).  Lane (r = lane % R, s = lane / R) handles row r
// and chunks s*CPL .. s*CPL+CPL-1 (CPL = 8/SL) of each of its super-blocks,
// so one wave load still reads SL contiguous 16R-byte runs of the tiled
// layout.  SL is picked so that the 64/R * tiles workgroups spread evenly
// over the CUs; every output row's sum stays inside its workgroup (added in
// fixed lane/wave order: deterministic, no cross-workgroup traffic).  All of
// a wave's loads are issued first (x, scales, then chunks) so that staging x
// waits only for x.
//
// Arithmetic per 16-byte qs chunk (32 weights of one row: 16 low nibbles of
// sub-block 2g, 16 high nibbles of sub-block 2g+1):
//   * (w >> s) & 0x000F000F | 0x43004300 is a pair of bf16 values 128 + q
//     (exact), one op per two weights;
//   * v_dot2_f32_bf16 against x packed as bf16 pairs in the same nibble
//     order gives S = sum (128 + q) x = 128 * X + sum q x, X = sum x over the
//     16 weights;
//   * y += d*sc * (S - 128 X) - dmin*m * X, i.e. two fmas per 16 weights.
// x is rounded to bf16 (as in the GEMM's A operand); the weights enter exact.
// Each wave stages its slice of x into LDS as bf16 pairs in nibble order
// together with the 16-weight sums X.
constexpr int kQ4kMaxWaves = 16;
constexpr size_t kQ4kMaxLds = 64 * 1024;

// LDS bytes of the Q4_K GEMV: x pairs + sums for all K, and the reduction.
static size_t q4k_lds_bytes(int64_t nb, int m) {
  return (size_t)nb * 8 * m * (64 + 8) + (size_t)kQ4kMaxWaves * m * 64 * 4;
}

template <int M, int SB, int SL, typename OUT>
__global__ __launch_bounds__(kQ4kMaxWaves * 64) void gemv_q4k_kernel(
    WView w, int64_t n, int64_t nb, const float *__restrict__ x, int64_t ldx, OUT *__restrict__ y, int64_t ldy,
    const float *__restrict__ bias, int act) {
  constexpr int R = 64 / SL, CPL = 8 / SL;
  extern __shared__ __align__(16) uint8_t smem[];
  uint32_t(*xp)[M][16] = reinterpret_cast<uint32_t(*)[M][16]>(smem);                 // [chunk][m][16]
  float2(*xsum)[M] = reinterpret_cast<float2(*)[M]>(smem + (size_t)nb * 8 * M * 64);  // [chunk][m]
  float(*red)[M][64] = reinterpret_cast<float(*)[M][64]>(smem + (size_t)nb * 8 * M * 72);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int64_t tile = blockIdx.x / SL;
  const int rg = blockIdx.x - (int)(tile * SL);
  const int r = lane % R, sgrp = lane / R;
  const int trow = rg * R + r;  // row inside the 64-row tile
  const int64_t b0 = (int64_t)wave * SB;  // the launcher makes SB divide nb: no partial waves

  // 1. loads, oldest first in the order they are consumed: x (4 floats per
  //    lane and super-block), the scales, then the qs chunks.
  float xv[SB][M][4];
#pragma unroll
  for (int sb = 0; sb < SB; ++sb)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float *xr = x + m * ldx + (b0 + sb) * 256 + 4 * lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[sb][m][i] = xr[i];
    }
  uint4 q[SB][CPL];
  uint32_t dm[SB], s0[SB], s1[SB], s2[SB];
#pragma unroll
  for (int sb = 0; sb < SB; ++sb) {
    dm[sb] = bfrag::ld4(bfrag::rec_at(w, 0, 4, tile, b0 + sb, trow));
    const uint8_t *sp = bfrag::rec_at(w, 1, 12, tile, b0 + sb, trow);
    s0[sb] = bfrag::ld4(sp);
    s1[sb] = bfrag::ld4(sp + 4);
    s2[sb] = bfrag::ld4(sp + 8);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep this issue order
#pragma unroll
  for (int sb = 0; sb < SB; ++sb)
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      q[sb][i] = bfrag::ld16(bfrag::chunk_at(w, 2, 8, tile, b0 + sb, sgrp * CPL + i, trow));

  // 2. stage x: lane L packs weights 4L..4L+3 of each super-block: they are
  //    bytes 4j..4j+3 (j = L & 3) of chunk c = 2(L >> 4) + ((L >> 2) & 1),
  //    low nibbles if (L & 15) < 8, i.e. pair dwords 2j (x0, x2), 2j+1 (x1, x3).
  {
    const int c = 2 * (lane >> 4) + ((lane >> 2) & 1);
    const int half = ((lane & 15) >> 3) * 8;
    const int j = lane & 3;
#pragma unroll
    for (int sb = 0; sb < SB; ++sb) {
      const int64_t ch = (b0 + sb) * 8 + c;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const __bf16 v0 = (__bf16)xv[sb][m][0], v1 = (__bf16)xv[sb][m][1];
        const __bf16 v2 = (__bf16)xv[sb][m][2], v3 = (__bf16)xv[sb][m][3];
        bf16x2_t p0 = {v0, v2}, p1 = {v1, v3};
        uint2 pk;
        __builtin_memcpy(&pk.x, &p0, 4);
        __builtin_memcpy(&pk.y, &p1, 4);
        *reinterpret_cast<uint2 *>(&xp[ch][m][half + 2 * j]) = pk;
        float t = (float)v0 + (float)v1 + (float)v2 + (float)v3;
        t += __shfl_xor(t, 1);
        t += __shfl_xor(t, 2);
        if (j == 0) {
          if (half) xsum[ch][m].y = t;
          else xsum[ch][m].x = t;
        }
      }
    }
  }
  __syncthreads();

  // 3. dot products.  bf16 pair (128 + q, 128 + q').  Both constants live in
  //    VGPRs: gfx9 VOP3 encodings take no literal and one scalar operand, so
  //    only then does (v & mask) | bias become a single v_and_or_b32.
  uint32_t kMask = 0x000F000Fu, kBias = 0x43004300u;
  asm volatile("" : "+v"(kMask), "+v"(kBias));
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;
  // Chunks are consumed in two halves, each behind its own wait, so the
  // first half's arithmetic overlaps the second half's loads (the compiler
  // would otherwise wait for every chunk before the first dot product).
  constexpr int kLoads = SB * CPL, kFirst = kLoads / 2;  // chunks in the first half (may be 0)
  static_for<2>([&]<int HALF>() {
    // chunk loads issued after the last chunk of this half
    constexpr int after = HALF == 0 ? kLoads - kFirst : 0;
    constexpr int count = HALF == 0 ? kFirst : kLoads - kFirst;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((after & 15) | ((after >> 4) << 14) | (0xF << 8) | (7 << 4));
    static_for<count>([&]<int LI>() {
      constexpr int li = (HALF == 0 ? 0 : kFirst) + LI;
      constexpr int sb = li / CPL, i = li % CPL;
      const float d = h2f((uint16_t)(dm[sb] & 0xFFFF)), dmin = h2f((uint16_t)(dm[sb] >> 16));
      const int c = sgrp * CPL + i;  // compile-time when SL == 1
      const int g = c >> 1;
      // sub-blocks 2g (low nibbles) and 2g+1 (high): bytes (2g)&3, (2g+1)&3 of
      // the packed 6-bit scale/min words for sub-blocks 0-3 (g < 2) or 4-7
      const uint32_t scw = g < 2 ? (s0[sb] & 0x3F3F3F3Fu) : ((s2[sb] & 0x0F0F0F0Fu) | ((s0[sb] >> 2) & 0x30303030u));
      const uint32_t mw = g < 2 ? (s1[sb] & 0x3F3F3F3Fu) : (((s2[sb] >> 4) & 0x0F0F0F0Fu) | ((s1[sb] >> 2) & 0x30303030u));
      const int sh = 16 * (g & 1);
      const float dlo = d * (float)((scw >> sh) & 0xFFu), dhi = d * (float)((scw >> (sh + 8)) & 0xFFu);
      const float klo = __builtin_fmaf(128.f, dlo, dmin * (float)((mw >> sh) & 0xFFu));
      const float khi = __builtin_fmaf(128.f, dhi, dmin * (float)((mw >> (sh + 8)) & 0xFFu));
      const uint32_t wd[4] = {q[sb][i].x, q[sb][i].y, q[sb][i].z, q[sb][i].w};
      uint32_t pl[8], ph[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pl[2 * j] = (wd[j] & kMask) | kBias;
        pl[2 * j + 1] = ((wd[j] >> 8) & kMask) | kBias;
        ph[2 * j] = ((wd[j] >> 4) & kMask) | kBias;
        ph[2 * j + 1] = ((wd[j] >> 12) & kMask) | kBias;
      }
      const int64_t ch = (b0 + sb) * 8 + c;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4 *xr = reinterpret_cast<const uint4 *>(xp[ch][m]);
        const uint4 xa = xr[0], xb = xr[1], xc = xr[2], xd = xr[3];
        const uint32_t xl[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const uint32_t xh[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
        float sl = 0.f, sh2 = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) {
          bf16x2_t a, b;
          __builtin_memcpy(&a, &pl[k2], 4);
          __builtin_memcpy(&b, &xl[k2], 4);
          sl = __builtin_amdgcn_fdot2_f32_bf16(a, b, sl, false);
          __builtin_memcpy(&a, &ph[k2], 4);
          __builtin_memcpy(&b, &xh[k2], 4);
          sh2 = __builtin_amdgcn_fdot2_f32_bf16(a, b, sh2, false);
        }
        const float2 X = xsum[ch][m];
        acc[m] = __builtin_fmaf(dlo, sl, acc[m]);
        acc[m] = __builtin_fmaf(-klo, X.x, acc[m]);
        acc[m] = __builtin_fmaf(dhi, sh2, acc[m]);
        acc[m] = __builtin_fmaf(-khi, X.y, acc[m]);
      }
    });
  });

  // 4. add the partial sums in lane-group, then wave order
#pragma unroll
  for (int m = 0; m < M; ++m) red[wave][m][lane] = acc[m];
  __syncthreads();
  if (wave == 0 && lane < R) {
    const int64_t row = tile * kRowTile + rg * R + lane;
    if (row < n) {
      const float bv = bias ? bias[row] : 0.f;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float t = 0.f;
        for (int wv = 0; wv < nwaves; ++wv)
#pragma unroll
          for (int sg = 0; sg < SL; ++sg) t += red[wv][m][sg * R + lane];
        store1<OUT>(y + m * ldy + row, apply_act(t + bv, act));
      }
    }
  }
}

// Super-blocks per wave for the Q4_K path (0: use the generic kernel).
static int q4k_sb(int64_t nb, int64_t m) {
  if (q4k_lds_bytes(nb, (int)m) > kQ4kMaxLds) return 0;
  if (nb <= kQ4kMaxWaves) return 1;
  // two super-blocks per wave fit 128 VGPRs up to m = 4; SB must divide nb
  if (nb <= 2 * kQ4kMaxWaves && nb % 2 == 0 && m <= 4) return 2;
  return 0;
}

// Lane groups per row (rows per workgroup = 64 / SL): the split that spreads
// ntiles * SL workgroups most evenly over the CUs while every wave of the
// launch is resident at once (at most 16 waves per CU: a second round would
// pay the memory latency again); fewest workgroups on a tie.
static int q4k_sl(int64_t ntiles, int64_t waves_per_wg, int cus) {
  double best = -1.0;
  int pick = 1;
  for (int sl : {1, 2, 4, 8}) {
    const int64_t wgs = ntiles * sl;
    if (sl > 1 && wgs * waves_per_wg > (int64_t)cus * 16) break;
    const double eff = (double)wgs / (double)(((wgs + cus - 1) / cus) * cus);
    if (eff > best + 1e-9) {
      best = eff;
      pick = sl;
    }
  }
  return pick;
}

static int pick_ksplit(int64_t ntiles, int64_t k) {
  const int64_t units = k >> 5;
  int64_t ks = 1;
  // aim for >= 2 workgroups per CU on 256 CUs, with >= 2 units per wave
  while (ntiles * ks < 512 && units / (ks * 2) >= 2 * kGemvWaves) ks *= 2;
  return (int)ks;
}

size_t gemv_scratch_bytes(int type, int64_t m, int64_t n, int64_t k) {
  if (type == Q4_K && q4k_sb(k / 256, m)) return 0;
  const int64_t ntiles = (n + kRowTile - 1) / kRowTile;
  const int ks = pick_ksplit(ntiles, k);
  if (ks == 1) return 0;
  return (size_t)ks * m * ntiles * kRowTile * sizeof(float);
}

template <int M, int SB, int SL, typename OUT>
static void launch_gemv_q4k_sl(const WView &w, int64_t n, int64_t nb, const float *x, int64_t ldx, OUT *y,
                               int64_t ldy, const float *bias, int act, hipStream_t stream) {
  const int64_t ntiles = (n + kRowTile - 1) / kRowTile;
  const int waves = (int)(nb / SB);
  hipLaunchKernelGGL((gemv_q4k_kernel<M, SB, SL, OUT>), dim3((unsigned)(ntiles * SL)), dim3(waves * 64),
                     q4k_lds_bytes(nb, M), stream, w, n, nb, x, ldx, y, ldy, bias, act);
}

template <int M, int SB, typename OUT>
static void launch_gemv_q4k_sb(const WView &w, int64_t n, int64_t nb, const float *x, int64_t ldx, OUT *y,
                               int64_t ldy, const float *bias, int act, int cus, hipStream_t stream) {
  switch (q4k_sl((n + kRowTile - 1) / kRowTile, nb / SB, cus)) {
    case 1: launch_gemv_q4k_sl<M, SB, 1, OUT>(w, n, nb, x, ldx, y, ldy, bias, act, stream); break;
    case 2: launch_gemv_q4k_sl<M, SB, 2, OUT>(w, n, nb, x, ldx, y, ldy, bias, act, stream); break;
    case 4: launch_gemv_q4k_sl<M, SB, 4, OUT>(w, n, nb, x, ldx, y, ldy, bias, act, stream); break;
    default: launch_gemv_q4k_sl<M, SB, 8, OUT>(w, n, nb, x, ldx, y, ldy, bias, act, stream); break;
  }
}

template <int M, typename OUT>
static void launch_gemv_q4k(const WView &w, int64_t n, int64_t k, const float *x, int64_t ldx, OUT *y, int64_t ldy,
                            const float *bias, int act, int cus, hipStream_t stream) {
  const int64_t nb = k / 256;
  if (q4k_sb(nb, M) == 1)
    launch_gemv_q4k_sb<M, 1, OUT>(w, n, nb, x, ldx, y, ldy, bias, act, cus, stream);
  else if constexpr (M <= 4)
    launch_gemv_q4k_sb<M, 2, OUT>(w, n, nb, x, ldx, y, ldy, bias, act, cus, stream);
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
                          OUT *y, int64_t ldy, const float *bias, int act, float *partial, int cus,
                          hipStream_t stream) {
  if (TYPE == Q4_K && q4k_sb(k / 256, m)) {
    switch (m) {
      case 1: launch_gemv_q4k<1, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      case 2: launch_gemv_q4k<2, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      case 3: launch_gemv_q4k<3, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      case 4: launch_gemv_q4k<4, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      case 5: launch_gemv_q4k<5, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      case 6: launch_gemv_q4k<6, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      case 7: launch_gemv_q4k<7, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
      default: launch_gemv_q4k<8, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    }
  }
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
                       float *partial, int cus, hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  bool ok = dispatch_type(type, [&]<int T>() {
    if (y_type == F32)
      launch_gemv_m<T, float>(w, n, k, x, m, ldx, static_cast<float *>(y), ldy, bias, act, partial, cus,
                              stream);
    else
      launch_gemv_m<T, __bf16>(w, n, k, x, m, ldx, static_cast<__bf16 *>(y), ldy, bias, act, partial, cus,
                               stream);
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mq
