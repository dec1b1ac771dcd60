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
// Q4_K fast path (every skinny modulation linear of the FLUX / Qwen graphs):
// candle's own QMatMul algorithm for k-quants.  x is quantized to Q8_K
// (per 256 elements: iscale = -128 / (the element of largest magnitude, the
// first one on ties), q = min(round_half_away(iscale * x), 127), d = 1 / iscale,
// plus the sums of q over each 32-element sub-block), the weight nibbles
// enter integer dot products exactly, and per super-block
//   y += (d_w * d_x) * sum_s sc_s * sum_{i in s} q_w q_x
//      - (dmin_w * d_x) * sum_s m_s * sum_{i in s} q_x,
// the formula of candle's Q4_K x Q8_K vec_dot (k_quants.rs; restated in
// oracle/ggml_oracle.c vd_q45_K).  The integer parts are exact, so the result
// differs from candle's CPU path only in the order of the final f32 adds.
//
// Workgroup = R = 64/SL rows of one 64-row weight tile x all of K; wave w
// takes super-blocks [w*SB, (w+1)*SB) (SB = 1 or 2 dividing K/256, at most
// 16 waves, so K <= 8192).  Lane (r = lane % R, s = lane / R) handles row r
// and chunks s*CPL .. s*CPL+CPL-1 (CPL = 8/SL) of each of its super-blocks,
// so one wave load still reads SL contiguous 16R-byte runs of the tiled
// layout.  SL is picked so that the 64/R * tiles workgroups spread evenly
// over the CUs; every output row's sum stays inside its workgroup (added in
// fixed lane/wave order: deterministic, no cross-workgroup traffic).  All of
// a wave's loads are issued first (x, scales, then chunks) so that the Q8_K
// staging waits only for x.
//
// Arithmetic per 16-byte qs chunk c of a super-block (32 weights of one row:
// 16 low nibbles of sub-block 2g and 16 high nibbles of sub-block 2g+1,
// g = c / 2, elements 64g + 16(c&1) + t and 64g + 32 + 16(c&1) + t):
// word j's low nibbles (w & 0x0F0F0F0F) are elements 4j..4j+3 of the low run
// in byte order, the high nibbles ((w >> 4) & 0x0F0F0F0F) those of the high
// run, so each feeds one v_dot4_i32_i8 against four consecutive Q8_K bytes of
// x: 3 + 2M VALU ops per 8 weights.
constexpr int kQ4kMaxWaves = 16;
constexpr size_t kQ4kMaxLds = 64 * 1024;

// Cross-lane steps through DPP (no LDS round trip).  Lanes a step has no
// source for (rows outside ROW_MASK) keep their own value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
}
// Max over the wave, uniform: quad xor 1, quad xor 2, half-row mirror, row
// mirror give every lane its 16-lane row's max; row_bcast:15 (rows 1, 3) and
// row_bcast:31 (rows 2, 3) carry rows 0-2 into row 3; lane 63 holds the max.
__device__ __forceinline__ float wave_max(float v) {
  v = __builtin_fmaxf(v, __int_as_float(dpp<0xB1, 0xF>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x4E, 0xF>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x141, 0xF>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x140, 0xF>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x142, 0xA>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x143, 0xC>(__float_as_int(v))));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Sum over each aligned group of 8 lanes (a half row), in every lane of it.
__device__ __forceinline__ int sum8(int v) {
  v += dpp<0xB1, 0xF>(v);
  v += dpp<0x4E, 0xF>(v);
  v += dpp<0x141, 0xF>(v);
  return v;
}

// LDS bytes of the Q4_K GEMV: Q8_K x (256 quants, d, 8 sub-block sums per
// super-block and row of x) for all K, and the reduction.
static size_t q4k_lds_bytes(int64_t nb, int m) {
  return (size_t)nb * m * (256 + 4 + 32) + (size_t)kQ4kMaxWaves * m * 64 * 4;
}

template <int M, int SB, int SL, typename OUT>
__global__ __launch_bounds__(kQ4kMaxWaves * 64) void gemv_q4k_kernel(
    WView w, int64_t n, int64_t nb, const float *__restrict__ x, int64_t ldx, OUT *__restrict__ y, int64_t ldy,
    const float *__restrict__ bias, int act) {
  constexpr int R = 64 / SL, CPL = 8 / SL;
  const int nwaves = blockDim.x >> 6;
  extern __shared__ __align__(16) uint8_t smem[];
  uint32_t(*xq)[M][64] = reinterpret_cast<uint32_t(*)[M][64]>(smem);                         // [sb][m][dword]
  int32_t(*xb)[M][8] = reinterpret_cast<int32_t(*)[M][8]>(smem + (size_t)nb * M * 256);    // [sb][m][sub-block]
  float(*xd)[M] = reinterpret_cast<float(*)[M]>(smem + (size_t)nb * M * 288);              // [sb][m]
  float(*red)[M][64] = reinterpret_cast<float(*)[M][64]>(smem + (size_t)nb * M * 292);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
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

  // 2. Q8_K staging of this wave's super-blocks: lane L holds elements
  //    4L..4L+3 (sub-block L / 8).
#pragma unroll
  for (int sb = 0; sb < SB; ++sb) {
    const int64_t bg = b0 + sb;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      // largest magnitude over the wave, then the value of its first
      // occurrence in element order (lowest lane, lowest slot in the lane)
      const float a0 = __builtin_fabsf(xv[sb][m][0]), a1 = __builtin_fabsf(xv[sb][m][1]);
      const float a2 = __builtin_fabsf(xv[sb][m][2]), a3 = __builtin_fabsf(xv[sb][m][3]);
      const float amax = wave_max(__builtin_fmaxf(__builtin_fmaxf(a0, a1), __builtin_fmaxf(a2, a3)));
      const float cand = a0 == amax ? xv[sb][m][0]
                         : a1 == amax ? xv[sb][m][1]
                         : a2 == amax ? xv[sb][m][2]
                                      : xv[sb][m][3];
      const uint64_t hit = __ballot(a0 == amax || a1 == amax || a2 == amax || a3 == amax);
      const int first = hit ? __builtin_ctzll(hit) : 0;
      const float vmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cand), first));
      uint32_t packed = 0;
      int qsum = 0;
      float dx = 0.f;
      if (amax != 0.f) {
        const float iscale = -128.f / vmax;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = (int)__builtin_fminf(__builtin_roundf(iscale * xv[sb][m][i]), 127.f);
          qsum += v;
          packed |= (uint32_t)(v & 0xFF) << (8 * i);
        }
        dx = 1.f / iscale;
      }
      xq[bg][m][lane] = packed;
      qsum = sum8(qsum);
      if ((lane & 7) == 0) xb[bg][m][lane >> 3] = qsum;
      if (lane == 0) xd[bg][m] = dx;
    }
  }
  __syncthreads();

  // 3. integer dot products, consumed in two halves of the chunk loads, each
  //    behind its own wait, so the first half's arithmetic overlaps the
  //    second half's loads.
  int32_t S[SB][M];
#pragma unroll
  for (int sb = 0; sb < SB; ++sb)
#pragma unroll
    for (int m = 0; m < M; ++m) S[sb][m] = 0;
  constexpr int kLoads = SB * CPL, kFirst = kLoads / 2;  // chunks in the first half (may be 0)
  static_for<2>([&]<int HALF>() {
    constexpr int after = HALF == 0 ? kLoads - kFirst : 0;  // chunk loads issued after this half
    constexpr int count = HALF == 0 ? kFirst : kLoads - kFirst;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt((after & 15) | ((after >> 4) << 14) | (0xF << 8) | (7 << 4));
    static_for<count>([&]<int LI>() {
      constexpr int li = (HALF == 0 ? 0 : kFirst) + LI;
      constexpr int sb = li / CPL, i = li % CPL;
      const int c = sgrp * CPL + i;  // compile-time when SL == 1
      const int g = c >> 1, hs = c & 1;
      // sub-blocks 2g (low nibbles) and 2g+1 (high): bytes (2g)&3, (2g+1)&3 of
      // the packed 6-bit scale words for sub-blocks 0-3 (g < 2) or 4-7
      const uint32_t scw = g < 2 ? (s0[sb] & 0x3F3F3F3Fu) : ((s2[sb] & 0x0F0F0F0Fu) | ((s0[sb] >> 2) & 0x30303030u));
      const int sh = 16 * (g & 1);
      const int sclo = (int)((scw >> sh) & 0xFFu), schi = (int)((scw >> (sh + 8)) & 0xFFu);
      const uint32_t wd[4] = {q[sb][i].x, q[sb][i].y, q[sb][i].z, q[sb][i].w};
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = wd[j] & 0x0F0F0F0Fu;
        hi[j] = (wd[j] >> 4) & 0x0F0F0F0Fu;
      }
      const int64_t bg = b0 + sb;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4 xa = *reinterpret_cast<const uint4 *>(&xq[bg][m][16 * g + 4 * hs]);
        const uint4 xc = *reinterpret_cast<const uint4 *>(&xq[bg][m][16 * g + 8 + 4 * hs]);
        int il = __builtin_amdgcn_sdot4((int)lo[0], (int)xa.x, 0, false);
        il = __builtin_amdgcn_sdot4((int)lo[1], (int)xa.y, il, false);
        il = __builtin_amdgcn_sdot4((int)lo[2], (int)xa.z, il, false);
        il = __builtin_amdgcn_sdot4((int)lo[3], (int)xa.w, il, false);
        int ih = __builtin_amdgcn_sdot4((int)hi[0], (int)xc.x, 0, false);
        ih = __builtin_amdgcn_sdot4((int)hi[1], (int)xc.y, ih, false);
        ih = __builtin_amdgcn_sdot4((int)hi[2], (int)xc.z, ih, false);
        ih = __builtin_amdgcn_sdot4((int)hi[3], (int)xc.w, ih, false);
        S[sb][m] += __mul24(sclo, il) + __mul24(schi, ih);  // |il|, |ih| < 2^15: 24-bit products are exact
      }
    });
  });

  // 4. per super-block f32 combine: (d_w d_x) S - (dmin_w d_x) sum_s m_s B_s,
  //    the mins term once per row (lane group 0)
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
  for (int sb = 0; sb < SB; ++sb) {
    const int64_t bg = b0 + sb;
    const float d = h2f((uint16_t)(dm[sb] & 0xFFFF)), dmin = h2f((uint16_t)(dm[sb] >> 16));
    const uint32_t mlo = s1[sb] & 0x3F3F3F3Fu;
    const uint32_t mhi = ((s2[sb] >> 4) & 0x0F0F0F0Fu) | ((s1[sb] >> 2) & 0x30303030u);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float dx = xd[bg][m];
      int smin = 0;
      if (sgrp == 0) {
        const int4 ba = *reinterpret_cast<const int4 *>(&xb[bg][m][0]);
        const int4 bb = *reinterpret_cast<const int4 *>(&xb[bg][m][4]);
        smin = __mul24((int)(mlo & 0xFF), ba.x) + __mul24((int)((mlo >> 8) & 0xFF), ba.y) +
               __mul24((int)((mlo >> 16) & 0xFF), ba.z) + __mul24((int)(mlo >> 24), ba.w) +
               __mul24((int)(mhi & 0xFF), bb.x) + __mul24((int)((mhi >> 8) & 0xFF), bb.y) +
               __mul24((int)((mhi >> 16) & 0xFF), bb.z) + __mul24((int)(mhi >> 24), bb.w);
      }
      acc[m] = __builtin_fmaf(d * dx, (float)S[sb][m], acc[m]);
      acc[m] = __builtin_fmaf(-(dmin * dx), (float)smin, acc[m]);
    }
  }

  // 5. add the partial sums in lane-group, then wave order
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
