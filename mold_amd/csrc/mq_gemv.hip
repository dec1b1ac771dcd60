// mq_gemv.hip — skinny-M quantized GEMV, y[m, n] = x[m, :] . W[n, :] for
// m <= 8 (FLUX/Qwen adaLN modulation, final-layer modulation: m = batch).
//
// HBM-bound: every weight byte is read exactly once.  Q4_K weights take
// gemv_q4k_kernel and the other types gemv_frag_kernel (both below, one
// workgroup per CU over consecutive rows); where those do not apply (LDS
// bounds; for the other types also K not a multiple of 256 or m > 4) the
// generic kernel runs: a workgroup
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
        store1<OUT>(y + m * ldy + row, apply_act(s, act_at(act, row)));
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
  store1<OUT>(y + mm * ldy + row, apply_act(s, act_at(act, row)));
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
// HBM-bound layout of the work: one 512-thread workgroup per CU owns `rows`
// consecutive output rows (ceil(n / CUs): 72 at n = 18432, so every CU reads
// the same number of weight bytes) over all of K; where the LDS would not hold
// that many rows' partials (the steps' stacked modulation launches, ~1M rows)
// workgroups take fewer rows and several run on each CU in turn.  Thread t takes the
// (row, super-block) pairs p = t, t + 512, ... (row fastest, so a wave's
// 16-byte loads of one chunk plane read consecutive rows of the tiled
// layout).  x is loaded first and the weight loads start once the whole
// workgroup's x has landed (x, read by every workgroup, otherwise queues
// behind the weight stream in the memory system and the Q8_K staging, on
// which every dot waits, starts late); the staging then runs while the first
// pairs stream in: 16-lane group g (of 32) quantizes items g, g + 32, ...
// (item = one row of x over one super-block) into LDS, 16 elements per lane.
// Each pair's integer dot reads its 32 Q8_K bytes per 16-byte weight chunk
// from LDS: 3 + 2M VALU ops per 8 weights.  The pairs' f32 partials go to
// LDS and thread (row, m) adds them in super-block order (deterministic).
constexpr int kQ4kThreads = 512;
constexpr size_t kQ4kMaxLds = 96 * 1024;

// Cross-lane steps through DPP (no LDS round trip).  Lanes a step has no
// source for (rows outside ROW_MASK) keep their own value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, ROW_MASK, 0xF, false);
}
// Max / min over each aligned group of 16 lanes (a DPP row), in every lane of
// it: quad xor 1, quad xor 2, half-row mirror (quads 0 <-> 1), row mirror
// (half rows 0 <-> 1).
__device__ __forceinline__ float row16_max(float v) {
  v = __builtin_fmaxf(v, __int_as_float(dpp<0xB1, 0xF>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x4E, 0xF>(__float_as_int(v))));
  v = __builtin_fmaxf(v, __int_as_float(dpp<0x141, 0xF>(__float_as_int(v))));
  return __builtin_fmaxf(v, __int_as_float(dpp<0x140, 0xF>(__float_as_int(v))));
}
__device__ __forceinline__ int row16_min(int v) {
  v = min(v, dpp<0xB1, 0xF>(v));
  v = min(v, dpp<0x4E, 0xF>(v));
  v = min(v, dpp<0x141, 0xF>(v));
  return min(v, dpp<0x140, 0xF>(v));
}

// LDS of the Q4_K GEMV: x as given (f32 or bf16, 256 elements per
// super-block and row of x), its Q8_K form (256 quants, 8 sub-block sums and
// d), then one f32 partial per (super-block, row, m).  For x given already in
// Q8_K form (MQ_X_Q8K) the blocks are copied in as they are, kQ8kXBytes each.
__host__ __device__ inline size_t q4k_lds_bytes(int64_t nb, int m, int64_t rows, int xsize) {
  return (size_t)nb * m * (xsize < 0 ? kQ8kXBytes : 256 * xsize + 256 + 32 + 4) + (size_t)nb * rows * m * 4;
}

// One item (256 elements of one row of x) to Q8_K, held by a 16-lane group:
// lane l16 holds elements 16 l16 .. 16 l16 + 15 in v.  iscale = -128 / (the
// first element of largest magnitude), q = min(round_half_away(iscale x),
// 127), d = 1 / iscale (all zero for an all-zero item).  Returns the lane's 16
// quants packed, and in qsum the sum of its sub-block's 32 quants (lanes l16
// and l16 ^ 1 hold one sub-block).
__device__ __forceinline__ float q8k_quantize16(const float v[16], int l16, int lane, uint32_t packed[4], int &qsum) {
  // largest magnitude over the item, then the value of its first occurrence
  // in element order: the lowest element index holding it, taken from the
  // lane that owns that index (with no hit, as for an all-NaN item, element 3)
  float lmax = __builtin_fabsf(v[0]);
#pragma unroll
  for (int i = 1; i < 16; ++i) lmax = __builtin_fmaxf(lmax, __builtin_fabsf(v[i]));
  const float amax = row16_max(lmax);
  int first = 16;
  float cand = v[3];
#pragma unroll
  for (int i = 15; i >= 0; --i) {
    const bool hit = __builtin_fabsf(v[i]) == amax;
    first = hit ? i : first;
    cand = hit ? v[i] : cand;
  }
  const int gfirst = row16_min(first < 16 ? 16 * l16 + first : 256);
  const int src = (lane & ~15) + (gfirst < 256 ? gfirst >> 4 : 0);
  const float vmax = __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(cand)));
  packed[0] = packed[1] = packed[2] = packed[3] = 0u;
  qsum = 0;
  float dx = 0.f;
  if (amax != 0.f) {
    const float iscale = -128.f / vmax;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = (int)__builtin_fminf(__builtin_roundf(iscale * v[i]), 127.f);
      qsum += q;
      packed[i >> 2] |= (uint32_t)(q & 0xFF) << (8 * (i & 3));
    }
    dx = 1.f / iscale;
  }
  qsum += dpp<0xB1, 0xF>(qsum);  // the sub-block's other half (lane L ^ 1)
  return dx;
}

typedef __attribute__((address_space(3))) void lds_void_t;
// One direct global->LDS load: lane i's 16 bytes from g land at LDS byte
// address lds + 16 i (M0 carries the LDS address).  Issued as inline asm so
// that the compiler never holds an in-flight register for x; the kernel
// orders it with its own s_waitcnt before the barrier that publishes x.
// s_nop: one wait state between writing M0 and the instruction reading it.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// One (row, super-block) pair's weight bytes.
struct Q4kPair {
  uint4 q[8];
  uint32_t dm, s0, s1, s2;
};

template <int M, typename XT, typename OUT, bool kOne>
__global__ __launch_bounds__(kQ4kThreads) void gemv_q4k_kernel(
    WView w, int64_t n, int64_t nrows_mem, int nb, int rows, const XT *__restrict__ x, int64_t ldx,
    OUT *__restrict__ y, int64_t ldy, const float *__restrict__ bias, int act) {
  extern __shared__ __align__(16) uint8_t smem[];
  // x given in Q8_K form (MQ_X_Q8K): its blocks are copied into LDS as they are
  constexpr bool kQ8 = __is_same(XT, Q8kX);
  constexpr int kXs = kQ8 ? 0 : (int)sizeof(XT);
  const XT *xl = reinterpret_cast<const XT *>(smem);                          // [nb][M][256] x
  uint8_t *q8 = smem + (size_t)nb * M * 256 * kXs;
  uint32_t *xq = reinterpret_cast<uint32_t *>(q8);                            // [nb][M][64] packed i8
  int32_t *xs = reinterpret_cast<int32_t *>(q8 + (size_t)nb * M * 256);       // [nb][M][8]
  float *xd = reinterpret_cast<float *>(q8 + (size_t)nb * M * 288);           // [nb][M]
  float *red = reinterpret_cast<float *>(q8 + (size_t)nb * M * (kQ8 ? kQ8kXBytes : 292));  // [nb * rows][M]
  // item (super-block sb, row m of x): its 64 packed quant words, 8 sub-block
  // sums and d (kQ8: block m * nb + sb of the copied rows)
  auto x_words = [&](int sb, int m) -> const uint32_t * {
    if constexpr (kQ8) return reinterpret_cast<const uint32_t *>(q8 + (size_t)(m * nb + sb) * kQ8kXBytes);
    else return xq + (sb * M + m) * 64;
  };
  auto x_sums = [&](int sb, int m) -> const int32_t * {
    if constexpr (kQ8) return reinterpret_cast<const int32_t *>(q8 + (size_t)(m * nb + sb) * kQ8kXBytes + 256);
    else return xs + (sb * M + m) * 8;
  };
  auto x_d = [&](int sb, int m) -> float {
    if constexpr (kQ8) return *reinterpret_cast<const float *>(q8 + (size_t)(m * nb + sb) * kQ8kXBytes + 288);
    else return xd[sb * M + m];
  };
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int64_t r0 = (int64_t)blockIdx.x * rows;
  const int npairs = rows * nb;

  auto load_pair = [&](int p, Q4kPair &d) {
    const int sb = p / rows;
    int64_t row = r0 + (p - sb * rows);
    row = row < nrows_mem ? row : nrows_mem - 1;  // rows past the padded tiles re-read the last one
    const int64_t t = row >> 6;
    const int r = (int)(row & 63);
    // weights are read once per launch: non-temporal loads keep them from
    // displacing x and other reused data in L2 / Infinity Cache
    d.dm = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(bfrag::rec_at(w, 0, 4, t, sb, r)));
    const uint32_t *sp = reinterpret_cast<const uint32_t *>(bfrag::rec_at(w, 1, 12, t, sb, r));
    d.s0 = __builtin_nontemporal_load(sp);
    d.s1 = __builtin_nontemporal_load(sp + 1);
    d.s2 = __builtin_nontemporal_load(sp + 2);
#pragma unroll
    for (int c = 0; c < 8; ++c)
    {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(bfrag::chunk_at(w, 2, 8, t, sb, c, r)));
      d.q[c] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };

  // 1. x into LDS by direct loads (item j = sb * M + m is row m's elements
  //    sb*256 .. +255: one 1 KiB load for f32, half a wave's for bf16); once
  //    every wave's x has landed, the first pair's weights (index clamped, so
  //    every load is unconditional).
  const int nitems = nb * M;
  constexpr int kWaves = kQ4kThreads / 64;
  Q4kPair slot[kOne ? 1 : 2];
  if constexpr (kQ8) {
    // x's blocks (M rows of nb, contiguous) into LDS as they are, 1 KiB per
    // wave load (lanes past the end issue nothing), then at once the first
    // pair's weights: x, a few KiB that every workgroup reads, comes from L2
    // and is not queued behind them.  The wait leaves at most the pair's
    // weight loads in flight (10 or more vector loads, issued after x).
    const uint32_t lbase = (uint32_t)(uintptr_t)(lds_void_t *)smem;
    const int xbytes = nitems * kQ8kXBytes;
    const uint8_t *xb = reinterpret_cast<const uint8_t *>(x);
    for (int c = wave; c * 1024 < xbytes; c += kWaves)
      if (c * 1024 + 16 * lane < xbytes) dma16(xb + c * 1024 + 16 * lane, lbase + (uint32_t)(c * 1024));
    load_pair(tid < npairs ? tid : npairs - 1, slot[0]);
    asm volatile("s_waitcnt vmcnt(10)" ::: "memory");  // this wave's x
    __syncthreads();
  } else {
    const uint32_t lbase = (uint32_t)(uintptr_t)(lds_void_t *)smem;
    if constexpr (kXs == 4) {
      for (int j = wave; j < nitems; j += kWaves) {
        const int sb = j / M, m = j - sb * M;
        dma16(x + m * ldx + sb * 256 + 4 * lane, lbase + j * 1024);
      }
    } else {
      // two items per load: lanes 0-31 item j, lanes 32-63 item j + 1; for an
      // odd item count the last load issues lanes 0-31 only (lane i writes LDS
      // byte 16 i on, so lanes 32-63 would write past the x region, and past
      // the allocation when few rows' partials follow it)
      for (int j = 2 * wave; j < nitems; j += 2 * kWaves) {
        const int sb = (j + (lane >> 5)) / M, m = (j + (lane >> 5)) - sb * M;
        if (lane < 32 || j + 1 < nitems) dma16(x + m * ldx + sb * 256 + 8 * (lane & 31), lbase + j * 512);
      }
    }
  }
  if constexpr (!kQ8) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's x
    __syncthreads();
    load_pair(tid < npairs ? tid : npairs - 1, slot[0]);
  }

  // 2. Q8_K staging: one item per 16-lane group (32 groups, every one at
  //    once); lane L of a group holds elements 16L..16L+15, half of sub-block
  //    L / 2.
  const int g16 = tid >> 4, l16 = tid & 15;
  auto stage = [&](int j) {
    float v[16];
    if constexpr (kXs == 4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 t = *reinterpret_cast<const float4 *>(xl + j * 256 + 16 * l16 + 4 * c);
        v[4 * c] = t.x;
        v[4 * c + 1] = t.y;
        v[4 * c + 2] = t.z;
        v[4 * c + 3] = t.w;
      }
    } else {
      // bf16 -> f32 is exact: the 16 bits become the high half
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint4 t = *reinterpret_cast<const uint4 *>(xl + j * 256 + 16 * l16 + 8 * c);
        const uint32_t wd[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[8 * c + 2 * i] = __uint_as_float(wd[i] << 16);
          v[8 * c + 2 * i + 1] = __uint_as_float(wd[i] & 0xFFFF0000u);
        }
      }
    }
    uint32_t packed[4];
    int qsum;
    const float dx = q8k_quantize16(v, l16, tid & 63, packed, qsum);
    *reinterpret_cast<uint4 *>(xq + j * 64 + 4 * l16) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    if ((l16 & 1) == 0) xs[j * 8 + (l16 >> 1)] = qsum;
    if (l16 == 0) xd[j] = dx;
  };
  if constexpr (!kQ8) {
    for (int j = g16; j < nitems; j += kQ4kThreads / 16) stage(j);
    __syncthreads();
  }

  // 3. per pair: integer dot against Q8_K x, one f32 partial per m
  auto dot_pair = [&](int p, const Q4kPair &cur) {
    const bool valid = p < npairs;  // clamped pairs are computed, not stored
    p = valid ? p : npairs - 1;
    const int sb = p / rows;
    // 6-bit scales and mins of sub-blocks 0-3 (low 6 bits of bytes 0-3 / 4-7)
    // and 4-7 (nibbles of bytes 8-11 with the top 2 bits of bytes 0-3 / 4-7)
    const uint32_t sc03 = cur.s0 & 0x3F3F3F3Fu, m03 = cur.s1 & 0x3F3F3F3Fu;
    const uint32_t sc47 = (cur.s2 & 0x0F0F0F0Fu) | ((cur.s0 >> 2) & 0x30303030u);
    const uint32_t m47 = ((cur.s2 >> 4) & 0x0F0F0F0Fu) | ((cur.s1 >> 2) & 0x30303030u);
    int sc[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = (int)((sc03 >> (8 * i)) & 0xFFu);
      sc[4 + i] = (int)((sc47 >> (8 * i)) & 0xFFu);
    }
    int S[M];
#pragma unroll
    for (int m = 0; m < M; ++m) S[m] = 0;
    // The one-slot instances take this path at m = 1, and at m = 2 on x given
    // as Q8_K blocks (3072 -> 9216, same box: 2.2-2.8 % and 8.9 % faster; at
    // m = 2 on f32 x no change, so that one keeps the path below)
    if constexpr (M <= 2 && (!kOne || M == 1 || kQ8)) {
      // steps s = (g, m) in order g-major: chunks 2g and 2g+1 (32 bytes) hold
      // elements 64g + 0..31 in their low nibbles (sub-block 2g) and 64g +
      // 32..63 in their high nibbles (sub-block 2g+1), each in byte order; one
      // sdot4 chain of 8 per sub-block and row m of x.  The 64 Q8_K bytes of
      // step s + 1 are read from LDS while step s computes (two register slots).
      auto xload = [&](int g, int m, uint4 *dst) {
        const uint4 *xb = reinterpret_cast<const uint4 *>(x_words(sb, m) + 16 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = xb[i];
      };
      uint4 xbuf[2][4];
      xload(0, 0, xbuf[0]);
      uint32_t lo[8], hi[8];
      static_for<4 * M>([&]<int ST>() {
        constexpr int g = ST / M, m = ST % M;
        if constexpr (ST + 1 < 4 * M) xload((ST + 1) / M, (ST + 1) % M, xbuf[(ST + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this step's dots
        if constexpr (m == 0) {
          const uint32_t wd[8] = {cur.q[2 * g].x,     cur.q[2 * g].y,     cur.q[2 * g].z,     cur.q[2 * g].w,
                                  cur.q[2 * g + 1].x, cur.q[2 * g + 1].y, cur.q[2 * g + 1].z, cur.q[2 * g + 1].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            lo[i] = wd[i] & 0x0F0F0F0Fu;
            hi[i] = (wd[i] >> 4) & 0x0F0F0F0Fu;
          }
        }
        const uint4 *xv = xbuf[ST & 1];
        const uint32_t xl[8] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w, xv[1].x, xv[1].y, xv[1].z, xv[1].w};
        const uint32_t xh[8] = {xv[2].x, xv[2].y, xv[2].z, xv[2].w, xv[3].x, xv[3].y, xv[3].z, xv[3].w};
        int dl = 0, dh = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dl = __builtin_amdgcn_sdot4((int)lo[i], (int)xl[i], dl, false);
          dh = __builtin_amdgcn_sdot4((int)hi[i], (int)xh[i], dh, false);
        }
        // |dl|, |dh| <= 32 * 15 * 128 < 2^16: the 24-bit products are exact
        S[m] += __mul24(sc[2 * g], dl) + __mul24(sc[2 * g + 1], dh);
      });
    } else {
      // (m > 2, and the one-slot instance at m = 2 on f32 / bf16 x: the same
      // steps with the Q8_K bytes read at their use; two register slots of 16
      // per step would spill at m > 2)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // chunks 2g and 2g+1 (32 bytes): low nibbles are elements 64g + 0..31
        // (sub-block 2g), high nibbles elements 64g + 32..63 (sub-block 2g+1),
        // each in byte order; one sdot4 chain of 8 per sub-block
        const uint32_t wd[8] = {cur.q[2 * g].x,     cur.q[2 * g].y,     cur.q[2 * g].z,     cur.q[2 * g].w,
                                cur.q[2 * g + 1].x, cur.q[2 * g + 1].y, cur.q[2 * g + 1].z, cur.q[2 * g + 1].w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          lo[i] = wd[i] & 0x0F0F0F0Fu;
          hi[i] = (wd[i] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint32_t *xb = x_words(sb, m) + 16 * g;
          const uint4 x0 = *reinterpret_cast<const uint4 *>(xb);
          const uint4 x1 = *reinterpret_cast<const uint4 *>(xb + 4);
          const uint4 x2 = *reinterpret_cast<const uint4 *>(xb + 8);
          const uint4 x3 = *reinterpret_cast<const uint4 *>(xb + 12);
          const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
          const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
          int dl = 0, dh = 0;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            dl = __builtin_amdgcn_sdot4((int)lo[i], (int)xl[i], dl, false);
            dh = __builtin_amdgcn_sdot4((int)hi[i], (int)xh[i], dh, false);
          }
          // |dl|, |dh| <= 32 * 15 * 128 < 2^16: the 24-bit products are exact
          S[m] += __mul24(sc[2 * g], dl) + __mul24(sc[2 * g + 1], dh);
        }
      }
    }
    const float d = h2f((uint16_t)(cur.dm & 0xFFFF)), dmin = h2f((uint16_t)(cur.dm >> 16));
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int4 ba = *reinterpret_cast<const int4 *>(x_sums(sb, m));
      const int4 bb = *reinterpret_cast<const int4 *>(x_sums(sb, m) + 4);
      const int smin = __mul24((int)(m03 & 0xFF), ba.x) + __mul24((int)((m03 >> 8) & 0xFF), ba.y) +
                       __mul24((int)((m03 >> 16) & 0xFF), ba.z) + __mul24((int)(m03 >> 24), ba.w) +
                       __mul24((int)(m47 & 0xFF), bb.x) + __mul24((int)((m47 >> 8) & 0xFF), bb.y) +
                       __mul24((int)((m47 >> 16) & 0xFF), bb.z) + __mul24((int)(m47 >> 24), bb.w);
      const float dx = x_d(sb, m);
      if (valid) red[p * M + m] = __builtin_fmaf(d * dx, (float)S[m], -(dmin * dx) * (float)smin);
    }
  };
  // The second pairs (512 .. min(npairs, 1024) - 1, spread evenly over the
  // waves: lanes 0 .. per-1 of each) are issued only once the first pair has
  // landed, and the first pair's dot runs while they stream in.  All of a
  // launch's loads issued at once finish in an arbitrary order across the
  // chip, so each thread's pairs would land near the end of the stream and
  // every dot would run after it; in two waves the first pairs land at about
  // the middle and only the second pairs' dots follow the stream.  Pairs past
  // 1024 (K beyond 2 * 512 pairs' worth) load as they go.
  if constexpr (kOne) {
    // every pair of the workgroup is thread tid's slot 0
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    dot_pair(tid, slot[0]);
  } else {
    const int n2 = (npairs < 2 * kQ4kThreads ? npairs : 2 * kQ4kThreads) - kQ4kThreads;
    const int per = n2 > 0 ? (n2 + kWaves - 1) / kWaves : 0;
    const int p1 = kQ4kThreads + per * wave + lane;
    const bool has1 = lane < per && p1 < npairs;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the first pair has landed
    if (has1) load_pair(p1, slot[1]);
    dot_pair(tid, slot[0]);
    if (has1) dot_pair(p1, slot[1]);
    for (int p = tid + 2 * kQ4kThreads; p < npairs; p += kQ4kThreads) {
      load_pair(p, slot[0]);
      dot_pair(p, slot[0]);
    }
  }
  __syncthreads();

  // 4. thread (row, m) adds its row's partials in super-block order
  for (int t = tid; t < rows * M; t += kQ4kThreads) {
    const int m = t / rows, rl = t - m * rows;
    const int64_t row = r0 + rl;
    if (row >= n) continue;
    float acc = 0.f;
    for (int sb = 0; sb < nb; ++sb) acc += red[(sb * rows + rl) * M + m];
    if (bias) acc += bias[row];
    store1<OUT>(y + m * ldy + row, apply_act(acc, act_at(act, row)));
  }
}

// ---------------------------------------------------------------------------
// Streaming GEMV for the other types (f32 x, exact f32 weights): the same work
// layout as the Q4_K kernel (one 512-thread workgroup per CU over `rows`
// consecutive output rows and all of K, thread t taking the (row, unit) pairs
// t, t + 512, ... with the row fastest so a wave's 16-byte loads of one chunk
// plane read consecutive rows), with the weights decoded by the GEMM's
// per-type B-fragment decoders (mq_bfrag.h) in their f32 form: each is the
// exact value ggml's dequantize_row_* gives, and x . w accumulates in f32.  A
// unit is 256 weights (128 for Q8_0), split in the decoders' two halves; a
// thread's (row, unit, half) bytes are loaded into registers as whole 16-byte
// chunks and the next item's loads are issued before the current item is
// computed.  x is staged to LDS by direct loads (in the shadow of the first
// item's weight loads); the items' partials go to LDS and thread (row, m)
// adds them in (unit, half) order (deterministic).  At m = 1 a fragment's
// eight weights u[i] * a + b are not formed: its dot is a * (u . x) + b *
// sum(x), with the sums of x over each aligned run of 8 staged in LDS beside
// x (18 VALU operations per 8 weights instead of 24; at m = 2 that form
// spills, and from m = 3 on its per-row terms outweigh the saved decode).
constexpr int kFragThreads = 512;
constexpr size_t kFragMaxLds = 160 * 1024;  // gfx950's LDS per workgroup
constexpr int kFragMaxM = 4;  // larger m takes gemv_kernel
constexpr int kFragLinMaxM = 1;

__host__ __device__ inline size_t frag_lds_bytes(int64_t k, int m, int64_t rows, int64_t units) {
  const size_t sums = m <= kFragLinMaxM ? (size_t)m * (k / 8) * 4 : 0;
  return (size_t)m * k * 4 + sums + ((size_t)rows * units * 2 + 1) * m * 4;
}

template <int TYPE, int M, typename OUT>
__global__ __launch_bounds__(kFragThreads) void gemv_frag_kernel(WView w, int64_t n, int64_t nrows_mem, int units,
                                                                 int rows, const float *__restrict__ x, int64_t ldx,
                                                                 OUT *__restrict__ y, int64_t ldy,
                                                                 const float *__restrict__ bias, int act) {
  using TT = bfrag::T<TYPE>;
  constexpr int kU = TT::kUnitK, kP = kU / 64;
  constexpr bool kLin = M <= kFragLinMaxM;
  constexpr bool kLinAdd = TYPE != Q8_0;  // Q8_0's Lin8 form has b = 0
  extern __shared__ __align__(16) uint8_t smem[];
  const int64_t k = (int64_t)units * kU;
  float *xs = reinterpret_cast<float *>(smem);            // [M][k]
  float *sx = xs + (size_t)M * k;                         // [M][k / 8] (kLin)
  float *red = sx + (kLin ? (size_t)M * (k >> 3) : 0);    // [units * 2 * rows + 1][M]
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int64_t r0 = (int64_t)blockIdx.x * rows;
  // a work item is (row, unit, half h): the decoders' lane-half split, so a
  // thread holds one half unit's bytes (item p = (2 u + h) * rows + row)
  const int nitems = rows * units * 2;

  auto load_item = [&](int p, typename TT::Raw &d) {
    p = p < nitems ? p : nitems - 1;  // clamped: every load unconditional, in bounds
    const int uh = p / rows;
    int64_t row = r0 + (p - uh * rows);
    row = row < nrows_mem ? row : nrows_mem - 1;
    const int64_t t = row >> 6;
    const int r = (int)(row & 63), u = uh >> 1, h = uh & 1;
    // every weight byte is read once: nontemporal loads for the k-quants and
    // Q8_0 (1-4 % faster on the decode shapes); the 32-element block types,
    // whose scale loads are 2- and 4-byte words, measured up to 8 % slower
    // with them
    constexpr bool kNT = !(TYPE == Q4_0 || TYPE == Q4_1 || TYPE == Q5_0 || TYPE == Q5_1);
    TT::template load_prep<kNT>(d, w, t, r, u, h);
    static_for<kP>([&]<int G>() { TT::template reload<G, kNT>(d, w, t, r, u, h); });
  };
  auto dot_item = [&](int p, const typename TT::Raw &d) {
    const bool valid = p < nitems;
    p = valid ? p : nitems - 1;
    const int uh = p / rows, u = uh >> 1, h = uh & 1;
    typename TT::Sc sc;
    TT::prep(d, sc, h);
    // chunk(S, h) = chunk(S, 0) + h * dh for every slice S of both chunk
    // maps: the item's x (and run sums) start at one 32-bit LDS offset and
    // each slice adds a constant
    constexpr int dh = TT::chunk(0, 1) - TT::chunk(0, 0);
    static_assert(TT::chunk(1, 1) - TT::chunk(1, 0) == dh && TT::chunk(2, 1) - TT::chunk(2, 0) == dh &&
                  TT::chunk(3, 1) - TT::chunk(3, 0) == dh);
    const int e0 = u * kU + 8 * dh * h;
    const float *xi = xs + e0;
    const float *si = sx + (e0 >> 3);
    const int kk = units * kU;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.f;
    static_for<kP>([&]<int G>() {
      // keeps the x reads of one step together with their use
      asm volatile("" ::: "memory");
      static_for<4>([&]<int S>() {
        constexpr int e = 64 * G + 8 * TT::chunk(S, 0);
        if constexpr (kLin) {
          const bfrag::Lin8 v = TT::template frag<G, S, bfrag::Lin8>(d, sc);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const float4 xa = *reinterpret_cast<const float4 *>(xi + m * kk + e);
            const float4 xb = *reinterpret_cast<const float4 *>(xi + m * kk + e + 4);
            float t = v.u[0] * xa.x;
            t = __builtin_fmaf(v.u[1], xa.y, t);
            t = __builtin_fmaf(v.u[2], xa.z, t);
            t = __builtin_fmaf(v.u[3], xa.w, t);
            t = __builtin_fmaf(v.u[4], xb.x, t);
            t = __builtin_fmaf(v.u[5], xb.y, t);
            t = __builtin_fmaf(v.u[6], xb.z, t);
            t = __builtin_fmaf(v.u[7], xb.w, t);
            float a = __builtin_fmaf(v.a, t, acc[m]);
            if constexpr (kLinAdd) a = __builtin_fmaf(v.b, si[m * (kk >> 3) + (e >> 3)], a);
            acc[m] = a;
          }
        } else {
          const bfrag::f32x8 v = TT::template frag<G, S, bfrag::f32x8>(d, sc);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            const float4 xa = *reinterpret_cast<const float4 *>(xi + m * kk + e);
            const float4 xb = *reinterpret_cast<const float4 *>(xi + m * kk + e + 4);
            float a = acc[m];
            a = __builtin_fmaf(v[0], xa.x, a);
            a = __builtin_fmaf(v[1], xa.y, a);
            a = __builtin_fmaf(v[2], xa.z, a);
            a = __builtin_fmaf(v[3], xa.w, a);
            a = __builtin_fmaf(v[4], xb.x, a);
            a = __builtin_fmaf(v[5], xb.y, a);
            a = __builtin_fmaf(v[6], xb.z, a);
            a = __builtin_fmaf(v[7], xb.w, a);
            acc[m] = a;
          }
        }
      });
    });
    // unconditional store (a clamped item writes the spare slot): a
    // conditional one lets the compiler sink the whole decode into the branch
    const int slot = valid ? p : nitems;
#pragma unroll
    for (int m = 0; m < M; ++m) red[slot * M + m] = acc[m];
  };

  // 1. x into LDS by direct loads (item j = row m's elements 256 c .. +255:
  //    one 1 KiB wave load) and the first item's weights.  For the k-quants x
  //    goes first and the weights once it has landed (as in the Q4_K kernel: x
  //    then does not queue behind the weight stream; Q5_K / Q6_K 3-7 % faster
  //    at m = 1 on the decode shapes); for the 32-element types the weights go
  //    first and one wait covers both (x first measured -2 .. +3 % there).
  constexpr bool kXFirst = TYPE == Q2_K || TYPE == Q3_K || TYPE == Q5_K || TYPE == Q6_K;
  typename TT::Raw a, b;
  if (!kXFirst) load_item(tid, a);
  {
    const uint32_t lbase = (uint32_t)(uintptr_t)(lds_void_t *)smem;
    const int items = (int)(M * (k >> 8));
    const int64_t per_row = k >> 8;
    for (int j = wave; j < items; j += kFragThreads / 64) {
      const int m = (int)(j / per_row);
      const int64_t c = j - (int64_t)m * per_row;
      dma16(x + m * ldx + c * 256 + 4 * lane, lbase + (uint32_t)j * 1024);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if constexpr (kLin && kLinAdd) {
    // sums of x over each aligned run of 8 (row m's run j at m * k / 8 + j)
    const int nrun = (int)(M * (k >> 3));
    for (int c = tid; c < nrun; c += kFragThreads) {
      const float4 xa = *reinterpret_cast<const float4 *>(xs + 8 * (int64_t)c);
      const float4 xb = *reinterpret_cast<const float4 *>(xs + 8 * (int64_t)c + 4);
      sx[c] = ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
    }
    __syncthreads();
  }
  if (kXFirst) load_item(tid, a);

  // 2. items, the next one's loads in flight while the current one computes
  for (int p = tid;; p += 2 * kFragThreads) {
    load_item(p + kFragThreads, b);
    dot_item(p, a);
    if (p + kFragThreads >= nitems) break;
    load_item(p + 2 * kFragThreads, a);
    dot_item(p + kFragThreads, b);
    if (p + 2 * kFragThreads >= nitems) break;
  }
  __syncthreads();

  // 3. thread (row, m) adds its row's partials in (unit, half) order
  for (int t = tid; t < rows * M; t += kFragThreads) {
    const int m = t / rows, rl = t - m * rows;
    const int64_t row = r0 + rl;
    if (row >= n) continue;
    float acc = 0.f;
    for (int uh = 0; uh < 2 * units; ++uh) acc += red[(uh * rows + rl) * M + m];
    if (bias) acc += bias[row];
    store1<OUT>(y + m * ldy + row, apply_act(acc, act_at(act, row)));
  }
}

// Rows per workgroup of the streaming kernel (0: use gemv_kernel): one
// workgroup per CU; x and the partials must fit the LDS.
static int frag_rows(int type, int64_t n, int64_t k, int64_t m, int cus) {
  const int64_t unit = type == Q8_0 ? 128 : 256;
  if (type == Q4_K || k % 256 != 0 || m > kFragMaxM) return 0;
  int64_t rows = (n + cus - 1) / cus;
  if (rows < 1) rows = 1;
  while (rows > 8 && frag_lds_bytes(k, (int)m, rows, k / unit) > kFragMaxLds) rows = (rows + 1) / 2;
  if (frag_lds_bytes(k, (int)m, rows, k / unit) > kFragMaxLds) return 0;
  return (int)rows;
}

template <int TYPE, int M, typename OUT>
static void launch_gemv_frag(const WView &w, int64_t n, int64_t k, const float *x, int64_t ldx, OUT *y, int64_t ldy,
                             const float *bias, int act, int rows, hipStream_t stream) {
  constexpr int64_t unit = bfrag::T<TYPE>::kUnitK;
  const int units = (int)(k / unit);
  const int64_t wgs = (n + rows - 1) / rows;
  const int64_t nrows_mem = ((n + kRowTile - 1) / kRowTile) * kRowTile;
  hipLaunchKernelGGL((gemv_frag_kernel<TYPE, M, OUT>), dim3((unsigned)wgs), dim3(kFragThreads),
                     frag_lds_bytes(k, M, rows, units), stream, w, n, nrows_mem, units, rows, x, ldx, y, ldy, bias,
                     act);
}

template <int TYPE, typename OUT>
static void launch_gemv_frag_m(const WView &w, int64_t n, int64_t k, const float *x, int64_t m, int64_t ldx, OUT *y,
                               int64_t ldy, const float *bias, int act, int rows, hipStream_t stream) {
  switch (m) {
    case 1: launch_gemv_frag<TYPE, 1, OUT>(w, n, k, x, ldx, y, ldy, bias, act, rows, stream); break;
    case 2: launch_gemv_frag<TYPE, 2, OUT>(w, n, k, x, ldx, y, ldy, bias, act, rows, stream); break;
    case 3: launch_gemv_frag<TYPE, 3, OUT>(w, n, k, x, ldx, y, ldy, bias, act, rows, stream); break;
    default: launch_gemv_frag<TYPE, 4, OUT>(w, n, k, x, ldx, y, ldy, bias, act, rows, stream); break;
  }
}

// Rows per workgroup of the Q4_K path (0: use the generic kernel): one
// workgroup per CU, fewer rows when the LDS would not hold them.
static int q4k_rows(int64_t n, int64_t nb, int64_t m, int cus) {
  int64_t rows = (n + cus - 1) / cus;
  if (rows < 1) rows = 1;
  while (rows > 8 && q4k_lds_bytes(nb, (int)m, rows, 4) > kQ4kMaxLds) rows = (rows + 1) / 2;
  if (q4k_lds_bytes(nb, (int)m, rows, 4) > kQ4kMaxLds) return 0;
  return (int)rows;
}

// When a workgroup has at most one pair per thread, the single-slot instance
// runs it (no second register slot, no Q8_K prefetch: far fewer VGPRs).
static bool q4k_one_slot(int64_t nb, int rows) { return (int64_t)rows * nb <= kQ4kThreads; }

template <int M, typename XT, typename OUT>
static void launch_gemv_q4k(const WView &w, int64_t n, int64_t k, const XT *x, int64_t ldx, OUT *y, int64_t ldy,
                            const float *bias, int act, int cus, hipStream_t stream) {
  const int64_t nb = k / 256;
  const int rows = q4k_rows(n, nb, M, cus);
  const bool one = q4k_one_slot(nb, rows);
  const int64_t wgs = (n + rows - 1) / rows;
  const int64_t nrows_mem = ((n + kRowTile - 1) / kRowTile) * kRowTile;
  const size_t lds = q4k_lds_bytes(nb, M, rows, __is_same(XT, Q8kX) ? -1 : (int)sizeof(XT));
  if (one)
    hipLaunchKernelGGL((gemv_q4k_kernel<M, XT, OUT, true>), dim3((unsigned)wgs), dim3(kQ4kThreads), lds, stream, w,
                       n, nrows_mem, (int)nb, rows, x, ldx, y, ldy, bias, act);
  else
    hipLaunchKernelGGL((gemv_q4k_kernel<M, XT, OUT, false>), dim3((unsigned)wgs), dim3(kQ4kThreads), lds, stream, w,
                       n, nrows_mem, (int)nb, rows, x, ldx, y, ldy, bias, act);
}

static int pick_ksplit(int64_t ntiles, int64_t k) {
  const int64_t units = k >> 5;
  int64_t ks = 1;
  // aim for >= 2 workgroups per CU on 256 CUs, with >= 2 units per wave
  while (ntiles * ks < 512 && units / (ks * 2) >= 2 * kGemvWaves) ks *= 2;
  return (int)ks;
}

size_t gemv_scratch_bytes(int type, int64_t m, int64_t n, int64_t k, int cus) {
  if (type == Q4_K && q4k_rows(n, k / 256, m, cus)) return 0;
  if (frag_rows(type, n, k, m, cus)) return 0;
  const int64_t ntiles = (n + kRowTile - 1) / kRowTile;
  const int ks = pick_ksplit(ntiles, k);
  if (ks == 1) return 0;
  return (size_t)ks * m * ntiles * kRowTile * sizeof(float);
}

template <int TYPE, int M, typename OUT>
static void launch_gemv_t(const WView &w, int64_t n, int64_t k, const float *x, int64_t ldx, OUT *y,
                          int64_t ldy, const float *bias, int act, float *partial, hipStream_t stream) {
  const int64_t ntiles = (n + kRowTile - 1) / kRowTile;
  const int ks = partial ? pick_ksplit(ntiles, k) : 1;  // no partials buffer: whole K per workgroup
  const int64_t npad = ntiles * kRowTile;
  hipLaunchKernelGGL((gemv_kernel<TYPE, M, OUT>), dim3((unsigned)ntiles, ks), dim3(kGemvWaves * 64), 0,
                     stream, w, n, k, x, ldx, y, ldy, bias, act, partial, ks, npad);
  if (ks > 1) {
    const int64_t total = (int64_t)M * n;
    hipLaunchKernelGGL(gemv_reduce_kernel<OUT>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, partial, ks, (int64_t)M, n, npad, y, ldy, bias, act);
  }
}

template <typename XT, typename OUT>
static void launch_gemv_q4k_m(const WView &w, int64_t n, int64_t k, const XT *x, int64_t m, int64_t ldx, OUT *y,
                              int64_t ldy, const float *bias, int act, int cus, hipStream_t stream) {
  switch (m) {
    case 1: launch_gemv_q4k<1, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    case 2: launch_gemv_q4k<2, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    case 3: launch_gemv_q4k<3, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    case 4: launch_gemv_q4k<4, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    case 5: launch_gemv_q4k<5, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    case 6: launch_gemv_q4k<6, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    case 7: launch_gemv_q4k<7, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
    default: launch_gemv_q4k<8, XT, OUT>(w, n, k, x, ldx, y, ldy, bias, act, cus, stream); return;
  }
}

// x -> MQ_X_Q8K blocks: one 256-element item (row, super-block) per 16-lane
// group, 32 per workgroup, by the Q4_K GEMV's own quantization of its staged
// x (q8k_quantize16), so a GEMV on the blocks equals one on x bit for bit.
template <typename XT>
__global__ __launch_bounds__(512) void quantize_x_q8k_kernel(const XT *__restrict__ x, int64_t m, int64_t nb,
                                                             int64_t ldx, uint8_t *__restrict__ dst) {
  const int tid = threadIdx.x, l16 = tid & 15;
  const int64_t items = m * nb;
  const int64_t j0 = (int64_t)blockIdx.x * 32 + (tid >> 4);
  const bool valid = j0 < items;
  const int64_t j = valid ? j0 : items - 1;  // every lane joins the group's cross-lane steps
  const int64_t row = j / nb, sb = j - row * nb;
  const XT *src = x + row * ldx + sb * 256 + 16 * l16;
  float v[16];
  if constexpr (__is_same(XT, float)) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 t = reinterpret_cast<const float4 *>(src)[c];
      v[4 * c] = t.x;
      v[4 * c + 1] = t.y;
      v[4 * c + 2] = t.z;
      v[4 * c + 3] = t.w;
    }
  } else {
    // bf16 -> f32 is exact: the 16 bits become the high half
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint4 t = reinterpret_cast<const uint4 *>(src)[c];
      const uint32_t wd[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[8 * c + 2 * i] = __uint_as_float(wd[i] << 16);
        v[8 * c + 2 * i + 1] = __uint_as_float(wd[i] & 0xFFFF0000u);
      }
    }
  }
  uint32_t packed[4];
  int qsum;
  const float d = q8k_quantize16(v, l16, tid & 63, packed, qsum);
  if (!valid) return;
  uint8_t *blk = dst + j * kQ8kXBytes;
  *reinterpret_cast<uint4 *>(blk + 16 * l16) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  if ((l16 & 1) == 0) *reinterpret_cast<int32_t *>(blk + 256 + 2 * l16) = qsum;
  if (l16 == 0) *reinterpret_cast<float *>(blk + 288) = d;
  if (l16 >= 1 && l16 <= 3) *reinterpret_cast<uint32_t *>(blk + 288 + 4 * l16) = 0u;  // the 12 pad bytes
}

hipError_t launch_quantize_x_q8k(const void *x, int x_type, int64_t m, int64_t k, int64_t ldx, void *dst,
                                 hipStream_t stream) {
  const int64_t nb = k / 256, items = m * nb;
  if (items <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((items + 31) / 32);
  if (x_type == F32)
    hipLaunchKernelGGL((quantize_x_q8k_kernel<float>), dim3(grid), dim3(512), 0, stream,
                       static_cast<const float *>(x), m, nb, ldx, static_cast<uint8_t *>(dst));
  else
    hipLaunchKernelGGL((quantize_x_q8k_kernel<__bf16>), dim3(grid), dim3(512), 0, stream,
                       static_cast<const __bf16 *>(x), m, nb, ldx, static_cast<uint8_t *>(dst));
  return hipGetLastError();
}

template <int TYPE, typename OUT>
static void launch_gemv_m(const WView &w, int64_t n, int64_t k, const float *x, int64_t m, int64_t ldx,
                          OUT *y, int64_t ldy, const float *bias, int act, float *partial, hipStream_t stream) {
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

// The Q4_K kernel's direct x loads need 16-byte aligned rows of x.
static bool q4k_x_aligned(const void *x, int x_type, int64_t ldx) {
  const int64_t es = x_type == F32 ? 4 : 2;
  return (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (ldx * es) % 16 == 0;
}

bool gemv_reads_x_in_place(int type, int64_t m, int64_t n, int64_t k, const void *x, int x_type, int64_t ldx,
                           int cus) {
  if (x_type == MQ_X_Q8K) return gemv_takes_x_q8k(type, m, n, k, cus);
  return type == Q4_K && m >= 1 && m <= kGemvMaxM && q4k_rows(n, k / 256, m, cus) > 0 &&
         q4k_x_aligned(x, x_type, ldx);
}

bool gemv_takes_x_q8k(int type, int64_t m, int64_t n, int64_t k, int cus) {
  return type == Q4_K && m >= 1 && m <= kGemvMaxM && k % 256 == 0 && q4k_rows(n, k / 256, m, cus) > 0;
}

hipError_t launch_gemv(int type, const WView &w, int64_t n, int64_t k, const void *x, int x_type, int64_t m,
                       int64_t ldx, void *y, int y_type, int64_t ldy, const float *bias, int act,
                       float *partial, int cus, hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  if (x_type == MQ_X_Q8K) {  // the caller checked: Q4_K, m <= 8, q4k rows, aligned contiguous blocks
    const Q8kX *xq = static_cast<const Q8kX *>(x);
    if (y_type == F32)
      launch_gemv_q4k_m<Q8kX, float>(w, n, k, xq, m, ldx, static_cast<float *>(y), ldy, bias, act, cus, stream);
    else
      launch_gemv_q4k_m<Q8kX, __bf16>(w, n, k, xq, m, ldx, static_cast<__bf16 *>(y), ldy, bias, act, cus, stream);
    return hipGetLastError();
  }
  if (gemv_reads_x_in_place(type, m, n, k, x, x_type, ldx, cus)) {
    if (x_type == F32) {
      if (y_type == F32)
        launch_gemv_q4k_m<float, float>(w, n, k, static_cast<const float *>(x), m, ldx, static_cast<float *>(y),
                                        ldy, bias, act, cus, stream);
      else
        launch_gemv_q4k_m<float, __bf16>(w, n, k, static_cast<const float *>(x), m, ldx,
                                         static_cast<__bf16 *>(y), ldy, bias, act, cus, stream);
    } else {
      if (y_type == F32)
        launch_gemv_q4k_m<__bf16, float>(w, n, k, static_cast<const __bf16 *>(x), m, ldx,
                                         static_cast<float *>(y), ldy, bias, act, cus, stream);
      else
        launch_gemv_q4k_m<__bf16, __bf16>(w, n, k, static_cast<const __bf16 *>(x), m, ldx,
                                          static_cast<__bf16 *>(y), ldy, bias, act, cus, stream);
    }
    return hipGetLastError();
  }
  if (x_type != F32) return hipErrorInvalidValue;  // the other kernels read f32 x
  const float *xf = static_cast<const float *>(x);
  const int frows = frag_rows(type, n, k, m, cus);
  if (frows && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % 4 == 0) {
    bool ok = dispatch_type(type, [&]<int T>() {
      if constexpr (T != Q4_K) {
        if (y_type == F32)
          launch_gemv_frag_m<T, float>(w, n, k, xf, m, ldx, static_cast<float *>(y), ldy, bias, act, frows, stream);
        else
          launch_gemv_frag_m<T, __bf16>(w, n, k, xf, m, ldx, static_cast<__bf16 *>(y), ldy, bias, act, frows,
                                        stream);
      }
    });
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
  }
  bool ok = dispatch_type(type, [&]<int T>() {
    if (y_type == F32)
      launch_gemv_m<T, float>(w, n, k, xf, m, ldx, static_cast<float *>(y), ldy, bias, act, partial, stream);
    else
      launch_gemv_m<T, __bf16>(w, n, k, xf, m, ldx, static_cast<__bf16 *>(y), ldy, bias, act, partial, stream);
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mq
