// mq_gemm.hip — fused dequant -> bf16 MFMA GEMM for large-M quantized linears
// (FLUX / Qwen-Image token projections): y[m, n] = act(x[m, :] . W[n, :] + b[n]).
//
// Tiling for gfx950 (256 CUs in 8 XCDs, 64-wide waves, 160 KiB LDS per CU):
//   * workgroup = 4 waves, block tile 256 (m) x 256 (n), K step 64;
//   * wave w owns weight tile nt*4 + w (64 output features) for all 256 rows,
//     so every weight element is decoded exactly once per block tile and goes
//     straight from registers into the MFMA B operand (no LDS round trip);
//   * the bf16 activation tile 256 x 64 is staged through LDS (double
//     buffered, XOR-swizzled 16-byte chunks, one barrier per K step) and read
//     by all four waves;
//   * v_mfma_f32_32x32x16_bf16: per wave 8 (m) x 2 (n) accumulator tiles,
//     256 f32 accumulators per lane;
//   * blockIdx -> tile mapping gives each XCD a contiguous run of tiles that
//     share the same activation panel in its L2.
// Within a K step of 64, lane half h (lane / 32) supplies K elements
// {16h..16h+15} u {32+16h..32+16h+15} (four runs of 8).  MFMA slice s takes
// run c_s = (s/2)*4 + 2h + (s%2) of eight elements; the A operand reads the
// same run from LDS, so the K order inside a step is a permutation shared by
// both operands.
#include <utility>

#include "mq_bfrag.h"
#include "mq_kernels.h"

namespace mq {

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kGemmThreads = 256;

__device__ __forceinline__ bf16x8 to_bf16x8(const float v[8]) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)v[i];
  return r;
}

template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f.template operator()<I>(), ...);
}
// Calls f.template operator()<I>() for I = 0 .. N-1 (compile-time step index).
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

template <typename OUT>
__device__ __forceinline__ void store_out(OUT *p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float *p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<__bf16>(__bf16 *p, float v) { *p = (__bf16)v; }

template <int TYPE, typename OUT>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_kernel(
    WView w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *__restrict__ a, int64_t m,
    int64_t lda, OUT *__restrict__ y, int64_t ldy, const float *__restrict__ bias, int act, int tiles_m,
    int tiles_n) {
  constexpr TypeInfo ti = type_info(TYPE);
  __shared__ uint4 lds[2][kBM * kBK / 8];  // 2 x 32 KiB, row = 8 chunks of 16 B

  // ---- XCD-aware tile order: workgroup i runs on XCD i % 8; give each XCD a
  // contiguous range of tiles (row-major over n, so concurrent tiles on one
  // XCD share the activation panel).
  const int total = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int base = total >> 3, extra = total & 7;
  const int v = xcd * base + (xcd < extra ? xcd : extra) + local;
  const int mt = v / tiles_n, nt = v - mt * tiles_n;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t m0 = (int64_t)mt * kBM;
  const int64_t wt_raw = (int64_t)nt * (kBN / kRowTile) + wave;
  const int64_t wt = wt_raw < ntiles_w ? wt_raw : ntiles_w - 1;  // keep reads in bounds
  const int64_t ksteps = (k + kBK - 1) / kBK;

  f32x16 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // A staging: thread -> chunk c (8 bf16) of rows ar + 32*i.
  const int ac = tid & 7, ar = tid >> 3;
  uint4 areg[8];
  auto load_a = [&](int64_t ks) {
    const int64_t kc = ks * kBK + ac * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t row = m0 + ar + 32 * i;
      if (row < m)
        areg[i] = *reinterpret_cast<const uint4 *>(a + row * lda + kc);
      else
        areg[i] = make_uint4(0, 0, 0, 0);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = ar + 32 * i;
      lds[buf][row * 8 + (ac ^ (row & 7))] = areg[i];
    }
  };

  load_a(0);
  store_a(0);
  __syncthreads();

  for (int64_t ks = 0; ks < ksteps; ++ks) {
    const int buf = (int)(ks & 1);
    if (ks + 1 < ksteps) load_a(ks + 1);

    // B operands: 2 rows (l32, l32 + 32) x 4 runs of 8 K elements.
    bf16x8 bfrag[2][4];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int off = (s >> 1) * 32 + 16 * h + (s & 1) * 8;
        const int64_t kk = ks * kBK + off;
        float vals[8];
        if (kk < k) {
          const int64_t b = kk / ti.bs;
          decode8<TYPE>(w, wt, l32 + 32 * nb, b, (int)(kk - b * ti.bs), vals);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) vals[i] = 0.f;
        }
        bfrag[nb][s] = to_bf16x8(vals);
      }
    }

#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int chunk = (s >> 1) * 4 + 2 * h + (s & 1);
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const int row = mb * 32 + l32;
        const uint4 raw = lds[buf][row * 8 + (chunk ^ (row & 7))];
        bf16x8 afrag;
        __builtin_memcpy(&afrag, &raw, 16);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afrag, bfrag[nb][s], acc[mb][nb], 0, 0, 0);
      }
    }

    if (ks + 1 < ksteps) store_a(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds column l32 of each 32x32 tile, rows
  // 8*(e/4) + 4*h + (e%4).
  if (wt_raw >= ntiles_w) return;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = wt_raw * kRowTile + nb * 32 + l32;
    if (col >= n) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + mb * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < m) store_out<OUT>(y + row * ldy + col, apply_act(acc[mb][nb][e] + bv, act));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fast path (k % 256 == 0): per-type B decoders from mq_bfrag.h.
//   * each lane keeps the packed bytes of its two weight rows for the current
//     K unit (256 weights; 128 for Q8_0) and loads the next unit's while the
//     current one is consumed, so weight loads have a whole unit of MFMA work
//     to land;
//   * scales are unpacked once per unit, nibbles are masked in place and
//     turned into f32 with v_cvt_f32_ubyte, one fma applies scale and min,
//     v_cvt_pk_bf16_f32 packs the fragment — about 2.75 VALU ops per weight,
//     each weight decoded once per 256-row block tile;
//   * the activation tile goes global -> VGPR -> LDS one K step ahead, LDS
//     double buffered, XOR-swizzled, one barrier per step.
template <int TYPE, typename OUT>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_fast_kernel(
    WView w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *__restrict__ a, int64_t m, int64_t lda,
    OUT *__restrict__ y, int64_t ldy, const float *__restrict__ bias, int act, int tiles_m, int tiles_n) {
  using TT = bfrag::T<TYPE>;
  constexpr int kSteps = TT::kUnitK / kBK;
  __shared__ uint4 lds[2][kBM * kBK / 8];

  const int total = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int base = total >> 3, extra = total & 7;
  const int v = xcd * base + (xcd < extra ? xcd : extra) + local;
  const int mt = v / tiles_n, nt = v - mt * tiles_n;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t m0 = (int64_t)mt * kBM;
  const int64_t wt_raw = (int64_t)nt * (kBN / kRowTile) + wave;
  const int64_t wt = wt_raw < ntiles_w ? wt_raw : ntiles_w - 1;  // keep reads in bounds
  const int64_t units = k / TT::kUnitK;

  f32x16 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // A staging: thread -> chunk ac (8 bf16) of rows ar + 32 i; rows past m
  // read row m-1 (finite, never stored).
  const int ac = tid & 7, ar = tid >> 3;
  const __bf16 *arow[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t row = m0 + ar + 32 * i;
    row = row < m ? row : m - 1;
    arow[i] = a + row * lda + ac * 8;
  }
  uint4 a0, a1, a2, a3, a4, a5, a6, a7;
#define MQ_LOAD_A(ks)                                                           \
  do {                                                                          \
    const int64_t _o = (ks) * kBK;                                              \
    a0 = *reinterpret_cast<const uint4 *>(arow[0] + _o);                        \
    a1 = *reinterpret_cast<const uint4 *>(arow[1] + _o);                        \
    a2 = *reinterpret_cast<const uint4 *>(arow[2] + _o);                        \
    a3 = *reinterpret_cast<const uint4 *>(arow[3] + _o);                        \
    a4 = *reinterpret_cast<const uint4 *>(arow[4] + _o);                        \
    a5 = *reinterpret_cast<const uint4 *>(arow[5] + _o);                        \
    a6 = *reinterpret_cast<const uint4 *>(arow[6] + _o);                        \
    a7 = *reinterpret_cast<const uint4 *>(arow[7] + _o);                        \
  } while (0)
#define MQ_STORE_A(buf)                                                         \
  do {                                                                          \
    uint4 *_l = lds[buf];                                                       \
    _l[(ar + 0) * 8 + (ac ^ ((ar + 0) & 7))] = a0;                              \
    _l[(ar + 32) * 8 + (ac ^ ((ar + 32) & 7))] = a1;                            \
    _l[(ar + 64) * 8 + (ac ^ ((ar + 64) & 7))] = a2;                            \
    _l[(ar + 96) * 8 + (ac ^ ((ar + 96) & 7))] = a3;                            \
    _l[(ar + 128) * 8 + (ac ^ ((ar + 128) & 7))] = a4;                          \
    _l[(ar + 160) * 8 + (ac ^ ((ar + 160) & 7))] = a5;                          \
    _l[(ar + 192) * 8 + (ac ^ ((ar + 192) & 7))] = a6;                          \
    _l[(ar + 224) * 8 + (ac ^ ((ar + 224) & 7))] = a7;                          \
  } while (0)

  typename TT::Raw cur[2], nxt[2];
  TT::load(cur[0], w, wt, l32, 0, h);
  TT::load(cur[1], w, wt, l32 + 32, 0, h);
  MQ_LOAD_A(0);
  MQ_STORE_A(0);
  __syncthreads();

  for (int64_t u = 0; u < units; ++u) {
    typename TT::Sc sc[2];
    TT::prep(cur[0], sc[0], h);
    TT::prep(cur[1], sc[1], h);
    static_for<kSteps>([&]<int G>() {
      const int64_t ks = u * kSteps + G;
      constexpr int buf = G & 1;
      const bool more = ks + 1 < units * kSteps;
      if (more) MQ_LOAD_A(ks + 1);
      if constexpr (G == 0) {
        if (u + 1 < units) {
          TT::load(nxt[0], w, wt, l32, u + 1, h);
          TT::load(nxt[1], w, wt, l32 + 32, u + 1, h);
        }
      }
      bf16x8 bfr[2][4];
      TT::template decode<G>(cur[0], sc[0], bfr[0]);
      TT::template decode<G>(cur[1], sc[1], bfr[1]);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int chunk = TT::chunk(s, h);
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) {
          const int row = mb * 32 + l32;
          const uint4 raw = lds[buf][row * 8 + (chunk ^ (row & 7))];
          bf16x8 afrag;
          __builtin_memcpy(&afrag, &raw, 16);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afrag, bfr[nb][s], acc[mb][nb], 0, 0, 0);
        }
      }
      if (more) MQ_STORE_A(buf ^ 1);
      __syncthreads();
    });
    cur[0] = nxt[0];
    cur[1] = nxt[1];
  }

  if (wt_raw >= ntiles_w) return;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = wt_raw * kRowTile + nb * 32 + l32;
    if (col >= n) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + mb * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < m) store_out<OUT>(y + row * ldy + col, apply_act(acc[mb][nb][e] + bv, act));
      }
    }
  }
}

hipError_t launch_gemm(int type, const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a,
                       int64_t m, int64_t lda, void *y, int y_type, int64_t ldy, const float *bias, int act,
                       hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  const int tiles_m = (int)((m + kBM - 1) / kBM);
  const int tiles_n = (int)((n + kBN - 1) / kBN);
  const int grid = tiles_m * tiles_n;
  const bool fast = (k % 256) == 0 && lda % 8 == 0;
  bool ok = dispatch_type(type, [&]<int T>() {
    if (fast) {
      if (y_type == F32)
        hipLaunchKernelGGL((gemm_fast_kernel<T, float>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k,
                           ntiles_w, a, m, lda, static_cast<float *>(y), ldy, bias, act, tiles_m, tiles_n);
      else
        hipLaunchKernelGGL((gemm_fast_kernel<T, __bf16>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k,
                           ntiles_w, a, m, lda, static_cast<__bf16 *>(y), ldy, bias, act, tiles_m, tiles_n);
      return;
    }
    if (y_type == F32)
      hipLaunchKernelGGL((gemm_kernel<T, float>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k,
                         ntiles_w, a, m, lda, static_cast<float *>(y), ldy, bias, act, tiles_m, tiles_n);
    else
      hipLaunchKernelGGL((gemm_kernel<T, __bf16>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k,
                         ntiles_w, a, m, lda, static_cast<__bf16 *>(y), ldy, bias, act, tiles_m, tiles_n);
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace mq
