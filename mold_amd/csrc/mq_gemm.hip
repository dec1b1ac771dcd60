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
// Fast path (k % 256 == 0): 256 x 256 block tile, 8 waves (two per SIMD, so
// one wave's dequant VALU work co-issues with the other's MFMAs), K step 64.
//   * A (bf16 activations): 3-slot LDS ring filled by direct global->LDS
//     loads (global_load_lds_dwordx4, inline asm) two K steps ahead;
//   * B (weights): wave w decodes rows 32w..32w+31 of the block's 256 weight
//     rows for the NEXT K step (per-type decoders, mq_bfrag.h) and writes the
//     bf16 tile to a 2-slot LDS ring, so every weight is decoded once per
//     block tile; its packed bytes are reloaded into registers for the next
//     unit one step after their last use;
//   * MFMA: wave (wm = w&1, wn = w>>1) owns output rows 128wm.. and columns
//     64wn..: 4 x 2 tiles of v_mfma_f32_32x32x16_bf16 per 16-K slice;
//   * LDS rows are 128 B (64 bf16); 16-byte chunk c of row r sits in slot
//     c ^ ((r >> 1) & 7), so the 16 lanes of a ds_read_b128 quarter (16
//     consecutive rows) cover all 64 banks;
//   * one barrier per step: s_waitcnt vmcnt(4) (the only younger memory ops
//     are this step's four A loads) lgkmcnt(0), then s_barrier.
constexpr int kAStages = 3;
constexpr int MQ_ACT_NONE_ = 0;  // mq_act MQ_ACT_NONE
constexpr int kFastThreads = 512;
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void step_barrier(bool more) {
  if (more)
    asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One 1 KiB direct global->LDS load: lane i's 16 bytes from g land at LDS byte
// address lds + 16 i.  Issued as inline asm so that the compiler does not see
// an LDS write it cannot tell apart from the slot being read (it would wait
// for every outstanding load before each LDS access, which turns the two-step
// A prefetch into none); the kernel orders these loads with its own
// s_waitcnt at the step barrier.  The compiler's waits for its own loads then
// count fewer outstanding loads than there are, so they can only wait longer
// than needed, never shorter.  M0 carries the LDS address (no other code in
// these kernels uses M0); s_nop: one wait state between writing M0 and the
// LDS-DMA instruction that reads it.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ int lds_slot(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }

template <int TYPE, typename OUT>
__global__ __launch_bounds__(kFastThreads, 1) void gemm_fast_kernel(
    WView w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *__restrict__ a, int64_t m, int64_t lda,
    OUT *__restrict__ y, int64_t ldy, const float *__restrict__ bias, int act, int tiles_m, int tiles_n) {
  using TT = bfrag::T<TYPE>;
  constexpr int kSteps = TT::kUnitK / kBK;
  __shared__ uint4 lds_a[kAStages][kBM * kBK / 8];
  __shared__ uint4 lds_b[2][kBN * kBK / 8];

  const int total = tiles_m * tiles_n;
  const int bid = blockIdx.x;
  const int xcd = bid & 7, local = bid >> 3;
  const int base = total >> 3, extra = total & 7;
  const int v = xcd * base + (xcd < extra ? xcd : extra) + local;
  const int mt = v / tiles_n, nt = v - mt * tiles_n;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int wm = wave & 1, wn = wave >> 1;
  const int phase = (wave >> 2) & 1;
  const int swz = (l32 >> 1) & 7;  // LDS swizzle key of every row this lane touches
  const int64_t m0 = (int64_t)mt * kBM;
  const int64_t units = k / TT::kUnitK;
  const int64_t ksteps = units * kSteps;

  // decoder role: weight tile nt*4 + wave/2, row (wave&1)*32 + l32 of it
  const int64_t dt_raw = (int64_t)nt * (kBN / kRowTile) + (wave >> 1);
  const int64_t dt = dt_raw < ntiles_w ? dt_raw : ntiles_w - 1;  // keep reads in bounds
  const int drow = (wave & 1) * 32 + l32;
  const int brow = 32 * wave + l32;  // its row in the LDS B tile

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // A DMA: load i (0..3) of wave w fills LDS rows 8(4w+i)..+7 (1 KiB); lane
  // j fetches row 8(4w+i) + j/8, logical chunk (j&7) ^ ((row >> 1) & 7).
  // Rows past m read row m-1 (finite, never stored).
  int64_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 8 * (4 * wave + i) + (lane >> 3);
    int64_t row = m0 + r;
    row = row < m ? row : m - 1;
    aoff[i] = row * lda + (((lane & 7) ^ ((r >> 1) & 7)) * 8);
  }
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto dma_a = [&](uint4 *slot, int64_t ks) {
    const uint32_t dst = (uint32_t)(uintptr_t)(lds_void_t *)(slot + (32 * wave_u) * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(a + aoff[i] + ks * kBK, dst + 1024 * i);
  };

  typename TT::Raw raw;
  typename TT::Sc sc;
  auto decode_to = [&]<int G>(uint4 *__restrict__ dst) {
    static_for<4>([&]<int S>() {
      const bf16x8 f = TT::template frag<G, S>(raw, sc);
      uint4 q;
      __builtin_memcpy(&q, &f, 16);
      dst[brow * 8 + (TT::chunk(S, h) ^ swz)] = q;
    });
  };

  // prologue: unit 0's weight bytes, A(0), A(1); decode step 0
  TT::load_prep(raw, w, dt, drow, 0, h);
  static_for<kSteps>([&]<int G>() { TT::template reload<G>(raw, w, dt, drow, 0, h); });
  dma_a(lds_a[0], 0);
  if (ksteps > 1) dma_a(lds_a[1], 1);
  if (ksteps > 1)
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  TT::prep(raw, sc, h);
  decode_to.template operator()<0>(lds_b[0]);
  step_barrier(ksteps > 1);

  for (int64_t u = 0; u < units; ++u) {
    const bool next_unit = u + 1 < units;
    static_for<kSteps>([&]<int G>() {
      const int64_t ks = u * kSteps + G;
      // the pieces decoded last iteration (step G of unit u) are free: fetch
      // unit u+1's; unit u's scales were unpacked last iteration too.
      // Loads are issued unconditionally (the last unit re-reads itself, the
      // last two steps re-fetch the final A step into a slot nobody reads), so
      // the number of loads younger than any given one is the same on every
      // path and the compiler's wait counts stay exact.
      const int64_t un = next_unit ? u + 1 : u;
      TT::template reload<G>(raw, w, dt, drow, un, h);
      if constexpr (G == 0) TT::load_prep(raw, w, dt, drow, un, h);
      const bool more = ks + 2 < ksteps;
      const int64_t ka = more ? ks + 2 : ksteps - 1;
      // The step's four LDS slots (A being filled, A being read, B being
      // decoded into, B being read) are distinct, which the restrict
      // qualifiers tell the compiler.
      auto body = [&](uint4 *__restrict__ a_dst, const uint4 *__restrict__ a_src, uint4 *__restrict__ b_dst,
                      const uint4 *__restrict__ b_src) {
      dma_a(a_dst, ka);

      // decode the next step's weights into the other B slot
      auto decode_next = [&]() {
        if constexpr (G + 1 < kSteps) {
          decode_to.template operator()<G + 1>(b_dst);
        } else {
          if (next_unit) {
            TT::prep(raw, sc, h);
            decode_to.template operator()<0>(b_dst);
          }
        }
      };
      auto mfma_step = [&]() {
        // Every fragment row this lane reads has (row >> 1) & 7 == swz, so the
        // slot of slice S is fixed per lane and the 32-row tile offsets are
        // immediates: one address register per slice.
        const char *abase = reinterpret_cast<const char *>(a_src) + (wm * 128 + l32) * 128;
        const char *bbase = reinterpret_cast<const char *>(b_src) + (wn * 64 + l32) * 128;
        bf16x8 fr[2][6];  // [slot][B nb=0,1 | A mb=0..3]
        auto read_frags = [&](bf16x8 *dst, int S) {
          const int off = (TT::chunk(S, h) ^ swz) * 16;
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) dst[nb] = *reinterpret_cast<const bf16x8 *>(bbase + off + nb * 4096);
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) dst[2 + mb] = *reinterpret_cast<const bf16x8 *>(abase + off + mb * 4096);
        };
        read_frags(fr[0], 0);
        static_for<4>([&]<int S>() {
          if constexpr (S < 3) read_frags(fr[(S + 1) & 1], S + 1);
#pragma unroll
          for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
              acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[S & 1][2 + mb], fr[S & 1][nb], acc[mb][nb], 0,
                                                                    0, 0);
          // interleave: the next slice's six fragment reads between this
          // slice's eight MFMAs
          if constexpr (S < 3) {
            static_for<6>([&]<int I>() {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            });
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          } else {
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
          }
        });
      };
      // The two waves sharing a SIMD (w and w+4) run the step's halves in
      // opposite order, so one decodes (VALU) while the other runs MFMAs.
      if (phase) {
        decode_next();
        __builtin_amdgcn_sched_barrier(0);
        mfma_step();
      } else {
        mfma_step();
        __builtin_amdgcn_sched_barrier(0);
        decode_next();
      }
      };
      body(lds_a[(ks + 2) % kAStages], lds_a[ks % kAStages], lds_b[(ks + 1) & 1], lds_b[ks & 1]);
      step_barrier(more);
    });
  }

  const int64_t wt_out = (int64_t)nt * (kBN / kRowTile) + wn;
  if (wt_out >= ntiles_w) return;
  const int64_t row0 = m0 + wm * 128 + 4 * h;
  const int64_t col0 = wt_out * kRowTile + l32;
  if (m0 + kBM <= m && wt_out * kRowTile + kRowTile <= n && act == MQ_ACT_NONE_) {
    // full tile, no activation: unchecked stores
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float bv = bias ? bias[col0 + nb * 32] : 0.f;
      OUT *yc = y + row0 * ldy + col0 + nb * 32;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          store_out<OUT>(yc + (mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy, acc[mb][nb][e] + bv);
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = col0 + nb * 32;
    if (col >= n) continue;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = row0 + mb * 32 + 8 * (e >> 2) + (e & 3);
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
        hipLaunchKernelGGL((gemm_fast_kernel<T, float>), dim3(grid), dim3(kFastThreads), 0, stream, w, n, k,
                           ntiles_w, a, m, lda, static_cast<float *>(y), ldy, bias, act, tiles_m, tiles_n);
      else
        hipLaunchKernelGGL((gemm_fast_kernel<T, __bf16>), dim3(grid), dim3(kFastThreads), 0, stream, w, n, k,
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
