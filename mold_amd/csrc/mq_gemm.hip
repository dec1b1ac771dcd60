// mq_gemm.hip — fused dequant -> bf16 MFMA GEMM for large-M quantized linears
// (FLUX / Qwen-Image token projections): y[m, n] = act(x[m, :] . W[n, :] + b[n]).
//
// Both kernels tile for gfx950 (256 CUs in 8 XCDs, 64-wide waves, 160 KiB
// LDS per CU) the same way:
//   * workgroup = 4 waves (one per SIMD), block tile 256 (m) x 256 (n);
//   * wave w owns weight tile nt*4 + w (64 output features) for all 256 rows,
//     so every weight element is decoded exactly once per block tile and goes
//     straight from registers into the MFMA B operand (no LDS round trip);
//   * the bf16 activation tile is staged through LDS (XOR-swizzled 16-byte
//     chunks, one barrier per K step of 64) and read by all four waves;
//   * v_mfma_f32_32x32x16_bf16: per wave 8 (m) x 2 (n) accumulator tiles,
//     256 f32 accumulators per lane;
//   * blockIdx -> tile mapping gives each XCD a contiguous range of tiles that
//     share the same activation panel in its L2.
// gemm_fast_kernel (k a multiple of 256) decodes with the per-type fragment
// decoders of mq_bfrag.h and pipelines loads, decode and MFMAs; gemm_kernel
// handles any k with the generic 8-element decoder.
// Within a K step of 64, lane half h (lane / 32) supplies K elements
// {16h..16h+15} u {32+16h..32+16h+15} (four runs of 8) in gemm_kernel, and
// the per-type chunk order TT::chunk(s, h) in gemm_fast_kernel; the A operand
// reads the same runs from LDS, so the K order inside a step is a permutation
// shared by both operands.
#include <type_traits>
#include <utility>

#include "mq_bfrag.h"
#include "mq_kernels.h"

namespace mq {

#ifdef MQ_GEMM_TYPE
// Kernels of one weight type (this file is compiled once per type with
// -DMQ_GEMM_TYPE=<type>, so the types build in parallel).

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

// y = v, or with a gate (f32 output only) the gated residual update
// y = r + g * v of the DiT blocks, r read through its own pointer `res`
// (the same buffer as y): loads of r never wait behind stores of y.
template <typename OUT>
__device__ __forceinline__ void store_epi(OUT *p, const float *r, float v, const float *gate, float g) {
  if constexpr (std::is_same_v<OUT, float>) {
    if (gate) v = __builtin_fmaf(g, v, *r);
  }
  store_out<OUT>(p, v);
}

template <int TYPE, typename OUT>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_kernel(
    WView w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *__restrict__ a, int64_t m,
    int64_t lda, OUT *__restrict__ y, int64_t ldy, const float *__restrict__ bias,
    const float *__restrict__ gate, const float *__restrict__ res, int act, int tiles_m,
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
    const float g = gate ? gate[col] : 0.f;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + mb * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < m)
          store_epi<OUT>(y + row * ldy + col, res + row * ldy + col, act_out<OUT>(acc[mb][nb][e] + bv, act), gate, g);
      }
    }
  }
}

constexpr int MQ_ACT_NONE_ = 0;  // mq_act MQ_ACT_NONE
constexpr int kFastThreads = 256;
typedef __attribute__((address_space(3))) void lds_void_t;

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

// ---------------------------------------------------------------------------
// Fast path (k a multiple of the type's unit, 16-byte aligned activation
// rows): one wave per SIMD, 256 x 256 block tile, 4 waves, K step 64.
//   * wave w owns weight tile nt*4 + w (64 output features) for all 256 rows:
//     lane (l32, h) decodes weight rows l32 and l32 + 32 of that tile straight
//     into MFMA B operands (per-type decoders, mq_bfrag.h), so every weight
//     is decoded once per block tile and B never touches LDS;
//   * A (bf16 activations, 256 x 64 per step) goes global -> LDS by direct
//     loads (dma16) into a 4-slot ring three steps ahead, one barrier per
//     step; rows are 128 B with 16-byte chunk c of row r in slot
//     c ^ ((r >> 1) & 7), so the 16 lanes of a ds_read_b128 quarter hit
//     distinct banks;
//   * with one wave per SIMD each wave has 512 registers: the 8 x 2 tiles of
//     v_mfma_f32_32x32x16_bf16 accumulators (256 f32) sit in AGPRs, leaving
//     room to read the next slice's A fragments and decode its B operands
//     (the next step's first slice during the last slice) while the current
//     slice's 16 MFMAs run;
//   * XCD-aware tile order (workgroup i runs on XCD i % 8; each XCD gets a
//     contiguous run of tiles, row-major over n, sharing the x panel in L2);
//   * weight bytes for unit u+1 are fetched during unit u (one unit ahead);
//     every load is unconditional (the last unit re-reads itself), so the
//     compiler's wait counts are the same on every path.

template <int TYPE, typename OUT>
__global__ __launch_bounds__(kFastThreads, 1) void gemm_fast_kernel(
    WView w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *__restrict__ a, int64_t m, int64_t lda,
    OUT *__restrict__ y, int64_t ldy, const float *__restrict__ bias, const float *__restrict__ gate,
    const float *__restrict__ res, int act, int tiles_m, int tiles_n, int full_tiles, int kparts,
    float *__restrict__ partial) {
  using TT = bfrag::T<TYPE>;
  constexpr int kSteps = TT::kUnitK / kBK;
  // VALU instructions placed after each pair of MFMAs (the decode work per
  // MFMA differs by type; measured best per type)
  constexpr int kVpm = TYPE == Q8_0 ? 3 : (TYPE == Q4_K || TYPE == Q5_K) ? 6 : 8;
  __shared__ uint4 lds_a[4][kBM * kBK / 8];

  // Workgroups 0 .. full_tiles-1 run whole tiles (XCD-aware order over
  // them); the rest run K part `part` of tail tile full_tiles + (w / kparts):
  // the units [part * U / kparts, (part + 1) * U / kparts) of the U = k / 256,
  // written raw to `partial` for gemm_tail_reduce_kernel.
  const int bid = blockIdx.x;
  int v, part = -1;
  if (bid < full_tiles) {
    const int xcd = bid & 7, local = bid >> 3;
    const int base = full_tiles >> 3, extra = full_tiles & 7;
    v = xcd * base + (xcd < extra ? xcd : extra) + local;
  } else {
    const int t = bid - full_tiles;
    v = full_tiles + t / kparts;
    part = t - (t / kparts) * kparts;
  }
  const int mt = v / tiles_n, nt = v - mt * tiles_n;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int swz = (l32 >> 1) & 7;  // LDS swizzle key of every row this lane reads
  const int64_t m0 = (int64_t)mt * kBM;
  const int64_t all_units = k / TT::kUnitK;
  const int64_t ub = part < 0 ? 0 : part * all_units / kparts;                  // first unit
  const int64_t units = part < 0 ? all_units : (part + 1) * all_units / kparts - ub;
  const int64_t ksteps = units * kSteps;
  a += ub * TT::kUnitK;  // A columns of this K range
  const int64_t wt_raw = (int64_t)nt * (kBN / kRowTile) + wave;
  const int64_t wt = wt_raw < ntiles_w ? wt_raw : ntiles_w - 1;  // keep reads in bounds

  f32x16 acc[8][2];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // A: 4-slot LDS ring filled by direct global->LDS loads three K steps
  // ahead.  Load i (0..7) of wave w fills LDS rows 64w + 8i .. +7 (1 KiB);
  // lane j fetches row 64w + 8i + j/8, logical chunk (j&7) ^ ((row>>1)&7).
  // Rows past m read row m-1 (finite, never stored).
  int aoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 64 * wave + 8 * i + (lane >> 3);
    int64_t row = m0 + r;
    row = row < m ? row : m - 1;
    aoff[i] = (int)(row * lda + (((lane & 7) ^ ((r >> 1) & 7)) * 8));
  }
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  auto dma_a = [&](uint4 *slot, int64_t ks) {
    const uint32_t dst = (uint32_t)(uintptr_t)(lds_void_t *)(slot + 64 * 8 * wave_u);
#pragma unroll
    for (int i = 0; i < 8; ++i) dma16(a + aoff[i] + ks * kBK, dst + 1024 * i);
  };

  typename TT::Raw raw[2];
  typename TT::Sc sc[2];
  // Barrier between K steps (global loads stay in flight across it, which
  // __syncthreads would not allow).  At the end of step ks the A loads for step ks+1 (issued two steps
  // earlier) must have landed; younger than them are at least the 16 loads
  // for steps ks+2 and ks+3, so vmcnt(16) suffices and leaves the newest
  // weight reloads in flight.
  auto step_sync = [&]() { asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // A fragments of slice S from slot `slot`, and B operands of slice S of
  // step G from the unpacked weight bytes.
  bf16x8 af[2][8], bf[2][2];
  auto read_a = [&](bf16x8 *dst, const uint4 *__restrict__ slot, int S) {
    const char *abase = reinterpret_cast<const char *>(slot) + l32 * 128 + (TT::chunk(S, h) ^ swz) * 16;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) dst[mb] = *reinterpret_cast<const bf16x8 *>(abase + mb * 4096);
  };
  auto decode_b = [&]<int G, int S>(bf16x8 *dst) {
#pragma unroll
    for (int j = 0; j < 2; ++j) dst[j] = TT::template frag<G, S>(raw[j], sc[j]);
  };

  // prologue: unit 0's weight bytes and scales, A(0) and A(1) into slots 0, 1;
  // step 0's slice-0 operands
#pragma unroll
  for (int j = 0; j < 2; ++j) TT::load_prep(raw[j], w, wt, l32 + 32 * j, ub, h);
  static_for<kSteps>([&]<int G>() {
#pragma unroll
    for (int j = 0; j < 2; ++j) TT::template reload<G>(raw[j], w, wt, l32 + 32 * j, ub, h);
  });
  dma_a(lds_a[0], 0);
  dma_a(lds_a[1], ksteps > 1 ? 1 : 0);
  dma_a(lds_a[2], ksteps > 2 ? 2 : ksteps - 1);
#pragma unroll
  for (int j = 0; j < 2; ++j) TT::prep(raw[j], sc[j], h);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  read_a(af[0], lds_a[0], 0);
  decode_b.template operator()<0, 0>(bf[0]);

  for (int64_t u = 0; u < units; ++u) {
    const int64_t un = u + 1 < units ? u + 1 : u;
    static_for<kSteps>([&]<int G>() {
      const int64_t ks = u * kSteps + G;
      const int64_t kf = ks + 3 < ksteps ? ks + 3 : ksteps - 1;
      auto body = [&](const uint4 *__restrict__ a_cur, const uint4 *__restrict__ a_next,
                      uint4 *__restrict__ a_fill) {
        dma_a(a_fill, kf);
        static_for<4>([&]<int S>() {
          // operands of the next slice (slice 0 of the next step after S = 3)
          if constexpr (S < 3) {
            read_a(af[(S + 1) & 1], a_cur, S + 1);
            decode_b.template operator()<G, S + 1>(bf[(S + 1) & 1]);
          } else {
            // piece G is fully decoded: fetch unit u+1's (and its scale bytes
            // after step 0); unit u+1's scales are unpacked before its first
            // slice is decoded.
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              TT::template reload<G>(raw[j], w, wt, l32 + 32 * j, ub + un, h);
              if constexpr (G == 0) TT::load_prep(raw[j], w, wt, l32 + 32 * j, ub + un, h);
            }
            read_a(af[0], a_next, 0);
            if constexpr (G + 1 < kSteps) {
              decode_b.template operator()<G + 1, 0>(bf[0]);
            } else {
#pragma unroll
              for (int j = 0; j < 2; ++j) TT::prep(raw[j], sc[j], h);
              decode_b.template operator()<0, 0>(bf[0]);
            }
          }
#pragma unroll
          for (int mb = 0; mb < 8; ++mb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
              acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[S & 1][mb], bf[S & 1][nb], acc[mb][nb], 0,
                                                                    0, 0);
          static_for<8>([&]<int I>() {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, kVpm, 0);
          });
        });
      };
      body(lds_a[ks & 3], lds_a[(ks + 1) & 3], lds_a[(ks + 3) & 3]);
      step_sync();
    });
  }

  // no A load may still be in flight when the wave ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: lane holds column l32 of each 32x32 tile, rows
  // 8*(e/4) + 4*h + (e%4).
  if (wt_raw >= ntiles_w) return;
  if (part >= 0) {
    // raw sums of this K part: tile-local row-major [256][256] f32 block
    float *pt = partial + ((int64_t)(v - full_tiles) * kparts + part) * (kBM * kBN) + 4 * h * kBN + wave * 64 + l32;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e) pt[(mb * 32 + 8 * (e >> 2) + (e & 3)) * kBN + nb * 32] = acc[mb][nb][e];
    return;
  }
  const int64_t row0 = m0 + 4 * h;
  const int64_t col0 = wt_raw * kRowTile + l32;
  if (m0 + kBM <= m && wt_raw * kRowTile + kRowTile <= n && act == MQ_ACT_NONE_) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float bv = bias ? bias[col0 + nb * 32] : 0.f;
      OUT *yc = y + row0 * ldy + col0 + nb * 32;
      if constexpr (std::is_same_v<OUT, float>) {
        if (gate) {
          // residual rows of 32-row block mb + 1 are loaded before block mb is
          // stored: one memory latency per tile column, not one per element
          const float g = gate[col0 + nb * 32];
          const float *rc = res + row0 * ldy + col0 + nb * 32;
          float r[2][16];
#pragma unroll
          for (int e = 0; e < 16; ++e) r[0][e] = rc[(8 * (e >> 2) + (e & 3)) * ldy];
#pragma unroll
          for (int mb = 0; mb < 8; ++mb) {
            if (mb + 1 < 8) {
#pragma unroll
              for (int e = 0; e < 16; ++e) r[(mb + 1) & 1][e] = rc[((mb + 1) * 32 + 8 * (e >> 2) + (e & 3)) * ldy];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < 16; ++e)
              yc[(mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy] = __builtin_fmaf(g, acc[mb][nb][e] + bv, r[mb & 1][e]);
            __builtin_amdgcn_sched_barrier(0);
          }
          continue;
        }
      }
      {
#pragma unroll
        for (int mb = 0; mb < 8; ++mb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            store_out<OUT>(yc + (mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy, acc[mb][nb][e] + bv);
      }
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = col0 + nb * 32;
    if (col >= n) continue;
    const float bv = bias ? bias[col] : 0.f;
    const float g = gate ? gate[col] : 0.f;
    if constexpr (std::is_same_v<OUT, float>) {
      if (gate) {
        // as the full-tile path: block mb + 1's residual rows loaded before
        // block mb is stored; rows past m are neither read nor written
        float r[2][16];
        auto load_block = [&](int mb, float *dst) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int64_t row = row0 + mb * 32 + 8 * (e >> 2) + (e & 3);
            dst[e] = row < m ? res[row * ldy + col] : 0.f;
          }
        };
        load_block(0, r[0]);
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) {
          if (mb + 1 < 8) load_block(mb + 1, r[(mb + 1) & 1]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int64_t row = row0 + mb * 32 + 8 * (e >> 2) + (e & 3);
            if (row < m) y[row * ldy + col] = __builtin_fmaf(g, apply_act(acc[mb][nb][e] + bv, act), r[mb & 1][e]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        continue;
      }
    }
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = row0 + mb * 32 + 8 * (e >> 2) + (e & 3);
        if (row < m)
          store_epi<OUT>(y + row * ldy + col, res + row * ldy + col, act_out<OUT>(acc[mb][nb][e] + bv, act), gate, g);
      }
    }
  }
}

// Tail tiles split over K: y = epi(sum of the kparts raw sums in part order
// + bias), one thread per 4 columns of a tile row.
template <typename OUT>
__global__ __launch_bounds__(256) void gemm_tail_reduce_kernel(const float *__restrict__ partial, int kparts,
                                                               int full_tiles, int tiles_n, int64_t m, int64_t n,
                                                               OUT *__restrict__ y, int64_t ldy,
                                                               const float *__restrict__ bias,
                                                               const float *__restrict__ gate, int act, int vec) {
  const int tl = blockIdx.y;                            // tail tile
  const int idx = blockIdx.x * 256 + threadIdx.x;       // 0 .. 256 * 64 - 1
  const int r = idx >> 6, c = (idx & 63) * 4;
  const int v = full_tiles + tl;
  const int mt = v / tiles_n, nt = v - mt * tiles_n;
  const int64_t row = (int64_t)mt * kBM + r, col0 = (int64_t)nt * kBN + c;
  if (row >= m) return;
  const float *src = partial + (int64_t)tl * kparts * (kBM * kBN) + r * kBN + c;
  // every part's load is issued before the first add (no chain of
  // latencies), then the parts are added in order
  float4 t[kGemmMaxKParts];
#pragma unroll
  for (int p = 0; p < kGemmMaxKParts; ++p)
    if (p < kparts) t[p] = *reinterpret_cast<const float4 *>(src + (int64_t)p * (kBM * kBN));
  float4 s = t[0];
#pragma unroll
  for (int p = 1; p < kGemmMaxKParts; ++p) {
    if (p < kparts) {
      s.x += t[p].x;
      s.y += t[p].y;
      s.z += t[p].z;
      s.w += t[p].w;
    }
  }
  const float sv[4] = {s.x, s.y, s.z, s.w};
  OUT *yr = y + row * ldy + col0;
  if (vec && col0 + 3 < n) {
    // y, bias and gate rows are 16-byte aligned here (8 for bf16 y): one
    // vector access each
    float o[4];
    const float4 bv = bias ? *reinterpret_cast<const float4 *>(bias + col0) : make_float4(0.f, 0.f, 0.f, 0.f);
    o[0] = act_out<OUT>(sv[0] + bv.x, act);
    o[1] = act_out<OUT>(sv[1] + bv.y, act);
    o[2] = act_out<OUT>(sv[2] + bv.z, act);
    o[3] = act_out<OUT>(sv[3] + bv.w, act);
    if constexpr (std::is_same_v<OUT, float>) {
      float4 *yv = reinterpret_cast<float4 *>(yr);
      if (gate) {
        const float4 rv = *yv;
        const float4 gv = *reinterpret_cast<const float4 *>(gate + col0);
        *yv = make_float4(__builtin_fmaf(gv.x, o[0], rv.x), __builtin_fmaf(gv.y, o[1], rv.y),
                          __builtin_fmaf(gv.z, o[2], rv.z), __builtin_fmaf(gv.w, o[3], rv.w));
      } else {
        *yv = make_float4(o[0], o[1], o[2], o[3]);
      }
    } else {
      __bf16 h[4] = {(__bf16)o[0], (__bf16)o[1], (__bf16)o[2], (__bf16)o[3]};
      *reinterpret_cast<uint2 *>(yr) = *reinterpret_cast<const uint2 *>(h);
    }
    return;
  }
  if constexpr (std::is_same_v<OUT, float>) {
    if (gate) {
      // the four residual values are read before any is written
      float rv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) rv[j] = col0 + j < n ? yr[j] : 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (col0 + j < n)
          yr[j] = __builtin_fmaf(gate[col0 + j], apply_act(sv[j] + (bias ? bias[col0 + j] : 0.f), act), rv[j]);
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (col0 + j < n) store_out<OUT>(yr + j, act_out<OUT>(sv[j] + (bias ? bias[col0 + j] : 0.f), act));
}

template <int T>
hipError_t launch_gemm_type(const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a, int64_t m,
                            int64_t lda, void *y, int y_type, int64_t ldy, const float *bias, const float *gate,
                            int act, const GemmTail &tail, float *partial, hipStream_t stream) {
  const int tiles_m = (int)((m + kBM - 1) / kBM);
  const int tiles_n = (int)((n + kBN - 1) / kBN);
  const int grid = tiles_m * tiles_n;
  const float *res = gate ? static_cast<const float *>(y) : nullptr;  // the gated update reads y, then writes it
  if (gemm_fast_ok(m, k, lda)) {
    const bool split = partial && tail.kparts > 1;
    const int full = split ? tail.full_tiles : grid;
    const int kp = split ? tail.kparts : 1;
    const int wgs = full + (grid - full) * kp;
    if (y_type == F32)
      hipLaunchKernelGGL((gemm_fast_kernel<T, float>), dim3(wgs), dim3(kFastThreads), 0, stream, w, n, k, ntiles_w, a,
                         m, lda, static_cast<float *>(y), ldy, bias, gate, res, act, tiles_m, tiles_n, full, kp,
                         partial);
    else
      hipLaunchKernelGGL((gemm_fast_kernel<T, __bf16>), dim3(wgs), dim3(kFastThreads), 0, stream, w, n, k, ntiles_w,
                         a, m, lda, static_cast<__bf16 *>(y), ldy, bias, gate, res, act, tiles_m, tiles_n, full, kp,
                         partial);
    if (split) {
      const dim3 rgrid(kBM * kBN / 4 / 256, (unsigned)(grid - full));
      const uintptr_t ya = y_type == F32 ? 15 : 7;
      const int vec = (reinterpret_cast<uintptr_t>(y) & ya) == 0 && ldy % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(bias) & 15) == 0 && (reinterpret_cast<uintptr_t>(gate) & 15) == 0;
      if (y_type == F32)
        hipLaunchKernelGGL(gemm_tail_reduce_kernel<float>, rgrid, dim3(256), 0, stream, partial, kp, full, tiles_n, m,
                           n, static_cast<float *>(y), ldy, bias, gate, act, vec);
      else
        hipLaunchKernelGGL(gemm_tail_reduce_kernel<__bf16>, rgrid, dim3(256), 0, stream, partial, kp, full, tiles_n,
                           m, n, static_cast<__bf16 *>(y), ldy, bias, gate, act, vec);
    }
  } else if (y_type == F32) {
    hipLaunchKernelGGL((gemm_kernel<T, float>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k, ntiles_w,
                       a, m, lda, static_cast<float *>(y), ldy, bias, gate, res, act, tiles_m, tiles_n);
  } else {
    hipLaunchKernelGGL((gemm_kernel<T, __bf16>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k, ntiles_w,
                       a, m, lda, static_cast<__bf16 *>(y), ldy, bias, gate, res, act, tiles_m, tiles_n);
  }
  return hipGetLastError();
}

template hipError_t launch_gemm_type<MQ_GEMM_TYPE>(const WView &, int64_t, int64_t, int64_t, const __bf16 *,
                                                   int64_t, int64_t, void *, int, int64_t, const float *,
                                                   const float *, int, const GemmTail &, float *, hipStream_t);

#else  // the type dispatcher

GemmTail gemm_tail_plan(int64_t m, int64_t n, int64_t k, int cus) {
  const int64_t tiles = ((m + kGemmTile - 1) / kGemmTile) * ((n + kGemmTile - 1) / kGemmTile);
  const int64_t rem = tiles % cus;                 // tiles of the last, partial round
  const int64_t units = k / 256;
  GemmTail t{(int)tiles, 1};
  if (rem == 0 || units < 2) return t;
  int64_t kp = cus / rem;                          // K parts per tail tile: they fill one round
  kp = kp < units ? kp : units;
  kp = kp < kGemmMaxKParts ? kp : kGemmMaxKParts;
  if (kp < 2) return t;
  t.full_tiles = (int)(tiles - rem);
  t.kparts = (int)kp;
  return t;
}

size_t gemm_tail_bytes(const GemmTail &t, int64_t m, int64_t n) {
  const int64_t tiles = ((m + kGemmTile - 1) / kGemmTile) * ((n + kGemmTile - 1) / kGemmTile);
  if (t.kparts < 2) return 0;
  return (size_t)(tiles - t.full_tiles) * t.kparts * kGemmTile * kGemmTile * sizeof(float);
}

hipError_t launch_gemm(int type, const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a,
                       int64_t m, int64_t lda, void *y, int y_type, int64_t ldy, const float *bias,
                       const float *gate, int act, const GemmTail &tail, float *partial, hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  hipError_t err = hipErrorInvalidValue;
  dispatch_type(type, [&]<int T>() {
    err = launch_gemm_type<T>(w, n, k, ntiles_w, a, m, lda, y, y_type, ldy, bias, gate, act, tail, partial, stream);
  });
  return err;
}

#endif  // MQ_GEMM_TYPE

}  // namespace mq
