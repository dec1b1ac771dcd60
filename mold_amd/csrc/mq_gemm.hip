// mq_gemm.hip — fused dequant -> bf16 MFMA GEMM for large-M quantized linears
// (FLUX / Qwen-Image token projections): y[m, n] = act(x[m, :] . W[n, :] + b[n]).
//
// gemm_fast_kernel (k a whole number of the weight type's K units) is the
// path every BASELINE shape takes.  It is shaped for gfx950's CUs (4 SIMDs,
// 512 VGPRs per SIMD lane, 160 KiB LDS) so that every SIMD holds two waves
// (one wave's MFMAs run while the other decodes weights):
//   * large m: workgroup = 8 waves (two per SIMD), block tile 256 (m) x 256
//     (n), one workgroup per CU, so the 256 x 64 activation tile of a K step
//     is fetched once for 256 output features (against two 4-wave 256 x 128
//     workgroups per CU: 3-8 % faster on every large BASELINE shape, same
//     outputs); small m: 64- or 128-row tiles of 4 waves x 128 features, three
//     or four workgroups per CU;
//   * wave w owns output features 32w .. 32w+31 of the tile for all its
//     rows: lane (l32, h) decodes weight row l32 of that run straight into
//     the MFMA B operand (per-type decoders, mq_bfrag.h), so every weight is
//     decoded once per block tile and B never touches LDS;
//   * v_mfma_f32_32x32x16_bf16, 8 accumulator tiles (128 f32) per lane at 256
//     rows;
//   * the bf16 activation tile (rows x 64 per K step) goes global -> LDS one
//     step ahead by LDS DMA (global_load_lds_dwordx4: no VGPRs, no LDS
//     write instructions) through a 2-slot ring (2 x 32 KiB at 256 rows);
//     the step's weight loads are issued with it at the step's start and
//     both are awaited once, at the step barrier;
//   * rows are 128 B, chunk c of row r in slot c ^ ((r >> 1) & 7), so the
//     16 lanes of a ds_read_b128 / ds_write_b128 quarter hit distinct banks;
//   * XCD-aware tile order: workgroup i runs on XCD i % 8; each XCD gets a
//     contiguous run of the launch order, which takes row panels in pairs
//     and, inside a pair, weight tiles in turn (fast_tile), so the tiles in
//     flight on one XCD share two activation panels and each weight tile in
//     its L2.
// gemm_kernel handles any k with the generic 8-element decoder (256 x 256
// tiles, one workgroup per CU).
// Within a K step of 64, lane half h (lane / 32) supplies the per-type chunk
// order TT::chunk(s, h) (gemm_kernel: K elements {16h..16h+15} u
// {32+16h..32+16h+15}); the A operand reads the same runs from LDS, so the K
// order inside a step is a permutation shared by both operands.
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
// Output stores of whole tiles: y is never read back by the kernel, so f32
// outputs are stored nontemporal (they do not displace the activation panels
// and weight tiles other workgroups re-read from L2: headline 4608x3072->21504
// f32 ~0.7 % faster, same values).
template <typename OUT>
__device__ __forceinline__ void store_out_stream(OUT *p, float v) {
  if constexpr (std::is_same_v<OUT, float>)
    __builtin_nontemporal_store(v, p);
  else
    store_out<OUT>(p, v);
}

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
          store_epi<OUT>(y + row * ldy + col, res + row * ldy + col, act_out<OUT>(acc[mb][nb][e] + bv, act_at(act, col)),
                         gate, g);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fast path.  Block tile kFM x (32 kW), K step kFK; see the file comment.
constexpr int kFK = 64;
constexpr int MQ_ACT_NONE_ = 0;  // mq_act MQ_ACT_NONE
constexpr int MQ_ACT_GELU_ = 1;  // mq_act MQ_ACT_GELU_TANH (the only other value)

// 16 bytes per lane from sbase + voff straight into LDS: lane i of the wave
// writes LDS bytes lds + 16 i .. + 15 (global_load_lds_dwordx4, saddr form).
// sbase and lds must be wave-uniform.  The compiler does not track this load:
// its data may be read only after step_barrier.
__device__ __forceinline__ void dma16(const char *sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}

// Launch-order tile v -> (row panel mt, weight tile nt) of the fast kernel:
// groups of two row panels, weight-tile major inside a group, so the
// workgroups an XCD runs at once (consecutive v) pair up on each weight tile
// and its bytes serve both panels from L2 (about 1 % faster than row-major on
// the headline shape, same outputs).  gemm_tail_reduce_kernel maps tail tiles
// with the same function.
__device__ __forceinline__ void fast_tile(int v, int tiles_m, int tiles_n, int &mt, int &nt) {
  constexpr int G = 2;
  const int grp = v / (G * tiles_n), idx = v - grp * (G * tiles_n);
  const int gp = tiles_m - grp * G < G ? tiles_m - grp * G : G;  // panels in this group (the last may have 1)
  mt = grp * G + idx % gp;
  nt = idx / gp;
}

// Barrier between K steps: every load of this wave (weights and the LDS DMA
// of the next A tile) has landed and its LDS reads are complete, then every
// wave arrives.  The wait is the s_waitcnt builtin, so the compiler knows the
// weight loads are complete and adds no waits of its own before their use;
// the memory clobber keeps LDS accesses from moving across the barrier.
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) expcnt(7) lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

template <int TYPE, typename OUT, bool GATED, int kFM, int kW>
__global__ __launch_bounds__(64 * kW, 8 / kW) void gemm_fast_kernel(
    WView w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *__restrict__ a, int64_t m, int64_t lda,
    OUT *y, int64_t ldy, const float *__restrict__ bias, const float *__restrict__ gate, int act, int tiles_m,
    int tiles_n, int full_tiles, int kparts, float *__restrict__ partial) {
  using TT = bfrag::T<TYPE>;
  constexpr int kP = TT::kUnitK / kFK;  // K steps per weight unit
  constexpr int kMB = kFM / 32;         // 32-row MFMA blocks of the tile
  constexpr int kFNW = 32 * kW;         // output features of the tile
  constexpr int kDM = kFM / (8 * kW);   // A DMA loads per wave and step
  __shared__ uint4 lds_a[2][kFM * kFK / 8];

  // Workgroups 0 .. full_tiles-1 run whole tiles (XCD-aware order over
  // them); the rest run K part `part` of tail tile full_tiles + (w / kparts):
  // the units [part * U / kparts, (part + 1) * U / kparts) of the U = k / unit,
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
  int mt, nt;
  fast_tile(v, tiles_m, tiles_n, mt, nt);

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t m0 = (int64_t)mt * kFM;
  const int64_t c0 = (int64_t)nt * kFNW + 32 * wave;  // this wave's first output feature
  const int64_t wt_raw = c0 / kRowTile;              // its weight tile
  const int wrow = (int)(c0 - wt_raw * kRowTile) + l32;  // this lane's row in that tile
  const int64_t wt = wt_raw < ntiles_w ? wt_raw : ntiles_w - 1;  // keep reads in bounds
  const int64_t all_units = k / TT::kUnitK;
  const int64_t ub = part < 0 ? 0 : part * all_units / kparts;  // first unit
  const int64_t units = part < 0 ? all_units : (part + 1) * all_units / kparts - ub;
  const int64_t ksteps = units * kP;

  f32x16 acc[kMB];
#pragma unroll
  for (int i = 0; i < kMB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;

  // A staging by LDS DMA: load i (0 .. kMB-1) of wave `wave` fills LDS rows
  // 32 i + 8 wave .. +7 of a slot (1 KiB), lane -> row ar = tid / 8, LDS
  // chunk slot ac = tid % 8, so the lane fetches global chunk
  // ac ^ ((ar >> 1) & 7) ((ar + 32 i) >> 1 & 7 == ar >> 1 & 7).  Rows past m
  // re-read row m - 1: their products land only in accumulator rows that are
  // never stored.  Row offsets are per lane (voff), the K offset is in the
  // uniform base address.
  const int ac = tid & 7, ar = tid >> 3;
  const int gch = ac ^ ((ar >> 1) & 7);
  uint32_t voff[kDM];
#pragma unroll
  for (int i = 0; i < kDM; ++i) {
    const int64_t r = m0 + ar + 8 * kW * i < m ? m0 + ar + 8 * kW * i : m - 1;
    voff[i] = (uint32_t)((r * lda + gch * 8) * 2);
  }
  const uint32_t akb = (uint32_t)(ub * TT::kUnitK * 2);
  const uint32_t lds_wave = (uint32_t)(uintptr_t)(&lds_a[0][0]) + (uint32_t)(8 * 128 * wave);
  auto dma_a = [&](int64_t ks, int slot) {
    const uint64_t g = reinterpret_cast<uint64_t>(a) + akb + (uint64_t)ks * (kFK * 2);
    const char *sb = reinterpret_cast<const char *>(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(g >> 32)) << 32) |
                                                    (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)g));
#pragma unroll
    for (int i = 0; i < kDM; ++i)
      dma16(sb, voff[i],
            __builtin_amdgcn_readfirstlane(lds_wave + (uint32_t)(slot * (kFM * kFK * 2) + 8 * kW * 128 * i)));
  };
  const int swz = (l32 >> 1) & 7;  // LDS swizzle key of every row this lane reads
  auto read_a = [&](int slot, int mb, int S) -> bf16x8 {
    const char *p = reinterpret_cast<const char *>(lds_a[slot]) + l32 * 128 + ((TT::chunk(S, h) ^ swz) << 4) +
                    mb * 4096;
    return *reinterpret_cast<const bf16x8 *>(p);
  };

  typename TT::Raw raw;
  typename TT::Sc sc;
  // prologue: unit 0's weight bytes and scales, A(0) into slot 0
  TT::load_prep(raw, w, wt, wrow, ub, h);
  static_for<kP>([&]<int G>() { TT::template reload<G>(raw, w, wt, wrow, ub, h); });
  dma_a(0, 0);
  TT::prep(raw, sc, h);
  step_barrier();

  // Every load a step issues (A(ks+1) into the other slot, the weight piece
  // decoded in the previous step and, at a unit's first step, the next unit's
  // scale bytes) is issued at the step's start and awaited at its end, so each
  // has a whole step of MFMAs to land.  Piece G is last used in step G (kP >= 2
  // for every type), so at step G piece G-1 is free to take the next unit's
  // bytes, and at step 0 piece kP-1 takes this unit's.
  for (int64_t u = 0; u < units; ++u) {
    const int64_t un = u + 1 < units ? u + 1 : u;  // the last unit re-reads itself
    static_for<kP>([&]<int G>() {
      const int64_t ks = u * kP + G;
      const int64_t kn = ks + 1 < ksteps ? ks + 1 : ks;  // the last step re-reads itself
      const int slot = (int)(ks & 1);
      if constexpr (G == 0) {
        TT::template reload<kP - 1>(raw, w, wt, wrow, ub + u, h);
        TT::load_prep(raw, w, wt, wrow, ub + un, h);  // unpacked by prep after step kP-1
      } else {
        TT::template reload<G - 1>(raw, w, wt, wrow, ub + un, h);
      }
      dma_a(kn, slot ^ 1);  // the other slot was last read in step ks-1
      bf16x8 bf[2];
      bf[0] = TT::template frag<G, 0>(raw, sc);
      static_for<4>([&]<int S>() {
        if constexpr (S < 3) bf[(S + 1) & 1] = TT::template frag<G, S + 1>(raw, sc);
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
          acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(read_a(slot, mb, S), bf[S & 1], acc[mb], 0, 0, 0);
      });
      if constexpr (G == kP - 1) TT::prep(raw, sc, h);
      step_barrier();
    });
  }

  // ---- epilogue: lane holds output feature c0 + l32 of each 32 x 32 tile mb,
  // rows 8*(e/4) + 4*h + (e%4).
  if (c0 >= n) return;
  if (part >= 0) {
    // raw sums of this K part: tile-local row-major [256][128] f32 block
    float *pt = partial + ((int64_t)(v - full_tiles) * kparts + part) * (kFM * kFNW) + 4 * h * kFNW + 32 * wave + l32;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) pt[(mb * 32 + 8 * (e >> 2) + (e & 3)) * kFNW] = acc[mb][e];
    return;
  }
  const int64_t col = c0 + l32;
  const int64_t row0 = m0 + 4 * h;
  const bool colok = col < n;
  const int la = act_at(act, col);  // this lane's column's activation
  const float bv = bias && colok ? bias[col] : 0.f;
  OUT *yc = y + row0 * ldy + col;
  if constexpr (GATED) {
    // y = y + g * v: block mb + 1's residual rows are loaded before block mb
    // is stored (one memory latency per tile column, not one per element);
    // rows past m and columns past n are neither read nor written
    const float g = colok ? gate[col] : 0.f;
    float r[2][16];
    if (m0 + kFM <= m && c0 + 32 <= n && la == MQ_ACT_NONE_) {
      // whole tile, no activation (every gated linear of the block graphs):
      // no bounds checks
      auto load_full = [&](int mb, float *dst) {
#pragma unroll
        for (int e = 0; e < 16; ++e) dst[e] = yc[(mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy];
      };
      load_full(0, r[0]);
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        if (mb + 1 < kMB) load_full(mb + 1, r[(mb + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 16; ++e)
          yc[(mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy] = __builtin_fmaf(g, acc[mb][e] + bv, r[mb & 1][e]);
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
    auto load_block = [&](int mb, float *dst) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t ro = mb * 32 + 8 * (e >> 2) + (e & 3);
        dst[e] = colok && row0 + ro < m ? yc[ro * ldy] : 0.f;
      }
    };
    load_block(0, r[0]);
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb) {
      if (mb + 1 < kMB) load_block(mb + 1, r[(mb + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t ro = mb * 32 + 8 * (e >> 2) + (e & 3);
        if (colok && row0 + ro < m) yc[ro * ldy] = __builtin_fmaf(g, act_out<float>(acc[mb][e] + bv, la), r[mb & 1][e]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return;
  } else {
    if (m0 + kFM <= m && c0 + 32 <= n) {
      // whole tile: no row checks, the activation chosen once
      if (la == MQ_ACT_NONE_) {
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            store_out_stream<OUT>(yc + (mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy, acc[mb][e] + bv);
      } else {
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            store_out_stream<OUT>(yc + (mb * 32 + 8 * (e >> 2) + (e & 3)) * ldy, act_out<OUT>(acc[mb][e] + bv, MQ_ACT_GELU_));
      }
      return;
    }
    if (!colok) return;
#pragma unroll
    for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t ro = mb * 32 + 8 * (e >> 2) + (e & 3);
        if (row0 + ro < m) store_out<OUT>(yc + ro * ldy, act_out<OUT>(acc[mb][e] + bv, la));
      }
  }
}

// Tail tiles split over K: y = epi(sum of the kparts raw sums in part order
// + bias), one thread per 4 columns of a tile row.
template <typename OUT, int kFM, int kFN>
__global__ __launch_bounds__(256) void gemm_tail_reduce_kernel(const float *__restrict__ partial, int kparts,
                                                               int full_tiles, int tiles_n, int64_t m, int64_t n,
                                                               OUT *__restrict__ y, int64_t ldy,
                                                               const float *__restrict__ bias,
                                                               const float *__restrict__ gate, int act, int vec) {
  const int tl = blockIdx.y;                                  // tail tile
  const int idx = blockIdx.x * 256 + threadIdx.x;             // 0 .. kFM * kFN / 4 - 1
  const int r = idx / (kFN / 4), c = (idx % (kFN / 4)) * 4;
  const int v = full_tiles + tl;
  const int tiles_m = (int)((m + kFM - 1) / kFM);
  int mt, nt;
  fast_tile(v, tiles_m, tiles_n, mt, nt);
  const int64_t row = (int64_t)mt * kFM + r, col0 = (int64_t)nt * kFN + c;
  if (row >= m) return;
  const float *src = partial + (int64_t)tl * kparts * (kFM * kFN) + r * kFN + c;
  // every part's load is issued before the first add (no chain of
  // latencies), then the parts are added in order
  float4 t[kGemmMaxKParts];
#pragma unroll
  for (int p = 0; p < kGemmMaxKParts; ++p)
    if (p < kparts) t[p] = *reinterpret_cast<const float4 *>(src + (int64_t)p * (kFM * kFN));
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
    o[0] = act_out<OUT>(sv[0] + bv.x, act_at(act, col0));
    o[1] = act_out<OUT>(sv[1] + bv.y, act_at(act, col0 + 1));
    o[2] = act_out<OUT>(sv[2] + bv.z, act_at(act, col0 + 2));
    o[3] = act_out<OUT>(sv[3] + bv.w, act_at(act, col0 + 3));
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
          yr[j] = __builtin_fmaf(gate[col0 + j], act_out<float>(sv[j] + (bias ? bias[col0 + j] : 0.f), act_at(act, col0 + j)),
                                 rv[j]);
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (col0 + j < n) store_out<OUT>(yr + j, act_out<OUT>(sv[j] + (bias ? bias[col0 + j] : 0.f), act_at(act, col0 + j)));
}

template <typename OUT, bool GATED, int FM, int W>
static void launch_fast(const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a, int64_t m,
                        int64_t lda, void *y, int64_t ldy, const float *bias, const float *gate, int act,
                        int tiles_m, int tiles_n, int full, int kp, float *partial, int wgs, hipStream_t stream) {
  hipLaunchKernelGGL((gemm_fast_kernel<MQ_GEMM_TYPE, OUT, GATED, FM, W>), dim3(wgs), dim3(64 * W), 0, stream, w,
                     n, k, ntiles_w, a, m, lda, static_cast<OUT *>(y), ldy, bias, gate, act, tiles_m, tiles_n, full,
                     kp, partial);
}

// One weight type's fast GEMM with FM-row block tiles of W waves (W * 32
// output features), and the reduce of its split tail tiles.
template <int FM, int W>
static void launch_fast_fm(const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a, int64_t m,
                           int64_t lda, void *y, int y_type, int64_t ldy, const float *bias, const float *gate,
                           int act, const GemmTail &tail, float *partial, hipStream_t stream) {
  constexpr int FN = 32 * W;
  const int tiles_m = (int)((m + FM - 1) / FM);
  const int tiles_n = (int)((n + FN - 1) / FN);
  const int grid = tiles_m * tiles_n;
  const bool split = partial && tail.kparts > 1;
  const int full = split ? tail.full_tiles : grid;
  const int kp = split ? tail.kparts : 1;
  const int wgs = full + (grid - full) * kp;
  if (gate)
    launch_fast<float, true, FM, W>(w, n, k, ntiles_w, a, m, lda, y, ldy, bias, gate, act, tiles_m, tiles_n, full,
                                    kp, partial, wgs, stream);
  else if (y_type == F32)
    launch_fast<float, false, FM, W>(w, n, k, ntiles_w, a, m, lda, y, ldy, bias, nullptr, act, tiles_m, tiles_n,
                                     full, kp, partial, wgs, stream);
  else
    launch_fast<__bf16, false, FM, W>(w, n, k, ntiles_w, a, m, lda, y, ldy, bias, nullptr, act, tiles_m, tiles_n,
                                      full, kp, partial, wgs, stream);
  if (split) {
    const dim3 rgrid(FM * FN / 4 / 256, (unsigned)(grid - full));
    const uintptr_t ya = y_type == F32 ? 15 : 7;
    const int vec = (reinterpret_cast<uintptr_t>(y) & ya) == 0 && ldy % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(bias) & 15) == 0 && (reinterpret_cast<uintptr_t>(gate) & 15) == 0;
    if (y_type == F32)
      hipLaunchKernelGGL((gemm_tail_reduce_kernel<float, FM, FN>), rgrid, dim3(256), 0, stream, partial, kp, full,
                         tiles_n, m, n, static_cast<float *>(y), ldy, bias, gate, act, vec);
    else
      hipLaunchKernelGGL((gemm_tail_reduce_kernel<__bf16, FM, FN>), rgrid, dim3(256), 0, stream, partial, kp, full,
                         tiles_n, m, n, static_cast<__bf16 *>(y), ldy, bias, gate, act, vec);
  }
}

template <int T>
hipError_t launch_gemm_type(const WView &w, int64_t n, int64_t k, int64_t ntiles_w, const __bf16 *a, int64_t m,
                            int64_t lda, void *y, int y_type, int64_t ldy, const float *bias, const float *gate,
                            int act, const GemmTail &tail, float *partial, hipStream_t stream) {
  if (gemm_fast_ok(T, m, k, lda)) {
    if (tail.fm == 64)
      launch_fast_fm<64, 4>(w, n, k, ntiles_w, a, m, lda, y, y_type, ldy, bias, gate, act, tail, partial, stream);
    else if (tail.fm == 128)
      launch_fast_fm<128, 4>(w, n, k, ntiles_w, a, m, lda, y, y_type, ldy, bias, gate, act, tail, partial, stream);
    else
      launch_fast_fm<256, 8>(w, n, k, ntiles_w, a, m, lda, y, y_type, ldy, bias, gate, act, tail, partial, stream);
    return hipGetLastError();
  }
  const int tiles_m = (int)((m + kBM - 1) / kBM);
  const int tiles_n = (int)((n + kBN - 1) / kBN);
  const int grid = tiles_m * tiles_n;
  const float *res = gate ? static_cast<const float *>(y) : nullptr;  // the gated update reads y, then writes it
  if (y_type == F32)
    hipLaunchKernelGGL((gemm_kernel<T, float>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k, ntiles_w, a, m,
                       lda, static_cast<float *>(y), ldy, bias, gate, res, act, tiles_m, tiles_n);
  else
    hipLaunchKernelGGL((gemm_kernel<T, __bf16>), dim3(grid), dim3(kGemmThreads), 0, stream, w, n, k, ntiles_w, a, m,
                       lda, static_cast<__bf16 *>(y), ldy, bias, gate, res, act, tiles_m, tiles_n);
  return hipGetLastError();
}

template hipError_t launch_gemm_type<MQ_GEMM_TYPE>(const WView &, int64_t, int64_t, int64_t, const __bf16 *,
                                                   int64_t, int64_t, void *, int, int64_t, const float *,
                                                   const float *, int, const GemmTail &, float *, hipStream_t);

#else  // the type dispatcher

// Tail plan of the fast kernel: when the last round of tiles over the CUs'
// workgroup slots is partial, split each of those tail tiles into kp K parts.
// K parts of each tail tile for row tiles of fm (1: no split).  fill: the
// tail fills one round of the slots (the measure gemm_tile_m compares row
// tiles by).  The split a launch runs (!fill) is the same for 256-row tiles
// (one workgroup per CU); the 64- and 128-row tiles (four / three slots per
// CU) split to about two workgroups per CU instead, and 128-row parts walk at
// least three K units: each part walks more of K and the tail writes fewer
// partial sums (same-box sweeps at m = 77 .. 1024: T5 q / up at m = 512 / 77
// -8 / -13 %, FLUX text proj at m = 512 -10 %, Qwen text Q3_K / Q4_K at
// m = 256 / 77 -12 / -14 / -11 %, 768 x 3072 -> 3072 Q4_K -17 %; a Q5_K
// m = 77 with 64-row parts of three units, and 256-row tiles kept to three
// units, measured slower).
static int64_t tail_kparts(int type, int64_t m, int64_t n, int64_t k, int cus, int fm, int64_t *rem_out,
                           bool fill) {
  const int fn = gemm_tile_n(fm);
  const int64_t tiles = ((m + fm - 1) / fm) * ((n + fn - 1) / fn);
  const int64_t slots = (int64_t)cus * gemm_wgs_per_cu(fm);
  const int64_t rem = tiles % slots;  // tiles of the last, partial round
  const int64_t units = k / gemm_unit_k(type);
  if (rem_out) *rem_out = rem;
  if (rem == 0 || units < 2) return 1;
  const bool two = !fill && fm != 256;
  int64_t kp = (two ? 2 * (int64_t)cus : slots) / rem;  // workgroups the tail aims at, per tail tile
  const int64_t max_parts = !fill && fm == 128 ? units / 3 : units;
  kp = kp < max_parts ? kp : max_parts;
  kp = kp < kGemmMaxKParts ? kp : kGemmMaxKParts;
  return kp < 2 ? 1 : kp;
}

// Rows per block tile.  256-row tiles decode each weight once per 256 rows of
// x; for small m most of such a tile is padding, so up to 128 rows the tile
// shrinks to 64 or 128 rows (more tiles, three or four workgroups per CU),
// from 129 to 256 rows to 128, and above 256 rows to 128 for some launches of
// one partial round (below).  Up to 128 rows the launch is latency-bound:
// its time follows the K units each workgroup walks after the tail split
// (measured on the T5 / FLUX / Qwen shapes at m = 77 and 128: 0.71-0.85 of the
// 256-row time), so the candidate with fewer units per workgroup wins, 64
// rows on a tie.
int gemm_tile_m(int type, int64_t m, int64_t n, int64_t k, int cus) {
  if (m > 256) {
    // One partial round of 256-row tiles (few row panels, e.g. the T5 encoder
    // and the DiT text streams at m = 512): 128-row tiles, three workgroups
    // per CU, fill more of the chip.  They win when the 256-row tiles are few
    // (at most a quarter of the CUs) and K short, or when the 256-row tiles must
    // split K while the 128-row ones need not (no partial sums to write and
    // add); elsewhere the 256 x 256 tile's efficiency wins (measured A/B:
    // 4096 -> 4096 at m = 512 / 768 / 1024 / 2048 +14 / +5 / +2 / +12 %,
    // 3072 -> 3072 at m = 768 +9 %; T5 up / down and FLUX text qkv at m = 512
    // 2-7 % slower with 128 rows, every large shape 3-18 % slower).
    const int64_t t256 = ((m + 255) / 256) * ((n + gemm_tile_n(256) - 1) / gemm_tile_n(256));
    if (t256 >= (int64_t)cus * gemm_wgs_per_cu(256)) return 256;
    const int64_t kp256 = tail_kparts(type, m, n, k, cus, 256, nullptr, true);
    const int64_t kp128 = tail_kparts(type, m, n, k, cus, 128, nullptr, true);
    if ((t256 <= cus / 4 && k <= 4096) || (kp256 >= 2 && kp128 == 1)) return 128;
    return 256;
  }
  if (m > 128) return 128;
  const int64_t units = k / gemm_unit_k(type);
  int best = 64;
  int64_t best_depth = -1;
  for (int fm : {64, 128}) {
    const int64_t kp = tail_kparts(type, m, n, k, cus, fm, nullptr, true);
    const int64_t depth = (units + kp - 1) / kp;
    if (best_depth < 0 || depth < best_depth) {
      best = fm;
      best_depth = depth;
    }
  }
  return best;
}

GemmTail gemm_tail_plan(int type, int64_t m, int64_t n, int64_t k, int cus, bool split) {
  const int fm = gemm_tile_m(type, m, n, k, cus);
  const int fn = gemm_tile_n(fm);
  const int64_t tiles = ((m + fm - 1) / fm) * ((n + fn - 1) / fn);
  GemmTail t{(int)tiles, 1, fm};
  if (!split) return t;
  int64_t rem = 0;
  const int64_t kp = tail_kparts(type, m, n, k, cus, fm, &rem, false);
  if (kp < 2) return t;
  t.full_tiles = (int)(tiles - rem);
  t.kparts = (int)kp;
  return t;
}

size_t gemm_tail_bytes(const GemmTail &t, int64_t m, int64_t n) {
  const int fn = gemm_tile_n(t.fm);
  const int64_t tiles = ((m + t.fm - 1) / t.fm) * ((n + fn - 1) / fn);
  if (t.kparts < 2) return 0;
  return (size_t)(tiles - t.full_tiles) * t.kparts * t.fm * fn * sizeof(float);
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
