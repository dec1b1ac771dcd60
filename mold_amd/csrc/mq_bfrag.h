// mq_bfrag.h — per-type B-operand decoders for the fused dequant -> bf16 MFMA
// GEMM (v_mfma_f32_32x32x16_bf16).
//
// The GEMM walks K in "units" (256 weights for every type except Q8_0, whose
// unit is 128) split into steps of 64.  In a step a lane (l32 = lane % 32,
// h = lane / 32) supplies, for one weight row, 32 of the step's 64 K
// positions as four runs of 8 — one bf16x8 MFMA B fragment per 16-K slice s.
// Which 8-element chunk of the 64-element step slice s of half h holds is
// chunk(s, h); the A operand is read from LDS through the same map, so any
// permutation of K inside a step is allowed and each type picks the one that
// matches its GGUF bit layout (whole 16-byte loads, no nibble shuffling).
//
// Raw holds one row's packed bytes for a whole unit (loaded one unit ahead);
// decode<G> turns step G of it into bf16.  Every weight is produced as
// RNE_bf16 of the exact f32 value ggml's dequantize_row_* computes: each
// decoder uses one fma whose product is exact and whose sum is the one
// rounding ggml performs (or is exact), so the bf16 operand equals the
// bf16-rounded dequantized weight.
#pragma once

#include "mq_kernels.h"

namespace mq {
namespace bfrag {

// Byte e of w as f32 (v_cvt_f32_ubyte{e}).
template <int E>
__device__ __forceinline__ float ub(uint32_t w) {
  return (float)((w >> (8 * E)) & 0xFFu);
}

__device__ __forceinline__ bf16x8 pack8(const float v[8]) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)v[i];
  return r;
}

// The words reaching fma8 are already masked per byte; keeping them opaque
// stops the compiler from folding that mask into each byte extraction, so
// every byte converts with one v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t opaque(uint32_t w) {
  asm volatile("" : "+v"(w));
  return w;
}

// Eight fma(byte_e(word), a, b) for the bytes of two words, as bf16.
__device__ __forceinline__ bf16x8 fma8(uint32_t w0, uint32_t w1, float a, float b) {
  w0 = opaque(w0);
  w1 = opaque(w1);
  float v[8];
  v[0] = __builtin_fmaf(ub<0>(w0), a, b);
  v[1] = __builtin_fmaf(ub<1>(w0), a, b);
  v[2] = __builtin_fmaf(ub<2>(w0), a, b);
  v[3] = __builtin_fmaf(ub<3>(w0), a, b);
  v[4] = __builtin_fmaf(ub<0>(w1), a, b);
  v[5] = __builtin_fmaf(ub<1>(w1), a, b);
  v[6] = __builtin_fmaf(ub<2>(w1), a, b);
  v[7] = __builtin_fmaf(ub<3>(w1), a, b);
  return pack8(v);
}

// Addresses in the tiled-planar layout (mq_common.h).
__device__ __forceinline__ const uint8_t *chunk_at(const WView &w, int f, int nchunks, int64_t t, int64_t b,
                                                   int c, int r) {
  return w.base + w.plane[f] + (((t * w.nb + b) * nchunks + c) * kRowTile + r) * 16;
}
__device__ __forceinline__ const uint8_t *rec_at(const WView &w, int f, int size, int64_t t, int64_t b, int r) {
  return w.base + w.plane[f] + ((t * w.nb + b) * kRowTile + r) * size;
}
__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ uint32_t ld2(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

// chunk maps shared by several types
//   super-block types: lane half h holds offsets 16h..16h+15 and 32+16h..32+16h+15
//   32-element block types: lane half h holds block (2g + h), offsets 32h..32h+31
__device__ __forceinline__ constexpr int chunk_sb(int s, int h) { return 4 * (s >> 1) + 2 * h + (s & 1); }
__device__ __forceinline__ constexpr int chunk_b32(int s, int h) { return 4 * h + s; }

template <int TYPE>
struct T;

// ---------------------------------------------------------------- Q4_K
// ggml dequantize_row_q4_K: for group g (64 weights) y = d*sc[2g]*(qs[32g+l] & 15) - dmin*m[2g]
// and y = d*sc[2g+1]*(qs[32g+l] >> 4) - dmin*m[2g+1], l = 0..31; 6-bit scales
// and mins unpacked by get_scale_min_k4.  Lane half h loads qs chunk 2g+h.
template <>
struct T<Q4_K> {
  static constexpr int kUnitK = 256;
  __device__ static constexpr int chunk(int s, int h) { return chunk_sb(s, h); }
  struct Raw {
    uint4 q[4];
    uint32_t dm, s0, s1, s2;
  };
  struct Sc {
    float d, dmin, d16;
    uint32_t sc03, m03, sc47, m47;
  };
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r.q[g] = ld16(chunk_at(w, 2, 8, t, u, 2 * g + h, row));
    r.dm = ld4(rec_at(w, 0, 4, t, u, row));
    const uint8_t *sp = rec_at(w, 1, 12, t, u, row);
    r.s0 = ld4(sp);
    r.s1 = ld4(sp + 4);
    r.s2 = ld4(sp + 8);
  }
  __device__ static void prep(const Raw &r, Sc &s, int) {
    s.d = h2f((uint16_t)(r.dm & 0xFFFF));
    s.dmin = h2f((uint16_t)(r.dm >> 16));
    s.d16 = s.d * 0.0625f;
    s.sc03 = r.s0 & 0x3F3F3F3Fu;
    s.m03 = r.s1 & 0x3F3F3F3Fu;
    s.sc47 = (r.s2 & 0x0F0F0F0Fu) | ((r.s0 >> 2) & 0x30303030u);
    s.m47 = ((r.s2 >> 4) & 0x0F0F0F0Fu) | ((r.s1 >> 2) & 0x30303030u);
  }
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &s, bf16x8 f[4]) {
    const uint32_t scw = G < 2 ? s.sc03 : s.sc47, mw = G < 2 ? s.m03 : s.m47;
    constexpr int e0 = (2 * G) & 3, e1 = (2 * G + 1) & 3;
    const float dlo = s.d * ub<e0>(scw), mlo = s.dmin * ub<e0>(mw);
    // high nibbles are masked in place (16*q): fold 1/16 into the scale (exact)
    const float dhi = s.d16 * ub<e1>(scw), mhi = s.dmin * ub<e1>(mw);
    const uint4 q = r.q[G];
    f[0] = fma8(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, dlo, -mlo);
    f[1] = fma8(q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu, dlo, -mlo);
    f[2] = fma8(q.x & 0xF0F0F0F0u, q.y & 0xF0F0F0F0u, dhi, -mhi);
    f[3] = fma8(q.z & 0xF0F0F0F0u, q.w & 0xF0F0F0F0u, dhi, -mhi);
  }
};

// ---------------------------------------------------------------- Q5_K
// As Q4_K with a fifth bit: low nibbles of group g take qh[l] bit 2g, high
// nibbles bit 2g+1 (ggml dequantize_row_q5_K).  Lane half h loads qh chunk h.
template <>
struct T<Q5_K> {
  static constexpr int kUnitK = 256;
  __device__ static constexpr int chunk(int s, int h) { return chunk_sb(s, h); }
  struct Raw {
    uint4 q[4];
    uint4 qh;
    uint32_t dm, s0, s1, s2;
  };
  using Sc = T<Q4_K>::Sc;
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
#pragma unroll
    for (int g = 0; g < 4; ++g) r.q[g] = ld16(chunk_at(w, 3, 8, t, u, 2 * g + h, row));
    r.qh = ld16(chunk_at(w, 2, 2, t, u, h, row));
    r.dm = ld4(rec_at(w, 0, 4, t, u, row));
    const uint8_t *sp = rec_at(w, 1, 12, t, u, row);
    r.s0 = ld4(sp);
    r.s1 = ld4(sp + 4);
    r.s2 = ld4(sp + 8);
  }
  __device__ static void prep(const Raw &r, Sc &s, int) {
    s.d = h2f((uint16_t)(r.dm & 0xFFFF));
    s.dmin = h2f((uint16_t)(r.dm >> 16));
    s.d16 = s.d;
    s.sc03 = r.s0 & 0x3F3F3F3Fu;
    s.m03 = r.s1 & 0x3F3F3F3Fu;
    s.sc47 = (r.s2 & 0x0F0F0F0Fu) | ((r.s0 >> 2) & 0x30303030u);
    s.m47 = ((r.s2 >> 4) & 0x0F0F0F0Fu) | ((r.s1 >> 2) & 0x30303030u);
  }
  template <int B>
  __device__ static uint32_t lo5(uint32_t q, uint32_t qh) {
    return (q & 0x0F0F0F0Fu) | (((qh >> B) & 0x01010101u) << 4);
  }
  template <int B>
  __device__ static uint32_t hi5(uint32_t q, uint32_t qh) {
    return ((q >> 4) & 0x0F0F0F0Fu) | (((qh >> B) & 0x01010101u) << 4);
  }
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &s, bf16x8 f[4]) {
    const uint32_t scw = G < 2 ? s.sc03 : s.sc47, mw = G < 2 ? s.m03 : s.m47;
    constexpr int e0 = (2 * G) & 3, e1 = (2 * G + 1) & 3;
    const float dlo = s.d * ub<e0>(scw), mlo = s.dmin * ub<e0>(mw);
    const float dhi = s.d * ub<e1>(scw), mhi = s.dmin * ub<e1>(mw);
    const uint4 q = r.q[G], qh = r.qh;
    constexpr int b0 = 2 * G, b1 = 2 * G + 1;
    f[0] = fma8(lo5<b0>(q.x, qh.x), lo5<b0>(q.y, qh.y), dlo, -mlo);
    f[1] = fma8(lo5<b0>(q.z, qh.z), lo5<b0>(q.w, qh.w), dlo, -mlo);
    f[2] = fma8(hi5<b1>(q.x, qh.x), hi5<b1>(q.y, qh.y), dhi, -mhi);
    f[3] = fma8(hi5<b1>(q.z, qh.z), hi5<b1>(q.w, qh.w), dhi, -mhi);
  }
};

// ---------------------------------------------------------------- Q6_K
// ggml dequantize_row_q6_K, per 128-weight half H: weight 32p + l (p = 0..3,
// l = 0..31) is d * sc[8H + 2p + l/16] * (q - 32) with q = 4 bits of
// ql[64H + 32(p&1) + l] (low nibble for p < 2) | 2 bits (2p) of qh[32H + l].
// Step G covers H = G/2, p = 2(G&1) and 2(G&1)+1.  Lane half h holds
// l = 16h..16h+15: ql chunks 4H+h and 4H+2+h, qh chunk 2H+h, scales 8H+2p+h.
template <>
struct T<Q6_K> {
  static constexpr int kUnitK = 256;
  __device__ static constexpr int chunk(int s, int h) { return chunk_sb(s, h); }
  struct Raw {
    uint4 qla[2], qlb[2], qh[2];
    uint4 sc;
    uint32_t d;
  };
  struct Sc {
    float ds[8];  // d*sc for (H, p) = index 4H + p
  };
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
#pragma unroll
    for (int H = 0; H < 2; ++H) {
      r.qla[H] = ld16(chunk_at(w, 0, 8, t, u, 4 * H + h, row));
      r.qlb[H] = ld16(chunk_at(w, 0, 8, t, u, 4 * H + 2 + h, row));
      r.qh[H] = ld16(chunk_at(w, 1, 4, t, u, 2 * H + h, row));
    }
    r.sc = ld16(chunk_at(w, 2, 1, t, u, 0, row));
    r.d = ld2(rec_at(w, 3, 2, t, u, row));
  }
  __device__ static void prep(const Raw &r, Sc &s, int h) {
    const float d = h2f((uint16_t)r.d);
    const uint32_t sw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        // scale byte 8H + 2p + h = word 2H + p/2, byte 2(p&1) + h
        const int32_t v = (int8_t)(sw[2 * H + (p >> 1)] >> (8 * (2 * (p & 1) + h)));
        s.ds[4 * H + p] = d * (float)v;
      }
  }
  template <int SH, int HB>
  __device__ static uint32_t q6(uint32_t ql, uint32_t qh) {
    return ((ql >> SH) & 0x0F0F0F0Fu) | (((qh >> HB) & 0x03030303u) << 4);
  }
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &s, bf16x8 f[4]) {
    constexpr int H = G >> 1, p0 = 2 * (G & 1), p1 = p0 + 1, sh = 4 * (G & 1);
    const uint4 a = r.qla[H], b = r.qlb[H], qh = r.qh[H];
    const float d0 = s.ds[4 * H + p0], d1 = s.ds[4 * H + p1];
    // d*sc*(q-32) is exact in f32 (<= 24 significant bits): fma(q, ds, -32 ds)
    f[0] = fma8(q6<sh, 2 * p0>(a.x, qh.x), q6<sh, 2 * p0>(a.y, qh.y), d0, -32.f * d0);
    f[1] = fma8(q6<sh, 2 * p0>(a.z, qh.z), q6<sh, 2 * p0>(a.w, qh.w), d0, -32.f * d0);
    f[2] = fma8(q6<sh, 2 * p1>(b.x, qh.x), q6<sh, 2 * p1>(b.y, qh.y), d1, -32.f * d1);
    f[3] = fma8(q6<sh, 2 * p1>(b.z, qh.z), q6<sh, 2 * p1>(b.w, qh.w), d1, -32.f * d1);
  }
};

// ---------------------------------------------------------------- Q3_K
// ggml dequantize_row_q3_K: weight 128H + 32p + l is
// d * (sc6[8H + 2p + l/16] - 32) * (((qs[32H + l] >> 2p) & 3) - (hmask[l] bit (4H+p) ? 0 : 4)).
template <>
struct T<Q3_K> {
  static constexpr int kUnitK = 256;
  __device__ static constexpr int chunk(int s, int h) { return chunk_sb(s, h); }
  struct Raw {
    uint4 qs[2];  // chunk 2H + h
    uint4 hm;     // hmask chunk h
    uint32_t s0, s1, s2, d;
  };
  struct Sc {
    float dl[8];  // d*(sc-32) for (H, p) = 4H + p
  };
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    r.qs[0] = ld16(chunk_at(w, 1, 4, t, u, h, row));
    r.qs[1] = ld16(chunk_at(w, 1, 4, t, u, 2 + h, row));
    r.hm = ld16(chunk_at(w, 0, 2, t, u, h, row));
    const uint8_t *sp = rec_at(w, 2, 12, t, u, row);
    r.s0 = ld4(sp);
    r.s1 = ld4(sp + 4);
    r.s2 = ld4(sp + 8);
    r.d = ld2(rec_at(w, 3, 2, t, u, row));
  }
  __device__ static void prep(const Raw &r, Sc &s, int h) {
    const float d = h2f((uint16_t)r.d);
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        // j = 8H + 2p + h: low 4 bits from byte (2p + h) of s0/s1 (nibble H),
        // high 2 bits from byte 2(p&1)+h of s2, bit pair 2H + p/2.
        const int byte = 2 * (p & 1) + h;
        const uint32_t lw = (p >> 1) ? r.s1 : r.s0;
        const uint32_t lo = (lw >> (8 * byte + 4 * H)) & 15u;
        const uint32_t hi = (r.s2 >> (8 * byte + 2 * (2 * H + (p >> 1)))) & 3u;
        s.dl[4 * H + p] = d * (float)((int)(lo | (hi << 4)) - 32);
      }
  }
  template <int SH, int HB>
  __device__ static uint32_t q3(uint32_t qs, uint32_t hm) {
    // 3-bit value v = q2 + 4*hbit; weight = dl * (v - 4)
    return ((qs >> SH) & 0x03030303u) | (((hm >> HB) & 0x01010101u) << 2);
  }
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &s, bf16x8 f[4]) {
    constexpr int H = G >> 1, p0 = 2 * (G & 1), p1 = p0 + 1;
    const uint4 q = r.qs[H], hm = r.hm;
    const float d0 = s.dl[4 * H + p0], d1 = s.dl[4 * H + p1];
    f[0] = fma8(q3<2 * p0, 4 * H + p0>(q.x, hm.x), q3<2 * p0, 4 * H + p0>(q.y, hm.y), d0, -4.f * d0);
    f[1] = fma8(q3<2 * p0, 4 * H + p0>(q.z, hm.z), q3<2 * p0, 4 * H + p0>(q.w, hm.w), d0, -4.f * d0);
    f[2] = fma8(q3<2 * p1, 4 * H + p1>(q.x, hm.x), q3<2 * p1, 4 * H + p1>(q.y, hm.y), d1, -4.f * d1);
    f[3] = fma8(q3<2 * p1, 4 * H + p1>(q.z, hm.z), q3<2 * p1, 4 * H + p1>(q.w, hm.w), d1, -4.f * d1);
  }
};

// ---------------------------------------------------------------- Q2_K
// ggml dequantize_row_q2_K: weight 128H + 32p + l is
// d*(sc[8H+2p+l/16] & 15) * ((qs[32H + l] >> 2p) & 3) - dmin*(sc[..] >> 4).
template <>
struct T<Q2_K> {
  static constexpr int kUnitK = 256;
  __device__ static constexpr int chunk(int s, int h) { return chunk_sb(s, h); }
  struct Raw {
    uint4 qs[2];
    uint4 sc;
    uint32_t dm;
  };
  struct Sc {
    float dl[8], ml[8];
  };
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    r.qs[0] = ld16(chunk_at(w, 1, 4, t, u, h, row));
    r.qs[1] = ld16(chunk_at(w, 1, 4, t, u, 2 + h, row));
    r.sc = ld16(chunk_at(w, 0, 1, t, u, 0, row));
    r.dm = ld4(rec_at(w, 2, 4, t, u, row));
  }
  __device__ static void prep(const Raw &r, Sc &s, int h) {
    const float d = h2f((uint16_t)(r.dm & 0xFFFF)), dmin = h2f((uint16_t)(r.dm >> 16));
    const uint32_t sw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
#pragma unroll
    for (int H = 0; H < 2; ++H)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t v = (sw[2 * H + (p >> 1)] >> (8 * (2 * (p & 1) + h))) & 0xFFu;
        s.dl[4 * H + p] = d * (float)(v & 15);
        s.ml[4 * H + p] = dmin * (float)(v >> 4);
      }
  }
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &s, bf16x8 f[4]) {
    constexpr int H = G >> 1, p0 = 2 * (G & 1), p1 = p0 + 1;
    const uint4 q = r.qs[H];
    const float d0 = s.dl[4 * H + p0], m0 = s.ml[4 * H + p0];
    const float d1 = s.dl[4 * H + p1], m1 = s.ml[4 * H + p1];
    constexpr uint32_t M = 0x03030303u;
    f[0] = fma8((q.x >> 2 * p0) & M, (q.y >> 2 * p0) & M, d0, -m0);
    f[1] = fma8((q.z >> 2 * p0) & M, (q.w >> 2 * p0) & M, d0, -m0);
    f[2] = fma8((q.x >> 2 * p1) & M, (q.y >> 2 * p1) & M, d1, -m1);
    f[3] = fma8((q.z >> 2 * p1) & M, (q.w >> 2 * p1) & M, d1, -m1);
  }
};

// ------------------------------------------------------ 32-weight blocks
// Unit = 8 blocks (Q8_0: 4); in step G lane half h decodes block 2G + h, whose
// weights 0..31 fill slices 0..3 in order (chunk_b32).

// ggml dequantize_row_q4_0: y[j] = ((qs[j] & 15) - 8) * d, y[j+16] = ((qs[j] >> 4) - 8) * d.
// ggml dequantize_row_q4_1: y[j] = (qs[j] & 15) * d + m, y[j+16] = (qs[j] >> 4) * d + m.
template <int TYPE>
struct T4_32 {
  static constexpr int kUnitK = 256;
  static constexpr bool kMin = TYPE == Q4_1;
  __device__ static constexpr int chunk(int s, int h) { return chunk_b32(s, h); }
  struct Raw {
    uint4 q[4];
    uint32_t d[4];
  };
  struct Sc {};
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t b = 8 * u + 2 * g + h;
      r.q[g] = ld16(chunk_at(w, 1, 1, t, b, 0, row));
      r.d[g] = kMin ? ld4(rec_at(w, 0, 4, t, b, row)) : ld2(rec_at(w, 0, 2, t, b, row));
    }
  }
  __device__ static void prep(const Raw &, Sc &, int) {}
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &, bf16x8 f[4]) {
    const float d = h2f((uint16_t)(r.d[G] & 0xFFFF));
    const float lo_b = kMin ? h2f((uint16_t)(r.d[G] >> 16)) : -8.f * d;
    const float d16 = d * 0.0625f;
    const uint4 q = r.q[G];
    f[0] = fma8(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, d, lo_b);
    f[1] = fma8(q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu, d, lo_b);
    f[2] = fma8(q.x & 0xF0F0F0F0u, q.y & 0xF0F0F0F0u, d16, lo_b);
    f[3] = fma8(q.z & 0xF0F0F0F0u, q.w & 0xF0F0F0F0u, d16, lo_b);
  }
};
template <>
struct T<Q4_0> : T4_32<Q4_0> {};
template <>
struct T<Q4_1> : T4_32<Q4_1> {};

// ggml dequantize_row_q5_0: y[j] = ((qs[j] & 15 | bit j of qh << 4) - 16) * d,
// y[j+16] = ((qs[j] >> 4 | bit j+16 of qh << 4) - 16) * d.  Q5_1: (..) * d + m.
template <int TYPE>
struct T5_32 {
  static constexpr int kUnitK = 256;
  static constexpr bool kMin = TYPE == Q5_1;
  __device__ static constexpr int chunk(int s, int h) { return chunk_b32(s, h); }
  struct Raw {
    uint4 q[4];
    uint32_t d[4], qh[4];
  };
  struct Sc {};
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t b = 8 * u + 2 * g + h;
      r.q[g] = ld16(chunk_at(w, 2, 1, t, b, 0, row));
      r.d[g] = kMin ? ld4(rec_at(w, 0, 4, t, b, row)) : ld2(rec_at(w, 0, 2, t, b, row));
      r.qh[g] = ld4(rec_at(w, 1, 4, t, b, row));
    }
  }
  __device__ static void prep(const Raw &, Sc &, int) {}
  // bits 4i..4i+3 of qh spread to bit 4 of bytes 0..3
  __device__ static uint32_t spread(uint32_t qh, int sh) {
    return ((((qh >> sh) & 15u) * 0x00204081u) & 0x01010101u) << 4;
  }
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &, bf16x8 f[4]) {
    const float d = h2f((uint16_t)(r.d[G] & 0xFFFF));
    const float b = kMin ? h2f((uint16_t)(r.d[G] >> 16)) : -16.f * d;
    const uint4 q = r.q[G];
    const uint32_t qh = r.qh[G];
    constexpr uint32_t L = 0x0F0F0F0Fu;
    f[0] = fma8((q.x & L) | spread(qh, 0), (q.y & L) | spread(qh, 4), d, b);
    f[1] = fma8((q.z & L) | spread(qh, 8), (q.w & L) | spread(qh, 12), d, b);
    f[2] = fma8(((q.x >> 4) & L) | spread(qh, 16), ((q.y >> 4) & L) | spread(qh, 20), d, b);
    f[3] = fma8(((q.z >> 4) & L) | spread(qh, 24), ((q.w >> 4) & L) | spread(qh, 28), d, b);
  }
};
template <>
struct T<Q5_0> : T5_32<Q5_0> {};
template <>
struct T<Q5_1> : T5_32<Q5_1> {};

// ggml dequantize_row_q8_0: y[j] = qs[j] * d.  The signed byte is read as
// u = q + 128 (xor 0x80) so that fma(u, d, -128 d) = q*d exactly.
template <>
struct T<Q8_0> {
  static constexpr int kUnitK = 128;
  __device__ static constexpr int chunk(int s, int h) { return chunk_b32(s, h); }
  struct Raw {
    uint4 q[2][2];
    uint32_t d[2];
  };
  struct Sc {};
  __device__ static void load(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int64_t b = 4 * u + 2 * g + h;
      r.q[g][0] = ld16(chunk_at(w, 1, 2, t, b, 0, row));
      r.q[g][1] = ld16(chunk_at(w, 1, 2, t, b, 1, row));
      r.d[g] = ld2(rec_at(w, 0, 2, t, b, row));
    }
  }
  __device__ static void prep(const Raw &, Sc &, int) {}
  template <int G>
  __device__ static void decode(const Raw &r, const Sc &, bf16x8 f[4]) {
    const float d = h2f((uint16_t)r.d[G]);
    const float b = -128.f * d;
    constexpr uint32_t X = 0x80808080u;
    const uint4 a = r.q[G][0], c = r.q[G][1];
    f[0] = fma8(a.x ^ X, a.y ^ X, d, b);
    f[1] = fma8(a.z ^ X, a.w ^ X, d, b);
    f[2] = fma8(c.x ^ X, c.y ^ X, d, b);
    f[3] = fma8(c.z ^ X, c.w ^ X, d, b);
  }
};

}  // namespace bfrag
}  // namespace mq
