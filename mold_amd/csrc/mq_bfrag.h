// mq_bfrag.h — per-type B-operand decoders for the fused dequant -> bf16 MFMA
// GEMM (v_mfma_f32_32x32x16_bf16).
//
// The GEMM walks K in "units" (256 weights for every type except Q8_0, whose
// unit is 128) split into steps of 64.  In a step a lane (l32 = lane % 32,
// h = lane / 32) supplies, for one weight row, 32 of the step's 64 K
// positions as four runs of 8 — one bf16x8 MFMA B fragment per 16-K slice S.
// Which 8-element chunk of the 64-element step slice S of half h holds is
// chunk(S, h); the A operand is read from LDS through the same map, so any
// permutation of K inside a step is allowed and each type picks the one that
// matches its GGUF bit layout (whole 16-byte loads, no nibble shuffling).
//
// Per type:
//   Raw              one row's packed bytes of one unit, held in registers;
//   load_prep(u)     loads the pieces prep() consumes (scales, d, ...);
//   reload<G>(u)     loads the pieces whose last use is step G — called for
//                    unit u+1 right after step G of unit u, so every weight
//                    load has about a unit of MFMA work to land;
//   prep()           unpacks the unit's scales into Sc once;
//   frag<G, S>()     the bf16x8 B fragment of slice S of step G (frag<G, S,
//                    f32x8>: the same eight weights exact in f32, for the GEMV).
// Every weight is produced as RNE_bf16 of the exact f32 value ggml's
// dequantize_row_* computes: each decoder uses one fma whose product is exact
// and whose addition is the one rounding ggml performs (or is exact).
#pragma once

#include "mq_kernels.h"

namespace mq {
namespace bfrag {

// Byte e of w as f32 (v_cvt_f32_ubyte{e}).
template <int E>
__device__ __forceinline__ float ub(uint32_t w) {
  return (float)((w >> (8 * E)) & 0xFFu);
}

// Signed byte e of w as f32.
template <int E>
__device__ __forceinline__ float sb(uint32_t w) {
  return (float)(int8_t)(w >> (8 * E));
}

// The words reaching fma8 are already masked per byte; keeping them opaque
// stops the compiler from folding that mask into each byte extraction, so
// every byte converts with one v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t opaque(uint32_t w) {
  asm volatile("" : "+v"(w));
  return w;
}

typedef float f32x8 __attribute__((ext_vector_type(8)));

// The eight weights of a fragment as u[i] * a + b before that fma is taken:
// the f32 GEMV forms x . w as a * (x . u) + b * sum(x), which saves the
// decode fma of every weight.
struct Lin8 {
  float u[8];
  float a, b;
};

// Eight fma(byte_e(word), a, b) for the bytes of two words: the exact f32
// weights (O = f32x8), those rounded to bf16 (O = bf16x8, the MFMA B
// fragment), or the bytes and (a, b) unapplied (O = Lin8).
template <typename O = bf16x8>
__device__ __forceinline__ O fma8(uint32_t w0, uint32_t w1, float a, float b) {
  w0 = opaque(w0);
  w1 = opaque(w1);
  if constexpr (__is_same(O, Lin8)) {
    return Lin8{{ub<0>(w0), ub<1>(w0), ub<2>(w0), ub<3>(w0), ub<0>(w1), ub<1>(w1), ub<2>(w1), ub<3>(w1)}, a, b};
  }
  float v[8];
  v[0] = __builtin_fmaf(ub<0>(w0), a, b);
  v[1] = __builtin_fmaf(ub<1>(w0), a, b);
  v[2] = __builtin_fmaf(ub<2>(w0), a, b);
  v[3] = __builtin_fmaf(ub<3>(w0), a, b);
  v[4] = __builtin_fmaf(ub<0>(w1), a, b);
  v[5] = __builtin_fmaf(ub<1>(w1), a, b);
  v[6] = __builtin_fmaf(ub<2>(w1), a, b);
  v[7] = __builtin_fmaf(ub<3>(w1), a, b);
  if constexpr (__is_same(O, f32x8)) {
    O r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = v[i];
    return r;
  } else {
    // one v_cvt_pk_bf16_f32 per adjacent pair, each into its own 32-bit lane
    // of the fragment (element-wise conversions were sometimes paired with a
    // zero register and reassembled with v_perm / v_alignbit)
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 p = __builtin_convertvector((f32x2){v[2 * j], v[2 * j + 1]}, bf16x2);
      __builtin_memcpy(&u[j], &p, 4);
    }
    O r;
    __builtin_memcpy(&r, u, 16);
    return r;
  }
}

// Words (x, y) for even slices, (z, w) for odd ones.
template <int S>
__device__ __forceinline__ uint32_t w0of(const uint4 &q) {
  return (S & 1) ? q.z : q.x;
}
template <int S>
__device__ __forceinline__ uint32_t w1of(const uint4 &q) {
  return (S & 1) ? q.w : q.y;
}

// Addresses in the tiled-planar layout (mq_common.h).
__device__ __forceinline__ const uint8_t *chunk_at(const WView &w, int f, int nchunks, int64_t t, int64_t b,
                                                   int c, int r) {
  return w.base + w.plane[f] + (((t * w.nb + b) * nchunks + c) * kRowTile + r) * 16;
}
__device__ __forceinline__ const uint8_t *rec_at(const WView &w, int f, int size, int64_t t, int64_t b, int r) {
  return w.base + w.plane[f] + ((t * w.nb + b) * kRowTile + r) * size;
}
// Weight loads; NT = nontemporal (for kernels that read each weight byte once:
// the streaming GEMV; the GEMM re-reads weight tiles through L2 and keeps the
// default).
template <bool NT = false>
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
  if constexpr (NT) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}
template <bool NT = false>
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
  else return *reinterpret_cast<const uint32_t *>(p);
}
template <bool NT = false>
__device__ __forceinline__ uint32_t ld2(const uint8_t *p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
  else return *reinterpret_cast<const uint16_t *>(p);
}

// chunk maps shared by several types
//   super-block types: lane half h holds offsets 16h..16h+15 and 32+16h..32+16h+15
//   32-element block types: lane half h holds block (2G + h), offsets 32h..32h+31
__device__ __forceinline__ constexpr int chunk_sb(int s, int h) { return 4 * (s >> 1) + 2 * h + (s & 1); }
__device__ __forceinline__ constexpr int chunk_b32(int s, int h) { return 4 * h + s; }

template <int TYPE>
struct T;

// ---------------------------------------------------------- Q4_K, Q5_K
// ggml dequantize_row_q4_K: for group g (64 weights) y = d*sc[2g]*(qs[32g+l] & 15) - dmin*m[2g]
// and y = d*sc[2g+1]*(qs[32g+l] >> 4) - dmin*m[2g+1], l = 0..31; 6-bit scales
// and mins unpacked by get_scale_min_k4.  Lane half h loads qs chunk 2g+h.
// ggml dequantize_row_q5_K adds a fifth bit: low nibbles of group g take
// qh[l] bit 2g, high nibbles bit 2g+1.  Lane half h loads qh chunk h.
template <int TYPE>
struct TK45 {
  static constexpr bool kFive = TYPE == Q5_K;
  static constexpr int kUnitK = 256;
  static constexpr int kQsField = kFive ? 3 : 2;
  __device__ static constexpr int chunk(int s, int h) { return chunk_sb(s, h); }
  struct Raw {
    uint4 q[4];
    uint4 qh;  // Q5_K only
    uint32_t dm, s0, s1, s2;
  };
  struct Sc {
    float d, dmin, d16;
    uint32_t sc03, m03, sc47, m47;
    uint4 qh;
  };
  template <bool NT = false>
  __device__ static void load_prep(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    r.dm = ld4<NT>(rec_at(w, 0, 4, t, u, row));
    const uint8_t *sp = rec_at(w, 1, 12, t, u, row);
    r.s0 = ld4<NT>(sp);
    r.s1 = ld4<NT>(sp + 4);
    r.s2 = ld4<NT>(sp + 8);
    if constexpr (kFive) r.qh = ld16<NT>(chunk_at(w, 2, 2, t, u, h, row));
  }
  template <int G, bool NT = false>
  __device__ static void reload(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    r.q[G] = ld16<NT>(chunk_at(w, kQsField, 8, t, u, 2 * G + h, row));
  }
  __device__ static void prep(const Raw &r, Sc &s, int) {
    s.d = h2f((uint16_t)(r.dm & 0xFFFF));
    s.dmin = h2f((uint16_t)(r.dm >> 16));
    s.d16 = kFive ? s.d : s.d * 0.0625f;
    s.sc03 = r.s0 & 0x3F3F3F3Fu;
    s.m03 = r.s1 & 0x3F3F3F3Fu;
    s.sc47 = (r.s2 & 0x0F0F0F0Fu) | ((r.s0 >> 2) & 0x30303030u);
    s.m47 = ((r.s2 >> 4) & 0x0F0F0F0Fu) | ((r.s1 >> 2) & 0x30303030u);
    if constexpr (kFive) s.qh = r.qh;
  }
  template <int G, int S, typename O = bf16x8>
  __device__ static O frag(const Raw &r, const Sc &s) {
    const uint32_t scw = G < 2 ? s.sc03 : s.sc47, mw = G < 2 ? s.m03 : s.m47;
    constexpr bool hi = S >= 2;
    constexpr int e = (2 * G + (hi ? 1 : 0)) & 3;
    // Q4_K high nibbles are masked in place (16*q): 1/16 is folded into d16 (exact)
    const float dl = (hi ? s.d16 : s.d) * ub<e>(scw), ml = s.dmin * ub<e>(mw);
    uint32_t a = w0of<S>(r.q[G]), b = w1of<S>(r.q[G]);
    if constexpr (!kFive) {
      const uint32_t M = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
      a &= M;
      b &= M;
    } else {
      constexpr int bit = 2 * G + (hi ? 1 : 0);
      const uint32_t ha = w0of<S>(s.qh), hb = w1of<S>(s.qh);
      a = ((hi ? a >> 4 : a) & 0x0F0F0F0Fu) | (((ha >> bit) & 0x01010101u) << 4);
      b = ((hi ? b >> 4 : b) & 0x0F0F0F0Fu) | (((hb >> bit) & 0x01010101u) << 4);
    }
    return fma8<O>(a, b, dl, -ml);
  }
};
template <>
struct T<Q4_K> : TK45<Q4_K> {};
template <>
struct T<Q5_K> : TK45<Q5_K> {};

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
  template <bool NT = false>
  __device__ static void load_prep(Raw &r, const WView &w, int64_t t, int row, int64_t u, int) {
    r.sc = ld16<NT>(chunk_at(w, 2, 1, t, u, 0, row));
    r.d = ld2<NT>(rec_at(w, 3, 2, t, u, row));
  }
  template <int G, bool NT = false>
  __device__ static void reload(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    if constexpr (G & 1) {  // the half's pieces are last used by step 2H+1
      constexpr int H = G >> 1;
      r.qla[H] = ld16<NT>(chunk_at(w, 0, 8, t, u, 4 * H + h, row));
      r.qlb[H] = ld16<NT>(chunk_at(w, 0, 8, t, u, 4 * H + 2 + h, row));
      r.qh[H] = ld16<NT>(chunk_at(w, 1, 4, t, u, 2 * H + h, row));
    }
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
  template <int G, int S, typename O = bf16x8>
  __device__ static O frag(const Raw &r, const Sc &s) {
    constexpr int H = G >> 1, p = 2 * (G & 1) + (S >> 1), sh = 4 * (G & 1);
    const uint4 &ql = (S >> 1) ? r.qlb[H] : r.qla[H];
    const uint32_t a = ((w0of<S>(ql) >> sh) & 0x0F0F0F0Fu) | (((w0of<S>(r.qh[H]) >> (2 * p)) & 0x03030303u) << 4);
    const uint32_t b = ((w1of<S>(ql) >> sh) & 0x0F0F0F0Fu) | (((w1of<S>(r.qh[H]) >> (2 * p)) & 0x03030303u) << 4);
    const float ds = s.ds[4 * H + p];
    // d*sc*(q-32) is exact in f32 (<= 24 significant bits): fma(q, ds, -32 ds)
    return fma8<O>(a, b, ds, -32.f * ds);
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
    uint4 hm;
  };
  template <bool NT = false>
  __device__ static void load_prep(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    r.hm = ld16<NT>(chunk_at(w, 0, 2, t, u, h, row));
    const uint8_t *sp = rec_at(w, 2, 12, t, u, row);
    r.s0 = ld4<NT>(sp);
    r.s1 = ld4<NT>(sp + 4);
    r.s2 = ld4<NT>(sp + 8);
    r.d = ld2<NT>(rec_at(w, 3, 2, t, u, row));
  }
  template <int G, bool NT = false>
  __device__ static void reload(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    if constexpr (G & 1) r.qs[G >> 1] = ld16<NT>(chunk_at(w, 1, 4, t, u, 2 * (G >> 1) + h, row));
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
    s.hm = r.hm;
  }
  template <int G, int S, typename O = bf16x8>
  __device__ static O frag(const Raw &r, const Sc &s) {
    constexpr int H = G >> 1, p = 2 * (G & 1) + (S >> 1), hb = 4 * H + p;
    // 3-bit value v = q2 + 4*hbit; weight = dl * (v - 4), exact
    const uint32_t a = ((w0of<S>(r.qs[H]) >> (2 * p)) & 0x03030303u) | (((w0of<S>(s.hm) >> hb) & 0x01010101u) << 2);
    const uint32_t b = ((w1of<S>(r.qs[H]) >> (2 * p)) & 0x03030303u) | (((w1of<S>(s.hm) >> hb) & 0x01010101u) << 2);
    const float dl = s.dl[4 * H + p];
    return fma8<O>(a, b, dl, -4.f * dl);
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
  template <bool NT = false>
  __device__ static void load_prep(Raw &r, const WView &w, int64_t t, int row, int64_t u, int) {
    r.sc = ld16<NT>(chunk_at(w, 0, 1, t, u, 0, row));
    r.dm = ld4<NT>(rec_at(w, 2, 4, t, u, row));
  }
  template <int G, bool NT = false>
  __device__ static void reload(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    if constexpr (G & 1) r.qs[G >> 1] = ld16<NT>(chunk_at(w, 1, 4, t, u, 2 * (G >> 1) + h, row));
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
  template <int G, int S, typename O = bf16x8>
  __device__ static O frag(const Raw &r, const Sc &s) {
    constexpr int H = G >> 1, p = 2 * (G & 1) + (S >> 1);
    constexpr uint32_t M = 0x03030303u;
    return fma8<O>((w0of<S>(r.qs[H]) >> (2 * p)) & M, (w1of<S>(r.qs[H]) >> (2 * p)) & M, s.dl[4 * H + p],
                -s.ml[4 * H + p]);
  }
};

// ------------------------------------------------------ 32-weight blocks
// Unit = 8 blocks (Q8_0: 4); in step G lane half h decodes block 2G + h, whose
// weights 0..31 fill slices 0..3 in order (chunk_b32).
//
// ggml dequantize_row_q4_0: y[j] = ((qs[j] & 15) - 8) * d, y[j+16] = ((qs[j] >> 4) - 8) * d.
// ggml dequantize_row_q4_1: y[j] = (qs[j] & 15) * d + m, y[j+16] = (qs[j] >> 4) * d + m.
// ggml dequantize_row_q5_0: y[j] = ((qs[j] & 15 | bit j of qh << 4) - 16) * d,
// y[j+16] = ((qs[j] >> 4 | bit j+16 of qh << 4) - 16) * d.  Q5_1: (..) * d + m.
template <int TYPE>
struct T32 {
  static constexpr int kUnitK = 256;
  static constexpr bool kMin = TYPE == Q4_1 || TYPE == Q5_1;
  static constexpr bool kFive = TYPE == Q5_0 || TYPE == Q5_1;
  static constexpr int kQsField = kFive ? 2 : 1;
  __device__ static constexpr int chunk(int s, int h) { return chunk_b32(s, h); }
  struct Raw {
    uint4 q[4];
    uint32_t d[4], qh[4];
  };
  struct Sc {};
  template <bool NT = false>
  __device__ static void load_prep(Raw &, const WView &, int64_t, int, int64_t, int) {}
  template <int G, bool NT = false>
  __device__ static void reload(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    const int64_t b = 8 * u + 2 * G + h;
    r.q[G] = ld16<NT>(chunk_at(w, kQsField, 1, t, b, 0, row));
    r.d[G] = kMin ? ld4<NT>(rec_at(w, 0, 4, t, b, row)) : ld2<NT>(rec_at(w, 0, 2, t, b, row));
    if constexpr (kFive) r.qh[G] = ld4<NT>(rec_at(w, 1, 4, t, b, row));
  }
  __device__ static void prep(const Raw &, Sc &, int) {}
  // bits sh..sh+3 of qh spread to bit 4 of bytes 0..3
  __device__ static uint32_t spread(uint32_t qh, int sh) {
    return ((((qh >> sh) & 15u) * 0x00204081u) & 0x01010101u) << 4;
  }
  template <int G, int S, typename O = bf16x8>
  __device__ static O frag(const Raw &r, const Sc &) {
    const float d = h2f((uint16_t)(r.d[G] & 0xFFFF));
    constexpr bool hi = S >= 2;
    uint32_t a = w0of<S>(r.q[G]), b = w1of<S>(r.q[G]);
    if constexpr (!kFive) {
      const float add = kMin ? h2f((uint16_t)(r.d[G] >> 16)) : -8.f * d;
      const uint32_t M = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
      // high nibbles masked in place are 16*q: scale by d/16 (exact)
      return fma8<O>(a & M, b & M, hi ? d * 0.0625f : d, add);
    } else {
      const float add = kMin ? h2f((uint16_t)(r.d[G] >> 16)) : -16.f * d;
      constexpr int bit0 = 16 * (S >> 1) + 8 * (S & 1);
      a = ((hi ? a >> 4 : a) & 0x0F0F0F0Fu) | spread(r.qh[G], bit0);
      b = ((hi ? b >> 4 : b) & 0x0F0F0F0Fu) | spread(r.qh[G], bit0 + 4);
      return fma8<O>(a, b, d, add);
    }
  }
};
template <>
struct T<Q4_0> : T32<Q4_0> {};
template <>
struct T<Q4_1> : T32<Q4_1> {};
template <>
struct T<Q5_0> : T32<Q5_0> {};
template <>
struct T<Q5_1> : T32<Q5_1> {};

// ggml dequantize_row_q8_0: y[j] = qs[j] * d.  The signed byte is read as
// u = q + 128 (xor 0x80) so that fma(u, d, -128 d) = q*d exactly; the Lin8
// form takes q itself (a = d, b = 0).
template <>
struct T<Q8_0> {
  static constexpr int kUnitK = 128;
  __device__ static constexpr int chunk(int s, int h) { return chunk_b32(s, h); }
  struct Raw {
    uint4 q[2][2];
    uint32_t d[2];
  };
  struct Sc {};
  template <bool NT = false>
  __device__ static void load_prep(Raw &, const WView &, int64_t, int, int64_t, int) {}
  template <int G, bool NT = false>
  __device__ static void reload(Raw &r, const WView &w, int64_t t, int row, int64_t u, int h) {
    const int64_t b = 4 * u + 2 * G + h;
    r.q[G][0] = ld16<NT>(chunk_at(w, 1, 2, t, b, 0, row));
    r.q[G][1] = ld16<NT>(chunk_at(w, 1, 2, t, b, 1, row));
    r.d[G] = ld2<NT>(rec_at(w, 0, 2, t, b, row));
  }
  __device__ static void prep(const Raw &, Sc &, int) {}
  template <int G, int S, typename O = bf16x8>
  __device__ static O frag(const Raw &r, const Sc &) {
    const float d = h2f((uint16_t)r.d[G]);
    constexpr uint32_t X = 0x80808080u;
    const uint4 &q = r.q[G][S >> 1];
    if constexpr (__is_same(O, Lin8)) {
      // the signed bytes themselves (v_cvt_f32_i32 of a sign-extended byte), b = 0
      const uint32_t w0 = opaque(w0of<S>(q)), w1 = opaque(w1of<S>(q));
      return Lin8{{sb<0>(w0), sb<1>(w0), sb<2>(w0), sb<3>(w0), sb<0>(w1), sb<1>(w1), sb<2>(w1), sb<3>(w1)}, d, 0.f};
    }
    return fma8<O>(w0of<S>(q) ^ X, w1of<S>(q) ^ X, d, -128.f * d);
  }
};

}  // namespace bfrag
}  // namespace mq
