// mq_common.h — GGUF block geometry, the device ("tiled planar") weight
// layout, and the exact per-type decoders shared by every kernel.
//
// Device layout.  GGUF blocks are byte-packed structs whose sizes (18, 34,
// 110, 210 bytes ...) leave most fields unaligned.  On upload each weight is
// split into one plane per block field and the rows are grouped into tiles of
// 64 (kRowTile).  For tile t, block b, row r (0..63) and byte j of field f:
//   * fields whose size is a multiple of 16 bytes are "chunked":
//       plane_f + (((t*nb + b)*(size/16) + j/16)*64 + r)*16 + j%16
//     so the 64 rows' 16-byte chunks lie next to each other (one 1 KiB,
//     fully coalesced wave load per chunk);
//   * small fields (2, 4, 12 bytes) are "records":
//       plane_f + ((t*nb + b)*64 + r)*size + j.
// Every 16-byte chunk is 16-byte aligned and every record is aligned to its
// natural size.  Rows past n in the last tile are zero bytes (zero scale, so
// they decode to 0).  The transform is a byte permutation: download inverts it.
//
// Decoders reproduce ggml's dequantize_row_* (restated in
// oracle/ggml_oracle.c) term for term: every product (f16 scale x small
// integer) is exact in f32 and at most one rounding follows, so results are
// bit-identical to candle's `QTensor::dequantize` for every input.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

constexpr int kRowTile = 64;
constexpr int kMaxFields = 5;

enum TypeId : int {
  F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8,
  Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, BF16 = 30
};

struct Field {
  int16_t off;   // byte offset inside the GGUF block
  int16_t size;  // bytes
};

struct TypeInfo {
  int id;
  int bs;        // elements per block
  int ts;        // bytes per block
  int nf;        // number of fields
  Field f[kMaxFields];
  const char *name;
};

// Field order follows the GGUF struct member order (ggml-common.h).
__host__ __device__ constexpr TypeInfo type_info(int id) {
  switch (id) {
    case Q4_0: return {Q4_0, 32, 18, 2, {{0, 2}, {2, 16}}, "Q4_0"};
    case Q4_1: return {Q4_1, 32, 20, 2, {{0, 4}, {4, 16}}, "Q4_1"};
    case Q5_0: return {Q5_0, 32, 22, 3, {{0, 2}, {2, 4}, {6, 16}}, "Q5_0"};
    case Q5_1: return {Q5_1, 32, 24, 3, {{0, 4}, {4, 4}, {8, 16}}, "Q5_1"};
    case Q8_0: return {Q8_0, 32, 34, 2, {{0, 2}, {2, 32}}, "Q8_0"};
    case Q2_K: return {Q2_K, 256, 84, 3, {{0, 16}, {16, 64}, {80, 4}}, "Q2_K"};
    case Q3_K: return {Q3_K, 256, 110, 4, {{0, 32}, {32, 64}, {96, 12}, {108, 2}}, "Q3_K"};
    case Q4_K: return {Q4_K, 256, 144, 3, {{0, 4}, {4, 12}, {16, 128}}, "Q4_K"};
    case Q5_K: return {Q5_K, 256, 176, 4, {{0, 4}, {4, 12}, {16, 32}, {48, 128}}, "Q5_K"};
    case Q6_K: return {Q6_K, 256, 210, 4, {{0, 128}, {128, 64}, {192, 16}, {208, 2}}, "Q6_K"};
    default: return {-1, 0, 0, 0, {}, "?"};
  }
}

__host__ __device__ constexpr bool is_quant(int id) { return type_info(id).bs > 0; }

// Geometry of one device-resident weight.
struct Geo {
  int64_t n;                   // rows (output features)
  int64_t k;                   // columns (input features)
  int64_t nb;                  // blocks per row
  int64_t ntiles;              // ceil(n / 64)
  int64_t plane[kMaxFields];   // byte offset of each field plane
  int64_t bytes;               // total device bytes
};

inline Geo make_geo(int id, int64_t n, int64_t k) {
  const TypeInfo ti = type_info(id);
  Geo g{};
  g.n = n;
  g.k = k;
  g.nb = k / ti.bs;
  g.ntiles = (n + kRowTile - 1) / kRowTile;
  int64_t off = 0;
  for (int f = 0; f < ti.nf; ++f) {
    g.plane[f] = off;
    off += g.ntiles * g.nb * kRowTile * ti.f[f].size;
    off = (off + 255) & ~int64_t(255);
  }
  g.bytes = off;
  return g;
}

// Address of byte j of field (size `size`, plane offset `plane`) of block b,
// row r of tile t.
__host__ __device__ inline int64_t field_offset(int64_t plane, int size, int64_t nb, int64_t t,
                                                int64_t b, int r, int j) {
  if ((size & 15) == 0)
    return plane + (((t * nb + b) * (size >> 4) + (j >> 4)) * kRowTile + r) * 16 + (j & 15);
  return plane + ((t * nb + b) * kRowTile + r) * size + j;
}

// ------------------------------------------------------------ device helpers

__device__ __forceinline__ float h2f(uint16_t u) {
  _Float16 h;
  __builtin_memcpy(&h, &u, 2);
  return (float)h;
}

template <typename T>
__device__ __forceinline__ T ld(const uint8_t *p) {
  return *reinterpret_cast<const T *>(p);
}

// Per-type accessor bound to one weight: base pointer + geometry.
struct WView {
  const uint8_t *base;
  int64_t nb;
  int64_t plane[kMaxFields];
};

template <int F, int SIZE>
__device__ __forceinline__ const uint8_t *fptr(const WView &w, int64_t t, int64_t b, int r, int j) {
  return w.base + field_offset(w.plane[F], SIZE, w.nb, t, b, r, j);
}

// 6-bit scale and min j of a Q4_K / Q5_K super-block (ggml get_scale_min_k4)
// from its 12 scale bytes as little-endian words s0, s1, s2.  For j < 4 they
// are the low 6 bits of bytes j and j + 4; for j >= 4 the nibbles of byte j + 4
// with the top 2 bits of bytes j - 4 and j: all eight at once as the bytes of
// four words, then byte j & 3 of the pair for j (word operations throughout:
// indexing the 12 bytes by a run-time j cost the dequantizer most of its time).
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &mn) {
  const uint32_t scw = j < 4 ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
  const uint32_t mw = j < 4 ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
  const int sh = 8 * (j & 3);
  sc = (int)((scw >> sh) & 0xFFu);
  mn = (int)((mw >> sh) & 0xFFu);
}

// Six-bit Q3_K scale j (0..15), still offset by 32 (ggml dequantize_row_q3_K),
// from the 12 scale bytes as words s0, s1, s2: the low 4 bits are the low
// (j < 8) or high nibble of byte j & 7, the high 2 bits are bits 2 (j >> 2)
// and up of byte 8 + (j & 3).
__device__ __forceinline__ int q3k_scale(int j, uint32_t s0, uint32_t s1, uint32_t s2) {
  const uint32_t lw = ((j & 4) ? s1 : s0) >> (4 * (j >> 3));
  const int low = (int)((lw >> (8 * (j & 3))) & 0xFu);
  const int high = (int)((s2 >> (8 * (j & 3) + 2 * (j >> 2))) & 3u);
  return low | (high << 4);
}

// Decode the 8 consecutive elements e0..e0+7 (e0 % 8 == 0) of block b of row
// r in tile t into f32, exactly as ggml's dequantize_row_* produces them.
template <int TYPE>
__device__ __forceinline__ void decode8(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]);

template <>
__device__ __forceinline__ void decode8<Q4_0>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const float d = h2f(ld<uint16_t>(fptr<0, 2>(w, t, b, r, 0)));
  const uint2 q = ld<uint2>(fptr<1, 16>(w, t, b, r, e0 & 15));
  const int sh = e0 >= 16 ? 4 : 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const int v = (int)((word >> (8 * (i & 3) + sh)) & 0xF) - 8;
    out[i] = (float)v * d;
  }
}

template <>
__device__ __forceinline__ void decode8<Q4_1>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const uint32_t dm = ld<uint32_t>(fptr<0, 4>(w, t, b, r, 0));
  const float d = h2f((uint16_t)(dm & 0xFFFF)), m = h2f((uint16_t)(dm >> 16));
  const uint2 q = ld<uint2>(fptr<1, 16>(w, t, b, r, e0 & 15));
  const int sh = e0 >= 16 ? 4 : 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const int v = (int)((word >> (8 * (i & 3) + sh)) & 0xF);
    out[i] = (float)v * d + m;
  }
}

template <>
__device__ __forceinline__ void decode8<Q5_0>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const float d = h2f(ld<uint16_t>(fptr<0, 2>(w, t, b, r, 0)));
  const uint32_t qh = ld<uint32_t>(fptr<1, 4>(w, t, b, r, 0));
  const uint2 q = ld<uint2>(fptr<2, 16>(w, t, b, r, e0 & 15));
  const int sh = e0 >= 16 ? 4 : 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const int lo = (int)((word >> (8 * (i & 3) + sh)) & 0xF);
    const int hi = (int)((qh >> (e0 + i)) & 1) << 4;
    out[i] = (float)((lo | hi) - 16) * d;
  }
}

template <>
__device__ __forceinline__ void decode8<Q5_1>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const uint32_t dm = ld<uint32_t>(fptr<0, 4>(w, t, b, r, 0));
  const float d = h2f((uint16_t)(dm & 0xFFFF)), m = h2f((uint16_t)(dm >> 16));
  const uint32_t qh = ld<uint32_t>(fptr<1, 4>(w, t, b, r, 0));
  const uint2 q = ld<uint2>(fptr<2, 16>(w, t, b, r, e0 & 15));
  const int sh = e0 >= 16 ? 4 : 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const int lo = (int)((word >> (8 * (i & 3) + sh)) & 0xF);
    const int hi = (int)((qh >> (e0 + i)) & 1) << 4;
    out[i] = (float)(lo | hi) * d + m;
  }
}

template <>
__device__ __forceinline__ void decode8<Q8_0>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const float d = h2f(ld<uint16_t>(fptr<0, 2>(w, t, b, r, 0)));
  const uint2 q = ld<uint2>(fptr<1, 32>(w, t, b, r, e0));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const int v = (int)(int8_t)((word >> (8 * (i & 3))) & 0xFF);
    out[i] = (float)v * d;
  }
}

template <>
__device__ __forceinline__ void decode8<Q2_K>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const uint32_t dm = ld<uint32_t>(fptr<2, 4>(w, t, b, r, 0));
  const float d = h2f((uint16_t)(dm & 0xFFFF)), dmin = h2f((uint16_t)(dm >> 16));
  const int sc = *fptr<0, 16>(w, t, b, r, e0 >> 4);
  const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
  const int byte0 = 32 * (e0 >> 7) + (e0 & 31);
  const int sh = 2 * ((e0 & 127) >> 5);
  const uint2 q = ld<uint2>(fptr<1, 64>(w, t, b, r, byte0));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const int v = (int)((word >> (8 * (i & 3) + sh)) & 3);
    out[i] = dl * (float)v - ml;
  }
}

template <>
__device__ __forceinline__ void decode8<Q3_K>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const float d = h2f(ld<uint16_t>(fptr<3, 2>(w, t, b, r, 0)));
  const uint8_t *sp = fptr<2, 12>(w, t, b, r, 0);
  const float dl = d * (float)(q3k_scale(e0 >> 4, ld<uint32_t>(sp), ld<uint32_t>(sp + 4), ld<uint32_t>(sp + 8)) - 32);
  const int byte0 = 32 * (e0 >> 7) + (e0 & 31);
  const int sh = 2 * ((e0 & 127) >> 5);
  const uint2 q = ld<uint2>(fptr<1, 64>(w, t, b, r, byte0));
  const uint2 hm = ld<uint2>(fptr<0, 32>(w, t, b, r, e0 & 31));
  const int hb = e0 >> 5;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    const uint32_t hword = i < 4 ? hm.x : hm.y;
    const int lo = (int)((word >> (8 * (i & 3) + sh)) & 3);
    const int h = (int)((hword >> (8 * (i & 3) + hb)) & 1);
    out[i] = dl * (float)(lo - (h ? 0 : 4));
  }
}

template <int FIVE>
__device__ __forceinline__ void decode8_k45(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const uint32_t dm = ld<uint32_t>(fptr<0, 4>(w, t, b, r, 0));
  const float d = h2f((uint16_t)(dm & 0xFFFF)), dmin = h2f((uint16_t)(dm >> 16));
  const uint8_t *sp = fptr<1, 12>(w, t, b, r, 0);
  int sc, mn;
  scale_min_k4(e0 >> 5, ld<uint32_t>(sp), ld<uint32_t>(sp + 4), ld<uint32_t>(sp + 8), sc, mn);
  const float d1 = d * (float)sc, m1 = dmin * (float)mn;
  const int g = e0 >> 6, hi = (e0 >> 5) & 1, l0 = e0 & 31;
  const uint2 q = ld<uint2>(fptr<FIVE ? 3 : 2, 128>(w, t, b, r, 32 * g + l0));
  uint2 qh = {0, 0};
  if (FIVE) qh = ld<uint2>(fptr<2, 32>(w, t, b, r, l0));
  const int hb = e0 >> 5;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t word = i < 4 ? q.x : q.y;
    int v = (int)((word >> (8 * (i & 3) + 4 * hi)) & 0xF);
    if (FIVE) {
      const uint32_t hword = i < 4 ? qh.x : qh.y;
      v += ((hword >> (8 * (i & 3) + hb)) & 1) ? 16 : 0;
    }
    out[i] = d1 * (float)v - m1;
  }
}

template <>
__device__ __forceinline__ void decode8<Q4_K>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  decode8_k45<0>(w, t, r, b, e0, out);
}

template <>
__device__ __forceinline__ void decode8<Q5_K>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  decode8_k45<1>(w, t, r, b, e0, out);
}

template <>
__device__ __forceinline__ void decode8<Q6_K>(const WView &w, int64_t t, int r, int64_t b, int e0, float out[8]) {
  const float d = h2f(ld<uint16_t>(fptr<3, 2>(w, t, b, r, 0)));
  const int H = e0 >> 7, p = (e0 & 127) >> 5, l0 = e0 & 31;
  const int sc = (int)(int8_t)*fptr<2, 16>(w, t, b, r, 8 * H + 2 * p + (l0 >> 4));
  const float ds = d * (float)sc;
  const uint2 ql = ld<uint2>(fptr<0, 128>(w, t, b, r, 64 * H + 32 * (p & 1) + l0));
  const uint2 qh = ld<uint2>(fptr<1, 64>(w, t, b, r, 32 * H + l0));
  const int lsh = (p >> 1) * 4, hsh = 2 * p;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lw = i < 4 ? ql.x : ql.y;
    const uint32_t hw = i < 4 ? qh.x : qh.y;
    const int lo = (int)((lw >> (8 * (i & 3) + lsh)) & 0xF);
    const int h = (int)((hw >> (8 * (i & 3) + hsh)) & 3);
    out[i] = ds * (float)((lo | (h << 4)) - 32);
  }
}

// Dispatch a functor templated on the weight type.
template <typename Fn>
inline bool dispatch_type(int id, Fn &&fn) {
  switch (id) {
    case Q4_0: fn.template operator()<Q4_0>(); return true;
    case Q4_1: fn.template operator()<Q4_1>(); return true;
    case Q5_0: fn.template operator()<Q5_0>(); return true;
    case Q5_1: fn.template operator()<Q5_1>(); return true;
    case Q8_0: fn.template operator()<Q8_0>(); return true;
    case Q2_K: fn.template operator()<Q2_K>(); return true;
    case Q3_K: fn.template operator()<Q3_K>(); return true;
    case Q4_K: fn.template operator()<Q4_K>(); return true;
    case Q5_K: fn.template operator()<Q5_K>(); return true;
    case Q6_K: fn.template operator()<Q6_K>(); return true;
    default: return false;
  }
}

inline WView make_view(const void *base, const Geo &g) {
  WView v{};
  v.base = static_cast<const uint8_t *>(base);
  v.nb = g.nb;
  for (int f = 0; f < kMaxFields; ++f) v.plane[f] = g.plane[f];
  return v;
}

}  // namespace mq
