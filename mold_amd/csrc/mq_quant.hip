// mq_quant.hip — f32 [n, k] on the device -> GGUF blocks (candle
// QTensor::quantize / quantize_onto, called by mold at
// crates/mold-inference/src/flux/pipeline.rs:219-229 (FP8 -> Q8_0 cache) and
// crates/mold-inference/src/flux/lora.rs:849 (LoRA re-quantize)).
//
// The block contents follow ggml's reference quantizers (quantize_row_*_ref,
// make_qx_quants, make_q3_quants, make_qkx2_quants; ggml, MIT License,
// Copyright (c) 2023-2024 The ggml authors).  To produce byte-identical
// blocks the arithmetic is performed in the same order with IEEE
// single-precision operations: FMA contraction is disabled in this file,
// divisions and square roots are the correctly rounded ones, and
// nearest_int() uses the same 1.5*2^23 magic add.  Byte identity is held
// against that ggml restatement only.  Whether candle's k_quants port makes
// the same bytes is unpinned: its source is not available here, and its
// Q2_K/Q4_K/Q5_K from_float may use make_qkx1_quants instead of
// make_qkx2_quants.  Q4_0/Q4_1/Q5_0/Q5_1/Q8_0 have a single formula.
// One thread quantizes one block; raw blocks go to a staging buffer that the
// upload path then permutes into the tiled device layout.
#include <utility>

#include "mq_kernels.h"

#pragma clang fp contract(off)

namespace mq {
namespace {

constexpr float kGroupMaxEps = 1e-15f;

__device__ __forceinline__ int nearest_int(float f) {
  const float v = f + 12582912.f;
  int i;
  __builtin_memcpy(&i, &v, 4);
  return (i & 0x007fffff) - 0x00400000;
}

// f32 -> f16, round to nearest even.  The empty asm pins `f` in a register:
// without it the backend folds a preceding multiply into the conversion as
// v_fma_mix(a, b, +0), which turns a -0 product (e.g. 0 * -1/8 for an all-zero
// Q4_0 block) into +0 and changes the stored scale bits.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm volatile("" : "+v"(f));
  _Float16 h = (_Float16)f;
  uint16_t u;
  __builtin_memcpy(&u, &h, 2);
  return u;
}

__device__ __forceinline__ void put16(uint8_t *p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xFF);
  p[1] = (uint8_t)(v >> 8);
}

template <typename T>
__device__ __forceinline__ T mn(T a, T b) { return a < b ? a : b; }
template <typename T>
__device__ __forceinline__ T mx(T a, T b) { return a > b ? a : b; }

// ------------------------------------------------------------ 32-element types

__device__ void q_q4_0(const float *x, uint8_t *o) {
  float amax = 0.f, vmax = 0.f;
  for (int j = 0; j < 32; ++j)
    if (amax < fabsf(x[j])) { amax = fabsf(x[j]); vmax = x[j]; }
  const float d = vmax / -8;
  const float id = d ? 1.0f / d : 0.0f;
  put16(o, f2h(d));
  for (int j = 0; j < 16; ++j) {
    const float x0 = x[j] * id, x1 = x[16 + j] * id;
    const uint8_t a = (uint8_t)mn<int>(15, (int8_t)(x0 + 8.5f));
    const uint8_t b = (uint8_t)mn<int>(15, (int8_t)(x1 + 8.5f));
    o[2 + j] = (uint8_t)(a | (b << 4));
  }
}

__device__ void q_q4_1(const float *x, uint8_t *o) {
  float vmin = 3.402823466e+38f, vmax = -3.402823466e+38f;
  for (int j = 0; j < 32; ++j) {
    if (x[j] < vmin) vmin = x[j];
    if (x[j] > vmax) vmax = x[j];
  }
  const float d = (vmax - vmin) / 15;
  const float id = d ? 1.0f / d : 0.0f;
  put16(o, f2h(d));
  put16(o + 2, f2h(vmin));
  for (int j = 0; j < 16; ++j) {
    const float x0 = (x[j] - vmin) * id, x1 = (x[16 + j] - vmin) * id;
    const uint8_t a = (uint8_t)mn<int>(15, (int8_t)(x0 + 0.5f));
    const uint8_t b = (uint8_t)mn<int>(15, (int8_t)(x1 + 0.5f));
    o[4 + j] = (uint8_t)(a | (b << 4));
  }
}

__device__ void q_q5_0(const float *x, uint8_t *o) {
  float amax = 0.f, vmax = 0.f;
  for (int j = 0; j < 32; ++j)
    if (amax < fabsf(x[j])) { amax = fabsf(x[j]); vmax = x[j]; }
  const float d = vmax / -16;
  const float id = d ? 1.0f / d : 0.0f;
  put16(o, f2h(d));
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const float x0 = x[j] * id, x1 = x[16 + j] * id;
    const uint8_t a = (uint8_t)mn<int>(31, (int8_t)(x0 + 16.5f));
    const uint8_t b = (uint8_t)mn<int>(31, (int8_t)(x1 + 16.5f));
    o[6 + j] = (uint8_t)((a & 0xF) | ((b & 0xF) << 4));
    qh |= ((uint32_t)(a & 0x10) >> 4) << j;
    qh |= ((uint32_t)(b & 0x10) >> 4) << (j + 16);
  }
  for (int i = 0; i < 4; ++i) o[2 + i] = (uint8_t)(qh >> (8 * i));
}

__device__ void q_q5_1(const float *x, uint8_t *o) {
  float vmin = x[0], vmax = x[0];
  for (int j = 1; j < 32; ++j) {
    if (x[j] < vmin) vmin = x[j];
    if (x[j] > vmax) vmax = x[j];
  }
  const float d = (vmax - vmin) / 31;
  const float id = d ? 1.0f / d : 0.0f;
  put16(o, f2h(d));
  put16(o + 2, f2h(vmin));
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const float x0 = (x[j] - vmin) * id, x1 = (x[16 + j] - vmin) * id;
    const uint8_t a = (uint8_t)(x0 + 0.5f);
    const uint8_t b = (uint8_t)(x1 + 0.5f);
    o[8 + j] = (uint8_t)((a & 0xF) | ((b & 0xF) << 4));
    qh |= ((uint32_t)(a & 0x10) >> 4) << j;
    qh |= ((uint32_t)(b & 0x10) >> 4) << (j + 16);
  }
  for (int i = 0; i < 4; ++i) o[4 + i] = (uint8_t)(qh >> (8 * i));
}

__device__ void q_q8_0(const float *x, uint8_t *o) {
  float amax = 0.f;
  for (int j = 0; j < 32; ++j) amax = mx(amax, fabsf(x[j]));
  const float d = amax / 127;
  const float id = d ? 1.0f / d : 0.0f;
  put16(o, f2h(d));
  for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

// ------------------------------------------------------------- k-quant helpers

// Scale and min search over a group of n values (ggml make_qkx2_quants).
__device__ float qkx2(int n, int nmax, const float *x, const float *w, uint8_t *L, float *the_min, uint8_t *Laux,
                      float rmin, float rdelta, int nstep, bool use_mad) {
  float vmin = x[0], vmax = x[0];
  float sum_w = w[0];
  float sum_x = sum_w * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < vmin) vmin = x[i];
    if (x[i] > vmax) vmax = x[i];
    sum_w += w[i];
    sum_x += w[i] * x[i];
  }
  if (vmin > 0) vmin = 0;
  if (vmax == vmin) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *the_min = -vmin;
    return 0.f;
  }
  float iscale = nmax / (vmax - vmin);
  float scale = 1 / iscale;
  float best = 0;
  for (int i = 0; i < n; ++i) {
    const int l = nearest_int(iscale * (x[i] - vmin));
    L[i] = (uint8_t)mx(0, mn(nmax, l));
    float diff = scale * L[i] + vmin - x[i];
    diff = use_mad ? fabsf(diff) : diff * diff;
    best += w[i] * diff;
  }
  if (nstep < 1) {
    *the_min = -vmin;
    return scale;
  }
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (vmax - vmin);
    float sum_l = 0, sum_l2 = 0, sum_xl = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * (x[i] - vmin));
      l = mx(0, mn(nmax, l));
      Laux[i] = (uint8_t)l;
      sum_l += w[i] * l;
      sum_l2 += w[i] * l * l;
      sum_xl += w[i] * l * x[i];
    }
    const float D = sum_w * sum_l2 - sum_l * sum_l;
    if (D > 0) {
      float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
      float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
      if (this_min > 0) {
        this_min = 0;
        this_scale = sum_xl / sum_l2;
      }
      float mad = 0;
      for (int i = 0; i < n; ++i) {
        float diff = this_scale * Laux[i] + this_min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        mad += w[i] * diff;
      }
      if (mad < best) {
        for (int i = 0; i < n; ++i) L[i] = Laux[i];
        best = mad;
        scale = this_scale;
        vmin = this_min;
      }
    }
  }
  *the_min = -vmin;
  return scale;
}

// Symmetric scale search with weights x^2 (ggml make_qx_quants, rmse_type 1).
__device__ float qx_rmse1(int n, int nmax, const float *x, int8_t *L) {
  float vmax = 0, amax = 0;
  for (int i = 0; i < n; ++i)
    if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); vmax = x[i]; }
  if (amax < kGroupMaxEps) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = -nmax / vmax;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = mx(-nmax, mn(nmax - 1, l));
    L[i] = (int8_t)(l + nmax);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 ? sumlx / suml2 : 0.0f;
  float best = scale * sumlx;
  for (int is = -9; is <= 9; ++is) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1f * is) / vmax;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * x[i]);
      l = mx(-nmax, mn(nmax - 1, l));
      const float w = x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; ++i) {
        const int l = nearest_int(iscale * x[i]);
        L[i] = (int8_t)(nmax + mx(-nmax, mn(nmax - 1, l)));
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

// Q3_K group search (ggml make_q3_quants with do_rmse).
__device__ float q3_group(int n, int nmax, const float *x, int8_t *L) {
  float vmax = 0, amax = 0;
  for (int i = 0; i < n; ++i)
    if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); vmax = x[i]; }
  if (amax < kGroupMaxEps) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  const float iscale = -nmax / vmax;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = mx(-nmax, mn(nmax - 1, l));
    L[i] = (int8_t)l;
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  for (int itry = 0; itry < 5; ++itry) {
    int changed = 0;
    for (int i = 0; i < n; ++i) {
      const float w = x[i] * x[i];
      float slx = sumlx - w * x[i] * L[i];
      if (slx > 0) {
        float sl2 = suml2 - w * L[i] * L[i];
        int nl = nearest_int(x[i] * sl2 / slx);
        nl = mx(-nmax, mn(nmax - 1, nl));
        if (nl != L[i]) {
          slx += w * x[i] * nl;
          sl2 += w * nl * nl;
          if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
            L[i] = (int8_t)nl;
            sumlx = slx;
            suml2 = sl2;
            ++changed;
          }
        }
      }
    }
    if (!changed) break;
  }
  for (int i = 0; i < n; ++i) L[i] = (int8_t)(L[i] + nmax);
  return sumlx / suml2;
}

__device__ __forceinline__ void unpack_k4(int j, const uint8_t *q, int &sc, int &m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

__device__ __forceinline__ void pack_k4(uint8_t *s, int j, uint8_t ls, uint8_t lm) {
  if (j < 4) {
    s[j] = ls;
    s[j + 4] = lm;
  } else {
    s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
    s[j - 4] |= (uint8_t)((ls >> 4) << 6);
    s[j] |= (uint8_t)((lm >> 4) << 6);
  }
}

__device__ __forceinline__ float h2f_dev(uint16_t u) { return h2f(u); }

// ------------------------------------------------------------- k-quant blocks
// Byte offsets follow the GGUF structs (see type_info in mq_common.h).

__device__ void q_q2_K(const float *x, uint8_t *o) {
  uint8_t L[256], Laux[16];
  float wts[16], mins[16], scales[16];
  uint8_t *sc = o, *qs = o + 16;
  float max_scale = 0, max_min = 0;
  for (int j = 0; j < 16; ++j) {
    for (int l = 0; l < 16; ++l) wts[l] = fabsf(x[16 * j + l]);
    scales[j] = qkx2(16, 3, x + 16 * j, wts, L + 16 * j, &mins[j], Laux, -0.5f, 0.1f, 15, true);
    if (scales[j] > max_scale) max_scale = scales[j];
    if (mins[j] > max_min) max_min = mins[j];
  }
  uint16_t dh, mh;
  if (max_scale > 0) {
    const float iscale = 15.f / max_scale;
    for (int j = 0; j < 16; ++j) sc[j] = (uint8_t)nearest_int(iscale * scales[j]);
    dh = f2h(max_scale / 15.f);
  } else {
    for (int j = 0; j < 16; ++j) sc[j] = 0;
    dh = f2h(0.f);
  }
  if (max_min > 0) {
    const float iscale = 15.f / max_min;
    for (int j = 0; j < 16; ++j) sc[j] |= (uint8_t)(nearest_int(iscale * mins[j]) << 4);
    mh = f2h(max_min / 15.f);
  } else {
    mh = f2h(0.f);
  }
  put16(o + 80, dh);
  put16(o + 82, mh);
  for (int j = 0; j < 16; ++j) {
    const float d = h2f_dev(dh) * (sc[j] & 0xF);
    if (!d) continue;
    const float dm = h2f_dev(mh) * (sc[j] >> 4);
    for (int i = 0; i < 16; ++i) {
      const int l = nearest_int((x[16 * j + i] + dm) / d);
      L[16 * j + i] = (uint8_t)mx(0, mn(3, l));
    }
  }
  for (int j = 0; j < 256; j += 128)
    for (int l = 0; l < 32; ++l)
      qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
}

__device__ void q_q3_K(const float *x, uint8_t *o) {
  int8_t L[256];
  float scales[16];
  uint8_t *hmask = o, *qs = o + 32, *sc = o + 96;
  float max_scale = 0, amax = 0;
  for (int j = 0; j < 16; ++j) {
    scales[j] = q3_group(16, 4, x + 16 * j, L + 16 * j);
    if (fabsf(scales[j]) > amax) { amax = fabsf(scales[j]); max_scale = scales[j]; }
  }
  for (int j = 0; j < 12; ++j) sc[j] = 0;
  uint16_t dh;
  if (max_scale) {
    const float iscale = -32.f / max_scale;
    for (int j = 0; j < 16; ++j) {
      int8_t l = (int8_t)nearest_int(iscale * scales[j]);
      l = (int8_t)(mx(-32, mn(31, (int)l)) + 32);
      if (j < 8) sc[j] = l & 0xF;
      else sc[j - 8] |= (uint8_t)((l & 0xF) << 4);
      l >>= 4;
      sc[j % 4 + 8] |= (uint8_t)(l << (2 * (j / 4)));
    }
    dh = f2h(1 / iscale);
  } else {
    dh = f2h(0.f);
  }
  put16(o + 108, dh);
  for (int j = 0; j < 16; ++j) {
    int8_t s = j < 8 ? (int8_t)(sc[j] & 0xF) : (int8_t)(sc[j - 8] >> 4);
    s = (int8_t)((s | (((sc[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32);
    const float d = h2f_dev(dh) * s;
    if (!d) continue;
    for (int i = 0; i < 16; ++i) {
      int l = nearest_int(x[16 * j + i] / d);
      l = mx(-4, mn(3, l));
      L[16 * j + i] = (int8_t)(l + 4);
    }
  }
  for (int j = 0; j < 32; ++j) hmask[j] = 0;
  int m = 0;
  uint8_t hm = 1;
  for (int j = 0; j < 256; ++j) {
    if (L[j] > 3) {
      hmask[m] |= hm;
      L[j] -= 4;
    }
    if (++m == 32) { m = 0; hm <<= 1; }
  }
  for (int j = 0; j < 256; j += 128)
    for (int l = 0; l < 32; ++l)
      qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
}

template <bool FIVE>
__device__ void q_q45_K(const float *x, uint8_t *o) {
  constexpr int nmax = FIVE ? 31 : 15;
  uint8_t L[256], Laux[32];
  float wts[32], mins[8], scales[8];
  uint8_t *sc = o + 4;
  float max_scale = 0, max_min = 0;
  for (int j = 0; j < 8; ++j) {
    float sum_x2 = 0;
    for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
    const float av_x = sqrtf(sum_x2 / 32);
    for (int l = 0; l < 32; ++l) wts[l] = av_x + fabsf(x[32 * j + l]);
    scales[j] = qkx2(32, nmax, x + 32 * j, wts, L + 32 * j, &mins[j], Laux, FIVE ? -0.5f : -1.f, 0.1f,
                     FIVE ? 15 : 20, false);
    if (scales[j] > max_scale) max_scale = scales[j];
    if (mins[j] > max_min) max_min = mins[j];
  }
  const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
  const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
  for (int j = 0; j < 12; ++j) sc[j] = 0;
  for (int j = 0; j < 8; ++j) {
    const uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
    const uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
    pack_k4(sc, j, mn<uint8_t>(63, ls), mn<uint8_t>(63, lm));
  }
  const uint16_t dh = f2h(max_scale / 63.f), mh = f2h(max_min / 63.f);
  put16(o, dh);
  put16(o + 2, mh);
  for (int j = 0; j < 8; ++j) {
    int s, m;
    unpack_k4(j, sc, s, m);
    const float d = h2f_dev(dh) * s;
    if (!d) continue;
    const float dm = h2f_dev(mh) * m;
    for (int i = 0; i < 32; ++i) {
      const int l = nearest_int((x[32 * j + i] + dm) / d);
      L[32 * j + i] = (uint8_t)mx(0, mn(nmax, l));
    }
  }
  if (!FIVE) {
    uint8_t *q = o + 16;
    for (int j = 0; j < 256; j += 64) {
      for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
      q += 32;
    }
  } else {
    uint8_t *qh = o + 16, *ql = o + 48;
    for (int j = 0; j < 32; ++j) qh[j] = 0;
    uint8_t m1 = 1, m2 = 2;
    for (int n = 0; n < 256; n += 64) {
      for (int j = 0; j < 32; ++j) {
        int l1 = L[n + j];
        if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
        int l2 = L[n + j + 32];
        if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
        ql[j] = (uint8_t)(l1 | (l2 << 4));
      }
      m1 <<= 2;
      m2 <<= 2;
      ql += 32;
    }
  }
}

__device__ void q_q6_K(const float *x, uint8_t *o) {
  int8_t L[256];
  float scales[16];
  uint8_t *ql = o, *qh = o + 128;
  int8_t *sc = reinterpret_cast<int8_t *>(o + 192);
  float max_scale = 0, max_abs = 0;
  for (int ib = 0; ib < 16; ++ib) {
    scales[ib] = qx_rmse1(16, 32, x + 16 * ib, L + 16 * ib);
    if (fabsf(scales[ib]) > max_abs) { max_abs = fabsf(scales[ib]); max_scale = scales[ib]; }
  }
  if (max_abs < kGroupMaxEps) {
    for (int i = 0; i < 210; ++i) o[i] = 0;
    put16(o + 208, f2h(0.f));
    return;
  }
  const float iscale = -128.f / max_scale;
  const uint16_t dh = f2h(1 / iscale);
  put16(o + 208, dh);
  for (int ib = 0; ib < 16; ++ib) sc[ib] = (int8_t)mn(127, nearest_int(iscale * scales[ib]));
  for (int j = 0; j < 16; ++j) {
    const float d = h2f_dev(dh) * sc[j];
    if (!d) continue;
    for (int i = 0; i < 16; ++i) {
      int l = nearest_int(x[16 * j + i] / d);
      l = mx(-32, mn(31, l));
      L[16 * j + i] = (int8_t)(l + 32);
    }
  }
  for (int j = 0; j < 256; j += 128) {
    for (int l = 0; l < 32; ++l) {
      const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF;
      const uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
      ql[l] = (uint8_t)(q1 | (q3 << 4));
      ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
      qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                        ((L[j + l + 96] >> 4) << 6));
    }
    ql += 64;
    qh += 32;
  }
}

template <int TYPE>
__device__ __forceinline__ void quant_block(const float *x, uint8_t *o) {
  if constexpr (TYPE == Q4_0) q_q4_0(x, o);
  else if constexpr (TYPE == Q4_1) q_q4_1(x, o);
  else if constexpr (TYPE == Q5_0) q_q5_0(x, o);
  else if constexpr (TYPE == Q5_1) q_q5_1(x, o);
  else if constexpr (TYPE == Q8_0) q_q8_0(x, o);
  else if constexpr (TYPE == Q2_K) q_q2_K(x, o);
  else if constexpr (TYPE == Q3_K) q_q3_K(x, o);
  else if constexpr (TYPE == Q4_K) q_q45_K<false>(x, o);
  else if constexpr (TYPE == Q5_K) q_q45_K<true>(x, o);
  else q_q6_K(x, o);
}

template <typename F, int... I>
__device__ __forceinline__ void static_for_q_impl(F &&f, std::integer_sequence<int, I...>) {
  (f.template operator()<I>(), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for_q(F &&f) {
  static_for_q_impl(f, std::make_integer_sequence<int, N>{});
}

// FP8 E4M3 ("fn": bias 7, no infinities, S.1111.111 is NaN) to f32, exact.
__device__ __forceinline__ float e4m3_to_f32(uint8_t b) {
  const uint32_t sign = (uint32_t)(b & 0x80) << 24;
  const uint32_t e = (b >> 3) & 0xF, m = b & 7;
  if (e == 0xF && m == 7) return __uint_as_float(sign | 0x7FC00000u);
  if (e == 0) {
    const float v = (float)m * 0.001953125f;  // m / 8 * 2^-6
    return sign ? -v : v;
  }
  return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

// One thread per block: copy the block's inputs to private memory (f32 as
// given, or FP8 E4M3 decoded exactly and multiplied by `scale`; with VEC the
// rows are 16-byte aligned and the inputs come as 16-byte loads), quantize
// into a private block image and put it in LDS; the workgroup's 64 blocks,
// contiguous in the raw staging buffer, then leave as 16-byte stores (one
// byte store per output byte had left the FP8 -> Q8_0 pass at ~7 % of HBM).
template <int TYPE, bool FP8, bool VEC>
__global__ __launch_bounds__(64) void quantize_kernel(const void *__restrict__ src, int64_t ld, int64_t n,
                                                      int64_t nb, float scale, uint8_t *__restrict__ dst) {
  constexpr TypeInfo ti = type_info(TYPE);
  __shared__ __align__(16) uint8_t stage[64 * ti.ts];
  const int64_t total = n * nb;
  const int64_t i0 = (int64_t)blockIdx.x * 64;
  const int64_t i = i0 + threadIdx.x;
  if (i < total) {
    const int64_t row = i / nb, b = i - row * nb;
    float x[ti.bs];
    if constexpr (FP8) {
      const uint8_t *p = static_cast<const uint8_t *>(src) + row * ld + b * ti.bs;
      if constexpr (VEC) {
#pragma unroll
        for (int c = 0; c < ti.bs / 16; ++c) {
          const uint4 v = reinterpret_cast<const uint4 *>(p)[c];
          const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int j = 0; j < 16; ++j) x[16 * c + j] = e4m3_to_f32((uint8_t)(wd[j >> 2] >> (8 * (j & 3)))) * scale;
        }
      } else {
        for (int j = 0; j < ti.bs; ++j) x[j] = e4m3_to_f32(p[j]) * scale;
      }
    } else {
      const float *p = static_cast<const float *>(src) + row * ld + b * ti.bs;
      if constexpr (VEC) {
#pragma unroll
        for (int c = 0; c < ti.bs / 4; ++c) {
          const float4 v = reinterpret_cast<const float4 *>(p)[c];
          x[4 * c] = v.x;
          x[4 * c + 1] = v.y;
          x[4 * c + 2] = v.z;
          x[4 * c + 3] = v.w;
        }
      } else {
        for (int j = 0; j < ti.bs; ++j) x[j] = p[j];
      }
    }
    uint8_t o[ti.ts];
    quant_block<TYPE>(x, o);
    for (int j = 0; j < ti.ts; ++j) stage[threadIdx.x * ti.ts + j] = o[j];
  }
  __syncthreads();
  // blocks i0 .. i0 + nblk - 1 are bytes i0 * ts .. of dst (i0 * ts is a
  // multiple of 64 * ts, so 16-byte aligned in the 256-byte aligned buffer)
  const int64_t nblk = total - i0 < 64 ? total - i0 : 64;
  const int bytes = (int)nblk * ti.ts;
  uint8_t *q = dst + i0 * ti.ts;
  const int whole = bytes & ~15;
  for (int o = 16 * (int)threadIdx.x; o < whole; o += 16 * 64)
    *reinterpret_cast<uint4 *>(q + o) = *reinterpret_cast<const uint4 *>(stage + o);
  for (int o = whole + (int)threadIdx.x; o < bytes; o += 64) q[o] = stage[o];
}

// A block image's bytes [OFF, OFF + 4) as a little-endian word (constant
// offsets, so the image stays in registers).
template <int OFF>
__device__ __forceinline__ uint32_t image_word(const uint8_t *o) {
  return (uint32_t)o[OFF] | ((uint32_t)o[OFF + 1] << 8) | ((uint32_t)o[OFF + 2] << 16) | ((uint32_t)o[OFF + 3] << 24);
}

// Field F of a block image into the tiled planes at (tile-block tb, row r):
// a 16-byte column per chunk of a chunked field, one run for a record (the
// same places the repack writes).
template <int TYPE, int F>
__device__ __forceinline__ void store_field(uint8_t *tiled, const Geo &g, int64_t tb, int r, const uint8_t *o) {
  constexpr TypeInfo ti = type_info(TYPE);
  constexpr int size = ti.f[F].size, off = ti.f[F].off;
  if constexpr (size % 16 == 0) {
    static_for_q<size / 16>([&]<int C>() {
      const uint4 v = make_uint4(image_word<off + 16 * C>(o), image_word<off + 16 * C + 4>(o),
                                 image_word<off + 16 * C + 8>(o), image_word<off + 16 * C + 12>(o));
      *reinterpret_cast<uint4 *>(tiled + g.plane[F] + ((tb * (size / 16) + C) * kRowTile + r) * 16) = v;
    });
  } else if constexpr (size == 4) {
    *reinterpret_cast<uint32_t *>(tiled + g.plane[F] + (tb * kRowTile + r) * 4) = image_word<off>(o);
  } else {
    static_assert(size == 2, "record fields of the 32-element types are 2 or 4 bytes");
    *reinterpret_cast<uint16_t *>(tiled + g.plane[F] + (tb * kRowTile + r) * 2) =
        (uint16_t)((uint32_t)o[off] | ((uint32_t)o[off + 1] << 8));
  }
}

// The 32-element types straight into the device layout: one 64-thread
// workgroup per (4 consecutive blocks, 64-row tile t); thread r quantizes row
// t * 64 + r's blocks (a 128-byte run of FP8 or 512 bytes of f32: whole cache
// lines; rows past n: zeros, as the repack writes them) and stores each
// block's fields where the repack would put them, so there is no raw staging
// and no repack pass (the repack reads these 18-34-byte blocks 2 bytes at a
// time).
constexpr int kQtBlocks = 4;

template <int TYPE, bool FP8, bool VEC>
__global__ __launch_bounds__(64) void quantize_tiled_kernel(const void *__restrict__ src, int64_t ld, Geo g,
                                                            float scale, uint8_t *__restrict__ tiled) {
  constexpr TypeInfo ti = type_info(TYPE);
  static_assert(ti.bs == 32, "32-element block types only");
  const int64_t t = blockIdx.y;
  const int r = threadIdx.x;
  const int64_t row = t * kRowTile + r;
#pragma unroll
  for (int j = 0; j < kQtBlocks; ++j) {
    const int64_t b = (int64_t)blockIdx.x * kQtBlocks + j;
    if (b >= g.nb) break;  // uniform across the workgroup
    uint8_t o[ti.ts];
    if (row < g.n) {
      float x[32];
      if constexpr (FP8) {
        const uint8_t *p = static_cast<const uint8_t *>(src) + row * ld + b * 32;
        if constexpr (VEC) {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const uint4 v = reinterpret_cast<const uint4 *>(p)[c];
            const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 16; ++i) x[16 * c + i] = e4m3_to_f32((uint8_t)(wd[i >> 2] >> (8 * (i & 3)))) * scale;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 32; ++i) x[i] = e4m3_to_f32(p[i]) * scale;
        }
      } else {
        const float *p = static_cast<const float *>(src) + row * ld + b * 32;
        if constexpr (VEC) {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const float4 v = reinterpret_cast<const float4 *>(p)[c];
            x[4 * c] = v.x;
            x[4 * c + 1] = v.y;
            x[4 * c + 2] = v.z;
            x[4 * c + 3] = v.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 32; ++i) x[i] = p[i];
        }
      }
      quant_block<TYPE>(x, o);
    } else {
#pragma unroll
      for (int i = 0; i < ti.ts; ++i) o[i] = 0;
    }
    const int64_t tb = t * g.nb + b;
    static_for_q<ti.nf>([&]<int F>() { store_field<TYPE, F>(tiled, g, tb, r, o); });
  }
}

template <bool FP8>
hipError_t launch_quantize_tiled_src(int type, const void *src, int64_t ld, float scale, void *tiled, const Geo &g,
                                     hipStream_t stream) {
  if (g.n == 0 || g.nb == 0) return hipSuccess;
  const int64_t es = FP8 ? 1 : 4;
  const bool vec = (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (ld * es) % 16 == 0;
  const dim3 grid((unsigned)((g.nb + kQtBlocks - 1) / kQtBlocks), (unsigned)g.ntiles);
  bool ok = false;
  auto go = [&]<int T>() {
    if (vec)
      hipLaunchKernelGGL((quantize_tiled_kernel<T, FP8, true>), grid, dim3(64), 0, stream, src, ld, g, scale,
                         static_cast<uint8_t *>(tiled));
    else
      hipLaunchKernelGGL((quantize_tiled_kernel<T, FP8, false>), grid, dim3(64), 0, stream, src, ld, g, scale,
                         static_cast<uint8_t *>(tiled));
    ok = true;
  };
  switch (type) {
    case Q4_0: go.template operator()<Q4_0>(); break;
    case Q4_1: go.template operator()<Q4_1>(); break;
    case Q5_0: go.template operator()<Q5_0>(); break;
    case Q5_1: go.template operator()<Q5_1>(); break;
    case Q8_0: go.template operator()<Q8_0>(); break;
    default: break;
  }
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

template <bool FP8>
hipError_t launch_quantize_src(int type, const void *src, int64_t ld, int64_t n, int64_t k, float scale,
                               void *dst_raw, hipStream_t stream) {
  const TypeInfo ti = type_info(type);
  const int64_t nb = k / ti.bs;
  const int64_t total = n * nb;
  if (total == 0) return hipSuccess;
  if ((reinterpret_cast<uintptr_t>(dst_raw) & 15) != 0) return hipErrorInvalidValue;
  // 16-byte source loads need every block's first element 16-byte aligned
  const int64_t es = FP8 ? 1 : 4;
  const bool vec = (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (ld * es) % 16 == 0 && (ti.bs * es) % 16 == 0;
  const unsigned grid = (unsigned)((total + 63) / 64);
  bool ok = dispatch_type(type, [&]<int T>() {
    if (vec)
      hipLaunchKernelGGL((quantize_kernel<T, FP8, true>), dim3(grid), dim3(64), 0, stream, src, ld, n, nb, scale,
                         static_cast<uint8_t *>(dst_raw));
    else
      hipLaunchKernelGGL((quantize_kernel<T, FP8, false>), dim3(grid), dim3(64), 0, stream, src, ld, n, nb, scale,
                         static_cast<uint8_t *>(dst_raw));
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize(int type, const float *src, int64_t ld, int64_t n, int64_t k, void *dst_raw,
                           hipStream_t stream) {
  return launch_quantize_src<false>(type, src, ld, n, k, 1.0f, dst_raw, stream);
}

hipError_t launch_quantize_fp8(int type, const uint8_t *src, int64_t ld, int64_t n, int64_t k, float scale,
                               void *dst_raw, hipStream_t stream) {
  return launch_quantize_src<true>(type, src, ld, n, k, scale, dst_raw, stream);
}

bool quantize_tiled_ok(int type) { return type == Q4_0 || type == Q4_1 || type == Q5_0 || type == Q5_1 || type == Q8_0; }

hipError_t launch_quantize_tiled(int type, const void *src, bool fp8, int64_t ld, float scale, void *tiled,
                                 const Geo &g, hipStream_t stream) {
  return fp8 ? launch_quantize_tiled_src<true>(type, src, ld, scale, tiled, g, stream)
             : launch_quantize_tiled_src<false>(type, src, ld, 1.0f, tiled, g, stream);
}

}  // namespace mq
