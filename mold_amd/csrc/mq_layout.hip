// mq_layout.hip — GGUF blocks <-> device tiled-planar layout (see mq_common.h),
// dense dequantize, and the f32 -> bf16 activation staging used by the GEMM.
#include <utility>

#include "mq_kernels.h"

namespace mq {

// Largest power of two (at most 16) dividing v.
constexpr int pow2_div(int v) {
  int a = 1;
  while (a < 16 && v % (2 * a) == 0) a *= 2;
  return a;
}

template <int U>
struct UnitT;
template <> struct UnitT<1> { using type = uint8_t; };
template <> struct UnitT<2> { using type = uint16_t; };
template <> struct UnitT<4> { using type = uint32_t; };
template <> struct UnitT<8> { using type = uint2; };
template <> struct UnitT<16> { using type = uint4; };

// Moves SIZE bytes in units of U bytes (both sides U-aligned); zero: store zeros.
template <int U, int SIZE>
__device__ __forceinline__ void move_bytes(uint8_t *d, const uint8_t *s, bool zero) {
  using T = typename UnitT<U>::type;
#pragma unroll
  for (int i = 0; i < SIZE / U; ++i) {
    T v{};
    if (!zero) v = reinterpret_cast<const T *>(s)[i];
    reinterpret_cast<T *>(d)[i] = v;
  }
}

// Field F of block (tile t, block b), row r: between the raw block at `raw`
// and the tiled planes at `tiled`.  A chunked field moves as 16-byte columns
// (the wave's 64 rows of one column are one contiguous KiB), a record as one
// run; units are the largest both sides' alignment allows.  With ALIGNED (the
// raw buffer starts on 16 bytes) the raw side's alignment is fixed by the
// block size and the field offset, since rows start at multiples of the
// block size; otherwise the raw side moves bytes.
template <int TYPE, bool ALIGNED, int F>
__device__ __forceinline__ void repack_field(uint8_t *raw, uint8_t *tiled, const Geo &g, int64_t tb, int r,
                                             bool inverse, bool zero) {
  constexpr TypeInfo ti = type_info(TYPE);
  constexpr int size = ti.f[F].size, off = ti.f[F].off;
  constexpr int ua = !ALIGNED ? 1
                     : pow2_div(ti.ts) < pow2_div(off == 0 ? 16 : off) ? pow2_div(ti.ts)
                                                                        : pow2_div(off == 0 ? 16 : off);
  if constexpr (size % 16 == 0) {
#pragma unroll
    for (int c = 0; c < size / 16; ++c) {
      uint8_t *tp = tiled + g.plane[F] + ((tb * (size / 16) + c) * kRowTile + r) * 16;
      uint8_t *rp = raw + off + 16 * c;
      if (inverse) move_bytes<ua, 16>(rp, tp, false);
      else move_bytes<ua, 16>(tp, rp, zero);
    }
  } else {
    constexpr int u = ua < pow2_div(size) ? ua : pow2_div(size);
    uint8_t *tp = tiled + g.plane[F] + (tb * kRowTile + r) * size;
    uint8_t *rp = raw + off;
    if (inverse) move_bytes<u, size>(rp, tp, false);
    else move_bytes<u, size>(tp, rp, zero);
  }
}

// One thread per (row, block); a wave holds the 64 rows of one tile for one
// block, so every write of the tiled side (and every read, inverse) is a
// contiguous run and each thread reads its own block's bytes.  inverse=false:
// raw -> tiled over the padded rows, the rows past n of the last tile written
// as zeros (no separate clear); inverse=true: tiled -> raw over the n real
// rows.  Upload/download only, never on the hot path.
template <int TYPE, bool ALIGNED>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                     Geo g, int inverse) {
  constexpr TypeInfo ti = type_info(TYPE);
  const int r = threadIdx.x & (kRowTile - 1);
  const int64_t pairs = g.ntiles * g.nb, row_bytes = g.nb * ti.ts;
  uint8_t *raw_base = inverse ? dst : const_cast<uint8_t *>(src);
  uint8_t *tiled = inverse ? const_cast<uint8_t *>(src) : dst;
  for (int64_t tb = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); tb < pairs; tb += (int64_t)gridDim.x * 4) {
    const int64_t t = tb / g.nb, b = tb - t * g.nb;
    const int64_t n = t * kRowTile + r;
    const bool real = n < g.n;
    if (inverse && !real) continue;
    uint8_t *raw = raw_base + (real ? n : 0) * row_bytes + b * ti.ts;
    [&]<int... F>(std::integer_sequence<int, F...>) {
      (repack_field<TYPE, ALIGNED, F>(raw, tiled, g, tb, r, inverse != 0, !real), ...);
    }(std::make_integer_sequence<int, ti.nf>{});
  }
}

hipError_t launch_repack(int type, const void *src, void *dst, const Geo &g, bool inverse,
                         hipStream_t stream) {
  const int64_t pairs = g.ntiles * g.nb;
  if (pairs == 0) return hipSuccess;
  const int64_t want = (pairs + 3) / 4;
  const int blocks = (int)(want < 65536 ? want : 65536);
  const bool aligned = ((reinterpret_cast<uintptr_t>(inverse ? dst : src)) & 15) == 0;
  bool ok = dispatch_type(type, [&]<int T>() {
    if (aligned)
      hipLaunchKernelGGL((repack_kernel<T, true>), dim3(blocks), dim3(256), 0, stream,
                         static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), g, inverse ? 1 : 0);
    else
      hipLaunchKernelGGL((repack_kernel<T, false>), dim3(blocks), dim3(256), 0, stream,
                         static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), g, inverse ? 1 : 0);
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

// ------------------------------------------------------------- dequantize

template <typename OUT>
__device__ __forceinline__ void store8(OUT *dst, const float v[8]);

template <>
__device__ __forceinline__ void store8<float>(float *dst, const float v[8]) {
  reinterpret_cast<float4 *>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4 *>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// Half outputs are the f32 dequantized value rounded once more to nearest
// even.  pin() keeps that f32 value in a register: otherwise the backend fuses
// the decoder's last multiply-add into the conversion (v_fma_mix*_f16), which
// rounds the exact product-sum straight to f16 and can differ in the last bit.
__device__ __forceinline__ float pin(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <>
__device__ __forceinline__ void store8<__bf16>(__bf16 *dst, const float v[8]) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)pin(v[i]);
  *reinterpret_cast<bf16x8 *>(dst) = r;
}

template <>
__device__ __forceinline__ void store8<_Float16>(_Float16 *dst, const float v[8]) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (_Float16)pin(v[i]);
  *reinterpret_cast<f16x8 *>(dst) = r;
}

// Fallback for k % 256 != 0 (legacy 32-element types only): one thread per 8
// consecutive outputs of a row, decoding straight from the tiled layout.
template <int TYPE, typename OUT>
__global__ void dequant_kernel(WView w, int64_t n, int64_t k, OUT *__restrict__ dst) {
  constexpr TypeInfo ti = type_info(TYPE);
  const int64_t groups_per_row = k >> 3;
  const int64_t total = n * groups_per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / groups_per_row;
    const int64_t kk = (i - row * groups_per_row) << 3;
    const int64_t b = kk / ti.bs;
    const int e0 = (int)(kk - b * ti.bs);
    float v[8];
    decode8<TYPE>(w, row / kRowTile, (int)(row % kRowTile), b, e0, v);
    store8<OUT>(dst + row * k + kk, v);
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Blocks of one 256-element column step, and the LDS bytes their records take
// for one 64-row tile.
template <int TYPE>
constexpr int dq_blocks() {
  return 256 / type_info(TYPE).bs;
}
template <int TYPE>
constexpr int dq_lds_bytes() {
  return kRowTile * type_info(TYPE).ts * dq_blocks<TYPE>();
}

// One workgroup per (64-row tile, 256-element column step).  In the tiled
// layout the records of one tile's consecutive blocks are contiguous in every
// field plane, so the workgroup first copies them to LDS with coalesced
// 16-byte loads (each weight byte is read from HBM once), then decodes from
// LDS with the same decode8 as the other paths (an LDS WView: one block row
// of the tile layout with nb = blocks per step).  Decode mapping: lane =
// 8 rows x 8 consecutive 8-element groups, so each store instruction writes
// eight 256-byte row segments (f32; 128 bytes for halves), and the LDS reads
// of a wave touch 8 rows x at most 2 chunks (no more than 2-way bank
// conflicts).  Needs k % 256 == 0.
template <int TYPE, typename OUT>
__global__ __launch_bounds__(256) void dequant_tile_kernel(WView w, int64_t n, int64_t k, OUT *__restrict__ dst) {
  constexpr TypeInfo ti = type_info(TYPE);
  constexpr int BPW = dq_blocks<TYPE>();
  __shared__ uint4 lds[dq_lds_bytes<TYPE>() / 16];
  const int tid = threadIdx.x;
  const int64_t t = blockIdx.y;
  const int64_t step = blockIdx.x;
  const int64_t b0 = step * BPW;
  WView lv;
  lv.base = reinterpret_cast<const uint8_t *>(lds);
  lv.nb = BPW;
  int off = 0;
#pragma unroll
  for (int f = 0; f < ti.nf; ++f) {
    const int bytes = kRowTile * ti.f[f].size * BPW;  // a multiple of 128
    const u32x4 *src = reinterpret_cast<const u32x4 *>(w.base + w.plane[f] + (t * w.nb + b0) * kRowTile * ti.f[f].size);
    u32x4 *ldst = reinterpret_cast<u32x4 *>(lds) + off / 16;
    for (int i = tid; i < bytes / 16; i += 256) ldst[i] = __builtin_nontemporal_load(&src[i]);
    lv.plane[f] = off;
    off += bytes;
  }
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  const int r8 = lane >> 3, g8 = lane & 7;
#pragma unroll 2
  for (int it = 0; it < 8; ++it) {
    const int pair = wave * 8 + it;  // (row octet, group octet) of the 8 x 4 in the tile step
    const int row = 8 * (pair >> 2) + r8;
    const int e = 64 * (pair & 3) + 8 * g8;  // element within the 256-element step
    float v[8];
    decode8<TYPE>(lv, 0, row, e / ti.bs, e % ti.bs, v);
    const int64_t grow = t * kRowTile + row;
    if (grow < n) store8<OUT>(dst + grow * k + step * 256 + e, v);
  }
}

hipError_t launch_dequant(int type, const WView &w, int64_t n, int64_t k, void *dst, int dst_type,
                          hipStream_t stream) {
  const int64_t total = n * (k >> 3);
  if (total == 0) return hipSuccess;
  if (k % 256 == 0) {
    const dim3 grid((unsigned)(k / 256), (unsigned)((n + kRowTile - 1) / kRowTile));
    bool ok = dispatch_type(type, [&]<int T>() {
      if (dst_type == F32)
        hipLaunchKernelGGL((dequant_tile_kernel<T, float>), grid, dim3(256), 0, stream, w, n, k,
                           static_cast<float *>(dst));
      else if (dst_type == BF16)
        hipLaunchKernelGGL((dequant_tile_kernel<T, __bf16>), grid, dim3(256), 0, stream, w, n, k,
                           static_cast<__bf16 *>(dst));
      else
        hipLaunchKernelGGL((dequant_tile_kernel<T, _Float16>), grid, dim3(256), 0, stream, w, n, k,
                           static_cast<_Float16 *>(dst));
    });
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
  }
  const int threads = 256;
  const int64_t want = (total + threads - 1) / threads;
  const int blocks = (int)(want < 262144 ? want : 262144);
  bool ok = dispatch_type(type, [&]<int T>() {
    if (dst_type == F32)
      hipLaunchKernelGGL((dequant_kernel<T, float>), dim3(blocks), dim3(threads), 0, stream, w, n, k,
                         static_cast<float *>(dst));
    else if (dst_type == BF16)
      hipLaunchKernelGGL((dequant_kernel<T, __bf16>), dim3(blocks), dim3(threads), 0, stream, w, n, k,
                         static_cast<__bf16 *>(dst));
    else
      hipLaunchKernelGGL((dequant_kernel<T, _Float16>), dim3(blocks), dim3(threads), 0, stream, w, n,
                         k, static_cast<_Float16 *>(dst));
  });
  if (!ok) return hipErrorInvalidValue;
  return hipGetLastError();
}

// ------------------------------------------------------- dense GGUF tensors

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return (float)v;  // exact from f16 and bf16
}

template <typename OUT>
__device__ __forceinline__ OUT from_f32(float v) {
  return (OUT)v;  // f32 -> f16 / bf16: round to nearest even
}

// One thread per 4 consecutive elements of a row (grid-stride over rows x
// column groups); the last group of a row may be partial.
template <typename IN, typename OUT>
__global__ __launch_bounds__(256) void convert_kernel(const IN *__restrict__ src, int64_t lds, int64_t n, int64_t k,
                                                      OUT *__restrict__ dst, int64_t ldd) {
  const int64_t gpr = (k + 3) >> 2;
  const int64_t total = n * gpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / gpr;
    const int64_t c0 = (i - row * gpr) << 2;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c0 + j < k) dst[row * ldd + c0 + j] = from_f32<OUT>(to_f32(src[row * lds + c0 + j]));
  }
}

template <typename IN>
static hipError_t convert_from(const IN *src, int64_t lds, int64_t n, int64_t k, void *dst, int dst_type,
                               int64_t ldd, hipStream_t stream) {
  const int64_t total = n * ((k + 3) >> 2);
  const int64_t want = (total + 255) / 256;
  const int blocks = (int)(want < 65536 ? want : 65536);
  if (dst_type == F32)
    hipLaunchKernelGGL((convert_kernel<IN, float>), dim3(blocks), dim3(256), 0, stream, src, lds, n, k,
                       static_cast<float *>(dst), ldd);
  else if (dst_type == F16)
    hipLaunchKernelGGL((convert_kernel<IN, _Float16>), dim3(blocks), dim3(256), 0, stream, src, lds, n, k,
                       static_cast<_Float16 *>(dst), ldd);
  else if (dst_type == BF16)
    hipLaunchKernelGGL((convert_kernel<IN, __bf16>), dim3(blocks), dim3(256), 0, stream, src, lds, n, k,
                       static_cast<__bf16 *>(dst), ldd);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_convert(const void *src, int src_type, int64_t lds, int64_t n, int64_t k, void *dst,
                          int dst_type, int64_t ldd, hipStream_t stream) {
  if (n <= 0 || k <= 0) return hipSuccess;
  switch (src_type) {
    case F32: return convert_from(static_cast<const float *>(src), lds, n, k, dst, dst_type, ldd, stream);
    case F16: return convert_from(static_cast<const _Float16 *>(src), lds, n, k, dst, dst_type, ldd, stream);
    case BF16: return convert_from(static_cast<const __bf16 *>(src), lds, n, k, dst, dst_type, ldd, stream);
    default: return hipErrorInvalidValue;
  }
}

// ------------------------------------------------- activation staging (GEMM A)

// x[m, k] (f32 or bf16, row stride ldx) -> bf16 [m, kp] with zeros in
// columns k..kp-1.  One thread per 8 output columns.
template <typename IN>
__global__ void stage_bf16_kernel(const IN *__restrict__ x, int64_t m, int64_t k, int64_t ldx,
                                  __bf16 *__restrict__ out, int64_t kp) {
  const int64_t gpr = kp >> 3;
  const int64_t total = m * gpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / gpr;
    const int64_t c = (i - row * gpr) << 3;
    bf16x8 r;
    const IN *src = x + row * ldx + c;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (c + j < k) ? (__bf16)(float)src[j] : (__bf16)0.0f;
    *reinterpret_cast<bf16x8 *>(out + row * kp + c) = r;
  }
}

// f32 rows with k a multiple of 8, 4-aligned row stride, 16-byte aligned x:
// two 16-byte loads and one 16-byte store per thread, a 2-D grid (column
// groups x rows, rows strided by gridDim.y), no divides.
__global__ __launch_bounds__(256) void stage_bf16_vec_kernel(const float4 *__restrict__ x, int64_t m, int64_t k,
                                                             int64_t ldx4, bf16x8 *__restrict__ out, int64_t kp) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 8-column group
  if (g >= (kp >> 3)) return;
  for (int64_t row = blockIdx.y; row < m; row += gridDim.y) {
    bf16x8 r;
    if (8 * g < k) {
      const float4 a = x[row * ldx4 + 2 * g], b = x[row * ldx4 + 2 * g + 1];
      r[0] = (__bf16)a.x; r[1] = (__bf16)a.y; r[2] = (__bf16)a.z; r[3] = (__bf16)a.w;
      r[4] = (__bf16)b.x; r[5] = (__bf16)b.y; r[6] = (__bf16)b.z; r[7] = (__bf16)b.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = (__bf16)0.0f;
    }
    out[row * (kp >> 3) + g] = r;
  }
}

hipError_t launch_stage_bf16(const void *x, int x_type, int64_t m, int64_t k, int64_t ldx, __bf16 *out,
                             int64_t kp, hipStream_t stream) {
  const int64_t total = m * (kp >> 3);
  if (total == 0) return hipSuccess;
  if (x_type == F32 && k % 8 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const int64_t groups = kp >> 3;
    const unsigned gx = (unsigned)((groups + 255) / 256);
    const unsigned gy = (unsigned)(m < 65535 ? m : 65535);
    hipLaunchKernelGGL(stage_bf16_vec_kernel, dim3(gx, gy), dim3(256), 0, stream, static_cast<const float4 *>(x), m,
                       k, ldx / 4, reinterpret_cast<bf16x8 *>(out), kp);
    return hipGetLastError();
  }
  const int threads = 256;
  const int64_t want = (total + threads - 1) / threads;
  const int blocks = (int)(want < 262144 ? want : 262144);
  if (x_type == F32)
    hipLaunchKernelGGL(stage_bf16_kernel<float>, dim3(blocks), dim3(threads), 0, stream,
                       static_cast<const float *>(x), m, k, ldx, out, kp);
  else
    hipLaunchKernelGGL(stage_bf16_kernel<__bf16>, dim3(blocks), dim3(threads), 0, stream,
                       static_cast<const __bf16 *>(x), m, k, ldx, out, kp);
  return hipGetLastError();
}

__global__ void widen_bf16_kernel(const __bf16 *__restrict__ x, int64_t m, int64_t k, int64_t ldx,
                                  float *__restrict__ out) {
  const int64_t total = m * k;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / k, c = i - row * k;
    out[i] = (float)x[row * ldx + c];
  }
}

hipError_t launch_widen_bf16(const __bf16 *x, int64_t m, int64_t k, int64_t ldx, float *out,
                             hipStream_t stream) {
  const int64_t total = m * k;
  if (total == 0) return hipSuccess;
  const int64_t want = (total + 255) / 256;
  const int blocks = (int)(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(widen_bf16_kernel, dim3(blocks), dim3(256), 0, stream, x, m, k, ldx, out);
  return hipGetLastError();
}

}  // namespace mq
