// mq_api.hip — the C ABI declared in include/moldq.h: contexts, HBM arena,
// weight upload/download, dequantize and the quantized matmul dispatcher.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <new>
#include <string>

#include "../../include/moldq.h"
#include "mq_kernels.h"

using namespace mq;

struct mq_ctx {
  int device = 0;
  int cu_count = 0;
  // HBM arena: one allocation, bump-allocated by uploads, freed with the ctx.
  uint8_t *arena = nullptr;
  size_t arena_size = 0;
  size_t arena_used = 0;
  // Scratch: activation staging and GEMV partial sums.
  void *scratch = nullptr;
  size_t scratch_size = 0;
  // GEMM tail-tile partial sums, one buffer per stream (so GEMMs with
  // in-place bf16 x may run concurrently on different streams).
  struct StreamBuf {
    hipStream_t stream = nullptr;
    void *p = nullptr;
    size_t size = 0;
  };
  static constexpr int kTailStreams = 4;
  StreamBuf tail[kTailStreams];
  int tail_used = 0;
};

struct mq_qtensor {
  mq_ctx *ctx = nullptr;
  int dtype = 0;
  int64_t n = 0, k = 0;
  Geo geo{};
  uint8_t *data = nullptr;
  bool in_arena = false;
  size_t gguf_bytes = 0;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(MQ_E_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(expr, what)                       \
  do {                                            \
    hipError_t _e = (expr);                       \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

// Make ctx->device current for the duration of a call; restore afterwards.
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    ok = (prev == dev) || (hipSetDevice(dev) == hipSuccess);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

size_t gguf_row_bytes(int dtype, int64_t k) {
  const TypeInfo ti = type_info(dtype);
  return (size_t)(k / ti.bs) * ti.ts;
}

int check_weight_shape(int dtype, int64_t n, int64_t k, size_t nbytes) {
  if (!is_quant(dtype)) return fail(MQ_E_INVALID, "dtype %d is not a supported GGUF block type", dtype);
  const TypeInfo ti = type_info(dtype);
  if (n <= 0 || k <= 0) return fail(MQ_E_INVALID, "weight shape [%lld, %lld] must be positive", (long long)n, (long long)k);
  if (k % ti.bs != 0)
    return fail(MQ_E_INVALID, "%s needs k %% %d == 0, got k=%lld", ti.name, ti.bs, (long long)k);
  const size_t want = gguf_row_bytes(dtype, k) * (size_t)n;
  if (nbytes != want)
    return fail(MQ_E_INVALID, "%s [%lld, %lld] is %zu bytes, got %zu", ti.name, (long long)n, (long long)k, want, nbytes);
  return MQ_OK;
}

int alloc_weight(mq_ctx *ctx, mq_qtensor *t) {
  const size_t bytes = (size_t)t->geo.bytes;
  const size_t aligned_used = (ctx->arena_used + 255) & ~size_t(255);
  if (ctx->arena && aligned_used + bytes <= ctx->arena_size) {
    t->data = ctx->arena + aligned_used;
    t->in_arena = true;
    ctx->arena_used = aligned_used + bytes;
    return MQ_OK;
  }
  hipError_t e = hipMalloc(&t->data, bytes);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) for weight failed: %s", bytes, hipGetErrorString(e));
  t->in_arena = false;
  return MQ_OK;
}

int ensure_scratch(mq_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->scratch_size) return MQ_OK;
  if (ctx->scratch) {
    // earlier work on any stream may still read the old buffer
    HIP_TRY(hipDeviceSynchronize(), "hipDeviceSynchronize before scratch growth");
    HIP_TRY(hipFree(ctx->scratch), "hipFree scratch");
    ctx->scratch = nullptr;
    ctx->scratch_size = 0;
  }
  const size_t sz = (bytes + (1 << 20) - 1) & ~size_t((1 << 20) - 1);
  hipError_t e = hipMalloc(&ctx->scratch, sz);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) for scratch failed: %s", sz, hipGetErrorString(e));
  ctx->scratch_size = sz;
  return MQ_OK;
}

WView view_of(const mq_qtensor *w) { return make_view(w->data, w->geo); }

// The stream's tail-partial buffer of at least `bytes`, or NULL when the
// context already serves kTailStreams other streams (the GEMM then runs every
// tile whole) or the allocation fails.
float *tail_buffer(mq_ctx *ctx, hipStream_t s, size_t bytes) {
  mq_ctx::StreamBuf *b = nullptr;
  for (int i = 0; i < ctx->tail_used; ++i)
    if (ctx->tail[i].stream == s) b = &ctx->tail[i];
  if (!b) {
    if (ctx->tail_used == mq_ctx::kTailStreams) return nullptr;
    b = &ctx->tail[ctx->tail_used++];
    b->stream = s;
  }
  if (b->size < bytes) {
    if (b->p) {
      if (hipStreamSynchronize(s) != hipSuccess) return nullptr;  // earlier work on s may still read it
      (void)hipFree(b->p);
      b->p = nullptr;
      b->size = 0;
    }
    const size_t sz = (bytes + (1 << 20) - 1) & ~size_t((1 << 20) - 1);
    if (hipMalloc(&b->p, sz) != hipSuccess) {
      b->p = nullptr;
      return nullptr;
    }
    b->size = sz;
  }
  return static_cast<float *>(b->p);
}

// GEMM: stage activations as bf16 [m, kp] (kp multiple of 64, zero padded)
// unless bf16 x can be read in place, then the fused dequant-MFMA kernel.
int run_gemm(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx, void *y,
             int y_dtype, int64_t ldy, const float *bias, const float *gate, int act, hipStream_t s) {
  const WView wv = view_of(w);
  const int64_t n = w->n, k = w->k;
  const int64_t kp = (k + 63) / 64 * 64;
  const __bf16 *a = nullptr;
  int64_t lda = 0;
  const bool direct = x_dtype == MQ_BF16 && k == kp && (ldx % 8) == 0 &&
                      (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  if (direct) {
    a = static_cast<const __bf16 *>(x);
    lda = ldx;
  } else {
    int rc = ensure_scratch(ctx, (size_t)m * kp * sizeof(__bf16));
    if (rc) return rc;
    __bf16 *st = static_cast<__bf16 *>(ctx->scratch);
    hipError_t e = launch_stage_bf16(x, x_dtype, m, k, ldx, st, kp, s);
    if (e != hipSuccess) return hip_fail(e, "stage activations");
    a = st;
    lda = kp;
  }
  GemmTail tail = gemm_tail_plan(w->dtype, m, n, k, ctx->cu_count);
  float *partial = nullptr;
  if (tail.kparts > 1 && gemm_fast_ok(w->dtype, m, k, lda)) partial = tail_buffer(ctx, s, gemm_tail_bytes(tail, m, n));
  hipError_t e = launch_gemm(w->dtype, wv, n, k, w->geo.ntiles, a, m, lda, y, y_dtype, ldy, bias, gate, act, tail,
                             partial, s);
  if (e != hipSuccess) return hip_fail(e, "gemm launch");
  return MQ_OK;
}

}  // namespace

namespace mq {
// Shared with the host-only translation units (GGUF reader).
int set_error(int code, const char *msg) {
  g_err = msg;
  return code;
}
}  // namespace mq

extern "C" {

const char *mq_last_error(void) { return g_err.c_str(); }
int mq_version(void) { return MOLDQ_VERSION; }

int mq_block_size(int dtype) {
  if (dtype == MQ_F32 || dtype == MQ_F16 || dtype == MQ_BF16) return 1;
  return type_info(dtype).bs;
}

int mq_type_size(int dtype) {
  if (dtype == MQ_F32) return 4;
  if (dtype == MQ_F16 || dtype == MQ_BF16) return 2;
  return type_info(dtype).ts;
}

int mq_ctx_create(int device_ordinal, mq_ctx **out) {
  if (!out) return fail(MQ_E_INVALID, "mq_ctx_create: out is NULL");
  *out = nullptr;
  int count = 0;
  HIP_TRY(hipGetDeviceCount(&count), "hipGetDeviceCount");
  if (device_ordinal < 0 || device_ordinal >= count)
    return fail(MQ_E_INVALID, "device ordinal %d out of range (%d devices)", device_ordinal, count);
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device_ordinal), "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MQ_E_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only", device_ordinal,
                prop.gcnArchName);
  mq_ctx *c = new (std::nothrow) mq_ctx();
  if (!c) return fail(MQ_E_OOM, "out of host memory");
  c->device = device_ordinal;
  c->cu_count = prop.multiProcessorCount;
  *out = c;
  return MQ_OK;
}

void mq_ctx_destroy(mq_ctx *ctx) {
  if (!ctx) return;
  DeviceGuard g(ctx->device);
  (void)hipDeviceSynchronize();
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  for (int i = 0; i < ctx->tail_used; ++i)
    if (ctx->tail[i].p) (void)hipFree(ctx->tail[i].p);
  if (ctx->arena) (void)hipFree(ctx->arena);
  delete ctx;
}

int mq_ctx_reserve_arena(mq_ctx *ctx, size_t bytes) {
  if (!ctx) return fail(MQ_E_INVALID, "ctx is NULL");
  if (ctx->arena) return fail(MQ_E_INVALID, "arena already reserved (%zu bytes)", ctx->arena_size);
  DeviceGuard g(ctx->device);
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) for arena failed: %s", bytes, hipGetErrorString(e));
  ctx->arena = static_cast<uint8_t *>(p);
  ctx->arena_size = bytes;
  ctx->arena_used = 0;
  return MQ_OK;
}

int mq_ctx_reserve_scratch(mq_ctx *ctx, size_t bytes) {
  if (!ctx) return fail(MQ_E_INVALID, "ctx is NULL");
  DeviceGuard g(ctx->device);
  return ensure_scratch(ctx, bytes);
}

static int make_tensor(mq_ctx *ctx, int dtype, int64_t n, int64_t k, mq_qtensor **out) {
  mq_qtensor *t = new (std::nothrow) mq_qtensor();
  if (!t) return fail(MQ_E_OOM, "out of host memory");
  t->ctx = ctx;
  t->dtype = dtype;
  t->n = n;
  t->k = k;
  t->geo = make_geo(dtype, n, k);
  t->gguf_bytes = gguf_row_bytes(dtype, k) * (size_t)n;
  int rc = alloc_weight(ctx, t);
  if (rc != MQ_OK) {
    delete t;
    return rc;
  }
  *out = t;
  return MQ_OK;
}

int mq_qtensor_from_device(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *dev_blocks, size_t nbytes,
                           void *stream, mq_qtensor **out) {
  if (!ctx || !out || !dev_blocks) return fail(MQ_E_INVALID, "mq_qtensor_from_device: NULL argument");
  *out = nullptr;
  int rc = check_weight_shape(dtype, n, k, nbytes);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  mq_qtensor *t = nullptr;
  rc = make_tensor(ctx, dtype, n, k, &t);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemsetAsync(t->data, 0, (size_t)t->geo.bytes, s);
  if (e == hipSuccess) e = launch_repack(dtype, dev_blocks, t->data, t->geo, false, s);
  if (e != hipSuccess) {
    mq_qtensor_free(t);
    return hip_fail(e, "repack to device layout");
  }
  *out = t;
  return MQ_OK;
}

int mq_qtensor_upload(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *host_blocks, size_t nbytes,
                      mq_qtensor **out) {
  if (!ctx || !out || !host_blocks) return fail(MQ_E_INVALID, "mq_qtensor_upload: NULL argument");
  *out = nullptr;
  int rc = check_weight_shape(dtype, n, k, nbytes);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  void *staging = nullptr;
  hipError_t e = hipMalloc(&staging, nbytes);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) staging failed: %s", nbytes, hipGetErrorString(e));
  e = hipMemcpy(staging, host_blocks, nbytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(staging);
    return hip_fail(e, "hipMemcpy H2D");
  }
  rc = mq_qtensor_from_device(ctx, dtype, n, k, staging, nbytes, nullptr, out);
  hipError_t se = hipStreamSynchronize(nullptr);
  (void)hipFree(staging);
  if (rc) return rc;
  if (se != hipSuccess) {
    mq_qtensor_free(*out);
    *out = nullptr;
    return hip_fail(se, "upload synchronize");
  }
  return MQ_OK;
}

int mq_quantize(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const float *src, int64_t ld, void *stream,
                mq_qtensor **out) {
  if (!ctx || !out || !src) return fail(MQ_E_INVALID, "mq_quantize: NULL argument");
  *out = nullptr;
  if (!is_quant(dtype)) return fail(MQ_E_INVALID, "mq_quantize: dtype %d is not a GGUF block type", dtype);
  if (n <= 0 || k <= 0 || ld < k)
    return fail(MQ_E_INVALID, "mq_quantize: bad shape n=%lld k=%lld ld=%lld", (long long)n, (long long)k, (long long)ld);
  const TypeInfo ti = type_info(dtype);
  if (k % ti.bs != 0) return fail(MQ_E_INVALID, "%s needs k %% %d == 0, got k=%lld", ti.name, ti.bs, (long long)k);
  DeviceGuard g(ctx->device);
  const size_t nbytes = gguf_row_bytes(dtype, k) * (size_t)n;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void *staging = nullptr;
  hipError_t e = hipMalloc(&staging, nbytes);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) staging failed: %s", nbytes, hipGetErrorString(e));
  e = launch_quantize(dtype, src, ld, n, k, staging, s);
  int rc = MQ_OK;
  if (e != hipSuccess) rc = hip_fail(e, "quantize launch");
  if (rc == MQ_OK) rc = mq_qtensor_from_device(ctx, dtype, n, k, staging, nbytes, stream, out);
  const hipError_t se = hipStreamSynchronize(s);
  (void)hipFree(staging);
  if (rc != MQ_OK) return rc;
  if (se != hipSuccess) {
    mq_qtensor_free(*out);
    *out = nullptr;
    return hip_fail(se, "quantize synchronize");
  }
  return MQ_OK;
}

int mq_qtensor_download(mq_ctx *ctx, const mq_qtensor *w, void *host_blocks, size_t nbytes) {
  if (!ctx || !w || !host_blocks) return fail(MQ_E_INVALID, "mq_qtensor_download: NULL argument");
  if (nbytes != w->gguf_bytes) return fail(MQ_E_INVALID, "download needs %zu bytes, got %zu", w->gguf_bytes, nbytes);
  DeviceGuard g(ctx->device);
  void *staging = nullptr;
  hipError_t e = hipMalloc(&staging, nbytes);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) staging failed", nbytes);
  e = launch_repack(w->dtype, w->data, staging, w->geo, true, nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e == hipSuccess) e = hipMemcpy(host_blocks, staging, nbytes, hipMemcpyDeviceToHost);
  (void)hipFree(staging);
  if (e != hipSuccess) return hip_fail(e, "download");
  return MQ_OK;
}

void mq_qtensor_free(mq_qtensor *w) {
  if (!w) return;
  if (w->data && !w->in_arena) {
    DeviceGuard g(w->ctx->device);
    (void)hipFree(w->data);
  }
  delete w;
}

int mq_qtensor_info(const mq_qtensor *w, int *dtype, int64_t *n, int64_t *k, size_t *gguf_bytes,
                    size_t *device_bytes) {
  if (!w) return fail(MQ_E_INVALID, "mq_qtensor_info: NULL tensor");
  if (dtype) *dtype = w->dtype;
  if (n) *n = w->n;
  if (k) *k = w->k;
  if (gguf_bytes) *gguf_bytes = w->gguf_bytes;
  if (device_bytes) *device_bytes = (size_t)w->geo.bytes;
  return MQ_OK;
}

int mq_dequantize(mq_ctx *ctx, const mq_qtensor *w, void *dst, int dst_dtype, void *stream) {
  if (!ctx || !w || !dst) return fail(MQ_E_INVALID, "mq_dequantize: NULL argument");
  if (dst_dtype != MQ_F32 && dst_dtype != MQ_F16 && dst_dtype != MQ_BF16)
    return fail(MQ_E_INVALID, "mq_dequantize: dst dtype %d must be F32, F16 or BF16", dst_dtype);
  if (reinterpret_cast<uintptr_t>(dst) & 15) return fail(MQ_E_INVALID, "mq_dequantize: dst must be 16-byte aligned");
  DeviceGuard g(ctx->device);
  hipError_t e = launch_dequant(w->dtype, view_of(w), w->n, w->k, dst, dst_dtype, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  return MQ_OK;
}

int mq_qmatmul(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx, void *y,
               int y_dtype, int64_t ldy, const float *bias, int act, void *stream) {
  if (!ctx || !w) return fail(MQ_E_INVALID, "mq_qmatmul: NULL ctx or weight");
  if (m < 0) return fail(MQ_E_INVALID, "mq_qmatmul: m=%lld < 0", (long long)m);
  if (m == 0) return MQ_OK;
  if (!x || !y) return fail(MQ_E_INVALID, "mq_qmatmul: NULL x or y");
  if (x_dtype != MQ_F32 && x_dtype != MQ_BF16) return fail(MQ_E_INVALID, "mq_qmatmul: x dtype %d must be F32 or BF16", x_dtype);
  if (y_dtype != MQ_F32 && y_dtype != MQ_BF16) return fail(MQ_E_INVALID, "mq_qmatmul: y dtype %d must be F32 or BF16", y_dtype);
  if (ldx < w->k) return fail(MQ_E_INVALID, "mq_qmatmul: ldx=%lld < k=%lld", (long long)ldx, (long long)w->k);
  if (ldy < w->n) return fail(MQ_E_INVALID, "mq_qmatmul: ldy=%lld < n=%lld", (long long)ldy, (long long)w->n);
  if (act != MQ_ACT_NONE && act != MQ_ACT_GELU_TANH) return fail(MQ_E_INVALID, "mq_qmatmul: unknown act %d", act);
  DeviceGuard g(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const WView wv = view_of(w);
  const int64_t n = w->n, k = w->k;

  if (m <= kGemvMaxM) {
    if (gemv_reads_x_in_place(w->dtype, m, n, k, x, x_dtype, ldx, ctx->cu_count)) {
      // Q4_K: f32 or bf16 x read in place, no scratch
      hipError_t e = launch_gemv(w->dtype, wv, n, k, x, x_dtype, m, ldx, y, y_dtype, ldy, bias, act, nullptr,
                                 ctx->cu_count, s);
      if (e != hipSuccess) return hip_fail(e, "gemv launch");
      return MQ_OK;
    }
    // otherwise x goes to scratch as contiguous f32 (widened from bf16, or
    // copied when its rows are not 16-byte aligned) unless it already is
    const void *xf = x;
    int64_t ldxf = ldx;
    const bool stage_x = x_dtype == MQ_BF16 || (reinterpret_cast<uintptr_t>(x) & 15) != 0 || (ldx % 4) != 0;
    size_t need = gemv_scratch_bytes(w->dtype, m, n, k, ctx->cu_count);
    size_t xoff = (need + 255) & ~size_t(255);
    if (stage_x) need = xoff + (size_t)m * k * sizeof(float);
    if (need) {
      int rc = ensure_scratch(ctx, need);
      if (rc) return rc;
    }
    if (stage_x) {
      float *xs = reinterpret_cast<float *>(static_cast<uint8_t *>(ctx->scratch) + xoff);
      hipError_t e = x_dtype == MQ_BF16
                         ? launch_widen_bf16(static_cast<const __bf16 *>(x), m, k, ldx, xs, s)
                         : hipMemcpy2DAsync(xs, k * sizeof(float), x, ldx * sizeof(float), k * sizeof(float), m,
                                            hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) return hip_fail(e, "stage activations for the GEMV");
      xf = xs;
      ldxf = k;
    }
    hipError_t e = launch_gemv(w->dtype, wv, n, k, xf, MQ_F32, m, ldxf, y, y_dtype, ldy, bias, act,
                               static_cast<float *>(ctx->scratch), ctx->cu_count, s);
    if (e != hipSuccess) return hip_fail(e, "gemv launch");
    return MQ_OK;
  }

  return run_gemm(ctx, w, x, x_dtype, m, ldx, y, y_dtype, ldy, bias, nullptr, act, s);
}

int mq_qmatmul_gated_add(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx,
                         float *y, int64_t ldy, const float *bias, const float *gate, void *stream) {
  if (!ctx || !w) return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: NULL ctx or weight");
  if (m < 0) return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: m=%lld < 0", (long long)m);
  if (m == 0) return MQ_OK;
  if (!x || !y || !gate) return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: NULL x, y or gate");
  if (x_dtype != MQ_F32 && x_dtype != MQ_BF16)
    return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: x dtype %d must be F32 or BF16", x_dtype);
  if (ldx < w->k) return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: ldx=%lld < k=%lld", (long long)ldx, (long long)w->k);
  if (ldy < w->n) return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: ldy=%lld < n=%lld", (long long)ldy, (long long)w->n);
  DeviceGuard g(ctx->device);
  // every m takes the GEMM kernel: its epilogue holds the gated update
  return run_gemm(ctx, w, x, x_dtype, m, ldx, y, MQ_F32, ldy, bias, gate, MQ_ACT_NONE, static_cast<hipStream_t>(stream));
}

}  // extern "C"
