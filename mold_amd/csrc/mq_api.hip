// mq_api.hip — the C ABI declared in include/moldq.h: contexts, HBM arena,
// weight upload/download, dequantize and the quantized matmul dispatcher.
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/moldq.h"
#include "mq_internal.h"
#include "mq_kernels.h"

using namespace mq;

// Scratch of mq_qmatmul_noalloc: one copy per GPU, reached from host code only
// through the per-device address that mq_ctx_create resolves (noalloc_scratch).
static __device__ __align__(256) uint8_t scratch[MQ_NOALLOC_SCRATCH_BYTES];

struct mq_ctx {
  int device = 0;
  int cu_count = 0;
  // HBM arena: one allocation, bump-allocated by uploads, freed with the ctx.
  uint8_t *arena = nullptr;
  size_t arena_size = 0;
  size_t arena_used = 0;
  // Per-stream workspaces: f32 -> bf16 activation staging, GEMM tail partial
  // sums, generic-GEMV partials and widened x.  A stream's workspace only
  // grows: the outgrown buffer is kept (retired) until the context is
  // destroyed, so no call synchronizes or frees, and work already queued (or
  // captured in a graph) never sees its buffer released.
  struct Ws {
    hipStream_t stream = nullptr;
    uint8_t *p = nullptr;
    size_t size = 0;
  };
  std::vector<Ws> ws;
  std::vector<void *> retired;
  // Streams whose GEMMs never split K over a partial last round of tiles
  // (mq_ctx_set_stream_tail_split).
  std::vector<hipStream_t> no_tail_split;
  size_t ws_floor = 0;  // mq_ctx_reserve_scratch: minimum size of every workspace
  // Upload staging: device buffers for raw GGUF blocks (grow, kept; the
  // second only for batched GGUF loads, which fill one while the other is
  // repacked), and for each upload thread two pinned host buffers and a copy
  // stream (allocated on the first large upload).  The repack runs on
  // upload_stream.
  uint8_t *dstage[2] = {};
  size_t dstage_size[2] = {};
  uint8_t *pinned[2 * mq::kUploadThreads] = {};
  hipStream_t copy_streams[mq::kUploadThreads] = {};
  hipStream_t upload_stream = nullptr;
  // Device address of this GPU's copy of `scratch` (mq_qmatmul_noalloc).
  uint8_t *noalloc_scratch = nullptr;
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

constexpr size_t kMiB = size_t(1) << 20;
size_t round_mib(size_t b) { return (b + kMiB - 1) & ~(kMiB - 1); }
size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// Dense GGUF tensors (biases, norm scales, embeddings and other tensors a
// block type cannot hold) are stored as they are in the file: row-major [n, k].
bool is_dense(int dtype) { return dtype == MQ_F32 || dtype == MQ_F16 || dtype == MQ_BF16; }
size_t dense_size(int dtype) { return dtype == MQ_F32 ? 4 : 2; }
const char *dense_name(int dtype) { return dtype == MQ_F32 ? "F32" : dtype == MQ_F16 ? "F16" : "BF16"; }

size_t gguf_row_bytes(int dtype, int64_t k) {
  if (is_dense(dtype)) return (size_t)k * dense_size(dtype);
  const TypeInfo ti = type_info(dtype);
  return (size_t)(k / ti.bs) * ti.ts;
}

int check_weight_shape(int dtype, int64_t n, int64_t k, size_t nbytes) {
  if (!is_quant(dtype) && !is_dense(dtype))
    return fail(MQ_E_INVALID, "dtype %d is not a GGUF block type or F32 / F16 / BF16", dtype);
  const char *name = is_dense(dtype) ? dense_name(dtype) : type_info(dtype).name;
  if (n <= 0 || k <= 0) return fail(MQ_E_INVALID, "weight shape [%lld, %lld] must be positive", (long long)n, (long long)k);
  if (!is_dense(dtype) && k % type_info(dtype).bs != 0)
    return fail(MQ_E_INVALID, "%s needs k %% %d == 0, got k=%lld", name, type_info(dtype).bs, (long long)k);
  const size_t want = gguf_row_bytes(dtype, k) * (size_t)n;
  if (nbytes != want)
    return fail(MQ_E_INVALID, "%s [%lld, %lld] is %zu bytes, got %zu", name, (long long)n, (long long)k, want, nbytes);
  return MQ_OK;
}

int alloc_weight(mq_ctx *ctx, mq_qtensor *t) {
  const size_t bytes = (size_t)t->geo.bytes;
  const size_t aligned_used = align256(ctx->arena_used);
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

// The workspace of stream s, at least `bytes` long.  Growth allocates a new
// buffer and retires the old one (no synchronization, no free).  A stream
// being captured into a graph cannot grow its workspace.
int stream_workspace(mq_ctx *ctx, hipStream_t s, size_t bytes, uint8_t **out) {
  *out = nullptr;
  mq_ctx::Ws *w = nullptr;
  for (auto &e : ctx->ws)
    if (e.stream == s) w = &e;
  if (!w) {
    ctx->ws.push_back(mq_ctx::Ws{s, nullptr, 0});
    w = &ctx->ws.back();
  }
  if (bytes <= w->size && w->p) {
    *out = w->p;
    return MQ_OK;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(MQ_E_INVALID,
                "stream is being captured and its workspace (%zu bytes) is smaller than the %zu bytes this call "
                "needs: run the call once on this stream before capturing or reserve the workspace with "
                "mq_ctx_reserve_stream_scratch",
                w->size, bytes);
  const size_t sz = round_mib(std::max({bytes, 2 * w->size, ctx->ws_floor}));
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) for the stream workspace failed: %s", sz, hipGetErrorString(e));
  if (w->p) ctx->retired.push_back(w->p);
  w->p = static_cast<uint8_t *>(p);
  w->size = sz;
  *out = w->p;
  return MQ_OK;
}

WView view_of(const mq_qtensor *w) { return make_view(w->data, w->geo); }

// Scratch layout of one quantized-matmul call.
struct Plan {
  bool gemv = false;
  bool stage_gemm = false;  // f32 (or unaligned bf16) x staged as bf16 for the GEMM
  bool stage_gemv = false;  // x widened / copied to contiguous f32 for the generic GEMV
  int64_t kp = 0;           // staged GEMM row length (k rounded up to 64)
  GemmTail tail{0, 1, kGemmTileM};
  size_t stage_off = 0, stage_bytes = 0;
  size_t part_off = 0, part_bytes = 0;  // GEMM tail partials or generic-GEMV K-split partials
  size_t total = 0;
};

Plan plan_qmatmul(const mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx,
                  bool gated, bool tail_split = true) {
  Plan p;
  const int64_t n = w->n, k = w->k;
  if (m <= kGemvMaxM && !gated) {
    p.gemv = true;
    if (gemv_reads_x_in_place(w->dtype, m, n, k, x, x_dtype, ldx, ctx->cu_count)) return p;  // no scratch
    p.stage_gemv = x_dtype == MQ_BF16 || (reinterpret_cast<uintptr_t>(x) & 15) != 0 || (ldx % 4) != 0;
    p.part_bytes = gemv_scratch_bytes(w->dtype, m, n, k, ctx->cu_count);
    p.stage_bytes = p.stage_gemv ? (size_t)m * k * sizeof(float) : 0;
  } else {
    p.kp = (k + 63) / 64 * 64;
    p.stage_gemm =
        !(x_dtype == MQ_BF16 && k == p.kp && (ldx % 8) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0);
    const int64_t lda = p.stage_gemm ? p.kp : ldx;
    p.stage_bytes = p.stage_gemm ? (size_t)m * p.kp * sizeof(__bf16) : 0;
    p.tail = gemm_tail_plan(w->dtype, m, n, k, ctx->cu_count, tail_split);
    if (p.tail.kparts > 1 && gemm_fast_ok(w->dtype, m, k, lda)) p.part_bytes = gemm_tail_bytes(p.tail, m, n);
    else p.tail.kparts = 1;
  }
  p.part_off = align256(p.stage_bytes);
  p.total = p.part_bytes ? p.part_off + p.part_bytes : p.stage_bytes;
  return p;
}

bool tail_split_on(const mq_ctx *ctx, hipStream_t s) {
  return std::find(ctx->no_tail_split.begin(), ctx->no_tail_split.end(), s) == ctx->no_tail_split.end();
}

// Runs one planned call with its scratch at `ws` (p.total bytes).
int run_qmatmul(mq_ctx *ctx, const mq_qtensor *w, const Plan &p, uint8_t *ws, const void *x, int x_dtype, int64_t m,
                int64_t ldx, void *y, int y_dtype, int64_t ldy, const float *bias, const float *gate, int act,
                hipStream_t s) {
  const WView wv = view_of(w);
  const int64_t n = w->n, k = w->k;
  float *partial = p.part_bytes ? reinterpret_cast<float *>(ws + p.part_off) : nullptr;
  if (p.gemv) {
    const void *xf = x;
    int xt = x_dtype;
    int64_t ldxf = ldx;
    if (p.stage_gemv) {
      float *xs = reinterpret_cast<float *>(ws + p.stage_off);
      hipError_t e = x_dtype == MQ_BF16
                         ? launch_widen_bf16(static_cast<const __bf16 *>(x), m, k, ldx, xs, s)
                         : hipMemcpy2DAsync(xs, k * sizeof(float), x, ldx * sizeof(float), k * sizeof(float), m,
                                            hipMemcpyDeviceToDevice, s);
      if (e != hipSuccess) return hip_fail(e, "stage activations for the GEMV");
      xf = xs;
      xt = MQ_F32;
      ldxf = k;
    }
    hipError_t e = launch_gemv(w->dtype, wv, n, k, xf, xt, m, ldxf, y, y_dtype, ldy, bias, act, partial,
                               ctx->cu_count, s);
    if (e != hipSuccess) return hip_fail(e, "gemv launch");
    return MQ_OK;
  }
  const __bf16 *a = static_cast<const __bf16 *>(x);
  int64_t lda = ldx;
  if (p.stage_gemm) {
    __bf16 *st = reinterpret_cast<__bf16 *>(ws + p.stage_off);
    hipError_t e = launch_stage_bf16(x, x_dtype, m, k, ldx, st, p.kp, s);
    if (e != hipSuccess) return hip_fail(e, "stage activations");
    a = st;
    lda = p.kp;
  }
  hipError_t e = launch_gemm(w->dtype, wv, n, k, w->geo.ntiles, a, m, lda, y, y_dtype, ldy, bias, gate, act, p.tail,
                             partial, s);
  if (e != hipSuccess) return hip_fail(e, "gemm launch");
  return MQ_OK;
}

int check_qmatmul_args(const char *fn, const mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m,
                       int64_t ldx, const void *y, int y_dtype, int64_t ldy, int act) {
  if (!ctx || !w) return fail(MQ_E_INVALID, "%s: NULL ctx or weight", fn);
  if (m < 0) return fail(MQ_E_INVALID, "%s: m=%lld < 0", fn, (long long)m);
  if (m == 0) return MQ_OK;
  if (!x || !y) return fail(MQ_E_INVALID, "%s: NULL x or y", fn);
  if (is_dense(w->dtype))
    return fail(MQ_E_UNSUPPORTED,
                "%s: the weight is a dense %s tensor; like candle's QMatMul::from_arc, dequantize it once "
                "(mq_dequantize) and use the device's dense matmul",
                fn, dense_name(w->dtype));
  if (x_dtype == MQ_X_Q8K) {
    if (!gemv_takes_x_q8k(w->dtype, m, w->n, w->k, ctx->cu_count))
      return fail(MQ_E_UNSUPPORTED, "%s: x in MQ_X_Q8K form needs a Q4_K weight, m <= %d and the GEMV's shape limits", fn,
                  kGemvMaxM);
    if (ldx != w->k || (reinterpret_cast<uintptr_t>(x) & 15) != 0)
      return fail(MQ_E_INVALID, "%s: MQ_X_Q8K x must be contiguous rows (ldx = k) at a 16-byte aligned address", fn);
  } else if (x_dtype != MQ_F32 && x_dtype != MQ_BF16) {
    return fail(MQ_E_INVALID, "%s: x dtype %d must be F32, BF16 or MQ_X_Q8K", fn, x_dtype);
  }
  if (y_dtype != MQ_F32 && y_dtype != MQ_BF16) return fail(MQ_E_INVALID, "%s: y dtype %d must be F32 or BF16", fn, y_dtype);
  if (ldx < w->k) return fail(MQ_E_INVALID, "%s: ldx=%lld < k=%lld", fn, (long long)ldx, (long long)w->k);
  if (ldy < w->n) return fail(MQ_E_INVALID, "%s: ldy=%lld < n=%lld", fn, (long long)ldy, (long long)w->n);
  if (act != MQ_ACT_NONE && act != MQ_ACT_GELU_TANH) return fail(MQ_E_INVALID, "%s: unknown act %d", fn, act);
  return MQ_OK;
}

int make_tensor(mq_ctx *ctx, int dtype, int64_t n, int64_t k, mq_qtensor **out) {
  mq_qtensor *t = new (std::nothrow) mq_qtensor();
  if (!t) return fail(MQ_E_OOM, "out of host memory");
  t->ctx = ctx;
  t->dtype = dtype;
  t->n = n;
  t->k = k;
  t->gguf_bytes = gguf_row_bytes(dtype, k) * (size_t)n;
  if (is_dense(dtype)) {  // stored as in the file: no tiles, no planes
    t->geo = Geo{};
    t->geo.n = n;
    t->geo.k = k;
    t->geo.nb = k;
    t->geo.bytes = (int64_t)t->gguf_bytes;
  } else {
    t->geo = make_geo(dtype, n, k);
  }
  int rc = alloc_weight(ctx, t);
  if (rc != MQ_OK) {
    delete t;
    return rc;
  }
  *out = t;
  return MQ_OK;
}

// Raw GGUF blocks already in device memory (at `raw`) into a new
// device-resident tensor, on stream s.  The repack kernel writes every byte
// of the tiled layout, padding rows included.
int tensor_from_raw(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *raw, hipStream_t s, mq_qtensor **out) {
  mq_qtensor *t = nullptr;
  int rc = make_tensor(ctx, dtype, n, k, &t);
  if (rc) return rc;
  hipError_t e = is_dense(dtype) ? hipMemcpyAsync(t->data, raw, t->gguf_bytes, hipMemcpyDeviceToDevice, s)
                                 : launch_repack(dtype, raw, t->data, t->geo, false, s);
  if (e != hipSuccess) {
    mq_qtensor_free(t);
    return hip_fail(e, "repack to device layout");
  }
  *out = t;
  return MQ_OK;
}

// The context's device staging buffer `slot` (0 or 1) for raw blocks, at
// least `bytes` long.  Callers have synchronized the work that used it before
// (uploads, quantize and download all return finished).
int device_stage(mq_ctx *ctx, size_t bytes, uint8_t **out, int slot = 0) {
  uint8_t *&buf = ctx->dstage[slot];
  size_t &size = ctx->dstage_size[slot];
  if (bytes > size) {
    if (buf) {
      HIP_TRY(hipFree(buf), "free upload staging");
      buf = nullptr;
      size = 0;
    }
    const size_t sz = round_mib(bytes);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) return fail(MQ_E_OOM, "hipMalloc(%zu) for upload staging failed: %s", sz, hipGetErrorString(e));
    buf = static_cast<uint8_t *>(p);
    size = sz;
  }
  *out = buf;
  return MQ_OK;
}

// Where a staged upload's bytes come from: an open file (pread at `offset`)
// or host memory.
struct UploadSource {
  int fd = -1;
  uint64_t offset = 0;
  const uint8_t *host = nullptr;
  // Fills dst with source bytes [pos, pos + len); false on a short read.
  bool read(uint8_t *dst, size_t pos, size_t len) const {
    if (host) {
      memcpy(dst, host + pos, len);
      return true;
    }
    size_t got = 0;
    while (got < len) {
      const ssize_t r = pread(fd, dst + got, len - got, (off_t)(offset + pos + got));
      if (r < 0 && errno == EINTR) continue;
      if (r <= 0) return false;
      got += (size_t)r;
    }
    return true;
  }
};

int upload_resources(mq_ctx *ctx) {
  if (!ctx->upload_stream)
    HIP_TRY(hipStreamCreateWithFlags(&ctx->upload_stream, hipStreamNonBlocking), "create upload stream");
  for (auto &s : ctx->copy_streams)
    if (!s) HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "create upload copy stream");
  for (auto &p : ctx->pinned)
    if (!p) HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&p), mq::kUploadChunk, hipHostMallocDefault), "hipHostMalloc");
  return MQ_OK;
}

// Copies `nbytes` of `src` to device memory `dst` and returns once every byte
// has landed.  The bytes are cut into T * rounds equal chunks (at most
// kUploadChunk, at least 1 MiB unless the tensor is smaller, multiples of
// 64 KiB), so every thread has the same work; chunk c belongs to thread
// c % T.  A thread fills its two pinned buffers in turn (file read or memcpy,
// the host-side cost that one thread cannot hide behind the PCIe copy) and
// queues each chunk's copy on its own stream; a buffer is refilled only after
// an event says its previous copy has left it.  The calling thread is thread 0.
int staged_h2d(mq_ctx *ctx, const UploadSource &src, uint8_t *dst, size_t nbytes) {
  if (nbytes == 0) return MQ_OK;
  int rc = upload_resources(ctx);
  if (rc) return rc;
  constexpr size_t kGrain = size_t(64) << 10, kMinChunk = size_t(1) << 20;
  const size_t nt_max = std::max<size_t>(1, std::min<size_t>(mq::kUploadThreads, (nbytes + kMinChunk - 1) / kMinChunk));
  const size_t rounds = (nbytes + nt_max * mq::kUploadChunk - 1) / (nt_max * mq::kUploadChunk);
  const size_t per = (nbytes + nt_max * rounds - 1) / (nt_max * rounds);
  const size_t chunk = std::min(mq::kUploadChunk, (per + kGrain - 1) / kGrain * kGrain);
  const size_t chunks = (nbytes + chunk - 1) / chunk;
  const int nt = (int)std::min(nt_max, chunks);
  struct Result {
    int code = MQ_OK;
    char msg[160] = {};
  };
  std::vector<Result> res(nt);
  std::atomic<bool> stop{false};
  auto work = [&](int t) {
    Result &r = res[t];
    auto bad = [&](int code, const char *what, size_t pos) {
      r.code = code;
      snprintf(r.msg, sizeof r.msg, "%s at byte %zu of a %zu-byte upload", what, pos, nbytes);
      stop.store(true);
    };
    hipStream_t s = ctx->copy_streams[t];
    hipEvent_t ev[2] = {nullptr, nullptr};
    if (hipSetDevice(ctx->device) != hipSuccess || hipEventCreateWithFlags(&ev[0], hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ev[1], hipEventDisableTiming) != hipSuccess) {
      bad(MQ_E_HIP, "upload thread set-up failed", 0);
    } else {
      bool used[2] = {false, false};
      int b = 0;
      for (size_t c = (size_t)t; c < chunks && !stop.load(std::memory_order_relaxed); c += (size_t)nt, b ^= 1) {
        const size_t pos = c * chunk, len = std::min(chunk, nbytes - pos);
        uint8_t *buf = ctx->pinned[2 * t + b];
        if (used[b] && hipEventSynchronize(ev[b]) != hipSuccess) {
          bad(MQ_E_HIP, "upload event wait failed", pos);
          break;
        }
        if (!src.read(buf, pos, len)) {
          bad(MQ_E_IO, "short read", (size_t)src.offset + pos);
          break;
        }
        if (hipMemcpyAsync(dst + pos, buf, len, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipEventRecord(ev[b], s) != hipSuccess) {
          bad(MQ_E_HIP, "async H2D copy failed", pos);
          break;
        }
        used[b] = true;
      }
    }
    // No copy may still read a pinned buffer once this call returns.
    if (hipStreamSynchronize(s) != hipSuccess && r.code == MQ_OK) bad(MQ_E_HIP, "upload copy stream failed", 0);
    for (auto e : ev)
      if (e) (void)hipEventDestroy(e);
  };
  std::vector<std::thread> pool;
  try {
    for (int t = 1; t < nt; ++t) pool.emplace_back(work, t);
  } catch (...) {  // fewer threads than asked for: stop the ones started
    stop.store(true);
    for (auto &th : pool) th.join();
    return fail(MQ_E_HIP, "could not start upload threads");
  }
  work(0);
  for (auto &th : pool) th.join();
  for (const Result &r : res)
    if (r.code != MQ_OK) return fail(r.code, "%s", r.msg);
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
  void *sp = nullptr;
  {
    DeviceGuard g(device_ordinal);
    HIP_TRY(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  }
  mq_ctx *c = new (std::nothrow) mq_ctx();
  if (!c) return fail(MQ_E_OOM, "out of host memory");
  c->device = device_ordinal;
  c->cu_count = prop.multiProcessorCount;
  c->noalloc_scratch = static_cast<uint8_t *>(sp);
  *out = c;
  return MQ_OK;
}

void mq_ctx_destroy(mq_ctx *ctx) {
  if (!ctx) return;
  DeviceGuard g(ctx->device);
  (void)hipDeviceSynchronize();
  for (auto &w : ctx->ws)
    if (w.p) (void)hipFree(w.p);
  for (void *p : ctx->retired) (void)hipFree(p);
  for (auto *p : ctx->dstage)
    if (p) (void)hipFree(p);
  for (auto *p : ctx->pinned)
    if (p) (void)hipHostFree(p);
  for (auto s : ctx->copy_streams)
    if (s) (void)hipStreamDestroy(s);
  if (ctx->upload_stream) (void)hipStreamDestroy(ctx->upload_stream);
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
  ctx->ws_floor = std::max(ctx->ws_floor, bytes);
  for (size_t i = 0; i < ctx->ws.size(); ++i) {
    uint8_t *p = nullptr;
    int rc = stream_workspace(ctx, ctx->ws[i].stream, bytes, &p);
    if (rc) return rc;
  }
  uint8_t *p = nullptr;
  return stream_workspace(ctx, nullptr, bytes, &p);  // the null stream's, now
}

int mq_ctx_reserve_stream_scratch(mq_ctx *ctx, void *stream, size_t bytes) {
  if (!ctx) return fail(MQ_E_INVALID, "ctx is NULL");
  DeviceGuard g(ctx->device);
  uint8_t *p = nullptr;
  return stream_workspace(ctx, static_cast<hipStream_t>(stream), bytes, &p);
}

int mq_ctx_set_stream_tail_split(mq_ctx *ctx, void *stream, int enabled) {
  if (!ctx) return fail(MQ_E_INVALID, "ctx is NULL");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  auto &v = ctx->no_tail_split;
  const auto it = std::find(v.begin(), v.end(), s);
  if (enabled && it != v.end()) v.erase(it);
  if (!enabled && it == v.end()) v.push_back(s);
  return MQ_OK;
}

int mq_qtensor_from_device(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *dev_blocks, size_t nbytes,
                           void *stream, mq_qtensor **out) {
  if (!ctx || !out || !dev_blocks) return fail(MQ_E_INVALID, "mq_qtensor_from_device: NULL argument");
  *out = nullptr;
  int rc = check_weight_shape(dtype, n, k, nbytes);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  return tensor_from_raw(ctx, dtype, n, k, dev_blocks, static_cast<hipStream_t>(stream), out);
}

int mq_qtensor_upload(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *host_blocks, size_t nbytes,
                      mq_qtensor **out) {
  if (!ctx || !out || !host_blocks) return fail(MQ_E_INVALID, "mq_qtensor_upload: NULL argument");
  *out = nullptr;
  int rc = check_weight_shape(dtype, n, k, nbytes);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  if (is_dense(dtype)) {  // no repack: the bytes go straight to their place
    mq_qtensor *t = nullptr;
    rc = make_tensor(ctx, dtype, n, k, &t);
    if (rc) return rc;
    const hipError_t e = hipMemcpy(t->data, host_blocks, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      mq_qtensor_free(t);
      return hip_fail(e, "hipMemcpy H2D");
    }
    *out = t;
    return MQ_OK;
  }
  uint8_t *st = nullptr;
  rc = device_stage(ctx, nbytes, &st);
  if (rc) return rc;
  if (nbytes > kUploadChunk) {  // large weights: the threaded pinned pipeline
    UploadSource src;
    src.host = static_cast<const uint8_t *>(host_blocks);
    rc = staged_h2d(ctx, src, st, nbytes);
    if (rc) return rc;
  } else {
    HIP_TRY(hipMemcpy(st, host_blocks, nbytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  rc = tensor_from_raw(ctx, dtype, n, k, st, nullptr, out);
  if (rc) return rc;
  hipError_t se = hipStreamSynchronize(nullptr);
  if (se != hipSuccess) {
    mq_qtensor_free(*out);
    *out = nullptr;
    return hip_fail(se, "upload synchronize");
  }
  return MQ_OK;
}

// Shared by mq_quantize and mq_quantize_fp8: quantize src (f32 or FP8 E4M3
// bytes) on `stream`, the 32-element block types straight into the tensor's
// device layout, the k-quants into the upload staging buffer, then repack.
static int quantize_common(mq_ctx *ctx, const char *fn, int dtype, int64_t n, int64_t k, const void *src, bool fp8,
                           int64_t ld, float scale, void *stream, mq_qtensor **out) {
  if (!ctx || !out || !src) return fail(MQ_E_INVALID, "%s: NULL argument", fn);
  *out = nullptr;
  if (n <= 0 || k <= 0 || ld < k)
    return fail(MQ_E_INVALID, "%s: bad shape n=%lld k=%lld ld=%lld", fn, (long long)n, (long long)k, (long long)ld);
  if (is_dense(dtype) && !fp8) {
    // QTensor::quantize(.., F32 / F16 / BF16): the values themselves, rounded to
    // nearest even when narrowing (mold stores its small tensors this way,
    // flux/pipeline.rs:223-228)
    DeviceGuard g(ctx->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    mq_qtensor *t = nullptr;
    int rc = make_tensor(ctx, dtype, n, k, &t);
    if (rc) return rc;
    hipError_t e = launch_convert(src, MQ_F32, ld, n, k, t->data, dtype, k, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      mq_qtensor_free(t);
      return hip_fail(e, "dense quantize");
    }
    *out = t;
    return MQ_OK;
  }
  if (!is_quant(dtype))
    return fail(MQ_E_INVALID, "%s: dtype %d is not a GGUF block type%s", fn, dtype, fp8 ? "" : " or F32 / F16 / BF16");
  const TypeInfo ti = type_info(dtype);
  if (k % ti.bs != 0) return fail(MQ_E_INVALID, "%s needs k %% %d == 0, got k=%lld", ti.name, ti.bs, (long long)k);
  DeviceGuard g(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (quantize_tiled_ok(dtype)) {
    // 32-element block types: quantized straight into the device layout
    mq_qtensor *t = nullptr;
    int rc = make_tensor(ctx, dtype, n, k, &t);
    if (rc) return rc;
    hipError_t e = launch_quantize_tiled(dtype, src, fp8, ld, scale, t->data, t->geo, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      mq_qtensor_free(t);
      return hip_fail(e, "quantize");
    }
    *out = t;
    return MQ_OK;
  }
  const size_t nbytes = gguf_row_bytes(dtype, k) * (size_t)n;
  uint8_t *st = nullptr;
  int rc = device_stage(ctx, nbytes, &st);
  if (rc) return rc;
  hipError_t e = fp8 ? launch_quantize_fp8(dtype, static_cast<const uint8_t *>(src), ld, n, k, scale, st, s)
                     : launch_quantize(dtype, static_cast<const float *>(src), ld, n, k, st, s);
  if (e != hipSuccess) return hip_fail(e, "quantize launch");
  rc = tensor_from_raw(ctx, dtype, n, k, st, s, out);
  if (rc) return rc;
  const hipError_t se = hipStreamSynchronize(s);
  if (se != hipSuccess) {
    mq_qtensor_free(*out);
    *out = nullptr;
    return hip_fail(se, "quantize synchronize");
  }
  return MQ_OK;
}

int mq_quantize(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const float *src, int64_t ld, void *stream,
                mq_qtensor **out) {
  return quantize_common(ctx, "mq_quantize", dtype, n, k, src, false, ld, 1.0f, stream, out);
}

int mq_quantize_fp8(mq_ctx *ctx, int dtype, int64_t n, int64_t k, const void *src, int64_t ld, float scale,
                    void *stream, mq_qtensor **out) {
  return quantize_common(ctx, "mq_quantize_fp8", dtype, n, k, src, true, ld, scale, stream, out);
}

int mq_qtensor_download(mq_ctx *ctx, const mq_qtensor *w, void *host_blocks, size_t nbytes) {
  if (!ctx || !w || !host_blocks) return fail(MQ_E_INVALID, "mq_qtensor_download: NULL argument");
  if (nbytes != w->gguf_bytes) return fail(MQ_E_INVALID, "download needs %zu bytes, got %zu", w->gguf_bytes, nbytes);
  DeviceGuard g(ctx->device);
  if (is_dense(w->dtype)) {
    HIP_TRY(hipMemcpy(host_blocks, w->data, nbytes, hipMemcpyDeviceToHost), "download");
    return MQ_OK;
  }
  uint8_t *st = nullptr;
  int rc = device_stage(ctx, nbytes, &st);
  if (rc) return rc;
  hipError_t e = launch_repack(w->dtype, w->data, st, w->geo, true, nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e == hipSuccess) e = hipMemcpy(host_blocks, st, nbytes, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "download");
  return MQ_OK;
}

int mq_qtensor_concat_rows(mq_ctx *ctx, const mq_qtensor *const *parts, int64_t count, mq_qtensor **out) {
  if (!ctx || !parts || !out || count <= 0) return fail(MQ_E_INVALID, "mq_qtensor_concat_rows: bad argument");
  *out = nullptr;
  int64_t n = 0;
  size_t bytes = 0;
  for (int64_t i = 0; i < count; ++i) {
    const mq_qtensor *p = parts[i];
    if (!p) return fail(MQ_E_INVALID, "mq_qtensor_concat_rows: part %lld is NULL", (long long)i);
    if (p->ctx != ctx) return fail(MQ_E_INVALID, "mq_qtensor_concat_rows: part %lld belongs to another context", (long long)i);
    if (p->dtype != parts[0]->dtype || p->k != parts[0]->k)
      return fail(MQ_E_INVALID, "mq_qtensor_concat_rows: part %lld is type %d with k = %lld, part 0 type %d with k = %lld",
                  (long long)i, p->dtype, (long long)p->k, parts[0]->dtype, (long long)parts[0]->k);
    n += p->n;
    bytes += p->gguf_bytes;
  }
  const int dtype = parts[0]->dtype;
  int rc = check_weight_shape(dtype, n, parts[0]->k, bytes);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  uint8_t *st = nullptr;
  rc = device_stage(ctx, bytes, &st);
  if (rc) return rc;
  // every part's GGUF bytes, in order, into the staging buffer (the inverse
  // repack writes its n real rows), then one repack of the whole
  size_t off = 0;
  for (int64_t i = 0; i < count; ++i) {
    const mq_qtensor *p = parts[i];
    const hipError_t e = is_dense(dtype) ? hipMemcpyAsync(st + off, p->data, p->gguf_bytes, hipMemcpyDeviceToDevice, nullptr)
                                         : launch_repack(dtype, p->data, st + off, p->geo, true, nullptr);
    if (e != hipSuccess) return hip_fail(e, "concat: part to GGUF blocks");
    off += p->gguf_bytes;
  }
  rc = tensor_from_raw(ctx, dtype, n, parts[0]->k, st, nullptr, out);
  if (rc) return rc;
  const hipError_t se = hipStreamSynchronize(nullptr);
  if (se != hipSuccess) {
    mq_qtensor_free(*out);
    *out = nullptr;
    return hip_fail(se, "concat synchronize");
  }
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (is_dense(w->dtype)) {
    const hipError_t e = w->dtype == dst_dtype
                             ? hipMemcpyAsync(dst, w->data, w->gguf_bytes, hipMemcpyDeviceToDevice, s)
                             : launch_convert(w->data, w->dtype, w->k, w->n, w->k, dst, dst_dtype, w->k, s);
    if (e != hipSuccess) return hip_fail(e, "dense dequantize");
    return MQ_OK;
  }
  hipError_t e = launch_dequant(w->dtype, view_of(w), w->n, w->k, dst, dst_dtype, s);
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  return MQ_OK;
}

int mq_qmatmul_workspace_size(mq_ctx *ctx, const mq_qtensor *w, int x_dtype, int64_t m, int gated, size_t *bytes) {
  if (!ctx || !w || !bytes) return fail(MQ_E_INVALID, "mq_qmatmul_workspace_size: NULL argument");
  if (m < 0) return fail(MQ_E_INVALID, "mq_qmatmul_workspace_size: m=%lld < 0", (long long)m);
  if (x_dtype != MQ_F32 && x_dtype != MQ_BF16 && x_dtype != MQ_X_Q8K)
    return fail(MQ_E_INVALID, "mq_qmatmul_workspace_size: x dtype %d must be F32, BF16 or MQ_X_Q8K", x_dtype);
  if (x_dtype == MQ_X_Q8K) {  // the GEMV reads it in place: no scratch
    if (!gemv_takes_x_q8k(w->dtype, m, w->n, w->k, ctx->cu_count) || gated)
      return fail(MQ_E_UNSUPPORTED, "mq_qmatmul_workspace_size: no MQ_X_Q8K GEMV for this weight and m");
    *bytes = 0;
    return MQ_OK;
  }
  if (is_dense(w->dtype))
    return fail(MQ_E_UNSUPPORTED, "mq_qmatmul_workspace_size: dense %s weights take no quantized matmul",
                dense_name(w->dtype));
  // a misaligned x pointer takes every staging path, so this is the bound
  // over all x placements and strides
  const void *worst = reinterpret_cast<const void *>(uintptr_t(1));
  *bytes = m == 0 ? 0 : plan_qmatmul(ctx, w, worst, x_dtype, m, w->k, gated != 0).total;
  return MQ_OK;
}

// mq_qmatmul with the activation on output columns act_col0 .. n-1 only.
static int qmatmul_cols(const char *fn, mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m,
                        int64_t ldx, void *y, int y_dtype, int64_t ldy, const float *bias, int act, int64_t act_col0,
                        void *stream) {
  int rc = check_qmatmul_args(fn, ctx, w, x, x_dtype, m, ldx, y, y_dtype, ldy, act);
  if (rc || m == 0) return rc;
  DeviceGuard g(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Plan p = plan_qmatmul(ctx, w, x, x_dtype, m, ldx, false, tail_split_on(ctx, s));
  uint8_t *ws = nullptr;
  if (p.total) {
    rc = stream_workspace(ctx, s, p.total, &ws);
    if (rc) return rc;
  }
  return run_qmatmul(ctx, w, p, ws, x, x_dtype, m, ldx, y, y_dtype, ldy, bias, nullptr, act_code(act, act_col0), s);
}

int mq_qmatmul(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx, void *y,
               int y_dtype, int64_t ldy, const float *bias, int act, void *stream) {
  return qmatmul_cols("mq_qmatmul", ctx, w, x, x_dtype, m, ldx, y, y_dtype, ldy, bias, act, 0, stream);
}

int mq_qmatmul_act_from(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx, void *y,
                        int y_dtype, int64_t ldy, const float *bias, int act, int64_t act_col0, void *stream) {
  if (!w) return fail(MQ_E_INVALID, "mq_qmatmul_act_from: NULL weight");
  if (act_col0 < 0 || act_col0 > w->n || w->n >= (int64_t(1) << 30))
    return fail(MQ_E_INVALID, "mq_qmatmul_act_from: act_col0=%lld outside 0 .. n=%lld (n below 2^30)",
                (long long)act_col0, (long long)w->n);
  return qmatmul_cols("mq_qmatmul_act_from", ctx, w, x, x_dtype, m, ldx, y, y_dtype, ldy, bias, act, act_col0,
                      stream);
}

int mq_quantize_x_q8k(mq_ctx *ctx, const void *x, int x_dtype, int64_t m, int64_t k, int64_t ldx, void *dst,
                      void *stream) {
  if (!ctx || ((!x || !dst) && m > 0)) return fail(MQ_E_INVALID, "mq_quantize_x_q8k: NULL argument");
  if (m < 0 || k <= 0 || k % 256 != 0 || ldx < k)
    return fail(MQ_E_INVALID, "mq_quantize_x_q8k: m=%lld, k=%lld (a multiple of 256), ldx=%lld", (long long)m,
                (long long)k, (long long)ldx);
  if (x_dtype != MQ_F32 && x_dtype != MQ_BF16)
    return fail(MQ_E_INVALID, "mq_quantize_x_q8k: x dtype %d must be F32 or BF16", x_dtype);
  const int64_t es = x_dtype == MQ_F32 ? 4 : 2;
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dst)) & 15) != 0 || (ldx * es) % 16 != 0)
    return fail(MQ_E_INVALID, "mq_quantize_x_q8k: x rows and dst must be 16-byte aligned");
  if (m == 0) return MQ_OK;
  DeviceGuard g(ctx->device);
  const hipError_t e = launch_quantize_x_q8k(x, x_dtype, m, k, ldx, dst, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "quantize x to Q8_K");
  return MQ_OK;
}

int mq_qmatmul_noalloc(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx, void *y,
                       int y_dtype, int64_t ldy, const float *bias, int act, void *stream) {
  int rc = check_qmatmul_args("mq_qmatmul_noalloc", ctx, w, x, x_dtype, m, ldx, y, y_dtype, ldy, act);
  if (rc || m == 0) return rc;
  DeviceGuard g(ctx->device);
  const Plan p =
      plan_qmatmul(ctx, w, x, x_dtype, m, ldx, false, tail_split_on(ctx, static_cast<hipStream_t>(stream)));
  if (p.total > MQ_NOALLOC_SCRATCH_BYTES)
    return fail(MQ_E_INVALID,
                "mq_qmatmul_noalloc: this call needs %zu bytes of scratch, more than its fixed %zu bytes "
                "(fewer rows, or bf16 x with 16-byte aligned rows, need less; mq_qmatmul has no limit)",
                p.total, (size_t)MQ_NOALLOC_SCRATCH_BYTES);
  // Every scratch byte the kernels read is written earlier in the same call
  // (staged rows and their zero padding, every split-K partial), so nothing
  // is cleared first.
  return run_qmatmul(ctx, w, p, ctx->noalloc_scratch, x, x_dtype, m, ldx, y, y_dtype, ldy, bias, nullptr, act,
                     static_cast<hipStream_t>(stream));
}

int mq_qmatmul_gated_add(mq_ctx *ctx, const mq_qtensor *w, const void *x, int x_dtype, int64_t m, int64_t ldx,
                         float *y, int64_t ldy, const float *bias, const float *gate, void *stream) {
  if (x_dtype == MQ_X_Q8K) return fail(MQ_E_UNSUPPORTED, "mq_qmatmul_gated_add: x in MQ_X_Q8K form takes the GEMV only");
  int rc = check_qmatmul_args("mq_qmatmul_gated_add", ctx, w, x, x_dtype, m, ldx, y, MQ_F32, ldy, MQ_ACT_NONE);
  if (rc || m == 0) return rc;
  if (!gate) return fail(MQ_E_INVALID, "mq_qmatmul_gated_add: NULL gate");
  DeviceGuard g(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // every m takes the GEMM kernel: its epilogue holds the gated update
  const Plan p = plan_qmatmul(ctx, w, x, x_dtype, m, ldx, true, tail_split_on(ctx, s));
  uint8_t *ws = nullptr;
  if (p.total) {
    rc = stream_workspace(ctx, s, p.total, &ws);
    if (rc) return rc;
  }
  return run_qmatmul(ctx, w, p, ws, x, x_dtype, m, ldx, y, MQ_F32, ldy, bias, gate, MQ_ACT_NONE, s);
}

}  // extern "C"

// ------------------------------------------------------------ GGUF upload
// Host-side piece of mq_gguf_load_tensor(s) (mq_gguf.cpp): each tensor's bytes
// go from the file through the threaded pinned pipeline (staged_h2d) into a
// device staging buffer, then the repack runs on the upload stream.  Tensors
// alternate between two staging buffers, so tensor i's repack (and the next
// tensor's hipMalloc) overlaps tensor i+1's file read and copy; a staging
// buffer is refilled once the event after its last repack has fired.
namespace mq {

int upload_from_file(mq_ctx *ctx, int fd, const UploadJob *jobs, int64_t count, mq_qtensor **out) {
  for (int64_t i = 0; i < count; ++i) out[i] = nullptr;
  size_t most = 0;
  for (int64_t i = 0; i < count; ++i) {
    const int rc = check_weight_shape(jobs[i].dtype, jobs[i].n, jobs[i].k, jobs[i].nbytes);
    if (rc) return rc;
    most = std::max(most, jobs[i].nbytes);
  }
  if (count == 0) return MQ_OK;
  DeviceGuard g(ctx->device);
  uint8_t *st[2] = {nullptr, nullptr};
  for (int b = 0; b < (count > 1 ? 2 : 1); ++b) {
    const int rc = device_stage(ctx, most, &st[b], b);
    if (rc) return rc;
  }
  int rc = upload_resources(ctx);
  if (rc) return rc;
  hipEvent_t done[2] = {nullptr, nullptr};
  for (auto &e : done)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      for (auto &d : done)
        if (d) (void)hipEventDestroy(d);
      return fail(MQ_E_HIP, "upload event create failed");
    }
  bool pending[2] = {false, false};
  int64_t made = 0;
  for (; made < count; ++made) {
    const UploadJob &j = jobs[made];
    const int b = (int)(made & 1);
    if (pending[b] && hipEventSynchronize(done[b]) != hipSuccess) {  // its last repack has read it
      rc = fail(MQ_E_HIP, "upload staging event wait failed");
      break;
    }
    UploadSource src;
    src.fd = fd;
    src.offset = j.offset;
    rc = staged_h2d(ctx, src, st[b], j.nbytes);
    if (rc) break;
    rc = tensor_from_raw(ctx, j.dtype, j.n, j.k, st[b], ctx->upload_stream, &out[made]);
    if (rc) break;
    if (hipEventRecord(done[b], ctx->upload_stream) != hipSuccess) {
      rc = fail(MQ_E_HIP, "upload staging event record failed");
      break;
    }
    pending[b] = true;
  }
  const hipError_t se = hipStreamSynchronize(ctx->upload_stream);
  for (auto e : done) (void)hipEventDestroy(e);
  if (rc == MQ_OK && se != hipSuccess) rc = hip_fail(se, "upload synchronize");
  if (rc != MQ_OK)
    for (int64_t i = 0; i < count; ++i) {
      mq_qtensor_free(out[i]);
      out[i] = nullptr;
    }
  return rc;
}

}  // namespace mq
