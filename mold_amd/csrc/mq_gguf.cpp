// mq_gguf.cpp — GGUF v2/v3 container reader (host side of weight residency).
//
// Restates the published GGUF layout that candle's gguf_file::Content::read
// parses (candle-core-mold 0.9.10, Cargo.lock:507; called at
// crates/mold-inference/src/flux/pipeline.rs:286-287 and through
// VarBuilder::from_gguf at :976):
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x {string key, u32 type, value}, n_tensors x {string name,
//   u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset},
//   padding to general.alignment (default 32), tensor data.
// Strings are u64 length + bytes.  Metadata values are skipped except
// general.alignment.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <memory>
#include <new>
#include <string>
#include <vector>

#include <fcntl.h>
#include <unistd.h>

#include "../../include/moldq.h"
#include "mq_internal.h"

namespace {

enum GType : uint32_t {
  U8 = 0, I8 = 1, U16 = 2, I16 = 3, U32 = 4, I32 = 5, F32T = 6, BOOL = 7, STR = 8, ARR = 9,
  U64 = 10, I64 = 11, F64 = 12
};

struct TensorInfo {
  std::string name;
  int n_dims = 0;
  int64_t dims[4] = {1, 1, 1, 1};
  int dtype = 0;
  uint64_t offset = 0;  // absolute file offset of the data
  size_t nbytes = 0;
};

}  // namespace

struct mq_gguf {
  std::string path;
  uint32_t version = 0;
  uint64_t alignment = 32;
  std::vector<TensorInfo> tensors;
};

namespace {

int gfail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return mq::set_error(code, buf);
}

struct Reader {
  FILE *f;
  bool ok = true;
  template <typename T>
  T get() {
    T v{};
    if (fread(&v, sizeof(T), 1, f) != 1) ok = false;
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > (1ull << 30)) {
      ok = false;
      return {};
    }
    std::string s(n, '\0');
    if (n && fread(&s[0], 1, n, f) != n) ok = false;
    return s;
  }
  void skip(uint64_t n) {
    if (fseeko(f, (off_t)n, SEEK_CUR) != 0) ok = false;
  }
};

size_t scalar_size(uint32_t t) {
  switch (t) {
    case U8: case I8: case BOOL: return 1;
    case U16: case I16: return 2;
    case U32: case I32: case F32T: return 4;
    case U64: case I64: case F64: return 8;
    default: return 0;
  }
}

// Skip one metadata value; returns its integer value for scalar int types.
bool skip_value(Reader &r, uint32_t type, uint64_t *as_int) {
  if (type == STR) {
    (void)r.str();
    return r.ok;
  }
  if (type == ARR) {
    const uint32_t et = r.get<uint32_t>();
    const uint64_t cnt = r.get<uint64_t>();
    if (!r.ok) return false;
    if (et == STR) {
      for (uint64_t i = 0; i < cnt && r.ok; ++i) (void)r.str();
    } else if (et == ARR) {
      for (uint64_t i = 0; i < cnt && r.ok; ++i)
        if (!skip_value(r, ARR, nullptr)) return false;
    } else {
      const size_t es = scalar_size(et);
      if (!es) return false;
      r.skip(es * cnt);
    }
    return r.ok;
  }
  const size_t sz = scalar_size(type);
  if (!sz) return false;
  uint64_t v = 0;
  if (fread(&v, sz, 1, r.f) != 1) return false;
  if (as_int) *as_int = v;
  return true;
}

}  // namespace

extern "C" {

int mq_gguf_open(const char *path, mq_gguf **out) {
  if (!path || !out) return gfail(MQ_E_INVALID, "mq_gguf_open: NULL argument");
  *out = nullptr;
  std::unique_ptr<FILE, int (*)(FILE *)> file(fopen(path, "rb"), fclose);
  if (!file) return gfail(MQ_E_IO, "cannot open %s", path);
  Reader r{file.get()};
  std::unique_ptr<mq_gguf> g(new (std::nothrow) mq_gguf());
  if (!g) return gfail(MQ_E_OOM, "out of host memory");
  g->path = path;
  const uint32_t magic = r.get<uint32_t>();
  g->version = r.get<uint32_t>();
  if (!r.ok || magic != 0x46554747u) return gfail(MQ_E_IO, "%s is not a GGUF file", path);
  if (g->version < 2 || g->version > 3)
    return gfail(MQ_E_IO, "GGUF version %u not supported (2 or 3)", g->version);
  const uint64_t n_tensors = r.get<uint64_t>();
  const uint64_t n_kv = r.get<uint64_t>();
  if (!r.ok || n_tensors > (1ull << 24) || n_kv > (1ull << 24))
    return gfail(MQ_E_IO, "%s: implausible tensor/metadata counts", path);
  for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
    const std::string key = r.str();
    const uint32_t type = r.get<uint32_t>();
    uint64_t iv = 0;
    if (!r.ok || !skip_value(r, type, &iv)) {
      r.ok = false;
      break;
    }
    if (key == "general.alignment" && (type == U32 || type == U64)) {
      if (iv == 0 || (iv & (iv - 1)) != 0 || iv > 65536)
        return gfail(MQ_E_IO, "%s: general.alignment %llu is not a power of two", path, (unsigned long long)iv);
      g->alignment = iv;
    }
  }
  for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
    TensorInfo t;
    t.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok || nd < 1 || nd > 4) {
      r.ok = false;
      break;
    }
    t.n_dims = (int)nd;
    bool dims_ok = true;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint64_t v = r.get<uint64_t>();
      dims_ok = dims_ok && v > 0 && v < (1ull << 40);
      t.dims[d] = (int64_t)v;
    }
    t.dtype = (int)r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (!r.ok) break;
    if (!dims_ok) return gfail(MQ_E_IO, "tensor %s: bad dimensions", t.name.c_str());
    int64_t elems = 1;
    for (int d = 0; d < t.n_dims; ++d) {
      if (elems > (int64_t(1) << 46) / t.dims[d]) return gfail(MQ_E_IO, "tensor %s: too large", t.name.c_str());
      elems *= t.dims[d];
    }
    const int bs = mq_block_size(t.dtype), ts = mq_type_size(t.dtype);
    if (bs <= 0 || ts <= 0 || t.dims[0] % bs != 0)
      return gfail(MQ_E_IO, "tensor %s: unsupported type %d or ne0 %lld", t.name.c_str(), t.dtype,
                   (long long)t.dims[0]);
    t.nbytes = (size_t)(elems / bs) * ts;
    g->tensors.push_back(std::move(t));
  }
  if (!r.ok) return gfail(MQ_E_IO, "%s: truncated or malformed GGUF header", path);
  const off_t pos = ftello(file.get());
  const uint64_t data_start = ((uint64_t)pos + g->alignment - 1) / g->alignment * g->alignment;
  fseeko(file.get(), 0, SEEK_END);
  const uint64_t fsize = (uint64_t)ftello(file.get());
  for (auto &t : g->tensors) {
    if (t.offset > fsize || t.offset % g->alignment != 0)
      return gfail(MQ_E_IO, "tensor %s: bad data offset %llu", t.name.c_str(), (unsigned long long)t.offset);
    t.offset += data_start;
    if (t.offset + t.nbytes > fsize) return gfail(MQ_E_IO, "tensor %s extends past end of file", t.name.c_str());
  }
  *out = g.release();
  return MQ_OK;
}

void mq_gguf_close(mq_gguf *g) { delete g; }

int64_t mq_gguf_tensor_count(const mq_gguf *g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t mq_gguf_find(const mq_gguf *g, const char *name) {
  if (!g || !name) return -1;
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) return (int64_t)i;
  return -1;
}

int mq_gguf_tensor_info(const mq_gguf *g, int64_t index, const char **name, int *dtype, int *n_dims,
                        int64_t dims[4], uint64_t *file_offset, size_t *nbytes) {
  if (!g || index < 0 || index >= (int64_t)g->tensors.size())
    return gfail(MQ_E_INVALID, "tensor index %lld out of range", (long long)index);
  const TensorInfo &t = g->tensors[(size_t)index];
  if (name) *name = t.name.c_str();
  if (dtype) *dtype = t.dtype;
  if (n_dims) *n_dims = t.n_dims;
  if (dims)
    for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
  if (file_offset) *file_offset = t.offset;
  if (nbytes) *nbytes = t.nbytes;
  return MQ_OK;
}

int mq_gguf_load_tensor(mq_ctx *ctx, const mq_gguf *g, int64_t index, mq_qtensor **out) {
  if (!g || !out || index < 0 || index >= (int64_t)g->tensors.size())
    return gfail(MQ_E_INVALID, "mq_gguf_load_tensor: bad argument");
  const TensorInfo &t = g->tensors[(size_t)index];
  if (mq_block_size(t.dtype) <= 1)
    return gfail(MQ_E_UNSUPPORTED, "tensor %s is dense (type %d); only GGUF block types upload", t.name.c_str(), t.dtype);
  int64_t rows = 1;
  for (int d = 1; d < t.n_dims; ++d) rows *= t.dims[d];
  if (!ctx) return gfail(MQ_E_INVALID, "mq_gguf_load_tensor: NULL ctx");
  const int fd = open(g->path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return gfail(MQ_E_IO, "cannot reopen %s", g->path.c_str());
  const int rc = mq::upload_from_file(ctx, t.dtype, rows, t.dims[0], fd, t.offset, t.nbytes, out);
  close(fd);
  return rc;
}

}  // extern "C"
