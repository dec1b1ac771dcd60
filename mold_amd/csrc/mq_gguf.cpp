// mq_gguf.cpp — GGUF v2/v3 container reader and writer (host side of weight
// residency and of mold's GGUF cache producers).
//
// Restates the published GGUF layout that candle's gguf_file::Content::read
// parses and gguf_file::write produces (candle-core-mold 0.9.10,
// Cargo.lock:507; read at crates/mold-inference/src/flux/pipeline.rs:286-287
// and through VarBuilder::from_gguf at :976; written by the FP8 -> Q8_0 cache
// at :240 and the embedding-patched cache at :541):
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x {string key, u32 type, value}, n_tensors x {string name,
//   u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset},
//   padding to general.alignment (default 32), tensor data, each tensor at an
//   offset (from the data start) that is a multiple of the alignment.
// Strings are u64 length + bytes.  Values: u8 i8 u16 i16 u32 i32 f32 bool
// string array u64 i64 f64 (type ids 0..12); an array is u32 element type,
// u64 count, elements.  The reader keeps every metadata value (nested arrays
// are kept as their type and length only).
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <memory>
#include <new>
#include <string>
#include <vector>

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

// One metadata value: scalars and numeric arrays as raw little-endian
// elements, strings (and string arrays) as std::string.
struct Kv {
  std::string key;
  uint32_t type = 0;       // GType of the value
  uint32_t elem_type = 0;  // element type (== type for scalars)
  uint64_t count = 1;      // elements (1 for scalars)
  std::vector<uint8_t> raw;
  std::vector<std::string> strs;
  bool nested = false;     // array of arrays: values not kept
};

}  // namespace

struct mq_gguf {
  std::string path;
  uint32_t version = 0;
  uint64_t alignment = 32;
  std::vector<Kv> kvs;
  std::vector<TensorInfo> tensors;
};

namespace {

int gfail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
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
  uint64_t fsize;  // bytes in the file: no length read from it may exceed what is left
  bool ok = true;
  template <typename T>
  T get() {
    T v{};
    if (fread(&v, sizeof(T), 1, f) != 1) ok = false;
    return v;
  }
  // Bytes between the read position and the end of the file.
  uint64_t left() const {
    const off_t pos = ftello(f);
    return pos < 0 || (uint64_t)pos > fsize ? 0 : fsize - (uint64_t)pos;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > (1ull << 30) || n > left()) {
      ok = false;
      return {};
    }
    std::string s(n, '\0');
    if (n && fread(&s[0], 1, n, f) != n) ok = false;
    return s;
  }
  bool bytes(void *dst, size_t n) {
    if (n && fread(dst, 1, n, f) != n) ok = false;
    return ok;
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

// Skips one array value (nested arrays), at most 8 levels deep.
bool skip_array(Reader &r, int depth) {
  const uint32_t et = r.get<uint32_t>();
  const uint64_t cnt = r.get<uint64_t>();
  if (!r.ok) return false;
  if (et == STR) {
    for (uint64_t i = 0; i < cnt && r.ok; ++i) (void)r.str();
  } else if (et == ARR) {
    if (depth > 8) return false;  // deeper nesting than any GGUF writer produces
    for (uint64_t i = 0; i < cnt && r.ok; ++i)
      if (!skip_array(r, depth + 1)) return false;
  } else {
    const size_t es = scalar_size(et);
    if (!es || cnt > (1ull << 34) / es || es * cnt > r.left()) return false;
    if (fseeko(r.f, (off_t)(es * cnt), SEEK_CUR) != 0) return false;
  }
  return r.ok;
}

bool read_value(Reader &r, Kv &kv) {
  if (kv.type == STR) {
    kv.elem_type = STR;
    kv.strs.push_back(r.str());
    return r.ok;
  }
  if (kv.type == ARR) {
    kv.elem_type = r.get<uint32_t>();
    kv.count = r.get<uint64_t>();
    if (!r.ok) return false;
    if (kv.elem_type == STR) {
      // every string holds at least its 8-byte length: a count the rest of
      // the file cannot hold is malformed, and nothing is reserved for it
      if (kv.count > (1ull << 26) || kv.count > r.left() / 8) return false;
      kv.strs.reserve(kv.count);
      for (uint64_t i = 0; i < kv.count && r.ok; ++i) kv.strs.push_back(r.str());
      return r.ok;
    }
    if (kv.elem_type == ARR) {
      kv.nested = true;
      for (uint64_t i = 0; i < kv.count && r.ok; ++i)
        if (!skip_array(r, 1)) return false;
      return r.ok;
    }
    const size_t es = scalar_size(kv.elem_type);
    if (!es || kv.count > (1ull << 30) / es || es * kv.count > r.left()) return false;
    kv.raw.resize(es * kv.count);
    return r.bytes(kv.raw.data(), kv.raw.size());
  }
  const size_t es = scalar_size(kv.type);
  if (!es) return false;
  kv.elem_type = kv.type;
  kv.raw.resize(es);
  return r.bytes(kv.raw.data(), es);
}

const Kv *kv_at(const mq_gguf *g, int64_t i) {
  if (!g || i < 0 || i >= (int64_t)g->kvs.size()) return nullptr;
  return &g->kvs[(size_t)i];
}

bool is_int_type(uint32_t t) {
  return t == U8 || t == I8 || t == U16 || t == I16 || t == U32 || t == I32 || t == U64 || t == I64 || t == BOOL;
}

int64_t int_at(const Kv &kv, uint64_t e) {
  const uint8_t *p = kv.raw.data() + e * scalar_size(kv.elem_type);
  switch (kv.elem_type) {
    case U8: case BOOL: return *p;
    case I8: return (int8_t)*p;
    case U16: { uint16_t v; memcpy(&v, p, 2); return v; }
    case I16: { int16_t v; memcpy(&v, p, 2); return v; }
    case U32: { uint32_t v; memcpy(&v, p, 4); return v; }
    case I32: { int32_t v; memcpy(&v, p, 4); return v; }
    case U64: { uint64_t v; memcpy(&v, p, 8); return (int64_t)v; }
    default: { int64_t v; memcpy(&v, p, 8); return v; }
  }
}

// Runs fn(), turning any C++ exception into a status code: nothing is thrown
// across the C ABI (an allocation the host cannot satisfy is MQ_E_OOM).
template <typename Fn>
int no_throw(const char *what, Fn &&fn) {
  try {
    return fn();
  } catch (const std::bad_alloc &) {
    return gfail(MQ_E_OOM, "%s: out of host memory", what);
  } catch (...) {
    return gfail(MQ_E_IO, "%s: unexpected failure", what);
  }
}

int gguf_open(const char *path, mq_gguf **out) {
  std::unique_ptr<FILE, int (*)(FILE *)> file(fopen(path, "rb"), fclose);
  if (!file) return gfail(MQ_E_IO, "cannot open %s", path);
  if (fseeko(file.get(), 0, SEEK_END) != 0) return gfail(MQ_E_IO, "cannot seek %s", path);
  const off_t fend = ftello(file.get());
  if (fend < 0 || fseeko(file.get(), 0, SEEK_SET) != 0) return gfail(MQ_E_IO, "cannot seek %s", path);
  Reader r{file.get(), (uint64_t)fend};
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
    Kv kv;
    kv.key = r.str();
    kv.type = r.get<uint32_t>();
    if (!r.ok || !read_value(r, kv)) {
      r.ok = false;
      break;
    }
    if (kv.key == "general.alignment") {
      if (kv.type != U32 && kv.type != U64) return gfail(MQ_E_IO, "%s: general.alignment is not an integer", path);
      const uint64_t iv = (uint64_t)int_at(kv, 0);
      if (iv == 0 || (iv & (iv - 1)) != 0 || iv > 65536)
        return gfail(MQ_E_IO, "%s: general.alignment %llu is not a power of two", path, (unsigned long long)iv);
      g->alignment = iv;
    }
    g->kvs.push_back(std::move(kv));
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
  const uint64_t fsize = r.fsize;
  for (auto &t : g->tensors) {
    if (t.offset > fsize || t.offset % g->alignment != 0)
      return gfail(MQ_E_IO, "tensor %s: bad data offset %llu", t.name.c_str(), (unsigned long long)t.offset);
    t.offset += data_start;
    if (t.offset + t.nbytes > fsize) return gfail(MQ_E_IO, "tensor %s extends past end of file", t.name.c_str());
  }
  *out = g.release();
  return MQ_OK;
}

}  // namespace

extern "C" {

int mq_gguf_open(const char *path, mq_gguf **out) {
  if (!path || !out) return gfail(MQ_E_INVALID, "mq_gguf_open: NULL argument");
  *out = nullptr;
  return no_throw("mq_gguf_open", [&] { return gguf_open(path, out); });
}

void mq_gguf_close(mq_gguf *g) { delete g; }

int mq_gguf_version(const mq_gguf *g) { return g ? (int)g->version : -1; }

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

int mq_gguf_read_tensor(const mq_gguf *g, int64_t index, void *dst, size_t nbytes) {
  if (!g || !dst || index < 0 || index >= (int64_t)g->tensors.size())
    return gfail(MQ_E_INVALID, "mq_gguf_read_tensor: bad argument");
  const TensorInfo &t = g->tensors[(size_t)index];
  if (nbytes != t.nbytes) return gfail(MQ_E_INVALID, "tensor %s is %zu bytes, got %zu", t.name.c_str(), t.nbytes, nbytes);
  const int fd = open(g->path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return gfail(MQ_E_IO, "cannot reopen %s", g->path.c_str());
  size_t got = 0;
  while (got < nbytes) {
    const ssize_t r = pread(fd, static_cast<uint8_t *>(dst) + got, nbytes - got, (off_t)(t.offset + got));
    if (r <= 0) break;
    got += (size_t)r;
  }
  close(fd);
  if (got != nbytes) return gfail(MQ_E_IO, "short read of tensor %s", t.name.c_str());
  return MQ_OK;
}

int64_t mq_gguf_kv_count(const mq_gguf *g) { return g ? (int64_t)g->kvs.size() : -1; }

int64_t mq_gguf_find_kv(const mq_gguf *g, const char *key) {
  if (!g || !key) return -1;
  for (size_t i = 0; i < g->kvs.size(); ++i)
    if (g->kvs[i].key == key) return (int64_t)i;
  return -1;
}

int mq_gguf_kv_info(const mq_gguf *g, int64_t index, const char **key, int *type, int *elem_type,
                    uint64_t *count) {
  const Kv *kv = kv_at(g, index);
  if (!kv) return gfail(MQ_E_INVALID, "metadata index %lld out of range", (long long)index);
  if (key) *key = kv->key.c_str();
  if (type) *type = (int)kv->type;
  if (elem_type) *elem_type = (int)kv->elem_type;
  if (count) *count = kv->count;
  return MQ_OK;
}

int mq_gguf_kv_int(const mq_gguf *g, int64_t index, uint64_t elem, int64_t *out) {
  const Kv *kv = kv_at(g, index);
  if (!kv || !out) return gfail(MQ_E_INVALID, "mq_gguf_kv_int: bad argument");
  if (kv->nested || !is_int_type(kv->elem_type))
    return gfail(MQ_E_INVALID, "metadata %s is not an integer or bool", kv->key.c_str());
  if (elem >= kv->count) return gfail(MQ_E_INVALID, "metadata %s: element %llu of %llu", kv->key.c_str(),
                                      (unsigned long long)elem, (unsigned long long)kv->count);
  *out = int_at(*kv, elem);
  return MQ_OK;
}

int mq_gguf_kv_float(const mq_gguf *g, int64_t index, uint64_t elem, double *out) {
  const Kv *kv = kv_at(g, index);
  if (!kv || !out) return gfail(MQ_E_INVALID, "mq_gguf_kv_float: bad argument");
  if (kv->nested || (kv->elem_type != F32T && kv->elem_type != F64))
    return gfail(MQ_E_INVALID, "metadata %s is not a float", kv->key.c_str());
  if (elem >= kv->count) return gfail(MQ_E_INVALID, "metadata %s: element %llu of %llu", kv->key.c_str(),
                                      (unsigned long long)elem, (unsigned long long)kv->count);
  if (kv->elem_type == F32T) {
    float v;
    memcpy(&v, kv->raw.data() + 4 * elem, 4);
    *out = v;
  } else {
    memcpy(out, kv->raw.data() + 8 * elem, 8);
  }
  return MQ_OK;
}

int mq_gguf_kv_str(const mq_gguf *g, int64_t index, uint64_t elem, const char **s, uint64_t *len) {
  const Kv *kv = kv_at(g, index);
  if (!kv || !s) return gfail(MQ_E_INVALID, "mq_gguf_kv_str: bad argument");
  if (kv->elem_type != STR) return gfail(MQ_E_INVALID, "metadata %s is not a string", kv->key.c_str());
  if (elem >= kv->strs.size()) return gfail(MQ_E_INVALID, "metadata %s: element %llu of %zu", kv->key.c_str(),
                                            (unsigned long long)elem, kv->strs.size());
  *s = kv->strs[(size_t)elem].c_str();
  if (len) *len = kv->strs[(size_t)elem].size();
  return MQ_OK;
}

int mq_gguf_load_tensors(mq_ctx *ctx, const mq_gguf *g, const int64_t *indices, int64_t count, mq_qtensor **out) {
  if (out)
    for (int64_t i = 0; i < count; ++i) out[i] = nullptr;
  if (!g || !out || count < 0 || (count > 0 && !indices))
    return gfail(MQ_E_INVALID, "mq_gguf_load_tensors: bad argument");
  if (!ctx) return gfail(MQ_E_INVALID, "mq_gguf_load_tensors: NULL ctx");
  if (count == 0) return MQ_OK;
  std::vector<mq::UploadJob> jobs;
  const int rj = no_throw("mq_gguf_load_tensors", [&] {
    jobs.resize((size_t)count);
    return MQ_OK;
  });
  if (rj) return rj;
  for (int64_t i = 0; i < count; ++i) {
    const int64_t index = indices[i];
    if (index < 0 || index >= (int64_t)g->tensors.size())
      return gfail(MQ_E_INVALID, "mq_gguf_load_tensors: index %lld out of range", (long long)index);
    const TensorInfo &t = g->tensors[(size_t)index];
    mq::UploadJob &j = jobs[(size_t)i];
    j.dtype = t.dtype;
    j.n = 1;
    for (int d = 1; d < t.n_dims; ++d) j.n *= t.dims[d];
    j.k = t.dims[0];
    j.offset = t.offset;
    j.nbytes = t.nbytes;
  }
  const int fd = open(g->path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return gfail(MQ_E_IO, "cannot reopen %s", g->path.c_str());
  const int rc = mq::upload_from_file(ctx, fd, jobs.data(), count, out);
  close(fd);
  return rc;
}

int mq_gguf_load_tensor(mq_ctx *ctx, const mq_gguf *g, int64_t index, mq_qtensor **out) {
  if (!g || !out || index < 0 || index >= (int64_t)g->tensors.size())
    return gfail(MQ_E_INVALID, "mq_gguf_load_tensor: bad argument");
  if (!ctx) return gfail(MQ_E_INVALID, "mq_gguf_load_tensor: NULL ctx");
  return mq_gguf_load_tensors(ctx, g, &index, 1, out);
}

}  // extern "C"

// ------------------------------------------------------------------ writer

namespace {

struct WTensor {
  std::string name;
  int dtype = 0;
  int n_dims = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  size_t nbytes = 0;
  std::vector<uint8_t> data;       // host copy, or
  const mq_qtensor *qt = nullptr;  // a device weight read back at finish
  mq_ctx *ctx = nullptr;
};

}  // namespace

struct mq_gguf_writer {
  std::string path;
  uint32_t alignment = 32;
  std::vector<Kv> kvs;
  std::vector<WTensor> tensors;
  bool finished = false;
};

namespace {

struct Out {
  FILE *f;
  bool ok = true;
  void bytes(const void *p, size_t n) {
    if (ok && n && fwrite(p, 1, n, f) != n) ok = false;
  }
  template <typename T>
  void put(T v) {
    bytes(&v, sizeof(T));
  }
  void str(const std::string &s) {
    put<uint64_t>(s.size());
    bytes(s.data(), s.size());
  }
  void pad_to(uint64_t pos, uint64_t align) {
    static const uint8_t zeros[256] = {0};
    uint64_t n = (align - pos % align) % align;
    while (n && ok) {
      const size_t c = n < sizeof(zeros) ? (size_t)n : sizeof(zeros);
      bytes(zeros, c);
      n -= c;
    }
  }
};

int add_kv(mq_gguf_writer *w, const char *key, uint32_t type, uint32_t elem_type, uint64_t count, const void *raw,
           size_t raw_bytes, const char *const *strs) {
  if (!w || !key) return gfail(MQ_E_INVALID, "GGUF writer: NULL writer or key");
  if (w->finished) return gfail(MQ_E_INVALID, "GGUF writer: already finished");
  for (const Kv &kv : w->kvs)
    if (kv.key == key) return gfail(MQ_E_INVALID, "GGUF writer: duplicate metadata key %s", key);
  return no_throw("GGUF writer metadata", [&] {
    Kv kv;
    kv.key = key;
    kv.type = type;
    kv.elem_type = elem_type;
    kv.count = count;
    if (raw_bytes) kv.raw.assign(static_cast<const uint8_t *>(raw), static_cast<const uint8_t *>(raw) + raw_bytes);
    if (strs)
      for (uint64_t i = 0; i < count; ++i) kv.strs.emplace_back(strs[i] ? strs[i] : "");
    w->kvs.push_back(std::move(kv));
    return (int)MQ_OK;
  });
}

int check_tensor_name(const mq_gguf_writer *w, const char *name) {
  if (!w || !name || !*name) return gfail(MQ_E_INVALID, "GGUF writer: NULL writer or empty tensor name");
  if (w->finished) return gfail(MQ_E_INVALID, "GGUF writer: already finished");
  for (const WTensor &t : w->tensors)
    if (t.name == name) return gfail(MQ_E_INVALID, "GGUF writer: duplicate tensor %s", name);
  return MQ_OK;
}

// Bytes of a tensor of `dtype` with GGUF dims (ne order), or 0 if invalid.
size_t tensor_bytes(int dtype, int n_dims, const int64_t *dims) {
  const int bs = mq_block_size(dtype), ts = mq_type_size(dtype);
  if (bs <= 0 || ts <= 0 || n_dims < 1 || n_dims > 4 || dims[0] % bs != 0) return 0;
  uint64_t elems = 1;
  for (int d = 0; d < n_dims; ++d) {
    if (dims[d] <= 0) return 0;
    elems *= (uint64_t)dims[d];
  }
  return (size_t)(elems / bs) * ts;
}

int writer_finish(mq_gguf_writer *w);

}  // namespace

extern "C" {

int mq_gguf_writer_create(const char *path, uint32_t alignment, mq_gguf_writer **out) {
  if (!path || !out) return gfail(MQ_E_INVALID, "mq_gguf_writer_create: NULL argument");
  *out = nullptr;
  if (alignment == 0) alignment = 32;
  if ((alignment & (alignment - 1)) != 0 || alignment > 65536)
    return gfail(MQ_E_INVALID, "GGUF alignment %u is not a power of two", alignment);
  return no_throw("mq_gguf_writer_create", [&] {
    std::unique_ptr<mq_gguf_writer> w(new mq_gguf_writer());
    w->path = path;
    w->alignment = alignment;
    if (alignment != 32) {
      const uint32_t a = alignment;
      const int rc = add_kv(w.get(), "general.alignment", U32, U32, 1, &a, 4, nullptr);
      if (rc) return rc;
    }
    *out = w.release();
    return (int)MQ_OK;
  });
}

void mq_gguf_writer_free(mq_gguf_writer *w) { delete w; }

int mq_gguf_writer_kv_scalar(mq_gguf_writer *w, const char *key, int type, const void *value) {
  const size_t es = scalar_size((uint32_t)type);
  if (!es || !value) return gfail(MQ_E_INVALID, "GGUF writer: metadata type %d is not a scalar type", type);
  if (key && strcmp(key, "general.alignment") == 0) return gfail(MQ_E_INVALID, "set general.alignment at create");
  return add_kv(w, key, (uint32_t)type, (uint32_t)type, 1, value, es, nullptr);
}

int mq_gguf_writer_kv_str(mq_gguf_writer *w, const char *key, const char *value) {
  if (!value) return gfail(MQ_E_INVALID, "GGUF writer: NULL string");
  return add_kv(w, key, STR, STR, 1, nullptr, 0, &value);
}

int mq_gguf_writer_kv_array(mq_gguf_writer *w, const char *key, int elem_type, const void *values, uint64_t count) {
  const size_t es = scalar_size((uint32_t)elem_type);
  if (!es) return gfail(MQ_E_INVALID, "GGUF writer: array element type %d is not a scalar type", elem_type);
  if (count && !values) return gfail(MQ_E_INVALID, "GGUF writer: NULL array");
  return add_kv(w, key, ARR, (uint32_t)elem_type, count, values, es * count, nullptr);
}

int mq_gguf_writer_kv_str_array(mq_gguf_writer *w, const char *key, const char *const *values, uint64_t count) {
  if (count && !values) return gfail(MQ_E_INVALID, "GGUF writer: NULL array");
  return add_kv(w, key, ARR, STR, count, nullptr, 0, values);
}

int mq_gguf_writer_add_tensor(mq_gguf_writer *w, const char *name, int dtype, int n_dims, const int64_t *dims,
                              const void *data, size_t nbytes) {
  int rc = check_tensor_name(w, name);
  if (rc) return rc;
  if (!dims || !data) return gfail(MQ_E_INVALID, "GGUF writer: NULL dims or data for %s", name);
  const size_t want = tensor_bytes(dtype, n_dims, dims);
  if (!want) return gfail(MQ_E_INVALID, "GGUF writer: tensor %s has bad type %d or dims", name, dtype);
  if (want != nbytes) return gfail(MQ_E_INVALID, "GGUF writer: tensor %s needs %zu bytes, got %zu", name, want, nbytes);
  WTensor t;
  t.dtype = dtype;
  t.n_dims = n_dims;
  for (int d = 0; d < n_dims; ++d) t.dims[d] = (uint64_t)dims[d];
  t.nbytes = nbytes;
  return no_throw("GGUF writer tensor", [&] {
    t.name = name;
    t.data.assign(static_cast<const uint8_t *>(data), static_cast<const uint8_t *>(data) + nbytes);
    w->tensors.push_back(std::move(t));
    return (int)MQ_OK;
  });
}

int mq_gguf_writer_add_qtensor(mq_gguf_writer *w, mq_ctx *ctx, const char *name, const mq_qtensor *qt, int n_dims,
                               const int64_t *dims) {
  int rc = check_tensor_name(w, name);
  if (rc) return rc;
  if (!ctx || !qt) return gfail(MQ_E_INVALID, "GGUF writer: NULL ctx or tensor for %s", name);
  int dtype = 0;
  int64_t n = 0, k = 0;
  size_t gb = 0;
  rc = mq_qtensor_info(qt, &dtype, &n, &k, &gb, nullptr);
  if (rc) return rc;
  WTensor t;
  t.dtype = dtype;
  if (n_dims == 0) {  // [n, k] as GGUF ne = {k, n}
    t.n_dims = 2;
    t.dims[0] = (uint64_t)k;
    t.dims[1] = (uint64_t)n;
  } else {
    if (!dims || n_dims < 1 || n_dims > 4 || dims[0] != k || tensor_bytes(dtype, n_dims, dims) != gb)
      return gfail(MQ_E_INVALID, "GGUF writer: dims of %s must have ne0 = %lld and %lld elements", name,
                   (long long)k, (long long)(n * k));
    t.n_dims = n_dims;
    for (int d = 0; d < n_dims; ++d) t.dims[d] = (uint64_t)dims[d];
  }
  t.nbytes = gb;
  t.qt = qt;
  t.ctx = ctx;
  return no_throw("GGUF writer tensor", [&] {
    t.name = name;
    w->tensors.push_back(std::move(t));
    return (int)MQ_OK;
  });
}

int mq_gguf_writer_finish(mq_gguf_writer *w) {
  if (!w) return gfail(MQ_E_INVALID, "mq_gguf_writer_finish: NULL writer");
  if (w->finished) return gfail(MQ_E_INVALID, "GGUF writer: already finished");
  return no_throw("mq_gguf_writer_finish", [&] { return writer_finish(w); });
}

}  // extern "C"

namespace {

int writer_finish(mq_gguf_writer *w) {
  const std::string tmp = w->path + ".tmp." + std::to_string((long long)getpid());
  FILE *f = fopen(tmp.c_str(), "wb");
  if (!f) return gfail(MQ_E_IO, "cannot create %s", tmp.c_str());
  Out o{f};
  o.put<uint32_t>(0x46554747u);
  o.put<uint32_t>(3);
  o.put<uint64_t>(w->tensors.size());
  o.put<uint64_t>(w->kvs.size());
  for (const Kv &kv : w->kvs) {
    o.str(kv.key);
    o.put<uint32_t>(kv.type);
    if (kv.type == ARR) {
      o.put<uint32_t>(kv.elem_type);
      o.put<uint64_t>(kv.count);
    }
    if (kv.elem_type == STR)
      for (const std::string &s : kv.strs) o.str(s);
    else
      o.bytes(kv.raw.data(), kv.raw.size());
  }
  uint64_t off = 0;
  for (const WTensor &t : w->tensors) {
    o.str(t.name);
    o.put<uint32_t>((uint32_t)t.n_dims);
    for (int d = 0; d < t.n_dims; ++d) o.put<uint64_t>(t.dims[d]);
    o.put<uint32_t>((uint32_t)t.dtype);
    o.put<uint64_t>(off);
    off += t.nbytes;
    off = (off + w->alignment - 1) / w->alignment * w->alignment;
  }
  uint64_t pos = (uint64_t)ftello(f);
  o.pad_to(pos, w->alignment);
  std::vector<uint8_t> buf;
  int rc = MQ_OK;
  uint64_t data_pos = 0;
  for (const WTensor &t : w->tensors) {
    if (!o.ok) break;
    const uint8_t *src = t.data.data();
    if (t.qt) {
      try {
        buf.resize(t.nbytes);
      } catch (...) {
        rc = gfail(MQ_E_OOM, "GGUF writer: cannot hold %zu bytes of %s", t.nbytes, t.name.c_str());
        break;
      }
      rc = mq_qtensor_download(t.ctx, t.qt, buf.data(), t.nbytes);
      if (rc) break;
      src = buf.data();
    }
    o.bytes(src, t.nbytes);
    data_pos += t.nbytes;
    o.pad_to(data_pos, w->alignment);
    data_pos = (data_pos + w->alignment - 1) / w->alignment * w->alignment;
  }
  const bool closed = fclose(f) == 0;
  if (rc == MQ_OK && (!o.ok || !closed)) rc = gfail(MQ_E_IO, "write to %s failed", tmp.c_str());
  if (rc == MQ_OK && rename(tmp.c_str(), w->path.c_str()) != 0)
    rc = gfail(MQ_E_IO, "cannot rename %s to %s", tmp.c_str(), w->path.c_str());
  if (rc != MQ_OK) {
    remove(tmp.c_str());
    return rc;
  }
  w->finished = true;
  return MQ_OK;
}

}  // namespace
