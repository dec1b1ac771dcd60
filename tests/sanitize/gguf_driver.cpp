// Sanitizer driver for libmoldq's GGUF reader and writer (mq_gguf.cpp), built
// on the CPU with AddressSanitizer + UndefinedBehaviorSanitizer.  The reader
// parses untrusted files, so besides a valid round trip it is fed every
// truncation of a valid file, crafted headers whose counts and lengths claim
// far more than the file holds, deep nesting, and seeded random byte
// mutations; every open must return a status code (no crash, no
// out-of-bounds access, no allocation the file cannot back), and a file that
// opens is queried through every accessor.  Prints "gguf_driver: ok".
// `gguf_driver table` prints the stub's block geometry for comparison with the
// built library.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "../../include/moldq.h"

namespace {

int g_failures = 0;

#define CHECK(cond)                                                      \
  do {                                                                   \
    if (!(cond)) {                                                       \
      fprintf(stderr, "CHECK failed at line %d: %s\n", __LINE__, #cond); \
      ++g_failures;                                                      \
    }                                                                    \
  } while (0)

std::vector<uint8_t> slurp(const std::string &p) {
  std::vector<uint8_t> b;
  FILE *f = fopen(p.c_str(), "rb");
  if (!f) return b;
  uint8_t buf[4096];
  size_t n;
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0) b.insert(b.end(), buf, buf + n);
  fclose(f);
  return b;
}

void dump(const std::string &p, const uint8_t *d, size_t n) {
  FILE *f = fopen(p.c_str(), "wb");
  if (!f) {
    perror("fopen");
    exit(2);
  }
  if (n) fwrite(d, 1, n, f);
  fclose(f);
}

// Every accessor on an open file: all metadata elements, all tensor infos
// and raw reads.  `strict`: names are found again by lookup (a mutated name
// may hold a NUL byte, which a C-string lookup cannot match).
void walk(mq_gguf *g, bool strict) {
  const int64_t nkv = mq_gguf_kv_count(g);
  for (int64_t i = 0; i < nkv; ++i) {
    const char *key = nullptr;
    int type = 0, et = 0;
    uint64_t cnt = 0;
    if (mq_gguf_kv_info(g, i, &key, &type, &et, &cnt) != MQ_OK) continue;
    CHECK(key != nullptr);
    if (strict) CHECK(mq_gguf_find_kv(g, key) >= 0);
    const uint64_t lim = cnt < 64 ? cnt : 64;
    for (uint64_t e = 0; e <= lim; ++e) {  // one past the end: an error, not a read
      int64_t iv;
      double fv;
      const char *s;
      uint64_t len;
      (void)mq_gguf_kv_int(g, i, e, &iv);
      (void)mq_gguf_kv_float(g, i, e, &fv);
      if (mq_gguf_kv_str(g, i, e, &s, &len) == MQ_OK) CHECK(strlen(s) <= len);
    }
  }
  const int64_t nt = mq_gguf_tensor_count(g);
  for (int64_t i = 0; i < nt; ++i) {
    const char *name = nullptr;
    int dt = 0, nd = 0;
    int64_t dims[4];
    uint64_t off = 0;
    size_t nb = 0;
    if (mq_gguf_tensor_info(g, i, &name, &dt, &nd, dims, &off, &nb) != MQ_OK) continue;
    if (strict) CHECK(mq_gguf_find(g, name) >= 0);
    if (nb <= (size_t(1) << 20)) {
      std::vector<uint8_t> buf(nb + 1);
      CHECK(mq_gguf_read_tensor(g, i, buf.data(), nb) == MQ_OK);
      CHECK(mq_gguf_read_tensor(g, i, buf.data(), nb + 1) == MQ_E_INVALID);
    }
    mq_qtensor *qt = nullptr;
    CHECK(mq_gguf_load_tensor(nullptr, g, i, &qt) != MQ_OK);  // no device here
  }
  // the batched load builds every job, then reaches the (device-less) upload
  std::vector<int64_t> idx;
  for (int64_t i = 0; i < nt; ++i) idx.push_back(nt - 1 - i);
  std::vector<mq_qtensor *> outs(idx.size() + 2, reinterpret_cast<mq_qtensor *>(&idx));
  int fake = 0;
  mq_ctx *ctx = reinterpret_cast<mq_ctx *>(&fake);
  CHECK(mq_gguf_load_tensors(ctx, g, idx.data(), nt, outs.data()) == (nt ? MQ_E_UNSUPPORTED : MQ_OK));
  for (int64_t i = 0; i < nt; ++i) CHECK(outs[(size_t)i] == nullptr);
  const int64_t bad[2] = {0, nt};
  CHECK(mq_gguf_load_tensors(ctx, g, bad, 2, outs.data()) == MQ_E_INVALID);
  CHECK(mq_gguf_load_tensors(ctx, g, nullptr, 1, outs.data()) == MQ_E_INVALID);
  CHECK(mq_gguf_load_tensors(nullptr, g, idx.data(), nt, outs.data()) == MQ_E_INVALID);
  for (auto &o : outs) o = reinterpret_cast<mq_qtensor *>(&idx);
  CHECK(mq_gguf_load_tensors(ctx, nullptr, idx.data(), nt, outs.data()) == MQ_E_INVALID);
  for (int64_t i = 0; i < nt; ++i) CHECK(outs[(size_t)i] == nullptr);  // cleared on every failure
  CHECK(mq_gguf_tensor_info(g, nt, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) == MQ_E_INVALID);
  CHECK(mq_gguf_kv_info(g, nkv, nullptr, nullptr, nullptr, nullptr) == MQ_E_INVALID);
}

// Opens `bytes` as a file; returns the status.  A file that opens is walked.
int open_bytes(const std::string &p, const std::vector<uint8_t> &bytes) {
  dump(p, bytes.data(), bytes.size());
  mq_gguf *g = nullptr;
  const int rc = mq_gguf_open(p.c_str(), &g);
  if (rc == MQ_OK) {
    CHECK(g != nullptr);
    walk(g, false);
    mq_gguf_close(g);
  } else {
    CHECK(g == nullptr);
    CHECK(rc == MQ_E_IO || rc == MQ_E_OOM);
  }
  return rc;
}

// A little-endian GGUF header builder for crafted files.
struct Buf {
  std::vector<uint8_t> b;
  template <typename T>
  Buf &put(T v) {
    const uint8_t *p = reinterpret_cast<const uint8_t *>(&v);
    b.insert(b.end(), p, p + sizeof(T));
    return *this;
  }
  Buf &str(const std::string &s) {
    put<uint64_t>(s.size());
    b.insert(b.end(), s.begin(), s.end());
    return *this;
  }
  Buf &head(uint64_t nt, uint64_t nkv) { return put<uint32_t>(0x46554747u).put<uint32_t>(3).put<uint64_t>(nt).put<uint64_t>(nkv); }
};

std::string write_valid(const std::string &dir) {
  const std::string p = dir + "/valid.gguf";
  mq_gguf_writer *w = nullptr;
  CHECK(mq_gguf_writer_create(p.c_str(), 64, &w) == MQ_OK);
  const uint8_t u8 = 200;
  const int32_t i32 = -7;
  const float f32 = 1.5f;
  const double f64 = -0.125;
  const int64_t i64 = -(int64_t(1) << 40);
  CHECK(mq_gguf_writer_kv_str(w, "general.architecture", "flux") == MQ_OK);
  CHECK(mq_gguf_writer_kv_scalar(w, "u8", 0, &u8) == MQ_OK);
  CHECK(mq_gguf_writer_kv_scalar(w, "i32", 5, &i32) == MQ_OK);
  CHECK(mq_gguf_writer_kv_scalar(w, "f32", 6, &f32) == MQ_OK);
  CHECK(mq_gguf_writer_kv_scalar(w, "f64", 12, &f64) == MQ_OK);
  CHECK(mq_gguf_writer_kv_scalar(w, "i64", 11, &i64) == MQ_OK);
  CHECK(mq_gguf_writer_kv_scalar(w, "u8", 0, &u8) == MQ_E_INVALID);  // duplicate key
  const int16_t arr[3] = {1, -2, 3};
  CHECK(mq_gguf_writer_kv_array(w, "arr.i16", 3, arr, 3) == MQ_OK);
  const char *strs[3] = {"a", "", "ccc"};
  CHECK(mq_gguf_writer_kv_str_array(w, "arr.str", strs, 3) == MQ_OK);
  CHECK(mq_gguf_writer_kv_array(w, "arr.empty", 4, nullptr, 0) == MQ_OK);
  std::vector<uint8_t> q4k(2 * 144);
  for (size_t i = 0; i < q4k.size(); ++i) q4k[i] = (uint8_t)(i * 37 + 11);
  const int64_t dq[2] = {256, 2};
  CHECK(mq_gguf_writer_add_tensor(w, "blk.0.weight", MQ_Q4_K, 2, dq, q4k.data(), q4k.size()) == MQ_OK);
  CHECK(mq_gguf_writer_add_tensor(w, "blk.0.weight", MQ_Q4_K, 2, dq, q4k.data(), q4k.size()) == MQ_E_INVALID);
  CHECK(mq_gguf_writer_add_tensor(w, "bad", MQ_Q4_K, 2, dq, q4k.data(), q4k.size() - 1) == MQ_E_INVALID);
  const float norm[7] = {0, 1, 2, 3, 4, 5, 6};
  const int64_t dn[1] = {7};
  CHECK(mq_gguf_writer_add_tensor(w, "norm.scale", MQ_F32, 1, dn, norm, sizeof(norm)) == MQ_OK);
  const uint16_t half[12] = {0x3c00, 0x4000, 0xbc00, 0, 1, 2, 3, 4, 5, 6, 7, 8};
  const int64_t dh[3] = {4, 1, 3};
  CHECK(mq_gguf_writer_add_tensor(w, "half", MQ_F16, 3, dh, half, sizeof(half)) == MQ_OK);
  CHECK(mq_gguf_writer_finish(w) == MQ_OK);
  CHECK(mq_gguf_writer_finish(w) == MQ_E_INVALID);
  mq_gguf_writer_free(w);

  mq_gguf *g = nullptr;
  CHECK(mq_gguf_open(p.c_str(), &g) == MQ_OK);
  if (g) {
    CHECK(mq_gguf_version(g) == 3);
    CHECK(mq_gguf_tensor_count(g) == 3);
    const int64_t ia = mq_gguf_find_kv(g, "arr.str");
    const char *s = nullptr;
    uint64_t len = 0;
    CHECK(ia >= 0 && mq_gguf_kv_str(g, ia, 2, &s, &len) == MQ_OK && len == 3 && memcmp(s, "ccc", 3) == 0);
    int64_t iv = 0;
    CHECK(mq_gguf_kv_int(g, mq_gguf_find_kv(g, "arr.i16"), 1, &iv) == MQ_OK && iv == -2);
    double fv = 0;
    CHECK(mq_gguf_kv_float(g, mq_gguf_find_kv(g, "f32"), 0, &fv) == MQ_OK && fv == 1.5);
    const int64_t it = mq_gguf_find(g, "blk.0.weight");
    std::vector<uint8_t> back(q4k.size());
    CHECK(it >= 0 && mq_gguf_read_tensor(g, it, back.data(), back.size()) == MQ_OK && back == q4k);
    walk(g, true);
    mq_gguf_close(g);
  }
  return p;
}

void crafted(const std::string &dir) {
  const std::string p = dir + "/crafted.gguf";
  struct Case {
    const char *what;
    Buf b;
  };
  std::vector<Case> cases;
  // metadata arrays whose counts claim far more than the file holds
  cases.push_back({"u8 array of 2^29", Buf().head(0, 1)});
  cases.back().b.str("a").put<uint32_t>(9).put<uint32_t>(0).put<uint64_t>(uint64_t(1) << 29);
  cases.push_back({"f64 array of 2^27", Buf().head(0, 1)});
  cases.back().b.str("a").put<uint32_t>(9).put<uint32_t>(12).put<uint64_t>(uint64_t(1) << 27);
  cases.push_back({"string array of 2^26", Buf().head(0, 1)});
  cases.back().b.str("a").put<uint32_t>(9).put<uint32_t>(8).put<uint64_t>(uint64_t(1) << 26);
  cases.push_back({"string array of 2^63", Buf().head(0, 1)});
  cases.back().b.str("a").put<uint32_t>(9).put<uint32_t>(8).put<uint64_t>(uint64_t(1) << 63);
  cases.push_back({"string of 2^30 bytes", Buf().head(0, 1)});
  cases.back().b.put<uint64_t>(uint64_t(1) << 30).put<uint32_t>(0x41414141);
  cases.push_back({"string of 2^64-1 bytes", Buf().head(0, 1)});
  cases.back().b.put<uint64_t>(~uint64_t(0));
  cases.push_back({"array of arrays of 2^40", Buf().head(0, 1)});
  cases.back().b.str("a").put<uint32_t>(9).put<uint32_t>(9).put<uint64_t>(uint64_t(1) << 40);
  {
    Buf b = Buf().head(0, 1);
    b.str("deep").put<uint32_t>(9);
    for (int i = 0; i < 200; ++i) b.put<uint32_t>(9).put<uint64_t>(1);
    b.put<uint32_t>(0).put<uint64_t>(1).put<uint8_t>(1);
    cases.push_back({"arrays nested 200 deep", b});
  }
  cases.push_back({"unknown value type", Buf().head(0, 1)});
  cases.back().b.str("a").put<uint32_t>(77).put<uint64_t>(0);
  cases.push_back({"alignment not a power of two", Buf().head(0, 1)});
  cases.back().b.str("general.alignment").put<uint32_t>(4).put<uint32_t>(48);
  cases.push_back({"alignment as a string", Buf().head(0, 1)});
  cases.back().b.str("general.alignment").put<uint32_t>(8).str("32");
  cases.push_back({"2^24+1 tensors", Buf().head((uint64_t(1) << 24) + 1, 0)});
  cases.push_back({"five dims", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(5);
  cases.push_back({"zero dim", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(1).put<uint64_t>(0).put<uint32_t>(0).put<uint64_t>(0);
  cases.push_back({"element count overflow", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(4).put<uint64_t>(uint64_t(1) << 39).put<uint64_t>(uint64_t(1) << 39)
      .put<uint64_t>(uint64_t(1) << 39).put<uint64_t>(uint64_t(1) << 39).put<uint32_t>(0).put<uint64_t>(0);
  cases.push_back({"ne0 not a block multiple", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(1).put<uint64_t>(100).put<uint32_t>(MQ_Q4_K).put<uint64_t>(0);
  cases.push_back({"unknown tensor type", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(1).put<uint64_t>(32).put<uint32_t>(99).put<uint64_t>(0);
  cases.push_back({"misaligned offset", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(1).put<uint64_t>(4).put<uint32_t>(MQ_F32).put<uint64_t>(3);
  cases.push_back({"data past end", Buf().head(1, 0)});
  cases.back().b.str("t").put<uint32_t>(1).put<uint64_t>(1 << 20).put<uint32_t>(MQ_F32).put<uint64_t>(0);
  cases.push_back({"version 1", Buf()});
  cases.back().b.put<uint32_t>(0x46554747u).put<uint32_t>(1).put<uint64_t>(0).put<uint64_t>(0);
  cases.push_back({"bad magic", Buf()});
  cases.back().b.put<uint32_t>(0x46554748u).put<uint32_t>(3).put<uint64_t>(0).put<uint64_t>(0);
  cases.push_back({"empty file", Buf()});
  for (auto &c : cases) {
    const int rc = open_bytes(p, c.b.b);
    if (rc == MQ_OK) {
      fprintf(stderr, "crafted case opened: %s\n", c.what);
      ++g_failures;
    }
  }
}

}  // namespace

int main(int argc, char **argv) {
  if (argc > 1 && strcmp(argv[1], "table") == 0) {
    const int ids[] = {MQ_F32, MQ_F16, MQ_Q4_0, MQ_Q4_1, MQ_Q5_0, MQ_Q5_1, MQ_Q8_0, MQ_Q2_K,
                       MQ_Q3_K, MQ_Q4_K, MQ_Q5_K, MQ_Q6_K, MQ_BF16, 4, 9, 15, 99};
    for (int id : ids) printf("%d %d %d\n", id, mq_block_size(id), mq_type_size(id));
    return 0;
  }
  char tmpl[] = "/tmp/mq_gguf_san_XXXXXX";
  const char *dir = mkdtemp(tmpl);
  if (!dir) {
    perror("mkdtemp");
    return 2;
  }
  const std::string d = dir;
  const std::string valid = write_valid(d);
  const std::vector<uint8_t> good = slurp(valid);
  CHECK(good.size() > 64);

  // every truncation of the valid file
  const std::string tp = d + "/trunc.gguf";
  int opened = 0;
  for (size_t len = 0; len < good.size(); ++len) {
    std::vector<uint8_t> t(good.begin(), good.begin() + (long)len);
    if (open_bytes(tp, t) == MQ_OK) ++opened;
  }
  crafted(d);

  // seeded random mutations of the header region
  uint64_t s = 0x9E3779B97F4A7C15ull;
  auto rnd = [&]() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  };
  const std::string mp = d + "/mut.gguf";
  size_t hdr = good.size() < 512 ? good.size() : 512;
  int mut_opened = 0;
  for (int it = 0; it < 3000; ++it) {
    std::vector<uint8_t> m = good;
    const int flips = 1 + (int)(rnd() % 8);
    for (int f = 0; f < flips; ++f) {
      const size_t at = 4 + (size_t)(rnd() % (hdr - 4));
      switch (rnd() % 4) {
        case 0: m[at] ^= (uint8_t)(1u << (rnd() % 8)); break;
        case 1: m[at] = (uint8_t)rnd(); break;
        case 2: m[at] = 0xFF; break;
        default: m[at] = 0x00; break;
      }
    }
    if (rnd() % 8 == 0) m.resize((size_t)(rnd() % m.size()));
    if (open_bytes(mp, m) == MQ_OK) ++mut_opened;
  }
  unlink(valid.c_str());
  unlink(tp.c_str());
  unlink(mp.c_str());
  unlink((d + "/crafted.gguf").c_str());
  rmdir(dir);
  printf("gguf_driver: %zu truncations (%d opened: trailing padding only), 3000 mutations (%d opened)\n",
         good.size(), opened, mut_opened);
  if (g_failures) {
    printf("gguf_driver: %d failures\n", g_failures);
    return 1;
  }
  printf("gguf_driver: ok\n");
  return 0;
}
