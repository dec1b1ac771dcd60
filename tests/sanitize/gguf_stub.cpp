// Host-only stand-ins for the libmoldq symbols that mq_gguf.cpp calls, so the
// GGUF reader/writer links on the CPU without HIP for the sanitizer build.
// Tensor uploads and device read-backs report MQ_E_UNSUPPORTED here; the
// block-size table is checked against the built library's by
// tests/test_sanitizers.py.
#include <string>

#include "../../include/moldq.h"
#include "../../mold_amd/csrc/mq_internal.h"

namespace {
thread_local std::string g_err;
}

namespace mq {
int set_error(int code, const char *msg) {
  g_err = msg;
  return code;
}
int upload_from_file(mq_ctx *, int, const UploadJob *, int64_t count, mq_qtensor **out) {
  for (int64_t i = 0; i < count; ++i) out[i] = nullptr;
  return set_error(MQ_E_UNSUPPORTED, "no device in the sanitizer build");
}
}  // namespace mq

extern "C" {
const char *mq_last_error(void) { return g_err.c_str(); }

int mq_block_size(int dtype) {
  switch (dtype) {
    case MQ_F32: case MQ_F16: case MQ_BF16: return 1;
    case MQ_Q4_0: case MQ_Q4_1: case MQ_Q5_0: case MQ_Q5_1: case MQ_Q8_0: return 32;
    case MQ_Q2_K: case MQ_Q3_K: case MQ_Q4_K: case MQ_Q5_K: case MQ_Q6_K: return 256;
    default: return 0;
  }
}

int mq_type_size(int dtype) {
  switch (dtype) {
    case MQ_F32: return 4;
    case MQ_F16: case MQ_BF16: return 2;
    case MQ_Q4_0: return 18;
    case MQ_Q4_1: return 20;
    case MQ_Q5_0: return 22;
    case MQ_Q5_1: return 24;
    case MQ_Q8_0: return 34;
    case MQ_Q2_K: return 84;
    case MQ_Q3_K: return 110;
    case MQ_Q4_K: return 144;
    case MQ_Q5_K: return 176;
    case MQ_Q6_K: return 210;
    default: return 0;
  }
}

int mq_qtensor_info(const mq_qtensor *, int *, int64_t *, int64_t *, size_t *, size_t *) {
  return mq::set_error(MQ_E_UNSUPPORTED, "no device in the sanitizer build");
}
int mq_qtensor_download(mq_ctx *, const mq_qtensor *, void *, size_t) {
  return mq::set_error(MQ_E_UNSUPPORTED, "no device in the sanitizer build");
}
}
