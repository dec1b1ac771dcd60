// mq_internal.h — what the library's translation units share beyond the C ABI
// (plain C++, no HIP headers, so the host-only GGUF reader can include it).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/moldq.h"

// Size of the file-scope device array that mq_qmatmul_noalloc uses as its
// scratch (one copy per GPU, held until the process ends).
#define MQ_NOALLOC_SCRATCH_BYTES (size_t(64) << 20)

namespace mq {

// Pinned host chunk of the file -> HBM weight upload (two are used in turn).
constexpr size_t kUploadChunk = size_t(16) << 20;

// Sets the thread's mq_last_error() message and returns `code`.
int set_error(int code, const char *msg);

// Reads `nbytes` of raw GGUF blocks at `offset` of the open file `fd` and
// makes a device-resident [n, k] tensor of type `dtype` from them (pinned,
// double-buffered asynchronous copy, then the repack).  Returns finished.
int upload_from_file(mq_ctx *ctx, int dtype, int64_t n, int64_t k, int fd, uint64_t offset, size_t nbytes,
                     mq_qtensor **out);

}  // namespace mq
