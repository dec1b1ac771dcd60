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

// Host -> HBM weight upload (GGUF file or host buffer): kUploadThreads host
// threads take the tensor's chunks of kUploadChunk bytes in turn, each through
// its own two pinned buffers and its own copy stream.
#ifndef MQ_UPLOAD_THREADS
#define MQ_UPLOAD_THREADS 8
#endif
#ifndef MQ_UPLOAD_CHUNK_MIB
#define MQ_UPLOAD_CHUNK_MIB 2
#endif
constexpr int kUploadThreads = MQ_UPLOAD_THREADS;
constexpr size_t kUploadChunk = size_t(MQ_UPLOAD_CHUNK_MIB) << 20;

// Sets the thread's mq_last_error() message and returns `code`.
int set_error(int code, const char *msg);

// One tensor of a GGUF file to upload: `nbytes` of raw blocks (or dense
// values) at byte `offset`, making a device-resident [n, k] tensor of `dtype`.
struct UploadJob {
  int dtype = 0;
  int64_t n = 0, k = 0;
  uint64_t offset = 0;
  size_t nbytes = 0;
};

// Uploads `count` tensors of the open file `fd` (threaded pinned pipeline,
// then the repack; one tensor's repack overlaps the next one's copy).
// Returns finished; on failure every out[i] is NULL.
int upload_from_file(mq_ctx *ctx, int fd, const UploadJob *jobs, int64_t count, mq_qtensor **out);

}  // namespace mq
