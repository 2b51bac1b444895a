// Contexts, buffers, recording and profiling: the HIP counterpart of the
// Metal plumbing in crates/bobcat-metal/src/backend.rs:1083-1340 and
// crates/bobcat-metal/src/commands.rs:207-411.  One in-order stream per
// context replaces Metal 4's command buffers, residency sets and argument
// tables; a ticket is an event pair on that stream.
#include <cstdio>
#include <cstring>

#include "runtime.h"

static thread_local std::string g_last_error;

namespace bch {

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() { return BCH_OK; }

bool block_shape(uint32_t format, uint32_t *elements, uint32_t *bytes) {
  switch (format) {
    case BCH_F32: *elements = 1; *bytes = 4; return true;
    case BCH_F16: case BCH_BF16: *elements = 1; *bytes = 2; return true;
    case BCH_Q4_0: *elements = 32; *bytes = 18; return true;
    case BCH_Q8_0: *elements = 32; *bytes = 34; return true;
    case BCH_Q4K: *elements = 256; *bytes = 144; return true;
    case BCH_Q5K: *elements = 256; *bytes = 176; return true;
    case BCH_Q6K: *elements = 256; *bytes = 210; return true;
    default: return false;
  }
}

uint64_t matrix_bytes(uint32_t format, uint32_t n_rows, uint32_t n_cols) {
  return bch_row_bytes(format, n_cols) * n_rows;
}

// check_range (backend.rs:2771-2790): the view must belong to this context
// and hold `bytes` bytes past its offset.
int check_view(bch_ctx *ctx, const char *kernel, bch_view view, uint64_t bytes, void **ptr) {
  if (!view.buffer) return fail(BCH_ERR_ARGUMENT, "%s: null buffer", kernel);
  if (view.buffer->owner != ctx) return fail(BCH_ERR_FOREIGN_BUFFER, "the buffer belongs to another backend");
  const uint64_t len = view.buffer->len;
  if (view.offset > len || bytes > len - view.offset)
    return fail(BCH_ERR_OUT_OF_BOUNDS,
                "the %s launch needs %llu bytes at offset %llu of a %llu-byte buffer", kernel,
                (unsigned long long)bytes, (unsigned long long)view.offset,
                (unsigned long long)len);
  *ptr = static_cast<char *>(view.buffer->ptr) + view.offset;
  return BCH_OK;
}

void add_profile(bch_ctx *ctx, const LaunchInfo &info, double seconds) {
  for (auto &e : ctx->profile) {
    if (strcmp(e.name, info.name) == 0 && e.n_rows == info.n_rows && e.n_cols == info.n_cols) {
      e.calls++;
      e.seconds += seconds;
      e.bytes += info.weight_bytes;
      return;
    }
  }
  bch_profile_entry e{};
  snprintf(e.name, sizeof e.name, "%s", info.name);
  e.n_rows = info.n_rows;
  e.n_cols = info.n_cols;
  e.calls = 1;
  e.seconds = seconds;
  e.bytes = info.weight_bytes;
  ctx->profile.push_back(e);
}

}  // namespace bch

using namespace bch;

extern "C" {

const char *bch_last_error(void) { return g_last_error.c_str(); }

uint64_t bch_row_bytes(uint32_t format, uint32_t n_cols) {
  uint32_t e, b;
  if (!block_shape(format, &e, &b) || n_cols % e) return 0;
  return (uint64_t)(n_cols / e) * b;
}

int bch_open(bch_ctx **out) {
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(BCH_ERR_NO_DEVICE, "no HIP device");
  auto *ctx = new bch_ctx();
  if (hipSetDevice(0) != hipSuccess) {
    delete ctx;
    return fail(BCH_ERR_NO_DEVICE, "cannot select HIP device 0");
  }
  // Default priority, non-blocking with respect to the legacy stream.
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
    delete ctx;
    return fail(BCH_ERR_NO_DEVICE, "cannot create a HIP stream");
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) == hipSuccess) ctx->n_cus = prop.multiProcessorCount;
  // The device address of bch_matmul_noalloc's static scratch on this device.
  if (int rc = matmul_noalloc_setup(ctx->device)) {
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return rc;
  }
  *out = ctx;
  return BCH_OK;
}

void bch_close(bch_ctx *ctx) {
  if (!ctx) return;
  hipStreamSynchronize(ctx->stream);
  for (auto &p : ctx->pending) {
    hipEventDestroy(p.begin);
    hipEventDestroy(p.end);
  }
  if (ctx->begin_event) hipEventDestroy(ctx->begin_event);
  if (ctx->counters) hipFree(ctx->counters);
  if (ctx->scratch) hipFree(ctx->scratch);
  hipStreamDestroy(ctx->stream);
  delete ctx;
}

int bch_device_info(bch_ctx *ctx, char *name, size_t name_len, uint32_t *n_cus) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, ctx->device) != hipSuccess) return fail(BCH_ERR_NO_DEVICE, "no properties");
  if (name && name_len) snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  if (n_cus) *n_cus = prop.multiProcessorCount;
  return BCH_OK;
}

int bch_buffer_new(bch_ctx *ctx, uint64_t len, bch_buffer **out) {
  *out = nullptr;
  void *p = nullptr;
  // A zero-length buffer still gets a distinct allocation.
  if (hipMalloc(&p, len ? len : 256) != hipSuccess)
    return fail(BCH_ERR_ALLOCATION, "cannot allocate a buffer of %llu bytes", (unsigned long long)len);
  if (hipMemsetAsync(p, 0, len ? len : 256, ctx->stream) != hipSuccess ||
      hipStreamSynchronize(ctx->stream) != hipSuccess) {
    hipFree(p);
    return fail(BCH_ERR_ALLOCATION, "cannot clear a buffer of %llu bytes", (unsigned long long)len);
  }
  *out = new bch_buffer{ctx, p, len};
  return BCH_OK;
}

int bch_buffer_from_host(bch_ctx *ctx, const void *data, uint64_t len, bch_buffer **out) {
  BCH_TRY(bch_buffer_new(ctx, len, out));
  if (len && hipMemcpy((*out)->ptr, data, len, hipMemcpyHostToDevice) != hipSuccess) {
    bch_buffer_free(*out);
    *out = nullptr;
    return fail(BCH_ERR_ALLOCATION, "cannot copy %llu bytes to the device", (unsigned long long)len);
  }
  return BCH_OK;
}

void bch_buffer_free(bch_buffer *b) {
  if (!b) return;
  hipFree(b->ptr);
  delete b;
}

uint64_t bch_buffer_len(const bch_buffer *b) { return b ? b->len : 0; }
void *bch_buffer_device_ptr(const bch_buffer *b) { return b ? b->ptr : nullptr; }

static int cpu_access(bch_ctx *ctx, bch_view view, uint64_t bytes, void **ptr) {
  if (ctx->committed > ctx->waited || ctx->recording)
    return fail(BCH_ERR_BUSY, "the CPU cannot access a buffer while work is in flight");
  if (!view.buffer) return fail(BCH_ERR_ARGUMENT, "null buffer");
  if (view.buffer->owner != ctx) return fail(BCH_ERR_FOREIGN_BUFFER, "the buffer belongs to another backend");
  if (view.offset > view.buffer->len || bytes > view.buffer->len - view.offset)
    return fail(BCH_ERR_ACCESS, "CPU access of %llu bytes at offset %llu exceeds a %llu-byte buffer",
                (unsigned long long)bytes, (unsigned long long)view.offset,
                (unsigned long long)view.buffer->len);
  *ptr = static_cast<char *>(view.buffer->ptr) + view.offset;
  return BCH_OK;
}

int bch_write(bch_ctx *ctx, bch_view view, const void *data, uint64_t bytes) {
  void *p;
  BCH_TRY(cpu_access(ctx, view, bytes, &p));
  if (bytes && hipMemcpy(p, data, bytes, hipMemcpyHostToDevice) != hipSuccess)
    return fail(BCH_ERR_EXECUTION, "host-to-device copy failed");
  return BCH_OK;
}

int bch_read(bch_ctx *ctx, bch_view view, void *out, uint64_t bytes) {
  void *p;
  BCH_TRY(cpu_access(ctx, view, bytes, &p));
  if (bytes && hipMemcpy(out, p, bytes, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(BCH_ERR_EXECUTION, "device-to-host copy failed");
  return BCH_OK;
}

int bch_begin(bch_ctx *ctx) {
  if (ctx->recording) return fail(BCH_ERR_ALREADY_RECORDING, "a recording is already open");
  if (!ctx->begin_event) hipEventCreate(&ctx->begin_event);
  hipEventRecord(ctx->begin_event, ctx->stream);
  ctx->recording = true;
  return BCH_OK;
}

// Metal::discard (backend.rs:1249): work already handed to the stream still
// runs; the recording closes without a ticket.
void bch_discard(bch_ctx *ctx) { ctx->recording = false; }

void bch_barrier(bch_ctx *) {}

int bch_commit(bch_ctx *ctx, uint64_t *ticket) {
  if (!ctx->recording) return fail(BCH_ERR_NOT_RECORDING, "no recording is open");
  bch_ctx::Pending p;
  p.ticket = ++ctx->committed;
  hipEventCreate(&p.begin);
  hipEventCreate(&p.end);
  // The event recorded at bch_begin marks this ticket's start; the fresh
  // event takes its place for the next recording.
  std::swap(p.begin, ctx->begin_event);
  hipEventRecord(p.end, ctx->stream);
  ctx->pending.push_back(p);
  ctx->recording = false;
  if (ticket) *ticket = p.ticket;
  return BCH_OK;
}

int bch_wait(bch_ctx *ctx, uint64_t ticket, double *gpu_seconds) {
  double total = 0.0;
  int rc = BCH_OK;
  while (!ctx->pending.empty() && ctx->pending.front().ticket <= ticket) {
    auto p = ctx->pending.front();
    ctx->pending.erase(ctx->pending.begin());
    hipError_t e = hipEventSynchronize(p.end);
    if (e != hipSuccess && rc == BCH_OK)
      rc = fail(BCH_ERR_EXECUTION, "the GPU failed to run the work: %s", hipGetErrorString(e));
    float ms = 0.f;
    if (e == hipSuccess && hipEventElapsedTime(&ms, p.begin, p.end) == hipSuccess) total += ms * 1e-3;
    hipEventDestroy(p.begin);
    hipEventDestroy(p.end);
    if (p.ticket > ctx->waited) ctx->waited = p.ticket;
  }
  if (ticket > ctx->waited && ticket <= ctx->committed) ctx->waited = ticket;
  if (gpu_seconds) *gpu_seconds = total;
  return rc;
}

int bch_end(bch_ctx *ctx, double *gpu_seconds) {
  uint64_t t;
  BCH_TRY(bch_commit(ctx, &t));
  return bch_wait(ctx, t, gpu_seconds);
}

void bch_set_profiling(bch_ctx *ctx, int enabled) {
  ctx->profiling = enabled != 0;
  if (ctx->profiling) ctx->profile.clear();
}

uint32_t bch_profile_count(const bch_ctx *ctx) { return (uint32_t)ctx->profile.size(); }

int bch_profile_get(const bch_ctx *ctx, uint32_t index, bch_profile_entry *out) {
  if (index >= ctx->profile.size()) return fail(BCH_ERR_ARGUMENT, "profile index out of range");
  *out = ctx->profile[index];
  return BCH_OK;
}

}  // extern "C"

int bch::ctx_scratch(bch_ctx *ctx, uint64_t bytes, void **out) {
  if (bytes > ctx->scratch_bytes) {
    if (ctx->scratch) {
      hipStreamSynchronize(ctx->stream);
      hipFree(ctx->scratch);
      ctx->scratch = nullptr;
      ctx->scratch_bytes = 0;
    }
    if (hipMalloc(&ctx->scratch, bytes) != hipSuccess) {
      ctx->scratch = nullptr;
      return fail(BCH_ERR_ALLOCATION, "cannot allocate %llu bytes of scratch", (unsigned long long)bytes);
    }
    ctx->scratch_bytes = bytes;
  }
  *out = ctx->scratch;
  return BCH_OK;
}
