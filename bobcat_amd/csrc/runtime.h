// Host-side runtime shared by the op launchers: contexts, buffers, view
// checks, error reporting and the launch wrapper that implements recording
// and per-kernel profiling.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "../../include/bobcat_hip.h"

struct bch_buffer {
  bch_ctx *owner;
  void *ptr;
  uint64_t len;
};

struct bch_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool recording = false;
  // Tickets: commit k records events[k-1-first_event]; wait drains them.
  uint64_t committed = 0;
  uint64_t waited = 0;
  hipEvent_t begin_event = nullptr;  // recorded at bch_begin
  struct Pending {
    uint64_t ticket;
    hipEvent_t begin;
    hipEvent_t end;
  };
  std::vector<Pending> pending;
  bool profiling = false;
  std::vector<bch_profile_entry> profile;
  uint32_t n_cus = 0;
  // Set while a driver captures a graph: launches go to the capture stream
  // and skip profiling and synchronisation.
  bool capturing = false;
  // Zeroed split counters of the op-level attention launcher.
  uint32_t *counters = nullptr;
  // Scratch of the op-level launchers (ctx_scratch), grown on demand.
  void *scratch = nullptr;
  uint64_t scratch_bytes = 0;
};

namespace bch {

// Record `code` with a formatted message as this thread's last error and
// return it.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// At least `bytes` of the context's scratch memory; growing it waits for the
// work in flight (the old region may still be in use).
int ctx_scratch(bch_ctx *ctx, uint64_t bytes, void **out);
// Finds bch_matmul_noalloc's static scratch on `device` (current); bch_open calls it.
int matmul_noalloc_setup(int device);
int ok();

// Check `view` for `bytes` bytes on behalf of `kernel`; on success store the
// device address of its first byte.
int check_view(bch_ctx *ctx, const char *kernel, bch_view view, uint64_t bytes, void **ptr);

template <class T>
int view_ptr(bch_ctx *ctx, const char *kernel, bch_view view, uint64_t bytes, T **ptr) {
  void *p = nullptr;
  int rc = check_view(ctx, kernel, view, bytes, &p);
  *ptr = static_cast<T *>(p);
  return rc;
}

// Describes one launch for profiling (backend.rs:376-391).
struct LaunchInfo {
  const char *name;
  uint32_t n_rows;
  uint32_t n_cols;
  uint64_t weight_bytes;
};

void add_profile(bch_ctx *ctx, const LaunchInfo &info, double seconds);

// Record the launches `fn(stream)` performs.  Requires an open recording
// (Error::NotRecording otherwise).  While profiling, the launches run on
// their own and are timed with events.
template <class F>
int launch(bch_ctx *ctx, const LaunchInfo &info, F &&fn) {
  if (!ctx->recording && !ctx->capturing) return fail(BCH_ERR_NOT_RECORDING, "no recording is open");
  if (ctx->profiling && !ctx->capturing) {
    hipEvent_t a, b;
    hipEventCreate(&a);
    hipEventCreate(&b);
    hipEventRecord(a, ctx->stream);
    fn(ctx->stream);
    hipEventRecord(b, ctx->stream);
    hipError_t e = hipEventSynchronize(b);
    float ms = 0.f;
    hipEventElapsedTime(&ms, a, b);
    hipEventDestroy(a);
    hipEventDestroy(b);
    if (e != hipSuccess) return fail(BCH_ERR_EXECUTION, "%s: %s", info.name, hipGetErrorString(e));
    add_profile(ctx, info, ms * 1e-3);
  } else {
    fn(ctx->stream);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(BCH_ERR_EXECUTION, "%s launch: %s", info.name, hipGetErrorString(e));
  return BCH_OK;
}

inline uint32_t div_ceil(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Element count of a block of `format` and its bytes; false if unknown.
bool block_shape(uint32_t format, uint32_t *elements, uint32_t *bytes);
uint64_t matrix_bytes(uint32_t format, uint32_t n_rows, uint32_t n_cols);

}  // namespace bch

#define BCH_TRY(expr)          \
  do {                         \
    int _rc = (expr);          \
    if (_rc != BCH_OK) return _rc; \
  } while (0)
