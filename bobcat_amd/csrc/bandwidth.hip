// The read-bandwidth probe: the counterpart of read_sum and
// measure_bandwidth (crates/bobcat-metal/src/bandwidth.rs:20-34, 60+).  It
// gives the HBM rate a plain streaming read reaches on this device, the
// practical ceiling for the matrix-vector kernels.
#include "runtime.h"

namespace bch {

// Each thread sums float4 values at a stride of the grid, so neighbouring
// lanes read neighbouring 16-byte words.
__global__ void k_read_sum(const float4 *__restrict__ src, float *__restrict__ out, uint64_t n) {
  const uint64_t grid = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint64_t i = gid; i < n; i += grid) {
    const float4 v = src[i];
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  out[gid] = acc.x + acc.y + acc.z + acc.w;
}

}  // namespace bch

using namespace bch;

extern "C" int bch_read_sum(bch_ctx *ctx, bch_view src, uint64_t n_vectors, bch_view out, uint32_t n_threads) {
  if (n_threads == 0 || n_threads % 256)
    return fail(BCH_ERR_ARGUMENT, "read_sum needs a positive multiple of 256 threads, got %u", n_threads);
  const float4 *s;
  float *o;
  BCH_TRY(view_ptr(ctx, "read_sum", src, n_vectors * 16, &s));
  BCH_TRY(view_ptr(ctx, "read_sum", out, (uint64_t)n_threads * 4, &o));
  return launch(ctx, {"read_sum", 0, 0, n_vectors * 16},
                [&](hipStream_t st) { k_read_sum<<<n_threads / 256, 256, 0, st>>>(s, o, n_vectors); });
}
