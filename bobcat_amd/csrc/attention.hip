// Causal grouped-query attention over the KV cache, split over keys.
//
// Counterpart of Metal::attention (crates/bobcat-metal/src/backend.rs:
// 2150-2320) and its kernels attention_chunk / attention_wide /
// attention_combine (attention.metal:25-265, 489-531); the math is the CPU
// attention of lfm2.rs:520-556: softmax(q·k/√d)·v over positions 0..pos.
//
// One workgroup of 256 handles (KV head, split, query): the ≤4 query heads
// that share the KV head, over a contiguous range of keys.  Keys stream in
// tiles of 256, one key per thread for the scores (each thread reads its
// key's row with 16-byte loads and reuses it for every head of the group),
// then one output element per thread for P·V, with an online softmax
// across tiles.  Splits write (max, sum, unnormalised output) partials;
// the last split to finish for a (query, KV head) — found with an atomic
// counter that it resets to zero — combines them, so the whole attention
// is one launch and replays safely inside a HIP graph.
#include <cmath>

#include "device.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr uint32_t kAttnThreads = 256;
constexpr uint32_t kAttnTile = 256;
constexpr uint32_t kMaxGroup = 4;     // ATTENTION_MAX_GROUP (backend.rs:103)
constexpr uint32_t kMaxHeadDim = 256; // ATTENTION_MAX_HEAD_DIM (backend.rs:106)
constexpr uint32_t kChunk = 64;       // ATTENTION_CHUNK (backend.rs:84): splits <= ceil(n_ctx / 64)
constexpr uint32_t kQueryBatch = 64;  // ATTENTION_QUERY_BATCH (backend.rs:93)

template <bool HALF>
__device__ __forceinline__ void load8(const void *base, uint64_t idx, float *v) {
  if (HALF) {
    const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const __half *>(base) + idx);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = half_bits_to_float(ws[i] & 0xffffu);
      v[2 * i + 1] = half_bits_to_float(ws[i] >> 16);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx);
    const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(base) + idx + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <bool HALF>
__device__ __forceinline__ float load1(const void *base, uint64_t idx) {
  if (HALF) return __half2float(static_cast<const __half *>(base)[idx]);
  return static_cast<const float *>(base)[idx];
}

template <bool HALF>
__global__ __launch_bounds__(kAttnThreads) void k_attention(
    const float *__restrict__ q, const void *__restrict__ kc, const void *__restrict__ vc,
    float *__restrict__ partials, uint32_t *__restrict__ counters, float *__restrict__ out, uint32_t n_heads,
    uint32_t n_kv, uint32_t hd, uint32_t first_pos, const uint32_t *dpos, uint32_t splits, float scale) {
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, qi = blockIdx.z, tid = threadIdx.x;
  const uint32_t group = n_heads / n_kv;
  const uint32_t kv_dim = n_kv * hd;
  const uint32_t pos = first_pos + (dpos ? *dpos : 0u) + qi;
  const uint32_t n_keys = pos + 1;
  const uint32_t chunk = (n_keys + splits - 1) / splits;
  const uint32_t k0 = min(split * chunk, n_keys), k1 = min(k0 + chunk, n_keys);

  __shared__ float q_s[kMaxGroup * kMaxHeadDim];
  __shared__ float p_s[kMaxGroup][kAttnTile];
  __shared__ float m_s[kMaxGroup], l_s[kMaxGroup], alpha_s[kMaxGroup];
  __shared__ uint32_t last_s;

  const float *qbase = q + ((uint64_t)qi * n_heads + (uint64_t)kvh * group) * hd;
  for (uint32_t i = tid; i < group * hd; i += kAttnThreads) q_s[i] = qbase[i];
  if (tid < kMaxGroup) {
    m_s[tid] = -INFINITY;
    l_s[tid] = 0.f;
  }
  constexpr int kOut = kMaxGroup * kMaxHeadDim / kAttnThreads;  // outputs per thread
  float acc[kOut];
#pragma unroll
  for (int j = 0; j < kOut; j++) acc[j] = 0.f;
  __syncthreads();

  for (uint32_t t0 = k0; t0 < k1; t0 += kAttnTile) {
    const uint32_t len = min(kAttnTile, k1 - t0);
    // Scores: one key per thread.
    {
      float sc[kMaxGroup] = {0.f, 0.f, 0.f, 0.f};
      const uint32_t key = t0 + tid;
      if (tid < len) {
        const uint64_t row = (uint64_t)key * kv_dim + (uint64_t)kvh * hd;
        for (uint32_t d = 0; d < hd; d += 8) {
          float kv8[8];
          load8<HALF>(kc, row + d, kv8);
#pragma unroll
          for (uint32_t g = 0; g < kMaxGroup; g++) {
            if (g < group) {
              const float *qq = q_s + g * hd + d;
#pragma unroll
              for (int i = 0; i < 8; i++) sc[g] = fmaf(qq[i], kv8[i], sc[g]);
            }
          }
        }
      }
#pragma unroll
      for (uint32_t g = 0; g < kMaxGroup; g++)
        if (g < group) p_s[g][tid] = tid < len ? sc[g] * scale : -INFINITY;
    }
    __syncthreads();
    // Online softmax: wave g owns head g.
    {
      const uint32_t wave = tid / 64, lane = tid % 64;
      if (wave < group) {
        float mx = -INFINITY;
        for (uint32_t j = lane; j < kAttnTile; j += 64) mx = fmaxf(mx, p_s[wave][j]);
        mx = wave_max(mx);
        const float m_old = m_s[wave];
        const float m_new = fmaxf(m_old, mx);
        float sum = 0.f;
        for (uint32_t j = lane; j < kAttnTile; j += 64) {
          const float e = expf(p_s[wave][j] - m_new);
          p_s[wave][j] = e;
          sum += e;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
          const float alpha = expf(m_old - m_new);  // 0 on the first tile (m_old = -inf)
          alpha_s[wave] = alpha;
          l_s[wave] = l_s[wave] * alpha + sum;
          m_s[wave] = m_new;
        }
      }
    }
    __syncthreads();
    // P·V: output element o = g*hd + d per thread (kOut of them).
#pragma unroll
    for (int j = 0; j < kOut; j++) {
      const uint32_t o = tid + j * kAttnThreads;
      if (o < group * hd) {
        const uint32_t g = o / hd, d = o % hd;
        float a = acc[j] * alpha_s[g];
        const uint64_t base = (uint64_t)t0 * kv_dim + (uint64_t)kvh * hd + d;
        // Eight independent value loads in flight per step.
        uint32_t t = 0;
        for (; t + 8 <= len; t += 8) {
          float vv[8];
#pragma unroll
          for (int i = 0; i < 8; i++) vv[i] = load1<HALF>(vc, base + (uint64_t)(t + i) * kv_dim);
#pragma unroll
          for (int i = 0; i < 8; i++) a = fmaf(p_s[g][t + i], vv[i], a);
        }
        for (; t < len; t++) a = fmaf(p_s[g][t], load1<HALF>(vc, base + (uint64_t)t * kv_dim), a);
        acc[j] = a;
      }
    }
    __syncthreads();
  }

  const uint32_t stride = hd + 2;
  if (splits == 1) {
#pragma unroll
    for (int j = 0; j < kOut; j++) {
      const uint32_t o = tid + j * kAttnThreads;
      if (o < group * hd) {
        const uint32_t g = o / hd, d = o % hd;
        out[((uint64_t)qi * n_heads + kvh * group + g) * hd + d] = acc[j] / l_s[g];
      }
    }
    return;
  }
  // Partial of (query, head, split): [m, l, acc[hd]].
#pragma unroll
  for (int j = 0; j < kOut; j++) {
    const uint32_t o = tid + j * kAttnThreads;
    if (o < group * hd) {
      const uint32_t g = o / hd, d = o % hd;
      const uint32_t h = kvh * group + g;
      float *pp = partials + (((uint64_t)qi * n_heads + h) * splits + split) * stride;
      pp[2 + d] = acc[j];
      if (d == 0) {
        pp[0] = m_s[g];
        pp[1] = l_s[g];
      }
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&counters[qi * n_kv + kvh], 1u);
    last_s = prev == splits - 1;
  }
  __syncthreads();
  if (!last_s) return;
  __threadfence();
  // Combine the splits of the group's heads: rescale to the global max.
  for (uint32_t o = tid; o < group * hd; o += kAttnThreads) {
    const uint32_t g = o / hd, d = o % hd;
    const uint32_t h = kvh * group + g;
    const float *pp = partials + ((uint64_t)qi * n_heads + h) * splits * stride;
    float M = -INFINITY;
    for (uint32_t sp = 0; sp < splits; sp++) M = fmaxf(M, pp[sp * stride]);
    float L = 0.f, O = 0.f;
    for (uint32_t sp = 0; sp < splits; sp++) {
      const float m = pp[sp * stride];
      if (m == -INFINITY) continue;
      const float w = expf(m - M);
      L = fmaf(pp[sp * stride + 1], w, L);
      O = fmaf(pp[sp * stride + 2 + d], w, O);
    }
    out[((uint64_t)qi * n_heads + h) * hd + d] = O / L;
  }
  if (tid == 0) counters[qi * n_kv + kvh] = 0;
}

uint32_t attention_splits(uint32_t n_keys_max, uint32_t n_kv_heads, uint32_t n_cus) {
  const uint32_t max_splits = (n_keys_max + kChunk - 1) / kChunk;
  const uint32_t want = (2 * (n_cus ? n_cus : 256) + n_kv_heads - 1) / n_kv_heads;
  uint32_t s = std::min(max_splits, want);
  return s ? s : 1;
}

uint64_t attention_partial_floats(uint32_t n_queries, uint32_t n_heads, uint32_t head_dim, uint32_t splits) {
  return (uint64_t)n_queries * n_heads * splits * (head_dim + 4);  // decode partials: 4 + head_dim floats
}

void run_attention(hipStream_t s, const float *q, const void *k_cache, const void *v_cache, bool kv_half,
                   float *partials, uint32_t *counters, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                   uint32_t head_dim, uint32_t first_pos, const uint32_t *dpos, uint32_t n_queries, uint32_t splits) {
  const float scale = 1.0f / sqrtf((float)head_dim);
  dim3 grid(n_kv_heads, splits, n_queries);
  if (kv_half)
    k_attention<true><<<grid, kAttnThreads, 0, s>>>(q, k_cache, v_cache, partials, counters, out, n_heads, n_kv_heads,
                                                    head_dim, first_pos, dpos, splits, scale);
  else
    k_attention<false><<<grid, kAttnThreads, 0, s>>>(q, k_cache, v_cache, partials, counters, out, n_heads,
                                                     n_kv_heads, head_dim, first_pos, dpos, splits, scale);
}

}  // namespace bch

using namespace bch;

extern "C" {

uint64_t bch_attention_scratch_floats(uint32_t n_heads, uint32_t head_dim, uint32_t n_ctx, uint32_t n_queries) {
  return (uint64_t)std::min(n_queries, kQueryBatch) * n_heads * ((n_ctx + kChunk - 1) / kChunk) * (head_dim + 2);
}

int bch_attention(bch_ctx *ctx, bch_view q, bch_view k_cache, bch_view v_cache, int kv_half, bch_view scratch,
                  bch_view out, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t first_pos,
                  uint32_t n_queries, uint32_t n_ctx) {
  const uint64_t last_pos = (uint64_t)first_pos + n_queries;
  if (n_kv_heads == 0 || n_heads % n_kv_heads || n_heads / n_kv_heads > kMaxGroup || head_dim == 0 ||
      head_dim % 32 || head_dim > kMaxHeadDim || last_pos > n_ctx)
    return fail(BCH_ERR_ATTENTION_LIMITS,
                "the attention kernels need KV heads that divide the query heads into groups of up to %u, heads of a "
                "multiple of 32 floats up to %u, and positions inside the context, got %u and %u heads of %u floats "
                "at positions up to %llu of %u",
                kMaxGroup, kMaxHeadDim, n_heads, n_kv_heads, head_dim, (unsigned long long)last_pos, n_ctx);
  const uint64_t elem = kv_half ? 2 : 4;
  const uint64_t query_bytes = (uint64_t)n_queries * n_heads * head_dim * 4;
  const uint64_t cache_bytes = last_pos * n_kv_heads * head_dim * elem;
  const uint64_t scratch_floats = bch_attention_scratch_floats(n_heads, head_dim, n_ctx, n_queries);
  const float *qp;
  const void *kp, *vp;
  float *sp, *op;
  BCH_TRY(view_ptr(ctx, "attention", q, query_bytes, &qp));
  BCH_TRY(view_ptr(ctx, "attention", k_cache, cache_bytes, &kp));
  BCH_TRY(view_ptr(ctx, "attention", v_cache, cache_bytes, &vp));
  BCH_TRY(view_ptr(ctx, "attention", scratch, scratch_floats * 4, &sp));
  BCH_TRY(view_ptr(ctx, "attention", out, query_bytes, &op));
  if (reinterpret_cast<uintptr_t>(kp) % 16 || reinterpret_cast<uintptr_t>(vp) % 16)
    return fail(BCH_ERR_ARGUMENT, "attention: the caches must be 16-byte aligned");
  if (!ctx->counters) {
    if (hipMalloc(&ctx->counters, kQueryBatch * 256 * 4) != hipSuccess)
      return fail(BCH_ERR_ALLOCATION, "attention: cannot allocate split counters");
    hipMemset(ctx->counters, 0, kQueryBatch * 256 * 4);
  }
  if (n_kv_heads > 256) return fail(BCH_ERR_ATTENTION_LIMITS, "attention: at most 256 KV heads");
  return launch(ctx, {"attention", 0, 0, 0}, [&](hipStream_t s) {
    // Query batches of 64 share the scratch, as the reference's do.
    for (uint32_t q0 = 0; q0 < n_queries; q0 += kQueryBatch) {
      const uint32_t nq = std::min(kQueryBatch, n_queries - q0);
      const uint32_t splits = attention_splits(first_pos + q0 + nq, n_kv_heads, ctx->n_cus);
      const uint64_t off = (uint64_t)q0 * n_heads * head_dim;
      run_attention(s, qp + off, kp, vp, kv_half != 0, sp, ctx->counters, op + off, n_heads, n_kv_heads, head_dim,
                    first_pos + q0, nullptr, nq, splits);
    }
  });
}

}  // extern "C"
