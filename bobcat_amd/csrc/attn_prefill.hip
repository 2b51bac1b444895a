// Prefill attention on MFMA: causal GQA softmax(q·k/√d)·v for a batch of
// queries against the f16 KV cache (Metal::attention with n_queries > 1 and
// its attention_flash kernel, crates/bobcat-metal/src/backend.rs:2150-2320,
// attention.metal:289-480).
//
// One workgroup per (32 consecutive queries, KV head); wave w owns query
// head kv·G + w of that KV head (G ≤ 4 query heads per KV head), so the four
// waves share each key block's V tile in LDS.  Per block of 32 keys a wave
// computes S^T = K·Q^T (keys × queries) with v_mfma_f32_32x32x16_f16, so each
// lane holds 16 scores of one query: the online softmax needs one cross-lane
// move (lane l and l^32 share a query), and the lane's accumulator registers
// for keys 8j + 4·(l/32) + 0..3 are exactly the B operand of the next
// product, O^T += V^T·P^T on v_mfma_f32_32x32x8_f16.  The queries and the
// probabilities are split into f16 high and low parts (~22 bits) and both
// are multiplied; K and V are the cache's f16 values, so the products are
// exact and accumulate in f32.
#include <algorithm>
#include <cmath>

#include "device.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

typedef _Float16 ph4_t __attribute__((ext_vector_type(4)));
typedef _Float16 ph8_t __attribute__((ext_vector_type(8)));
typedef float pf16_t __attribute__((ext_vector_type(16)));

constexpr int kPrefQ = 32;        // queries per workgroup
constexpr int kPrefKeys = 32;     // keys per block
constexpr int kVtStride = 40;     // halves per V^T row in LDS (32 keys + padding)

// The output gate of gated attention (Qwen3.5, qwen35.rs:422-424): with
// `gate` set, output element d of (query z, head h) is multiplied by
// sigmoid(gate[z·query_stride + h·head_stride + d]).
struct AttnGate {
  const float *gate;
  uint32_t head_stride, query_stride;
  __device__ float at(uint32_t z, uint32_t head, uint32_t d) const {
    return gate ? 1.0f / (1.0f + expf(-gate[(uint64_t)z * query_stride + (uint64_t)head * head_stride + d])) : 1.f;
  }
};

template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill(const float *__restrict__ q, const _Float16 *__restrict__ kc,
                                                      const _Float16 *__restrict__ vc, float *__restrict__ out,
                                                      uint32_t n_heads, uint32_t n_kv, uint32_t first_pos,
                                                      uint32_t n_queries, uint32_t q_stride, uint32_t out_stride,
                                                      float scale, float *__restrict__ partials, AttnGate gate) {
  constexpr int KS = HD / 16;  // k-steps of the score product
  constexpr int OB = HD / 32;  // 32-row blocks of the output
  __shared__ _Float16 vt[HD * kVtStride];  // V^T of the current key block: [d][key]
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const uint32_t kv = blockIdx.y, q0 = blockIdx.x * kPrefQ;
  const uint32_t group = n_heads / n_kv;
  const bool active = (uint32_t)wave < group;
  const uint32_t head = kv * group + (active ? wave : 0);
  const uint32_t col = lane % 32, half_id = lane / 32;
  const uint32_t z = min(q0 + col, n_queries - 1);  // this lane's query (past the end: a copy, never stored)
  const uint32_t qpos = first_pos + q0 + col;
  const uint32_t kend = first_pos + min(q0 + kPrefQ, n_queries);  // keys of the block's last query, exclusive
  const uint64_t row_elems = (uint64_t)n_kv * HD;                 // cache elements per position
  // Key split blockIdx.z of gridDim.z: a contiguous run of whole 32-key
  // blocks of the tile's keys (possibly none, or none visible to a query:
  // that split's partial then has max -inf and sum 0, and weighs nothing in
  // the combine).
  const uint32_t n_blocks = (kend + kPrefKeys - 1) / kPrefKeys, n_split = gridDim.z, split = blockIdx.z;
  const uint32_t kb_lo = split * n_blocks / n_split * kPrefKeys, kb_hi = (split + 1) * n_blocks / n_split * kPrefKeys;

  // The query's k-step fragments as the B operand: Q[z][16·s + 8·half .. +8].
  ph8_t qh[KS], ql[KS];
  {
    const float *qr = q + (uint64_t)z * q_stride + (uint64_t)head * HD + 8 * half_id;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      const float4 a = *reinterpret_cast<const float4 *>(qr + 16 * s);
      const float4 b = *reinterpret_cast<const float4 *>(qr + 16 * s + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; j++) {
        qh[s][j] = (_Float16)v[j];
        ql[s][j] = (_Float16)(v[j] - (float)qh[s][j]);
      }
    }
  }

  pf16_t o[OB];
#pragma unroll
  for (int b = 0; b < OB; b++)
#pragma unroll
    for (int i = 0; i < 16; i++) o[b][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // Key block kb's loads: this thread's VP pieces of V (8 halves each,
  // staged transposed in LDS) and this lane's K fragments, both with
  // clamped rows (the staging zeroes V past kend; scores past it are
  // masked).  Each block's loads are issued one block ahead, before the
  // current block's MFMAs, so that the memory latency overlaps them
  // (loading in the block itself put a full round trip on every block).
  constexpr int VP = kPrefKeys * HD / 8 / 256;
  static_assert(VP >= 1 && kPrefKeys * HD / 8 == 256 * VP, "V pieces per thread");
  auto load_v = [&](uint32_t kb, ph8_t *v8) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < VP; p++) {
      const uint32_t c = tid + 256 * p, key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
      const uint32_t row = min(kb + key, kend - 1);
      v8[p] = *reinterpret_cast<const ph8_t *>(vc + (uint64_t)row * row_elems + (uint64_t)kv * HD + d0);
    }
  };
  auto load_k = [&](uint32_t kb, ph8_t *ka) __attribute__((always_inline)) {
    const uint32_t krow = min(kb + col, kend - 1);
    const _Float16 *kr = kc + (uint64_t)krow * row_elems + (uint64_t)kv * HD + 8 * half_id;
#pragma unroll
    for (int s = 0; s < KS; s++) ka[s] = *reinterpret_cast<const ph8_t *>(kr + 16 * s);
  };

  // (Heads of 256 hold a 32 x 256 f32 output tile per wave in registers:
  // they load each block in the block itself, as a second register set
  // would not fit.)
  constexpr bool kAhead = HD <= 128;
  auto block = [&](uint32_t kb, const ph8_t *ka, const ph8_t *vcur, ph8_t *kn, ph8_t *vn)
                   __attribute__((always_inline)) {
    // Stage V^T of keys kb .. kb+31 (zeros past kend).
    __syncthreads();
#pragma unroll
    for (int p = 0; p < VP; p++) {
      const uint32_t c = tid + 256 * p, key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
      const bool in = kb + key < kend;
#pragma unroll
      for (int j = 0; j < 8; j++) vt[(d0 + j) * kVtStride + key] = in ? vcur[p][j] : (_Float16)0.f;
    }
    __syncthreads();
    // The next block's loads (a clamped re-read past the split's end).
    if constexpr (kAhead) {
      const uint32_t nb = min(kb + kPrefKeys, kb_hi - kPrefKeys);
      load_v(nb, vn);
      load_k(nb, kn);
    }
    if (!active) return;

    // S^T = K·Q^T: lane supplies K[kb + col][16·s + 8·half .. +8].
    pf16_t sc;
#pragma unroll
    for (int i = 0; i < 16; i++) sc[i] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; s++) {
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[s], qh[s], sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[s], ql[s], sc, 0, 0, 0);
    }
    // sc[r] is the score of key kb + 8·(r/4) + 4·half + r%4 for this lane's query.
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t key = kb + 8 * (r / 4) + 4 * half_id + (r % 4);
      sc[r] = (key <= qpos && key < kend) ? sc[r] * scale : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // -inf while no key of this split has been visible to the query (a
    // causal split can start after it): the block then adds exact zeros.
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float corr = expf(m_run - m_use);
    m_run = m_new;
    float psum = 0.f;
    ph4_t ph[4], pl[4];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const float p = expf(sc[r] - m_use);
      psum += p;
      const _Float16 h = (_Float16)p;
      ph[r / 4][r % 4] = h;
      pl[r / 4][r % 4] = (_Float16)(p - (float)h);
    }
    l_run = l_run * corr + psum;
#pragma unroll
    for (int b = 0; b < OB; b++)
#pragma unroll
      for (int i = 0; i < 16; i++) o[b][i] *= corr;
    // O^T += V^T·P^T over 4 k-steps of 8 keys: lane supplies
    // V^T[32b + col][8j + 4·half .. +4] and P^T[8j + 4·half .. +4][col].
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int b = 0; b < OB; b++) {
        const ph4_t a = *reinterpret_cast<const ph4_t *>(vt + (32 * b + col) * kVtStride + 8 * j + 4 * half_id);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x8f16(a, ph[j], o[b], 0, 0, 0);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x8f16(a, pl[j], o[b], 0, 0, 0);
      }
    }
  };
  // Two register sets, alternating block by block.
  const uint32_t kb_end = min(kb_hi, (kend + kPrefKeys - 1) / kPrefKeys * kPrefKeys);
  if constexpr (kAhead) {
    if (kb_lo < kb_end) {
      ph8_t kA[KS], kB[KS], vA[VP], vB[VP];
      load_v(kb_lo, vA);
      load_k(kb_lo, kA);
      for (uint32_t kb = kb_lo; kb < kb_end; kb += 2 * kPrefKeys) {
        block(kb, kA, vA, kB, vB);
        if (kb + kPrefKeys < kb_end) block(kb + kPrefKeys, kB, vB, kA, vA);
      }
    }
  } else {
    for (uint32_t kb = kb_lo; kb < kb_end; kb += kPrefKeys) {
      ph8_t kA[KS], vA[VP];
      load_v(kb, vA);
      if (active) load_k(kb, kA);
      block(kb, kA, vA, nullptr, nullptr);
    }
  }
  if (!active) return;
  const float l_all = l_run + __shfl_xor(l_run, 32, 64);
  if (q0 + col >= n_queries) return;
  float inv = 1.f / l_all;
  float *orow = out + (uint64_t)(q0 + col) * out_stride + (uint64_t)head * HD;
  if (n_split > 1) {
    // Unnormalised partial (max, sum, output) of this split, combined by
    // k_attn_prefill_combine.
    float *pp = partials + (((uint64_t)(q0 + col) * n_heads + head) * n_split + split) * (HD + 2);
    if (half_id == 0) {
      pp[0] = m_run;
      pp[1] = l_all;
    }
    orow = pp + 2;
    inv = 1.f;
  }
#pragma unroll
  for (int b = 0; b < OB; b++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint32_t d = 32 * b + 8 * g + 4 * half_id;
      if (n_split > 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) orow[d + i] = o[b][4 * g + i];
      } else {
        *reinterpret_cast<float4 *>(orow + d) =
            float4{o[b][4 * g] * inv * gate.at(q0 + col, head, d), o[b][4 * g + 1] * inv * gate.at(q0 + col, head, d + 1),
                   o[b][4 * g + 2] * inv * gate.at(q0 + col, head, d + 2),
                   o[b][4 * g + 3] * inv * gate.at(q0 + col, head, d + 3)};
      }
    }
}

// Output of each (query, head) from its key splits' partials: one workgroup
// of HD threads per (query, head).
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_prefill_combine(const float *__restrict__ partials, float *__restrict__ out,
                                                              uint32_t n_heads, uint32_t n_split, uint32_t out_stride,
                                                              AttnGate gate) {
  const uint32_t slot = blockIdx.x, z = slot / n_heads, head = slot % n_heads, d = threadIdx.x;
  const float *pp = partials + (uint64_t)slot * n_split * (HD + 2);
  float M = -INFINITY;
  for (uint32_t sp = 0; sp < n_split; sp++) M = fmaxf(M, pp[sp * (HD + 2)]);
  float L = 0.f, O = 0.f;
  for (uint32_t sp = 0; sp < n_split; sp++) {
    const float w = expf(pp[sp * (HD + 2)] - M);
    L = fmaf(pp[sp * (HD + 2) + 1], w, L);
    O = fmaf(pp[sp * (HD + 2) + 2 + d], w, O);
  }
  out[(uint64_t)z * out_stride + (uint64_t)head * HD + d] = O / L * gate.at(z, head, d);
}

bool attn_prefill_mfma_supported(uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, bool kv_half) {
  return kv_half && n_kv && n_heads % n_kv == 0 && n_heads / n_kv <= 4 &&
         (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

uint64_t attn_prefill_partial_floats(uint32_t n_queries, uint32_t n_heads, uint32_t head_dim, uint32_t splits) {
  return (uint64_t)n_queries * n_heads * splits * (head_dim + 2);
}

uint32_t attn_prefill_splits(uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t first_pos,
                             uint32_t n_queries, uint64_t partial_floats) {
  if (!n_queries) return 1;
  // Enough workgroups for two per CU, at least kMinSplitBlocks 32-key blocks
  // per split of the batch's middle tile, and no more partials than the
  // scratch holds.
  constexpr uint32_t kTargetGroups = 512, kMinSplitBlocks = 2, kMaxSplits = 16;
  const uint32_t tiles = (n_queries + kPrefQ - 1) / kPrefQ;
  uint32_t want = (kTargetGroups + tiles * n_kv - 1) / (tiles * n_kv);
  const uint32_t mid_blocks = (first_pos + (n_queries + 1) / 2 + kPrefKeys - 1) / kPrefKeys;
  want = std::min(want, mid_blocks / kMinSplitBlocks);
  want = std::min<uint32_t>(want, kMaxSplits);
  const uint64_t per_split = (uint64_t)n_queries * n_heads * (head_dim + 2);
  want = (uint32_t)std::min<uint64_t>(want, partial_floats / per_split);
  return std::max<uint32_t>(want, 1);
}

void run_attn_prefill_mfma(hipStream_t s, const float *q, const void *k_cache, const void *v_cache, float *out,
                           uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t first_pos,
                           uint32_t n_queries, uint32_t q_stride, uint32_t out_stride, float scale, float *partials,
                           uint64_t partial_floats, const float *gate, uint32_t gate_head_stride,
                           uint32_t gate_query_stride) {
  if (!n_queries) return;
  const uint32_t n_split =
      partials ? attn_prefill_splits(n_heads, n_kv, head_dim, first_pos, n_queries, partial_floats) : 1;
  const dim3 grid((n_queries + kPrefQ - 1) / kPrefQ, n_kv, n_split);
  const _Float16 *kc = static_cast<const _Float16 *>(k_cache);
  const _Float16 *vc = static_cast<const _Float16 *>(v_cache);
  const AttnGate g{gate, gate_head_stride, gate_query_stride};
  auto go = [&](auto hd) {
    constexpr int HD = decltype(hd)::value;
    k_attn_prefill<HD><<<grid, 256, 0, s>>>(q, kc, vc, out, n_heads, n_kv, first_pos, n_queries, q_stride,
                                            out_stride, scale, partials, g);
    if (n_split > 1)
      k_attn_prefill_combine<HD><<<n_queries * n_heads, HD, 0, s>>>(partials, out, n_heads, n_split, out_stride, g);
  };
  if (head_dim == 64)
    go(std::integral_constant<int, 64>{});
  else if (head_dim == 128)
    go(std::integral_constant<int, 128>{});
  else
    go(std::integral_constant<int, 256>{});
}

}  // namespace bch

using namespace bch;

extern "C" int bch_attention_prefill(bch_ctx *ctx, bch_view q, bch_view k_cache, bch_view v_cache, bch_view out,
                                     uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t first_pos,
                                     uint32_t n_queries, uint32_t n_ctx) {
  const uint64_t last_pos = (uint64_t)first_pos + n_queries;
  if (!attn_prefill_mfma_supported(n_heads, n_kv_heads, head_dim, true) || last_pos > n_ctx)
    return fail(BCH_ERR_ATTENTION_LIMITS,
                "attention_prefill: f16 caches, heads of 64, 128 or 256, at most 4 query heads per KV head and positions "
                "inside the context, got %u and %u heads of %u at positions up to %llu of %u",
                n_heads, n_kv_heads, head_dim, (unsigned long long)last_pos, n_ctx);
  const uint64_t query_bytes = (uint64_t)n_queries * n_heads * head_dim * 4;
  const uint64_t cache_bytes = last_pos * n_kv_heads * head_dim * 2;
  const float *qp;
  const void *kp, *vp;
  float *op;
  BCH_TRY(view_ptr(ctx, "attention_prefill", q, query_bytes, &qp));
  BCH_TRY(view_ptr(ctx, "attention_prefill", k_cache, cache_bytes, &kp));
  BCH_TRY(view_ptr(ctx, "attention_prefill", v_cache, cache_bytes, &vp));
  BCH_TRY(view_ptr(ctx, "attention_prefill", out, query_bytes, &op));
  if (reinterpret_cast<uintptr_t>(kp) % 16 || reinterpret_cast<uintptr_t>(vp) % 16 ||
      reinterpret_cast<uintptr_t>(qp) % 16 || reinterpret_cast<uintptr_t>(op) % 16)
    return fail(BCH_ERR_ARGUMENT, "attention_prefill: operands must be 16-byte aligned");
  return launch(ctx, {"attention_prefill", 0, 0, 0}, [&](hipStream_t s) {
    run_attn_prefill_mfma(s, qp, kp, vp, op, n_heads, n_kv_heads, head_dim, first_pos, n_queries,
                          n_heads * head_dim, n_heads * head_dim, 1.0f / sqrtf((float)head_dim), nullptr, 0,
                          nullptr, 0, 0);
  });
}
