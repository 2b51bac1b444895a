// Mixture-of-experts kernels: the router and the weighted down projection of
// the experts it picks (the expert SwiGLU rows run through the persistent
// GEMV of gemv.hip).  Counterparts of moe_route / matvec_experts_down
// (crates/bobcat-metal/src/moe.metal:21-121, 237-307) and of the CPU
// Model::moe_block / route (crates/bobcat/src/lfm2.rs:413-440, 691-709).
#include <algorithm>
#include <cmath>

#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

// Orderable key of (value, index): larger values first, ties to the lower
// index (the order of the reference's stable descending sort).
__device__ __forceinline__ uint64_t route_key(float v, uint32_t index) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0;  // -0 ties +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - index);
}

// Wave 0 of a workgroup: the n_used experts of largest score + bias, ties to
// the lower expert, and their normalised weights, into out (ids, then
// weights as float bits).  Each expert's rank is the number of experts whose
// (score + bias, index) key is larger, counted by its lane over the keys in
// LDS (no cross-lane reductions on the critical path); ranks below n_used
// are the picks, in order.  score and bias are in LDS.
__device__ void pick_route(const float *score, const float *bias, uint32_t *__restrict__ out, uint32_t n_experts,
                           uint32_t n_used) {
  __shared__ uint64_t key_s[kMoeMaxExperts];
  __shared__ uint32_t pick_s[kMoeMaxUsed];
  __shared__ float pscore_s[kMoeMaxUsed];
  const uint32_t lane = threadIdx.x % 64;
  for (uint32_t e = lane; e < n_experts; e += 64) key_s[e] = route_key(score[e] + bias[e], e);
  __builtin_amdgcn_wave_barrier();
  for (uint32_t e = lane; e < n_experts; e += 64) {
    const uint64_t ke = key_s[e];
    uint32_t rank = 0;
    // Eight keys' reads in flight at a time (the count is independent of
    // the order; the clamped duplicates of the last block are not counted).
    for (uint32_t j0 = 0; j0 < n_experts; j0 += 8) {
      uint64_t kj[8];
#pragma unroll
      for (uint32_t u = 0; u < 8; u++) kj[u] = key_s[min(j0 + u, n_experts - 1)];
#pragma unroll
      for (uint32_t u = 0; u < 8; u++) rank += (j0 + u < n_experts && kj[u] > ke) ? 1u : 0u;
    }
    if (rank < n_used) {
      pick_s[rank] = e;
      pscore_s[rank] = score[e];
    }
  }
  __builtin_amdgcn_wave_barrier();
  // Every lane sums the picked scores in pick order (as the reference sums
  // the sorted picks); lane k < n_used writes pick k.
  float sum = 0.f;
  for (uint32_t k = 0; k < n_used; k++) sum += pscore_s[k];
  const float norm = sum + 1e-6f;  // transformers adds 1e-6 (lfm2.rs:703-705)
  if (lane < n_used) {
    out[lane] = pick_s[lane];
    out[n_used + lane] = __float_as_uint(pscore_s[lane] / norm);
  }
}

// One workgroup per token.  The token (RMS-normalised when norm_w is given,
// as rms_norm does: w·(x·scale)) is staged in LDS; wave w scores experts
// w, w+16, ... with the F32 router rows, their loads issued ahead; wave 0 then picks the n_used experts
// of largest sigmoid score + bias and writes their ids and normalised weights.
__global__ __launch_bounds__(1024) void k_moe_route(const float *__restrict__ x, const float *__restrict__ norm_w,
                                                    float eps, float *__restrict__ normed,
                                                    const float *__restrict__ router, const float *__restrict__ bias,
                                                    uint32_t *__restrict__ route, uint32_t n_cols, uint32_t n_experts,
                                                    uint32_t n_used) {
  extern __shared__ float xs[];
  __shared__ float red[16];
  __shared__ float score[kMoeMaxExperts], bias_s[kMoeMaxExperts];
  const uint32_t t = blockIdx.x, tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const float *row = x + (uint64_t)t * n_cols;
  // Router rows of this wave's experts (e0 + 16k), kU float4 per lane per
  // pass; the first pass is issued before the input is read, so its latency
  // overlaps the staging and the norm, and every pass issues all its loads
  // before the first multiply.
  constexpr int kU = 8, kE = 2;
  const uint32_t n4 = n_cols / 4;
  float4 w[kE][kU];
#define BCH_ROUTER_LOAD(e0, base)                                                                   \
  _Pragma("unroll") for (int k = 0; k < kE; k++) {                                                   \
    const uint32_t e_ = (e0) + 16 * k;                                                               \
    const float4 *r4_ = reinterpret_cast<const float4 *>(router + (uint64_t)min(e_, n_experts - 1) * n_cols); \
    _Pragma("unroll") for (int u = 0; u < kU; u++) {                                                 \
      const uint32_t i_ = (base) + lane + 64 * u;                                                    \
      w[k][u] = (e_ < n_experts && i_ < n4) ? r4_[i_] : make_float4(0.f, 0.f, 0.f, 0.f);             \
    }                                                                                                \
  }
  // The token's inputs and norm weights (two per thread for rows of up to
  // 2,048 columns) are requested before the router rows: memory returns in
  // issue order, so the norm waits for them alone.
  constexpr int kX = 2;
  float xv[kX], nv[kX];
#pragma unroll
  for (int j = 0; j < kX; j++) {
    const uint32_t i = min(tid + 1024 * j, n_cols - 1);
    xv[j] = row[i];
    nv[j] = norm_w ? norm_w[i] : 1.f;
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  BCH_ROUTER_LOAD(wave, 0u)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kX; j++) {
    const uint32_t i = tid + 1024 * j;
    ss = i < n_cols ? fmaf(xv[j], xv[j], ss) : ss;
  }
  for (uint32_t i = tid + 1024 * kX; i < n_cols; i += 1024) ss = fmaf(row[i], row[i], ss);
  float scale = 1.f;
  if (norm_w) {
    ss = block_sum<1024>(ss, red);
    scale = rsqrtf(ss / (float)n_cols + eps);
  }
#pragma unroll
  for (int j = 0; j < kX; j++) {
    const uint32_t i = tid + 1024 * j;
    if (i < n_cols) {
      const float v = norm_w ? nv[j] * (xv[j] * scale) : xv[j];
      xs[i] = v;
      if (norm_w) normed[(uint64_t)t * n_cols + i] = v;
    }
  }
  for (uint32_t i = tid + 1024 * kX; i < n_cols; i += 1024) {
    const float v = norm_w ? norm_w[i] * (row[i] * scale) : row[i];
    xs[i] = v;
    if (norm_w) normed[(uint64_t)t * n_cols + i] = v;
  }
  for (uint32_t i = tid; i < n_experts; i += 1024) bias_s[i] = bias[i];
  __syncthreads();
  // Each lane sums its columns in increasing order, then the wave sums.
  for (uint32_t e0 = wave; e0 < n_experts; e0 += 16 * kE) {
    float acc[kE];
#pragma unroll
    for (int k = 0; k < kE; k++) acc[k] = 0.f;
    for (uint32_t base = 0; base < n4; base += 64 * kU) {
      if (e0 != wave || base != 0) {
        BCH_ROUTER_LOAD(e0, base)
      }
#pragma unroll
      for (int u = 0; u < kU; u++) {
        const uint32_t i = base + lane + 64 * u;
        if (i < n4) {
          const float4 v = reinterpret_cast<const float4 *>(xs)[i];
#pragma unroll
          for (int k = 0; k < kE; k++)
            acc[k] = fmaf(w[k][u].x, v.x, fmaf(w[k][u].y, v.y, fmaf(w[k][u].z, v.z, fmaf(w[k][u].w, v.w, acc[k]))));
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kE; k++) {
      acc[k] = wave_sum(acc[k]);
      if (lane == 0 && e0 + 16 * k < n_experts) score[e0 + 16 * k] = 1.0f / (1.0f + expf(-acc[k]));
    }
  }
#undef BCH_ROUTER_LOAD
  __syncthreads();
  if (wave != 0) return;
  pick_route(score, bias_s, route + (uint64_t)t * 2 * n_used, n_experts, n_used);
}

// Routes of decode and prefill tokens with the router spread over the chip:
// one workgroup per (token, 4 experts), wave w scoring expert
// 4·blockIdx.y + w.  A workgroup issues its router row loads, the norm
// weights and the token's inputs at once, normalises the token for itself
// (as k_moe_route does; the first workgroup also stores it in `normed`) and
// hands its scores to the token's other workgroups through
// scores[token][expert] with device-scope stores.  The last to arrive, by
// counters[token] (left zeroed), picks the route.
__global__ __launch_bounds__(256) void k_moe_scores(const float *__restrict__ x, const float *__restrict__ norm_w,
                                                    float eps, float *__restrict__ normed,
                                                    const float *__restrict__ router, const float *__restrict__ bias,
                                                    float *__restrict__ scores, uint32_t *__restrict__ counters,
                                                    uint32_t *__restrict__ route, uint32_t n_cols, uint32_t n_experts,
                                                    uint32_t n_used) {
  extern __shared__ float xs[];
  __shared__ float red[4];
  __shared__ float score_s[kMoeMaxExperts], bias_s[kMoeMaxExperts];
  __shared__ uint32_t last_s;
  const uint32_t t = blockIdx.x, tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const uint32_t e = 4 * blockIdx.y + wave, n4 = n_cols / 4;
  constexpr int kU = 8, kX = 8;  // router float4 per lane per pass; input elements per thread held
  // The token's inputs and norm weights first, then the router row: memory
  // returns in issue order, so the norm waits for the inputs alone.  Loads
  // are unconditional (clamped indices), so the waits count exactly.
  const float *row = x + (uint64_t)t * n_cols;
  float xv[kX], nv[kX];
#pragma unroll
  for (int j = 0; j < kX; j++) {
    const uint32_t i = min(tid + 256 * j, n_cols - 1);
    xv[j] = row[i];
    nv[j] = norm_w ? norm_w[i] : 1.f;
  }
  const float bv = bias[min(tid, n_experts - 1)];  // for the route pick (n_experts <= 256 threads)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  const float4 *r4 = reinterpret_cast<const float4 *>(router + (uint64_t)min(e, n_experts - 1) * n_cols);
  float4 w[kU];
#pragma unroll
  for (int u = 0; u < kU; u++) w[u] = r4[min(lane + 64 * u, n4 - 1)];
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kX; j++) ss = tid + 256 * j < n_cols ? fmaf(xv[j], xv[j], ss) : ss;
  for (uint32_t i = tid + 256 * kX; i < n_cols; i += 256) ss = fmaf(row[i], row[i], ss);
  float scale = 1.f;
  if (norm_w) {
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    lds_barrier();
    ss = red[0] + red[1] + red[2] + red[3];
    scale = rsqrtf(ss / (float)n_cols + eps);
  }
  // Staged as rms_norm computes it: w·(x·scale).
#pragma unroll
  for (int j = 0; j < kX; j++) {
    const uint32_t i = tid + 256 * j;
    if (i < n_cols) xs[i] = norm_w ? nv[j] * (xv[j] * scale) : xv[j];
  }
  for (uint32_t i = tid + 256 * kX; i < n_cols; i += 256) xs[i] = norm_w ? norm_w[i] * (row[i] * scale) : row[i];
  if (tid < n_experts) bias_s[tid] = bv;
  lds_barrier();
  // Each lane sums its columns in increasing order, then the wave sums (the
  // order k_moe_route uses).
  if (e < n_experts) {
    float acc = 0.f;
    for (uint32_t base = 0; base < n4; base += 64 * kU) {
      if (base != 0) {
#pragma unroll
        for (int u = 0; u < kU; u++) {
          const uint32_t i = base + lane + 64 * u;
          w[u] = i < n4 ? r4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < kU; u++) {
        const uint32_t i = base + lane + 64 * u;
        if (i < n4) {
          const float4 v = reinterpret_cast<const float4 *>(xs)[i];
          acc = fmaf(w[u].x, v.x, fmaf(w[u].y, v.y, fmaf(w[u].z, v.z, fmaf(w[u].w, v.w, acc))));
        }
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) coherent_store(scores + (uint64_t)t * n_experts + e, 1.0f / (1.0f + expf(-acc)));
  }
  if (norm_w && blockIdx.y == 0)
    for (uint32_t i = tid; i < n_cols; i += 256) normed[(uint64_t)t * n_cols + i] = xs[i];
  // Hand-off to the token's last workgroup, by the hardware's ordering (as
  // in attn_decode.hip; an agent-scope release would write back the whole
  // L2): the scores are agent-scope atomic stores written through to the
  // coherence point, acknowledged before the barrier (s_waitcnt(0); the
  // signal fence keeps the compiler from sinking them), then counted in by
  // a device atomic, and the last workgroup reads them with agent-scope
  // atomic loads issued after its atomic returned.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&counters[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_s = prev == gridDim.y - 1;
  }
  __syncthreads();
  if (!last_s || wave != 0) return;
  for (uint32_t i = lane; i < n_experts; i += 64) score_s[i] = coherent_load(scores + (uint64_t)t * n_experts + i);
  __builtin_amdgcn_wave_barrier();
  pick_route(score_s, bias_s, route + (uint64_t)t * 2 * n_used, n_experts, n_used);
  if (lane == 0) coherent_store(&counters[t], 0u);
}

// y[r] += Σ_slot w_slot · (W_{e_slot} row r) · x_slot for one token.  A
// group of LPR lanes takes a row, lane i unit i, for every picked expert.
// Load order sets the latency: the route (scalar loads) and the USED inputs
// are requested first, every weight load of the workgroup's rows as soon as
// the route has arrived, and the inputs are staged in LDS (a padded slot
// per unit, as the GEMV does) while the weights are on their way.  The
// experts are added in route order.
template <class F, int LPR, int USED>
__global__ __launch_bounds__(256) void k_experts_down(const uint8_t *__restrict__ W, uint64_t rb, uint32_t n_rows,
                                                      uint32_t n_cols, const float *__restrict__ x,
                                                      const uint32_t *__restrict__ route, float *__restrict__ y) {
  constexpr int T = 256, G = T / LPR;
  constexpr uint32_t kSlot = F::kUnit + (F::kUnit >= 64 ? 4 : 0);
  // float4 of the inputs per thread held in registers (the rest, if any,
  // staged after the weights are requested).
  constexpr int kPer = std::min(8, (USED * LPR * (int)F::kUnit / 4 + T - 1) / T);
  extern __shared__ float4 xs4[];
  float *xs = reinterpret_cast<float *>(xs4);
  const uint32_t tid = threadIdx.x, n_units = n_cols / F::kUnit, per_input = n_units * kSlot;
  const uint32_t n4 = n_cols / 4, all4 = USED * n4;
  uint32_t ids[USED];
  float wts[USED];
#pragma unroll
  for (int k = 0; k < USED; k++) {
    ids[k] = route[k];
    wts[k] = __uint_as_float(route[USED + k]);
  }
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float4 xv[kPer];
#pragma unroll
  for (int j = 0; j < kPer; j++) xv[j] = x4[min(tid + j * T, all4 - 1)];
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t g = tid / LPR, li = tid % LPR;
  const bool active = li < n_units;
  const uint32_t unit = active ? li : 0u;
  const uint32_t r = blockIdx.x * G + g, rc = min(r, n_rows - 1);
  typename F::Raw raw[USED];
#pragma unroll
  for (int k = 0; k < USED; k++) raw[k] = F::fetch(W + ((uint64_t)ids[k] * n_rows + rc) * rb, unit);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // Staging: input k's element e goes to slot k·per_input + (e / kUnit)·kSlot
  // + e % kUnit.  Clamped duplicates rewrite the same value.
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const uint32_t i = min(tid + j * T, all4 - 1), k = i / n4, e = 4 * (i % n4);
    *reinterpret_cast<float4 *>(xs + k * per_input + (e / F::kUnit) * kSlot + e % F::kUnit) = xv[j];
  }
  for (uint32_t i = tid + kPer * T; i < all4; i += T) {
    const uint32_t k = i / n4, e = 4 * (i % n4);
    *reinterpret_cast<float4 *>(xs + k * per_input + (e / F::kUnit) * kSlot + e % F::kUnit) = x4[i];
  }
  lds_barrier();
  float dots[USED];
#pragma unroll
  for (int k = 0; k < USED; k++) {
    typename F::Frag f;
    F::from_lds(xs + k * per_input + unit * kSlot, f);
    dots[k] = group_sum<LPR>(active ? F::compute(raw[k], unit, f) : 0.f);
  }
  if (li == 0 && r < n_rows) {
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < USED; k++) acc += wts[k] * dots[k];
    y[r] += acc;
  }
}

void run_moe_route(hipStream_t s, const float *x, const float *norm_w, float eps, float *normed, const float *router,
                   const float *bias, uint32_t *route, uint32_t n_cols, uint32_t n_experts, uint32_t n_used,
                   uint32_t n_tokens, float *scores, uint32_t *counters) {
  const size_t lds = (size_t)n_cols * 4;
  static const bool lds_limit_set =
      hipFuncSetAttribute(reinterpret_cast<const void *>(k_moe_route), hipFuncAttributeMaxDynamicSharedMemorySize,
                          131072) == hipSuccess;
  (void)lds_limit_set;
  if (scores) {
    static const bool set = hipFuncSetAttribute(reinterpret_cast<const void *>(k_moe_scores),
                                                hipFuncAttributeMaxDynamicSharedMemorySize, 131072) == hipSuccess;
    (void)set;
    k_moe_scores<<<dim3(n_tokens, (n_experts + 3) / 4), 256, lds, s>>>(x, norm_w, eps, normed, router, bias, scores,
                                                                      counters, route, n_cols, n_experts, n_used);
    return;
  }
  k_moe_route<<<n_tokens, 1024, lds, s>>>(x, norm_w, eps, normed, router, bias, route, n_cols, n_experts, n_used);
}

template <class F, int LPR>
static void launch_down(hipStream_t s, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                        const uint32_t *route, uint32_t n_used, float *y, uint32_t n_cus) {
  constexpr uint32_t kSlot = F::kUnit + (F::kUnit >= 64 ? 4 : 0);
  const uint64_t rb = bch_row_bytes(F::kFormat, n_cols);
  const size_t lds = (size_t)n_used * (n_cols / F::kUnit) * kSlot * 4;
  const uint32_t groups = 256 / LPR;
  const uint32_t grid = (n_rows + groups - 1) / groups;  // one row per group
  switch (n_used) {
#define BCH_DOWN(U)                                                                                              \
  case U: {                                                                                                      \
    static const bool set = hipFuncSetAttribute(reinterpret_cast<const void *>(k_experts_down<F, LPR, U>),     \
                                                hipFuncAttributeMaxDynamicSharedMemorySize, 163840) == hipSuccess; \
    (void)set;                                                                                                   \
    k_experts_down<F, LPR, U><<<grid, 256, lds, s>>>(W, rb, n_rows, n_cols, x, route, y);                        \
    break;                                                                                                       \
  }
    BCH_DOWN(1) BCH_DOWN(2) BCH_DOWN(3) BCH_DOWN(4) BCH_DOWN(5) BCH_DOWN(6) BCH_DOWN(7) BCH_DOWN(8)
#undef BCH_DOWN
    default: break;
  }
}

template <class F>
static bool down_for(hipStream_t s, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                     const uint32_t *route, uint32_t n_used, float *y, uint32_t n_cus) {
  if (n_cols % F::kUnit) return false;
  const uint32_t n_units = n_cols / F::kUnit;
  constexpr uint32_t kSlot = F::kUnit + (F::kUnit >= 64 ? 4 : 0);
  if ((uint64_t)n_used * n_units * kSlot * 4 > 163840) return false;  // the inputs must fit in LDS
  if (n_units <= 4) launch_down<F, 4>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  else if (n_units <= 8) launch_down<F, 8>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  else if (n_units <= 16) launch_down<F, 16>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  else if (n_units <= 32) launch_down<F, 32>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  else if (n_units <= 64) launch_down<F, 64>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  else return false;
  return true;
}

bool run_experts_down(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                      const float *x, const uint32_t *route, uint32_t n_used, float *y, uint32_t n_cus) {
  if (n_used == 0 || n_used > kMoeMaxUsed) return false;
  if (format == Q4K::kFormat) return down_for<Q4K>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  if (format == F16::kFormat) return down_for<F16>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  if (format == F32::kFormat) return down_for<F32>(s, W, n_rows, n_cols, x, route, n_used, y, n_cus);
  return false;
}

// --- grouping for the batched experts --------------------------------------

// Entries v = token·n_used + slot grouped by expert (moe.metal:122-175 is
// the reference's kernel): offsets[e] is where expert e's entries start in
// `entries`, in token order, and offsets[n_experts] the total.  One
// workgroup of 16 waves; wave w takes a contiguous run of the entries.  The
// entries' experts are first copied to LDS as bytes (up to
// kGroupLdsEntries entries; larger batches read them from the route).  Each
// wave counts its run's entries per expert 64 at a time, one ballot per
// distinct expert among the 64; a prefix over (expert, wave) gives every
// wave its first slot for each expert; a second pass over the run places
// the entries, so each expert's entries keep their order.
constexpr int kGroupWaves = 16;
constexpr uint32_t kGroupLdsEntries = 16384;
static_assert(kMoeMaxExperts <= 256, "expert ids fit a byte");

__global__ __launch_bounds__(kGroupWaves * 64) void k_moe_group(const uint32_t *__restrict__ route,
                                                                uint32_t *__restrict__ offsets,
                                                                uint32_t *__restrict__ entries, uint32_t n_experts,
                                                                uint32_t n_used, uint32_t n_tokens) {
  __shared__ uint32_t slot[kGroupWaves][kMoeMaxExperts];  // per (wave, expert): count, then next slot
  __shared__ uint32_t total[kMoeMaxExperts];
  __shared__ uint8_t ids[kGroupLdsEntries];
  const uint32_t wave = threadIdx.x / 64, lane = threadIdx.x % 64, n_entries = n_used * n_tokens;
  auto route_expert = [&](uint32_t v) { return route[2ull * n_used * (v / n_used) + v % n_used]; };
  const bool staged = n_entries <= kGroupLdsEntries;
  if (staged)
    for (uint32_t v = threadIdx.x; v < n_entries; v += kGroupWaves * 64) ids[v] = (uint8_t)route_expert(v);
  for (uint32_t e = lane; e < n_experts; e += 64) slot[wave][e] = 0;
  __syncthreads();
  auto expert_of = [&](uint32_t v) -> uint32_t { return staged ? ids[v] : route_expert(v); };
  const uint32_t per = (n_entries + kGroupWaves * 64 - 1) / (kGroupWaves * 64) * 64;  // entries per wave
  const uint32_t v0 = min(wave * per, n_entries), v1 = min(v0 + per, n_entries);
  const uint64_t below = (1ull << lane) - 1;
  // For each distinct expert le among this slice's lanes (those with v < v1),
  // in order of the lowest lane holding it: fn(le, ballot of its lanes).
  auto distinct = [&](uint32_t e, bool valid, auto fn) {
    uint64_t todo = __ballot(valid);
    while (todo) {
      const uint32_t leader = (uint32_t)__ffsll((unsigned long long)todo) - 1;
      const uint32_t le = __shfl(e, leader, 64);
      const uint64_t mask = __ballot(valid && e == le);
      fn(le, mask);
      todo &= ~mask;
    }
  };
  for (uint32_t first = v0; first < v1; first += 64) {
    const uint32_t v = first + lane;
    const bool valid = v < v1;
    const uint32_t e = valid ? expert_of(v) : 0;
    distinct(e, valid, [&](uint32_t le, uint64_t mask) {
      if (lane == 0) slot[wave][le] += (uint32_t)__popcll(mask);
    });
  }
  __syncthreads();
  // Expert totals, their exclusive prefix (offsets), then each wave's first
  // slot per expert.
  for (uint32_t e = threadIdx.x; e < n_experts; e += kGroupWaves * 64) {
    uint32_t t = 0;
    for (int w = 0; w < kGroupWaves; w++) t += slot[w][e];
    total[e] = t;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t start = 0;
    for (uint32_t e = 0; e < n_experts; e++) {
      const uint32_t t = total[e];
      total[e] = start;
      offsets[e] = start;
      start += t;
    }
    offsets[n_experts] = start;
  }
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < n_experts; e += kGroupWaves * 64) {
    uint32_t start = total[e];
    for (int w = 0; w < kGroupWaves; w++) {
      const uint32_t c = slot[w][e];
      slot[w][e] = start;
      start += c;
    }
  }
  __syncthreads();
  for (uint32_t first = v0; first < v1; first += 64) {
    const uint32_t v = first + lane;
    const bool valid = v < v1;
    const uint32_t e = valid ? expert_of(v) : 0;
    distinct(e, valid, [&](uint32_t le, uint64_t mask) {
      const uint32_t base = slot[wave][le];
      if (valid && e == le) entries[base + (uint32_t)__popcll(mask & below)] = v;
      __builtin_amdgcn_wave_barrier();
      if (lane == 0) slot[wave][le] = base + (uint32_t)__popcll(mask);
      __builtin_amdgcn_wave_barrier();
    });
  }
}

// y[t] += Σ_s w_s · x[n_used·t + s], the sum in slot order first
// (moe.metal:177-200).  One thread per element.
__global__ void k_moe_combine(const float *__restrict__ x, const uint32_t *__restrict__ route, float *__restrict__ y,
                              uint32_t n_embd, uint32_t n_used, uint32_t n_tokens) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (uint64_t)n_tokens * n_embd) return;
  const uint64_t t = i / n_embd, d = i % n_embd;
  const uint32_t *r = route + 2 * n_used * t;
  float sum = 0.f;
  for (uint32_t k = 0; k < n_used; k++) sum += __uint_as_float(r[n_used + k]) * x[(t * n_used + k) * n_embd + d];
  y[i] += sum;
}

void run_moe_group(hipStream_t s, const uint32_t *route, uint32_t *offsets, uint32_t *entries, uint32_t n_experts,
                   uint32_t n_used, uint32_t n_tokens) {
  k_moe_group<<<1, kGroupWaves * 64, 0, s>>>(route, offsets, entries, n_experts, n_used, n_tokens);
}

void run_moe_combine(hipStream_t s, const float *x, const uint32_t *route, float *y, uint32_t n_embd,
                     uint32_t n_used, uint32_t n_tokens) {
  const uint64_t n = (uint64_t)n_tokens * n_embd;
  if (n) k_moe_combine<<<(uint32_t)((n + 255) / 256), 256, 0, s>>>(x, route, y, n_embd, n_used, n_tokens);
}

}  // namespace bch

// ---------------------------------------------------------------------
// C ABI (Metal::moe_route / matvec_experts_swiglu / matvec_experts_down /
// moe_group / matmul_experts / moe_combine / route_bytes,
// crates/bobcat-metal/src/backend.rs:1428-1731, 2724-2734).
// ---------------------------------------------------------------------

using namespace bch;

static int check_experts(uint32_t n_experts, uint32_t n_used) {
  if (n_experts > kMoeMaxExperts || n_used > kMoeMaxUsed || n_used == 0 || n_used > n_experts)
    return fail(BCH_ERR_EXPERT_LIMITS, "at most %u of %u experts per token, got %u of %u", kMoeMaxUsed,
                kMoeMaxExperts, n_used, n_experts);
  return BCH_OK;
}

static bool expert_format(uint32_t format) {
  return format == Q4K::kFormat || format == F16::kFormat || format == F32::kFormat;
}

extern "C" uint64_t bch_route_bytes(uint32_t n_used, uint32_t n_tokens) { return 2ull * n_used * n_tokens * 4; }

extern "C" int bch_moe_route(bch_ctx *ctx, bch_view x, const bch_norm *norm, bch_view normed, bch_view router,
                             bch_view bias, bch_view route, uint32_t n_cols, uint32_t n_experts, uint32_t n_used,
                             uint32_t n_tokens) {
  BCH_TRY(check_experts(n_experts, n_used));
  if (n_cols == 0 || n_cols % 4 || n_cols > 32768 || n_tokens == 0)
    return fail(BCH_ERR_ARGUMENT, "moe_route: %u columns (a positive multiple of 4 up to 32768), %u tokens", n_cols,
                n_tokens);
  const uint64_t token_bytes = (uint64_t)n_tokens * n_cols * 4;
  const float *xp, *rp, *bp, *nw = nullptr;
  float *np = nullptr;
  uint32_t *route_p;
  BCH_TRY(view_ptr(ctx, "moe_route", x, token_bytes, &xp));
  BCH_TRY(view_ptr(ctx, "moe_route", router, (uint64_t)n_experts * n_cols * 4, &rp));
  BCH_TRY(view_ptr(ctx, "moe_route", bias, (uint64_t)n_experts * 4, &bp));
  BCH_TRY(view_ptr(ctx, "moe_route", route, bch_route_bytes(n_used, n_tokens), &route_p));
  if (norm) {
    BCH_TRY(view_ptr(ctx, "moe_route", norm->weight, (uint64_t)n_cols * 4, &nw));
    BCH_TRY(view_ptr(ctx, "moe_route", normed, token_bytes, &np));
  }
  if (reinterpret_cast<uintptr_t>(rp) % 16)
    return fail(BCH_ERR_ARGUMENT, "moe_route: the router is not 16-byte aligned");
  const float eps = norm ? norm->eps : 0.f;
  return launch(ctx, {"moe_route", n_experts, n_cols, (uint64_t)n_experts * n_cols * 4}, [&](hipStream_t s) {
    run_moe_route(s, xp, nw, eps, np, rp, bp, route_p, n_cols, n_experts, n_used, n_tokens, nullptr, nullptr);
  });
}

extern "C" int bch_matvec_experts_swiglu(bch_ctx *ctx, uint32_t format, bch_view gate, bch_view up, uint32_t n_rows,
                                         uint32_t n_cols, uint32_t n_experts, bch_view x, bch_view route,
                                         uint32_t n_used, bch_view y, uint32_t n_tokens) {
  if (!expert_format(format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "format %u has no expert kernels", format);
  BCH_TRY(check_experts(n_experts, n_used));
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (rb == 0 || n_rows == 0 || n_tokens == 0)
    return fail(BCH_ERR_ARGUMENT, "matvec_experts_swiglu: %u x %u of format %u", n_rows, n_cols, format);
  const uint8_t *gp, *up_p;
  const float *xp;
  const uint32_t *rp;
  float *yp;
  const uint64_t stacked = rb * n_rows * n_experts;
  BCH_TRY(view_ptr(ctx, "matvec_experts_swiglu", gate, stacked, &gp));
  BCH_TRY(view_ptr(ctx, "matvec_experts_swiglu", up, stacked, &up_p));
  BCH_TRY(view_ptr(ctx, "matvec_experts_swiglu", x, (uint64_t)n_tokens * n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matvec_experts_swiglu", route, bch_route_bytes(n_used, n_tokens), &rp));
  BCH_TRY(view_ptr(ctx, "matvec_experts_swiglu", y, (uint64_t)n_tokens * n_used * n_rows * 4, &yp));
  if (reinterpret_cast<uintptr_t>(gp) % 16 || reinterpret_cast<uintptr_t>(up_p) % 16 ||
      reinterpret_cast<uintptr_t>(xp) % 16)
    return fail(BCH_ERR_ARGUMENT, "matvec_experts_swiglu: operands must be 16-byte aligned");
  bool ok = true;
  BCH_TRY(launch(ctx, {"matvec_experts_swiglu", n_rows, n_cols, 2 * rb * n_rows * n_used}, [&](hipStream_t s) {
    for (uint32_t t = 0; t < n_tokens && ok; t++)
      ok = fast_matvec_experts_swiglu(s, format, gp, up_p, n_rows, n_cols, rp + (uint64_t)t * 2 * n_used, n_used,
                                      xp + (uint64_t)t * n_cols, yp + (uint64_t)t * n_used * n_rows, ctx->n_cus);
  }));
  if (!ok) return fail(BCH_ERR_UNSUPPORTED_FORMAT, "matvec_experts_swiglu: rows of %u columns are too wide", n_cols);
  return BCH_OK;
}

extern "C" int bch_matvec_experts_down(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows,
                                       uint32_t n_cols, uint32_t n_experts, bch_view x, bch_view route,
                                       uint32_t n_used, bch_view y, uint32_t n_tokens) {
  if (!expert_format(format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "format %u has no expert kernels", format);
  BCH_TRY(check_experts(n_experts, n_used));
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (rb == 0 || n_rows == 0 || n_tokens == 0)
    return fail(BCH_ERR_ARGUMENT, "matvec_experts_down: %u x %u of format %u", n_rows, n_cols, format);
  const uint8_t *wp;
  const float *xp;
  const uint32_t *rp;
  float *yp;
  BCH_TRY(view_ptr(ctx, "matvec_experts_down", weights, rb * n_rows * n_experts, &wp));
  BCH_TRY(view_ptr(ctx, "matvec_experts_down", x, (uint64_t)n_tokens * n_used * n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matvec_experts_down", route, bch_route_bytes(n_used, n_tokens), &rp));
  BCH_TRY(view_ptr(ctx, "matvec_experts_down", y, (uint64_t)n_tokens * n_rows * 4, &yp));
  if (reinterpret_cast<uintptr_t>(wp) % 16 || reinterpret_cast<uintptr_t>(xp) % 16)
    return fail(BCH_ERR_ARGUMENT, "matvec_experts_down: operands must be 16-byte aligned");
  bool ok = true;
  BCH_TRY(launch(ctx, {"matvec_experts_down", n_rows, n_cols, rb * n_rows * n_used}, [&](hipStream_t s) {
    for (uint32_t t = 0; t < n_tokens && ok; t++)
      ok = run_experts_down(s, format, wp, n_rows, n_cols, xp + (uint64_t)t * n_used * n_cols,
                            rp + (uint64_t)t * 2 * n_used, n_used, yp + (uint64_t)t * n_rows, ctx->n_cus);
  }));
  if (!ok) return fail(BCH_ERR_UNSUPPORTED_FORMAT, "matvec_experts_down: rows of %u columns are too wide", n_cols);
  return BCH_OK;
}

extern "C" int bch_moe_group(bch_ctx *ctx, bch_view route, bch_view offsets, bch_view entries, uint32_t n_experts,
                             uint32_t n_used, uint32_t n_tokens) {
  BCH_TRY(check_experts(n_experts, n_used));
  const uint32_t *rp;
  uint32_t *op, *ep;
  BCH_TRY(view_ptr(ctx, "moe_group", route, bch_route_bytes(n_used, n_tokens), &rp));
  BCH_TRY(view_ptr(ctx, "moe_group", offsets, (uint64_t)(n_experts + 1) * 4, &op));
  BCH_TRY(view_ptr(ctx, "moe_group", entries, (uint64_t)n_used * n_tokens * 4, &ep));
  return launch(ctx, {"moe_group", 0, 0, 0},
                [&](hipStream_t s) { run_moe_group(s, rp, op, ep, n_experts, n_used, n_tokens); });
}

extern "C" int bch_matmul_experts(bch_ctx *ctx, uint32_t format, bch_view weights, const bch_view *up,
                                  uint32_t n_rows, uint32_t n_cols, uint32_t n_experts, bch_view x,
                                  int shared_input, bch_view offsets, bch_view entries, uint32_t n_used, bch_view y,
                                  uint32_t n_tokens) {
  if (!expert_format(format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "format %u has no expert kernels", format);
  BCH_TRY(check_experts(n_experts, n_used));
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (rb == 0 || n_rows == 0 || n_cols % 256)
    return fail(BCH_ERR_ARGUMENT, "matmul_experts: %u x %u needs columns in multiples of 256", n_rows, n_cols);
  const uint64_t entry_count = (uint64_t)n_used * n_tokens;
  const uint64_t input_rows = shared_input ? n_tokens : entry_count;
  const uint64_t stacked = rb * n_rows * n_experts;
  const uint8_t *wp, *upp = nullptr;
  const float *xp;
  const uint32_t *op, *ep;
  float *yp;
  BCH_TRY(view_ptr(ctx, "matmul_experts", weights, stacked, &wp));
  if (up) BCH_TRY(view_ptr(ctx, "matmul_experts", *up, stacked, &upp));
  BCH_TRY(view_ptr(ctx, "matmul_experts", x, input_rows * n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matmul_experts", y, entry_count * n_rows * 4, &yp));
  BCH_TRY(view_ptr(ctx, "matmul_experts", offsets, (uint64_t)(n_experts + 1) * 4, &op));
  BCH_TRY(view_ptr(ctx, "matmul_experts", entries, entry_count * 4, &ep));
  if (reinterpret_cast<uintptr_t>(wp) % 16 || reinterpret_cast<uintptr_t>(upp) % 16 ||
      reinterpret_cast<uintptr_t>(xp) % 16)
    return fail(BCH_ERR_ARGUMENT, "matmul_experts: operands must be 16-byte aligned");
  void *split = nullptr;
  BCH_TRY(ctx_scratch(ctx, matmul_split_bytes((uint32_t)input_rows, n_cols), &split));
  return launch(ctx, {"matmul_experts", n_rows, n_cols, stacked * (up ? 2 : 1)}, [&](hipStream_t s) {
    if (n_tokens)
      run_matmul_experts(s, format, wp, upp, n_rows, n_cols, n_experts, xp, shared_input != 0, op, ep, n_used, yp,
                         n_tokens, split);
  });
}

extern "C" int bch_moe_combine(bch_ctx *ctx, bch_view x, bch_view route, bch_view y, uint32_t n_embd,
                               uint32_t n_used, uint32_t n_tokens) {
  if (n_used == 0 || n_used > kMoeMaxUsed)
    return fail(BCH_ERR_EXPERT_LIMITS, "at most %u experts per token, got %u", kMoeMaxUsed, n_used);
  const float *xp;
  const uint32_t *rp;
  float *yp;
  const uint64_t n = (uint64_t)n_tokens * n_embd;
  BCH_TRY(view_ptr(ctx, "moe_combine", x, n * n_used * 4, &xp));
  BCH_TRY(view_ptr(ctx, "moe_combine", route, bch_route_bytes(n_used, n_tokens), &rp));
  BCH_TRY(view_ptr(ctx, "moe_combine", y, n * 4, &yp));
  return launch(ctx, {"moe_combine", 0, 0, 0},
                [&](hipStream_t s) { run_moe_combine(s, xp, rp, yp, n_embd, n_used, n_tokens); });
}
