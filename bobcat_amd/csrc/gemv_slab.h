// Slab GEMV for decode: every workgroup owns one contiguous slab of items
// (rows, SwiGLU pairs, conv channels) and issues the loads of ALL of its
// weights as its first instructions, before the input is staged.
//
// A decode GEMV moves a few MB to a few tens of MB and lasts a few µs, so
// what bounds it is how soon the bytes are requested, not how they are
// reused: with the whole slab in flight from the first cycle, each CU keeps
// ~50-100 KB of requests outstanding (8 TB/s × ~2 µs of latency is ~60 KB
// per CU), and the input staging, the RMS norm and the digit conversion
// run while the weights are on their way.  The item policies (row
// addressing, SwiGLU, the gated short convolution, accumulation into the
// residual, argmax partials) are those of the x-stationary kernel in
// gemv.h, and so are the per-unit arithmetic and the reduction order, so
// the two kernels give the same sums.
//
// Layout: a group of LPR lanes spans a row (lane i owns unit i, as in
// gemv.h).  Workgroup w owns a contiguous slab of n/grid items (the first
// n % grid workgroups one more); group g of
// the workgroup takes items g, g+G, g+2G, ... of the slab, at most MAXI.
#pragma once
#include <type_traits>

#include "gemv.h"

namespace bch {

// Where the input comes from: the vector x itself (PlainIn), or the decode
// attention's deferred split partials combined on the way in (SplitIn).
// load() issues a float4's loads (unconditional: the staging waits for them
// alone), finish() turns them into the float4.
struct PlainIn {
  using Raw = float4;
  __device__ Raw load(const float4 *x4, uint32_t i) const { return x4[i]; }
  __device__ float4 finish(const Raw &r, uint32_t) const { return r; }
};

// The combine of the decode attention's last workgroup (attn_decode.hip),
// for at most kDeferSplits splits: every slot's (max, sum) header and
// output quad are loaded whatever the split count (slots past it hold
// stale values and are selected away), so no address waits for *dpos.
template <bool GATE>
struct SplitIn {
  SplitOut a;
  struct Raw {
    float4 out, o[kDeferSplits], g;
    float2 ml[kDeferSplits];
  };
  __device__ Raw load(const float4 *x4, uint32_t i) const {
    Raw r;
    r.out = x4[i];
    const uint32_t e = 4 * i, h = e / a.head_dim, el = e % a.head_dim, stride = a.head_dim + 4;
#pragma unroll
    for (uint32_t sp = 0; sp < kDeferSplits; sp++) {
      const float *pp = a.partials + ((uint64_t)h * a.max_splits + min(sp, a.max_splits - 1)) * stride;
      r.ml[sp] = *reinterpret_cast<const float2 *>(pp);
      r.o[sp] = *reinterpret_cast<const float4 *>(pp + 4 + el);
    }
    if constexpr (GATE) r.g = *reinterpret_cast<const float4 *>(a.gate + (uint64_t)h * a.gate_head_stride + el);
    return r;
  }
  __device__ float4 finish(const Raw &r, uint32_t n_splits) const {
    if (n_splits > a.defer) return r.out;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t sp = 0; sp < kDeferSplits; sp++) M = sp < n_splits ? fmaxf(M, r.ml[sp].x) : M;
    float L = 0.f;
    float4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t sp = 0; sp < kDeferSplits; sp++) {
      if (sp < n_splits) {
        const float w = expf(r.ml[sp].x - M);
        L = fmaf(r.ml[sp].y, w, L);
        O.x = fmaf(r.o[sp].x, w, O.x);
        O.y = fmaf(r.o[sp].y, w, O.y);
        O.z = fmaf(r.o[sp].z, w, O.z);
        O.w = fmaf(r.o[sp].w, w, O.w);
      }
    }
    float4 v = {O.x / L, O.y / L, O.z / L, O.w / L};
    if constexpr (GATE) {
      v.x *= 1.0f / (1.0f + expf(-r.g.x));
      v.y *= 1.0f / (1.0f + expf(-r.g.y));
      v.z *= 1.0f / (1.0f + expf(-r.g.z));
      v.w *= 1.0f / (1.0f + expf(-r.g.w));
    }
    return v;
  }
};

template <class F, int LPR, int MAXI, bool NORM, class P, class In>
__device__ __forceinline__ void slab_body(const P &p, const float *__restrict__ x, const float *__restrict__ nw,
                                          float eps, uint32_t per, uint32_t rem, uint32_t n_units,
                                          uint32_t n_cols,
                                          const In &in) {
  constexpr int T = LPR <= 64 ? 256 : LPR;  // threads per workgroup
  constexpr int G = T / LPR;                // groups per workgroup
  constexpr int R = P::kRows;
  const int tid = threadIdx.x;
  const int g = tid / LPR, li = tid % LPR;
  const bool active = li < (int)n_units;
  const uint32_t unit = active ? (uint32_t)li : 0u;
  // Workgroups take `per` items each and the first `rem` one more (per and
  // rem come from the host: the slab's bounds gate the first weight
  // address, and a division here stood before it).
  const uint32_t begin = blockIdx.x * per + min(blockIdx.x, rem);
  const uint32_t end = begin + per + (blockIdx.x < rem ? 1u : 0u);

  // 1. The input (and norm weights) into registers, then every weight load
  // of the slab.  Memory returns in issue order, so the input goes first:
  // the staging below waits for it alone while the weights stream in.
  // float4 per thread: a row has at most LPR units of kUnit inputs.
  constexpr int kPer = (LPR * (int)F::kUnit / 4 + T - 1) / T;
  const uint32_t n4 = n_cols / 4;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 *w4 = reinterpret_cast<const float4 *>(nw);
  // Every load below is unconditional (indices clamped into range): a load
  // under a branch makes the compiler's wait counting fall back to waiting
  // for everything, which would hold the staging until the weights arrive.
  typename In::Raw xv[kPer];
  float4 wv[kPer];
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const uint32_t i = min(tid + k * T, n4 - 1);
    xv[k] = in.load(x4, i);
    if (NORM) wv[k] = w4[i];
  }
  // The deferred attention splits' count (only SplitIn reads it).
  uint32_t in_splits = 0;
  if constexpr (!std::is_same_v<In, PlainIn>) in_splits = *in.a.dpos / in.a.kps + 1;
  // Keep the compiler from moving these loads behind the weights.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // What the storing lanes read (a residual row, a conv channel's taps and
  // history): the lane or thread that stores item k loads it now too.
  constexpr bool kPreload = P::kPre;
  using Pre = typename PreOf<P>::type;
  Pre pre{};
  const uint32_t pre_k = LPR <= 64 ? (uint32_t)li : (uint32_t)tid;  // the item this lane stores
  if constexpr (kPreload) {
    const uint32_t item = LPR <= 64 ? begin + g + pre_k * G : begin + pre_k;
    pre = p.preload(min(item, end - 1));
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  typename F::Raw raw[MAXI * R];
#pragma unroll
  for (int k = 0; k < MAXI; k++) {
    const uint32_t item = min(begin + g + k * G, end - 1);
#pragma unroll
    for (int j = 0; j < R; j++) raw[k * R + j] = F::fetch(p.row(item, j), unit);
  }

  // 2. The input, times the norm weights, staged in LDS (padded unit slots).
  constexpr uint32_t kPad = F::kUnit >= 64 ? 4 : 0;
  constexpr uint32_t kSlot = F::kUnit + kPad;
  extern __shared__ float4 xs4[];
  float *xs = reinterpret_cast<float *>(xs4);
  // Branch-free as well, so the input loads stay where they were issued:
  // a clamped duplicate writes the same value to the same place and adds
  // nothing to the sum of squares.
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const uint32_t i = tid + k * T, ic = min(i, n4 - 1);
    float4 v = in.finish(xv[k], in_splits);
    if (NORM) {
      const float q = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, v.w * v.w)));
      ss += i < n4 ? q : 0.f;
      v.x *= wv[k].x, v.y *= wv[k].y, v.z *= wv[k].z, v.w *= wv[k].w;
    }
    const uint32_t e = 4 * ic;
    *reinterpret_cast<float4 *>(xs + (e / F::kUnit) * kSlot + e % F::kUnit) = v;
  }
  __shared__ float ss_s[T / 64];
  if (NORM) {
    ss = wave_sum(ss);
    if (tid % 64 == 0) ss_s[tid / 64] = ss;
  }
  lds_barrier();
  if constexpr (kDigitsOf<F>) {
    digitize_units<T, kSlot, (8 * LPR + T - 1) / T>(xs, n_units);
    lds_barrier();
  }
  typename F::Frag f;
  F::from_lds(xs + unit * kSlot, f);
  float scale = 1.f;
  if (NORM) {
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < T / 64; w++) ss += ss_s[w];
    scale = rsqrtf(ss / (float)n_cols + eps);  // f32: off the path to the first dot product
  }

  // 3. Dot products, reductions and stores, item by item.
  uint64_t best = 0;
  constexpr int W = LPR > 64 ? LPR / 64 : 1;
  __shared__ float red[(LPR > 64 ? MAXI * R * W : 1)];
#pragma unroll
  for (int k = 0; k < MAXI; k++) {
    const uint32_t item = begin + g + k * G;
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; j++) acc[j] = (active && item < end) ? F::compute(raw[k * R + j], unit, f) : 0.f;
    if constexpr (LPR <= 64) {
#pragma unroll
      for (int j = 0; j < R; j++) acc[j] = group_sum<LPR>(acc[j]);
      if (li == k % LPR && item < end) {
        if constexpr (kPreload) {
          if (pre_k == (uint32_t)k)
            p.store_pre(item, acc, scale, pre);
          else
            p.store(item, acc, scale);
        } else {
          p.store(item, acc, scale);
        }
        if constexpr (P::kArgmax) best = max(best, argmax_key(acc[0] * scale, item));
      }
    } else {
#pragma unroll
      for (int j = 0; j < R; j++) {
        const float t = wave_sum(acc[j]);
        if (tid % 64 == 0) red[(k * R + j) * W + tid / 64] = t;
      }
    }
  }
  if constexpr (LPR > 64) {
    lds_barrier();
    if (tid < MAXI) {
      const uint32_t item = begin + tid;
      if (item < end) {
        float v[R];
#pragma unroll
        for (int j = 0; j < R; j++) {
          float t = 0.f;
#pragma unroll
          for (int w = 0; w < W; w++) t += red[(tid * R + j) * W + w];
          v[j] = t;
        }
        if constexpr (kPreload)
          p.store_pre(item, v, scale, pre);
        else
          p.store(item, v, scale);
        if constexpr (P::kArgmax) best = max(best, argmax_key(v[0] * scale, item));
      }
    }
  }
  if constexpr (P::kArgmax) {
    __shared__ uint64_t best_s[T / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = ((uint64_t)__shfl_xor((uint32_t)(best >> 32), off, 64) << 32) |
                         (uint64_t)__shfl_xor((uint32_t)best, off, 64);
      best = max(best, o);
    }
    if (tid % 64 == 0) best_s[tid / 64] = best;
    lds_barrier();
    if (tid == 0) {
#pragma unroll
      for (int w = 1; w < T / 64; w++) best = max(best, best_s[w]);
      p.partials[blockIdx.x] = best;
    }
  }
}

template <class F, int LPR, int MAXI, bool NORM, class P>
__global__ __launch_bounds__(256) void k_slab(P p, const float *__restrict__ x, const float *__restrict__ nw,
                                              float eps, uint32_t per, uint32_t rem, uint32_t n_units,
                                              uint32_t n_cols) {
  slab_body<F, LPR, MAXI, NORM>(p, x, nw, eps, per, rem, n_units, n_cols, PlainIn{});
}
// The same with the input from an input policy (SplitIn).
template <class F, int LPR, int MAXI, bool NORM, class P, class In>
__global__ __launch_bounds__(256) void k_slab_in(P p, const float *__restrict__ x, const float *__restrict__ nw,
                                                 float eps, uint32_t per, uint32_t rem, uint32_t n_units,
                                                 uint32_t n_cols, In in) {
  slab_body<F, LPR, MAXI, NORM>(p, x, nw, eps, per, rem, n_units, n_cols, in);
}

// Launch with `grid` workgroups; the caller has checked that every group's
// share of its slab is at most MAXI items.
template <class F, int LPR, int MAXI, bool NORM, class P, class In = PlainIn>
static void launch_slab(hipStream_t s, uint32_t grid, const P &p, const float *x, const float *nw, float eps,
                        uint32_t n_items, uint32_t n_units, uint32_t n_cols, const In &in = In{}) {
  const uint32_t per = n_items / grid, rem = n_items % grid;
  constexpr int threads = LPR <= 64 ? 256 : LPR;
  constexpr uint32_t kSlot = F::kUnit + (F::kUnit >= 64 ? 4 : 0);
  const uint32_t lds = n_units * kSlot * 4;
  if constexpr (std::is_same_v<In, PlainIn>) {
    static const bool lds_limit_set =
        hipFuncSetAttribute(reinterpret_cast<const void *>(k_slab<F, LPR, MAXI, NORM, P>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 256 * kSlot * 4) == hipSuccess;
    (void)lds_limit_set;
    k_slab<F, LPR, MAXI, NORM, P><<<grid, threads, lds, s>>>(p, x, nw, eps, per, rem, n_units, n_cols);
  } else {
    static const bool lds_limit_set =
        hipFuncSetAttribute(reinterpret_cast<const void *>(k_slab_in<F, LPR, MAXI, NORM, P, In>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 256 * kSlot * 4) == hipSuccess;
    (void)lds_limit_set;
    k_slab_in<F, LPR, MAXI, NORM, P, In><<<grid, threads, lds, s>>>(p, x, nw, eps, per, rem, n_units, n_cols,
                                                                    in);
  }
}

// Workgroups of a slab launch: two per CU (the measured best; one per CU
// leaves a SIMD a single wave for the arithmetic at the end), or fewer when
// there are fewer item groups than that.
inline uint32_t slab_grid(uint32_t n_items, uint32_t groups, uint32_t n_cus) {
  return std::max(1u, std::min(2 * (n_cus ? n_cus : 256), div_ceil(n_items, groups)));
}
// Items per group for that grid (the largest share of any group).
inline uint32_t slab_maxi(uint32_t n_items, uint32_t groups, uint32_t grid) {
  return div_ceil(div_ceil(n_items, grid), groups);
}

}  // namespace bch
