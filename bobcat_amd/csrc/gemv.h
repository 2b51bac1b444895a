// x-stationary matrix-vector kernels for decode (the fast path behind
// run_matvec / run_matvec_swiglu / run_matvec3 / run_matvec_conv).
//
// A "group" of LPR lanes spans one whole row: lane i owns unit i of the row
// (formats.h: 64 weights of a Q4_K super-block, 8 of an F16 row, 4 of an
// F32 row) and keeps that unit's inputs in VGPRs for the kernel's life.
// The group then streams RPG items (an item is one output row, or the
// gate/up pair of a SwiGLU row, or the B/C/X rows of a conv channel) with
// the loop fully unrolled, so all of the items' weight loads are in flight
// together; per-item partial sums stay in registers and are reduced once at
// the end (shuffles inside a wave, LDS across the waves of a wide group).
// The workgroup first stages the input in LDS with coalesced loads (times
// the norm weights, with the sum of squares of an RMS norm reduced on the
// way), then every lane takes its unit's fragment from LDS.
//
// LPR is a power of two up to 64 (several groups per wave) or a multiple
// of 64 up to 256 (one group over several waves); rows wider than 256 units
// use the older per-unit kernel in matvec.hip.
#pragma once
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

__device__ __forceinline__ float silu_g(float v) { return v / (1.0f + expf(-v)); }

// --- item policies -----------------------------------------------------
// Each provides kRows (rows per item), row(item, j) and store(item, v[], scale).

// Orderable key of (value, index): larger values win, and among equal values
// the lower index wins (the tie rule of argmax, norm.metal:142-197).
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
  const uint32_t b = __float_as_uint(v) == 0x80000000u ? 0u : __float_as_uint(v);  // -0 ties +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - index);
}

template <bool ACC>
struct PlainItems {
  // Accumulating rows read y[item] with the batch's weights (preload), so
  // the read-modify-write at the end does not wait on memory.
  static constexpr bool kPre = ACC;
  static constexpr int kRows = 1;
  static constexpr bool kArgmax = false;
  const uint8_t *W;
  uint64_t rb;
  float *y;
  struct Pre {
    float y;
  };
  __device__ const uint8_t *row(uint32_t item, int) const { return W + (uint64_t)item * rb; }
  __device__ void store(uint32_t item, const float *v, float scale) const {
    const float t = v[0] * scale;
    y[item] = ACC ? y[item] + t : t;
  }
  __device__ Pre preload(uint32_t item) const { return Pre{y[item]}; }
  __device__ void store_pre(uint32_t item, const float *v, float scale, const Pre &pre) const {
    y[item] = pre.y + v[0] * scale;
  }
};

// Logits: rows stored as PlainItems<false>, plus one argmax partial per
// workgroup, so the next token needs no pass over the logits.
struct ArgmaxItems {
  static constexpr bool kPre = false;
  static constexpr int kRows = 1;
  static constexpr bool kArgmax = true;
  const uint8_t *W;
  uint64_t rb;
  float *y;
  uint64_t *partials;
  __device__ const uint8_t *row(uint32_t item, int) const { return W + (uint64_t)item * rb; }
  __device__ void store(uint32_t item, const float *v, float scale) const { y[item] = v[0] * scale; }
};

struct SwigluItems {
  static constexpr bool kPre = false;
  static constexpr int kRows = 2;
  static constexpr bool kArgmax = false;
  const uint8_t *Wg, *Wu;
  uint64_t rb;
  float *y;
  __device__ const uint8_t *row(uint32_t item, int j) const { return (j ? Wu : Wg) + (uint64_t)item * rb; }
  __device__ void store(uint32_t item, const float *v, float scale) const {
    y[item] = silu_g(v[0] * scale) * (v[1] * scale);
  }
};

// The SwiGLU rows of the experts a token's route picked: item i is row
// i % n_ff of the expert in route slot i / n_ff (gate and up stack the
// experts, n_ff rows each; lfm2.rs:128-142).
struct ExpertSwigluItems {
  static constexpr bool kPre = false;
  static constexpr int kRows = 2;
  static constexpr bool kArgmax = false;
  const uint8_t *Wg, *Wu;
  uint64_t rb;
  const uint32_t *ids;
  uint32_t n_ff;
  float *y;
  __device__ const uint8_t *row(uint32_t item, int j) const {
    const uint32_t slot = item / n_ff;
    const uint64_t r = (uint64_t)ids[slot] * n_ff + (item - slot * n_ff);
    return (j ? Wu : Wg) + r * rb;
  }
  __device__ void store(uint32_t item, const float *v, float scale) const {
    y[item] = silu_g(v[0] * scale) * (v[1] * scale);
  }
};

// The input projections of a Gated DeltaNet token in one launch
// (qwen35.rs:442-462): rows [0, r0) are the q/k/v channels, each followed by
// its causal convolution and SiLU as qwen35.rs:448-462 runs them (history
// [channel][k-1], the oldest first), rows [r0, r0+r1) the output gate z,
// then r2 rows of beta and r2 of alpha (raw; the recurrence gates them).
struct GdnInItems {
  // A q/k/v channel's taps and history are read with the batch's weights.
  static constexpr bool kPre = true;
  static constexpr int kRows = 1;
  static constexpr bool kArgmax = false;
  const uint8_t *Wqkv, *Wz, *Wb, *Wa;
  uint32_t r0, r1, r2;
  uint64_t rb;
  const float *taps;
  float *hist;
  uint32_t ksize;
  float *conv_out, *z, *beta, *alpha;
  __device__ const uint8_t *row(uint32_t item, int) const {
    if (item < r0) return Wqkv + (uint64_t)item * rb;
    if (item < r0 + r1) return Wz + (uint64_t)(item - r0) * rb;
    if (item < r0 + r1 + r2) return Wb + (uint64_t)(item - r0 - r1) * rb;
    return Wa + (uint64_t)(item - r0 - r1 - r2) * rb;
  }
  struct Pre {
    float t[kGdnMaxKernel], h[kGdnMaxKernel - 1];
  };
  __device__ Pre preload(uint32_t item) const {
    Pre pre{};
    if (item < r0) {
      const uint32_t past = ksize - 1;
#pragma unroll
      for (int k = 0; k < (int)kGdnMaxKernel; k++) pre.t[k] = (uint32_t)k < ksize ? taps[(uint64_t)item * ksize + k] : 0.f;
#pragma unroll
      for (int k = 0; k < (int)kGdnMaxKernel - 1; k++) pre.h[k] = (uint32_t)k < past ? hist[(uint64_t)item * past + k] : 0.f;
    }
    return pre;
  }
  // store() with the preloaded taps and history: the same operations in the
  // same order.
  __device__ void store_pre(uint32_t item, const float *v, float scale, const Pre &pre) const {
    const float y = v[0] * scale;
    if (item < r0) {
      const uint32_t past = ksize - 1;
      float *h = hist + (uint64_t)item * past;
      float last = 0.f;
#pragma unroll
      for (int k = 0; k < (int)kGdnMaxKernel; k++)
        if ((uint32_t)k == past) last = pre.t[k];
      float sum = last * y;
#pragma unroll
      for (int j = 0; j < (int)kGdnMaxKernel - 1; j++)
        if ((uint32_t)j < past) sum += pre.t[j] * pre.h[j];
      conv_out[item] = silu_g(sum);
#pragma unroll
      for (int j = 0; j < (int)kGdnMaxKernel - 2; j++)
        if ((uint32_t)j + 1 < past) h[j] = pre.h[j + 1];
      h[past - 1] = y;
    } else if (item < r0 + r1) {
      z[item - r0] = y;
    } else if (item < r0 + r1 + r2) {
      beta[item - r0 - r1] = y;
    } else {
      alpha[item - r0 - r1 - r2] = y;
    }
  }
  __device__ void store(uint32_t item, const float *v, float scale) const {
    const float y = v[0] * scale;
    if (item < r0) {
      const uint32_t past = ksize - 1;
      const float *tp = taps + (uint64_t)item * ksize;
      float *h = hist + (uint64_t)item * past;
      float sum = tp[past] * y;
      for (uint32_t j = 0; j < past; j++) sum += tp[j] * h[j];
      conv_out[item] = silu_g(sum);
      for (uint32_t j = 0; j + 1 < past; j++) h[j] = h[j + 1];
      h[past - 1] = y;
    } else if (item < r0 + r1) {
      z[item - r0] = y;
    } else if (item < r0 + r1 + r2) {
      beta[item - r0 - r1] = y;
    } else {
      alpha[item - r0 - r1 - r2] = y;
    }
  }
};

struct ThreeItems {
  static constexpr bool kPre = false;
  static constexpr int kRows = 1;
  static constexpr bool kArgmax = false;
  const uint8_t *W0, *W1, *W2;
  uint32_t r0, r1;
  uint64_t rb;
  float *y0, *y1, *y2;
  __device__ const uint8_t *row(uint32_t item, int) const {
    if (item < r0) return W0 + (uint64_t)item * rb;
    if (item < r0 + r1) return W1 + (uint64_t)(item - r0) * rb;
    return W2 + (uint64_t)(item - r0 - r1) * rb;
  }
  __device__ void store(uint32_t item, const float *v, float scale) const {
    const float t = v[0] * scale;
    if (item < r0)
      y0[item] = t;
    else if (item < r0 + r1)
      y1[item - r0] = t;
    else
      y2[item - r0 - r1] = t;
  }
};

// The gated short convolution of one channel (matvec.metal:386-454,
// lfm2.rs:456-475) on rows ch, n+ch, 2n+ch of the input projection.
struct ConvItems {
  // The channel's taps and history are read with the batch's weights.
  static constexpr bool kPre = true;
  static constexpr int kMaxTaps = 9;
  static constexpr int kRows = 3;
  static constexpr bool kArgmax = false;
  const uint8_t *W;
  uint64_t rb;
  uint32_t n_embd, ksize;
  const float *taps;
  float *history, *out;
  struct Pre {
    float t[kMaxTaps], h[kMaxTaps - 1];
  };
  __device__ const uint8_t *row(uint32_t ch, int j) const { return W + (uint64_t)(j * n_embd + ch) * rb; }
  __device__ Pre preload(uint32_t ch) const {
    Pre pre;
#pragma unroll
    for (int k = 0; k < kMaxTaps; k++) pre.t[k] = (uint32_t)k < ksize ? taps[(uint64_t)ch * ksize + k] : 0.f;
#pragma unroll
    for (int k = 0; k < kMaxTaps - 1; k++) pre.h[k] = (uint32_t)k + 1 < ksize ? history[k * n_embd + ch] : 0.f;
    return pre;
  }
  // store() with the preloaded taps and history: the same operations in the
  // same order.
  __device__ void store_pre(uint32_t ch, const float *v, float scale, const Pre &pre) const {
    const float b = v[0] * scale, c = v[1] * scale, xin = v[2] * scale;
    const float bx = b * xin;
    float last = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxTaps; k++)
      if ((uint32_t)k + 1 == ksize) last = pre.t[k];
    float sum = last * bx;
#pragma unroll
    for (int k = 0; k < kMaxTaps - 1; k++)
      if ((uint32_t)k + 1 < ksize) sum = fmaf(pre.t[k], pre.h[k], sum);
#pragma unroll
    for (int k = 0; k < kMaxTaps - 2; k++)
      if ((uint32_t)k + 2 < ksize) history[k * n_embd + ch] = pre.h[k + 1];
    history[(ksize - 2) * n_embd + ch] = bx;
    out[ch] = c * sum;
  }
  __device__ void store(uint32_t ch, const float *v, float scale) const {
    const float b = v[0] * scale, c = v[1] * scale, xin = v[2] * scale;
    const float *t = taps + (uint64_t)ch * ksize;
    const float bx = b * xin;
    float sum = t[ksize - 1] * bx;
    for (uint32_t k = 0; k + 1 < ksize; k++) sum = fmaf(t[k], history[k * n_embd + ch], sum);
    for (uint32_t k = 0; k + 2 < ksize; k++) history[k * n_embd + ch] = history[(k + 1) * n_embd + ch];
    history[(ksize - 2) * n_embd + ch] = bx;
    out[ch] = c * sum;
  }
};

// --- the kernel ----------------------------------------------------------

// The preloaded values of a policy with kPre, else nothing.
template <class P, bool = P::kPre>
struct PreOf {
  struct type {};
};
template <class P>
struct PreOf<P, true> {
  using type = typename P::Pre;
};


template <class F>
constexpr bool kDigitsOf = requires { F::kDigits; };

template <int LPR>
__device__ __forceinline__ float group_total(float v, float *lds_scratch, int slot) {
  if constexpr (LPR <= 64) {
    return group_sum<LPR>(v);
  } else {
    // One group per workgroup, LPR/64 waves: reduce in-wave, then in LDS.
    v = wave_sum(v);
    const int wave = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) lds_scratch[slot * (LPR / 64) + wave] = v;
    return 0.f;  // finished by the caller after a barrier
  }
}

template <class F, int LPR, int RPG, bool NORM, class P>
__global__ __launch_bounds__(256) void k_gemv(P p, const float *__restrict__ x, const float *__restrict__ nw,
                                              float eps, uint32_t n_items, uint32_t n_units, uint32_t n_cols) {
  constexpr int T = LPR <= 64 ? 256 : LPR;  // threads per workgroup
  constexpr int G = T / LPR;                // groups per workgroup
  constexpr int R = P::kRows;
  constexpr int N = RPG * R;                // rows per batch
  const int tid = threadIdx.x;
  const int g = tid / LPR, li = tid % LPR;
  const bool active = li < (int)n_units;
  const uint32_t unit = active ? (uint32_t)li : 0u;  // idle lanes read unit 0 and drop it
  const uint32_t n_batches = (n_items + RPG - 1) / RPG;
  const uint32_t stride = gridDim.x * G;
  uint32_t b = blockIdx.x * G + g;

  // Weight loads of a batch: issued ahead of the batch's arithmetic.  The
  // lane that stores item `it` of a batch (lane it, or thread it when a
  // group spans waves) also preloads what its store reads, when the policy
  // asks for it and every lane stores at most one item.
  constexpr bool kPreload = P::kPre && (LPR > 64 || LPR >= RPG);
  using Pre = typename PreOf<P>::type;
  const uint32_t my_item = LPR <= 64 ? (uint32_t)li : (uint32_t)tid;
  typename F::Raw ra[N], rb[N];
  Pre pa{}, pb{};
  auto fetch = [&](typename F::Raw *dst, Pre &pre, uint32_t batch) {
#pragma unroll
    for (int it = 0; it < RPG; it++) {
      const uint32_t item = min(batch * RPG + it, n_items - 1);
#pragma unroll
      for (int j = 0; j < R; j++) dst[it * R + j] = F::fetch(p.row(item, j), unit);
    }
    if constexpr (kPreload)
      if (my_item < (uint32_t)RPG && batch * RPG + my_item < n_items) pre = p.preload(batch * RPG + my_item);
  };
  // The input (times the norm weights) is staged once per workgroup in LDS
  // with coalesced loads, one padded slot of kSlot floats per unit, and each
  // lane then reads its unit's fragment from there.  (Loading each lane's
  // unit straight from memory would make every wave load touch 64 cache
  // lines.)  The x loads go out first and the weight loads right after, so
  // waiting for x does not wait for the weights.
  constexpr uint32_t kPad = F::kUnit >= 64 ? 4 : 0;  // spreads the fragment reads over the LDS banks
  constexpr uint32_t kSlot = F::kUnit + kPad;
  // float4 loads per thread per pass: wide rows (the down projection, 10752
  // inputs over 192 threads) take one pass, so no second round trip.
  constexpr int kPer = LPR > 64 && !NORM ? 16 : 8;
  extern __shared__ float4 xs4[];
  float *xs = reinterpret_cast<float *>(xs4);
  const uint32_t n4 = n_cols / 4;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const float4 *w4 = reinterpret_cast<const float4 *>(nw);
  float ss = 0.f;
  for (uint32_t base = 0; base < n4; base += kPer * T) {
    float4 xv[kPer], wv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const uint32_t i = base + tid + k * T;
      if (i < n4) {
        xv[k] = x4[i];
        if (NORM) wv[k] = w4[i];
      }
    }
    if (base == 0 && b < n_batches) fetch(ra, pa, b);
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const uint32_t i = base + tid + k * T;
      if (i < n4) {
        float4 v = xv[k];
        if (NORM) {
          ss = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
          v.x *= wv[k].x, v.y *= wv[k].y, v.z *= wv[k].z, v.w *= wv[k].w;
        }
        const uint32_t e = 4 * i;
        *reinterpret_cast<float4 *>(xs + (e / F::kUnit) * kSlot + e % F::kUnit) = v;
      }
    }
  }
  __shared__ float ss_s[T / 64];
  if (NORM) {
    ss = wave_sum(ss);
    if (tid % 64 == 0) ss_s[tid / 64] = ss;
  }
  __syncthreads();
  if constexpr (kDigitsOf<F>) {
    // Integer activations (Q4K8): the staged inputs become digit planes in place.
    digitize_units<T, kSlot, (8 * LPR + T - 1) / T>(xs, n_units);
    __syncthreads();
  }
  typename F::Frag f;
  F::from_lds(xs + unit * kSlot, f);
  float scale = 1.f;
  if (NORM) {
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < T / 64; w++) ss += ss_s[w];
    scale = rsqrtf(ss / (float)n_cols + eps);
  }
  constexpr int W = LPR > 64 ? LPR / 64 : 1;
  __shared__ float red[N * W];

  uint64_t best = 0;  // argmax key of the items this lane stored (P::kArgmax)

  // Reduce a batch over the group and store it.
  auto finish = [&](const typename F::Raw *cur, const Pre &pre, uint32_t batch) {
    float acc[N];
#pragma unroll
    for (int i = 0; i < N; i++) acc[i] = active ? F::compute(cur[i], unit, f) : 0.f;
    const uint32_t first = batch * RPG;
    if constexpr (LPR <= 64) {
#pragma unroll
      for (int i = 0; i < N; i++) acc[i] = group_sum<LPR>(acc[i]);
#pragma unroll
      for (int it = 0; it < RPG; it++) {
        if (li == it % LPR && first + it < n_items) {
          float v[R];
#pragma unroll
          for (int j = 0; j < R; j++) v[j] = acc[it * R + j];
          if constexpr (kPreload)
            p.store_pre(first + it, v, scale, pre);
          else
            p.store(first + it, v, scale);
          if constexpr (P::kArgmax) best = max(best, argmax_key(v[0] * scale, first + it));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < N; i++) {
        const float t = wave_sum(acc[i]);
        if (tid % 64 == 0) red[i * W + tid / 64] = t;
      }
      __syncthreads();
      if (tid < RPG && first + tid < n_items) {
        float v[R];
#pragma unroll
        for (int j = 0; j < R; j++) {
          float t = 0.f;
#pragma unroll
          for (int w = 0; w < W; w++) t += red[(tid * R + j) * W + w];
          v[j] = t;
        }
        if constexpr (kPreload)
          p.store_pre(first + tid, v, scale, pre);
        else
          p.store(first + tid, v, scale);
        if constexpr (P::kArgmax) best = max(best, argmax_key(v[0] * scale, first + tid));
      }
      __syncthreads();
    }
  };

  // Ping-pong between two register buffers: the next batch's loads are in
  // flight while the current batch is reduced.
  while (true) {
    if (b >= n_batches) break;
    if (b + stride < n_batches) fetch(rb, pb, b + stride);
    finish(ra, pa, b);
    b += stride;
    if (b >= n_batches) break;
    if (b + stride < n_batches) fetch(ra, pa, b + stride);
    finish(rb, pb, b);
    b += stride;
  }
  if constexpr (P::kArgmax) {
    // One partial per workgroup: the largest key over its lanes.
    __shared__ uint64_t best_s[T / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = ((uint64_t)__shfl_xor((uint32_t)(best >> 32), off, 64) << 32) |
                         (uint64_t)__shfl_xor((uint32_t)best, off, 64);
      best = max(best, o);
    }
    if (tid % 64 == 0) best_s[tid / 64] = best;
    __syncthreads();
    if (tid == 0) {
#pragma unroll
      for (int w = 1; w < T / 64; w++) best = max(best, best_s[w]);
      p.partials[blockIdx.x] = best;
    }
  }
}

// --- host side -------------------------------------------------------------

// Lanes per row for n_units units (0 when the x-stationary path does not apply).
inline int lanes_for(uint32_t n_units) {
  if (n_units > 256) return 0;
  if (n_units <= 64) {
    int l = 4;
    while (l < (int)n_units) l *= 2;
    return l;
  }
  return (int)((n_units + 63) / 64 * 64);
}

// Items per group: enough weight bytes in flight per lane without spilling,
// and enough workgroups to cover the chip.
template <class P>
static int rpg_for(uint32_t n_items, int lpr, uint32_t n_cus) {
  constexpr int R = P::kRows;
  const int groups_per_block = lpr <= 64 ? 256 / lpr : 1;
  // The argmax key costs the registers that keep 4 rows at 2 waves per SIMD.
  int rpg = R == 1 ? (P::kArgmax ? 2 : 4) : R == 2 ? 2 : 1;
  const uint32_t want_blocks = 2 * (n_cus ? n_cus : 256);
  while (rpg > 1 && (uint64_t)n_items < (uint64_t)want_blocks * groups_per_block * rpg) rpg /= 2;
  return rpg;
}

template <class F, int LPR, int RPG, bool NORM, class P>
static void launch_gemv(hipStream_t s, const P &p, const float *x, const float *nw, float eps, uint32_t n_items,
                        uint32_t n_units, uint32_t n_cols) {
  constexpr int threads = LPR <= 64 ? 256 : LPR;
  constexpr int G = threads / LPR;
  // Persistent groups: enough workgroups for `per_cu` per CU, each group
  // walking batches at a stride of the whole grid.
  constexpr uint32_t per_cu = 2;
  const uint32_t n_batches = div_ceil(n_items, RPG);
  uint32_t grid = std::max(1u, std::min(div_ceil(n_batches, G), per_cu * 256));
  if constexpr (P::kArgmax) grid = std::min(grid, kArgmaxPartials);
  // LDS for the staged input: one padded slot per unit (up to 68 KiB).
  constexpr uint32_t kSlot = F::kUnit + (F::kUnit >= 64 ? 4 : 0);
  const uint32_t lds = n_units * kSlot * 4;
  static const bool lds_limit_set =
      hipFuncSetAttribute(reinterpret_cast<const void *>(k_gemv<F, LPR, RPG, NORM, P>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, 256 * kSlot * 4) == hipSuccess;
  (void)lds_limit_set;
  k_gemv<F, LPR, RPG, NORM, P><<<grid, threads, lds, s>>>(p, x, nw, eps, n_items, n_units, n_cols);
}

// Formats outside the headline path (Q8_0, Q4_0, Q5_K, Q6_K) are built for one and
// two items per group only, which keeps the number of kernels down.
template <class F>
constexpr bool kFewBatches = F::kFormat == 8 || F::kFormat == 2 || F::kFormat == 14 || F::kFormat == 13;

// The largest items per group rpg_for picks for a policy.
template <class P>
constexpr int kMaxRpg = P::kRows == 1 ? (P::kArgmax ? 2 : 4) : P::kRows == 2 ? 2 : 1;

template <class F, int LPR, bool NORM, class P>
static void gemv_rpg(hipStream_t s, int rpg, const P &p, const float *x, const float *nw, float eps,
                     uint32_t n_items, uint32_t n_units, uint32_t n_cols) {
  constexpr int kMax = kFewBatches<F> ? std::min(2, kMaxRpg<P>) : kMaxRpg<P>;
  if constexpr (kMax >= 4) {
    if (rpg >= 4) return launch_gemv<F, LPR, 4, NORM>(s, p, x, nw, eps, n_items, n_units, n_cols);
  }
  if constexpr (kMax >= 2) {
    if (rpg >= 2) return launch_gemv<F, LPR, 2, NORM>(s, p, x, nw, eps, n_items, n_units, n_cols);
  }
  launch_gemv<F, LPR, 1, NORM>(s, p, x, nw, eps, n_items, n_units, n_cols);
}

// Which norm modes a policy is built for: the drivers always fuse the RMS
// norm into SwiGLU, the conv and DeltaNet input projections, q/k/v and the
// logits, and never into the experts' rows; other calls take the per-unit
// kernel of matvec.hip.
template <class P>
inline constexpr bool kNormBuilt = true;
template <class P>
inline constexpr bool kPlainBuilt = true;
template <> inline constexpr bool kPlainBuilt<SwigluItems> = false;
template <> inline constexpr bool kPlainBuilt<ConvItems> = false;
template <> inline constexpr bool kPlainBuilt<GdnInItems> = false;
template <> inline constexpr bool kPlainBuilt<ThreeItems> = false;
template <> inline constexpr bool kPlainBuilt<ArgmaxItems> = false;
template <> inline constexpr bool kNormBuilt<ExpertSwigluItems> = false;

template <class F, bool NORM, class P>
static bool gemv_dispatch(hipStream_t s, const P &p, const float *x, const float *nw, float eps, uint32_t n_items,
                          uint32_t n_cols, uint32_t n_cus) {
  if constexpr (NORM ? !kNormBuilt<P> : !kPlainBuilt<P>) {
    return false;
  } else {
  if (n_cols % F::kUnit) return false;  // a row must be whole units
  const uint32_t n_units = n_cols / F::kUnit;
  const int lpr = lanes_for(n_units);
  if (!lpr) return false;
  const int rpg = rpg_for<P>(n_items, lpr, n_cus);
  switch (lpr) {
    case 4: gemv_rpg<F, 4, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 8: gemv_rpg<F, 8, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 16: gemv_rpg<F, 16, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 32: gemv_rpg<F, 32, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 64: gemv_rpg<F, 64, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 128: gemv_rpg<F, 128, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 192: gemv_rpg<F, 192, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    case 256: gemv_rpg<F, 256, NORM>(s, rpg, p, x, nw, eps, n_items, n_units, n_cols); break;
    default: return false;
  }
  return true;
  }
}

template <class P>
static bool gemv_any(hipStream_t s, uint32_t format, const P &p, const float *x, const float *nw, float eps,
                     uint32_t n_items, uint32_t n_cols, uint32_t n_cus) {
  const bool norm = nw != nullptr;
  if (norm ? !kNormBuilt<P> : !kPlainBuilt<P>) return false;
  // Integer activations where a workgroup serves many rows (rows of at most
  // 64 units); for wide rows (the down projection: a few rows per
  // workgroup) converting the staged input costs more than it saves.
  if (format == Q4K::kFormat && n_cols <= 64 * 64)
    return norm ? gemv_dispatch<Q4K8, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<Q4K8, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format == Q4K::kFormat)
    return norm ? gemv_dispatch<Q4K, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<Q4K, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format == F16::kFormat)
    return norm ? gemv_dispatch<F16, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<F16, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format == Q6K::kFormat)
    return norm ? gemv_dispatch<Q6K, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<Q6K, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format == Q5K::kFormat)
    return norm ? gemv_dispatch<Q5K, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<Q5K, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format == Q8_0::kFormat)
    return norm ? gemv_dispatch<Q8_0, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<Q8_0, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format == Q4_0::kFormat)
    return norm ? gemv_dispatch<Q4_0, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
                : gemv_dispatch<Q4_0, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
  if (format != F32::kFormat) return false;
  return norm ? gemv_dispatch<F32, true>(s, p, x, nw, eps, n_items, n_cols, n_cus)
              : gemv_dispatch<F32, false>(s, p, x, nw, eps, n_items, n_cols, n_cus);
}

}  // namespace bch
