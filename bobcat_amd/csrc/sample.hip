// Token sampling on the GPU: the CLI's Sampler::sample
// (crates/bobcat-cli/src/sampler.rs:45-112) as one workgroup, so that a
// non-greedy decode also stays inside the captured graph.
//
// Steps, in the reference's (llama.cpp's) order:
//   1. repetition penalty on each distinct token of the last 64, in place;
//   2. temperature <= 0: argmax (ties to the lowest id);
//   3. top-k: a radix select finds the k-th largest logit and a scan-based
//      compaction keeps the k candidates (ties at the threshold by lowest
//      id), at most kMaxCandidates of them;
//   4. the candidates are sorted by logit (bitonic sort in LDS), then
//      softmax at temperature 1, the top-p prefix, the min-p floor, log and
//      softmax at the temperature, and a draw walking the sorted candidates.
// When more than kMaxCandidates candidates survive top-k (top_k = 0 keeps
// the whole vocabulary), nothing is sorted: every step that walks the
// sorted list (the top-p prefix and the draw) instead finds the rank where
// the cumulative mass crosses its target by a radix descent over the logits'
// ordered keys with mass histograms (sample_large below).
// The draw comes from a wyrand generator whose 64-bit state lives in device
// memory, so graph replays continue the stream.  Sums run as tree
// reductions/scans instead of the reference's sequential loops, so draws
// that land within rounding of a candidate boundary may differ.
#include <cmath>

#include "device.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr uint32_t kSampleThreads = 1024;
constexpr uint32_t kRepeatLastN = 64;  // REPEAT_LAST_N (sampler.rs:8-9)

__device__ __forceinline__ uint32_t ord_key(float v) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0;  // -0 ties +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// wyrand, the generator of fastrand 2 (the reference's Rng): state += c0;
// the 128-bit product state * (state ^ c1) folded to 64 bits.
__device__ __forceinline__ uint64_t wyrand(uint64_t *state) {
  const uint64_t s = *state + 0x2d358dccaa6c78a5ull;
  *state = s;
  const uint64_t t = s ^ 0x8bb84b93962eacc9ull;
  const uint64_t lo = s * t, hi = __umul64hi(s, t);
  return lo ^ hi;
}

// fastrand's f32 in [0, 1): 23 high bits of a 32-bit draw as the mantissa of
// a float in [1, 2), minus one.
__device__ __forceinline__ float wyrand_f32(uint64_t *state) {
  const uint32_t u = (uint32_t)wyrand(state);
  return __uint_as_float(0x3f800000u | (u >> 9)) - 1.0f;
}

// The draw of a sampling launch: the generator's next f32, advancing its
// state, or the caller's draw when the launch has no generator.
__device__ __forceinline__ float next_draw(const SampleArgs &a) {
  if (!a.rng) return a.draw;
  uint64_t st = *a.rng;
  const float u = wyrand_f32(&st);
  *a.rng = st;
  return u;
}

// Exclusive prefix sum of one value per thread over the workgroup; `total`
// receives the sum.  Uses shuffles within a wave and LDS across waves.
template <class T>
__device__ T block_scan(T v, T *lds16, T *total) {
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  T incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T o = __shfl_up(incl, off, 64);
    if (lane >= (uint32_t)off) incl += o;
  }
  if (lane == 63) lds16[wave] = incl;
  __syncthreads();
  T base = 0, sum = 0;
  for (uint32_t w = 0; w < kSampleThreads / 64; w++) {
    if (w < wave) base += lds16[w];
    sum += lds16[w];
  }
  __syncthreads();
  *total = sum;
  return base + incl - v;
}

// --- candidates beyond kMaxCandidates ------------------------------------
//
// Candidates are ranked by key descending, then id ascending (the sorted
// order of the reference, whose unstable sort leaves equal logits in an
// unspecified order).  A "cut" (key K, id I) keeps the candidates ranked at
// or before (K, I): key > K, or key == K and id <= I.
struct Cut {
  uint32_t key, id;
};

__device__ __forceinline__ bool before_cut(uint32_t key, uint32_t id, Cut c) {
  return key > c.key || (key == c.key && id <= c.id);
}

// The id of the j-th (0-based) element, in id order, among those with key K
// that pass `pred`; 0xffffffff when there are fewer.  Each thread scans a
// contiguous range, so the order is the id order.
template <class Pred>
__device__ uint32_t nth_tied_id(const float *logits, uint32_t n, uint32_t K, uint32_t j, Pred pred, uint32_t *u16,
                                uint32_t *result) {
  const uint32_t per = (n + kSampleThreads - 1) / kSampleThreads;
  const uint32_t lo = threadIdx.x * per, hi = min(n, lo + per);
  uint32_t cnt = 0;
  for (uint32_t i = lo; i < hi; i++) cnt += ord_key(logits[i]) == K && pred(i);
  if (threadIdx.x == 0) *result = 0xffffffffu;
  uint32_t total;
  const uint32_t base = block_scan<uint32_t>(cnt, u16, &total);
  if (j >= base && j < base + cnt) {
    uint32_t seen = base;
    for (uint32_t i = lo; i < hi; i++)
      if (ord_key(logits[i]) == K && pred(i)) {
        if (seen == j) {
          *result = i;
          break;
        }
        seen++;
      }
  }
  __syncthreads();
  const uint32_t r = *result;
  __syncthreads();
  return r;
}

// A float from its ordered key (the inverse of ord_key).
__device__ __forceinline__ float ord_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Weights are summed in 64-bit fixed point (2^-40 units): integer sums do
// not depend on the order the histogram's atomic adds land in, so a launch
// (and every replay of a captured graph) cuts at the same rank for the same
// inputs.  Weights lie in [0, 1] (probabilities) or are 1 (counts), so a
// sum over up to 2^23 candidates stays below 2^63.
constexpr double kMassOne = 1099511627776.0;  // 2^40
constexpr uint32_t kSampleMaxVocab = 1u << 23;
__device__ __forceinline__ uint64_t mass_fixed(float w) { return __double2ull_rn((double)w * kMassOne); }

// The first rank whose cumulative weight reaches `target` (>= when
// `inclusive`, > otherwise; target in 2^-40 units), among the elements
// passing `pred`, as a cut.  When the total weight never gets there
// (rounding), the cut is the last such element and `found` is false.  A
// radix descent over the 32-bit keys, 8 bits a pass, with weight
// histograms; the elements tied at the final key weigh the same, so the id
// of the crossing one follows by division.
template <class Pred, class Weight>
__device__ Cut mass_cut(const float *logits, uint32_t n, uint64_t target, bool inclusive, Pred pred, Weight weight,
                        uint64_t *bins, uint32_t *u16, uint32_t *sel_s, uint64_t *above_s, bool *found) {
  constexpr uint32_t kNone = 0xffffffffu;
  const uint32_t tid = threadIdx.x;
  uint32_t prefix = 0;
  uint64_t above = 0;  // weight of the keys above the current prefix
  bool reached = true;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (uint32_t i = tid; i < 256; i += kSampleThreads) bins[i] = 0;
    __syncthreads();
    const uint32_t hi_mask = shift == 24 ? 0u : ~0u << (shift + 8);
    for (uint32_t i = tid; i < n; i += kSampleThreads) {
      const float v = logits[i];
      const uint32_t key = ord_key(v);
      if ((key & hi_mask) == (prefix & hi_mask) && pred(i))
        atomicAdd(reinterpret_cast<unsigned long long *>(&bins[(key >> shift) & 255u]),
                  (unsigned long long)mass_fixed(weight(v)));
    }
    __syncthreads();
    if (tid == 0) {
      uint64_t acc = above;
      uint32_t bin = kNone, last = kNone;
      for (int b = 255; b >= 0; b--) {
        if (bins[b] == 0) continue;
        const uint64_t next = acc + bins[b];
        if (inclusive ? next >= target : next > target) {
          bin = (uint32_t)b;
          break;
        }
        acc = next;
        last = (uint32_t)b;
      }
      if (bin == kNone) {
        // Not reached: descend into the last bin with weight, if any.
        sel_s[0] = last;
        sel_s[1] = 0;
        *above_s = last == kNone ? acc : acc - bins[last];
      } else {
        sel_s[0] = bin;
        sel_s[1] = 1;
        *above_s = acc;
      }
    }
    __syncthreads();
    const uint32_t bin = sel_s[0];
    reached = reached && sel_s[1] != 0;
    above = *above_s;
    __syncthreads();
    if (bin == kNone) {  // nothing passes the predicate
      *found = false;
      return Cut{0u, 0u};
    }
    prefix |= bin << shift;
  }
  uint32_t c = 0;
  for (uint32_t i = tid; i < n; i += kSampleThreads) c += ord_key(logits[i]) == prefix && pred(i);
  uint32_t n_tied;
  block_scan<uint32_t>(c, u16, &n_tied);
  uint32_t j = n_tied - 1;
  if (reached) {
    // Ties before the crossing one: each weighs wk, and `above` + f·wk is
    // still short of the target for the f that precede it.
    const uint64_t wk = mass_fixed(weight(ord_value(prefix)));
    const uint64_t rem = target > above ? target - above : 0;
    uint64_t f = 0;
    if (wk > 0) f = inclusive ? (rem > 0 ? (rem - 1) / wk : 0) : rem / wk;
    if (f < (uint64_t)j) j = (uint32_t)f;
  }
  *found = reached;
  const uint32_t id = nth_tied_id(logits, n, prefix, j, pred, u16, sel_s);
  return Cut{prefix, id};
}

__device__ void sample_large(const SampleArgs &a, uint32_t k, uint64_t *bins, uint32_t *u16, float *f16s,
                             uint32_t *sel_s, uint64_t *above_s, uint32_t *token_s) {
  const uint32_t tid = threadIdx.x, n = a.n;
  const float *logits = a.logits;
  // 1. The top-k set as a cut (top_k = 0 or >= n keeps everything).
  Cut topk{0u, 0xffffffffu};
  if (k < n) {
    bool f;
    topk = mass_cut(
        logits, n, (uint64_t)k << 40, true, [](uint32_t) { return true; }, [](float) { return 1.0f; }, bins, u16,
        sel_s, above_s, &f);
  }
  auto in_topk = [&](uint32_t i) { return before_cut(ord_key(logits[i]), i, topk); };
  // 2. Softmax at temperature 1 over the candidates.
  float mx = -INFINITY;
  for (uint32_t i = tid; i < n; i += kSampleThreads)
    if (in_topk(i)) mx = fmaxf(mx, logits[i]);
  mx = block_max<kSampleThreads>(mx, f16s);
  float part = 0.f;
  for (uint32_t i = tid; i < n; i += kSampleThreads)
    if (in_topk(i)) part += expf(logits[i] - mx);
  const float S = block_sum<kSampleThreads>(part, f16s);
  auto prob = [=](float v) { return expf(v - mx) / S; };
  // 3. Top-p: the shortest prefix reaching top_p (all candidates when none does).
  bool reached = false;
  Cut topp = mass_cut(logits, n, mass_fixed(a.top_p), true, in_topk, prob, bins, u16, sel_s, above_s, &reached);
  if (!reached) topp = topk;
  // 4. Min-p: drop candidates below the first one's probability times min_p.
  const float floor_p = (1.0f / S) * a.min_p;
  auto kept = [&](uint32_t i) {
    const float v = logits[i];
    return in_topk(i) && before_cut(ord_key(v), i, topp) && prob(v) >= floor_p;
  };
  // 5. Temperature over the kept log-probabilities, then the draw.
  const float l0 = logf(1.0f / S);
  const float T = a.temperature;
  auto tq = [=](float v) { return expf((logf(expf(v - mx) / S) - l0) / T); };
  float qp = 0.f;
  for (uint32_t i = tid; i < n; i += kSampleThreads)
    if (kept(i)) qp += tq(logits[i]);
  const float Sq = block_sum<kSampleThreads>(qp, f16s);
  __shared__ float draw_s;
  if (tid == 0) draw_s = next_draw(a);
  __syncthreads();
  const float u = draw_s;
  bool got = false;
  const Cut c = mass_cut(logits, n, mass_fixed(u), false, kept, [=](float v) { return tq(v) / Sq; }, bins, u16, sel_s,
                         above_s, &got);
  if (tid == 0) *token_s = c.id;
  __syncthreads();
}

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleArgs a) {
  __shared__ float cval[kMaxCandidates];
  __shared__ uint32_t cidx[kMaxCandidates];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t u16[16];
  __shared__ float f16s[16];
  __shared__ uint64_t k16[16];
  __shared__ uint32_t prefix_s, remain_s, keep_s, token_s;
  __shared__ uint64_t large_bins[256];
  __shared__ uint32_t large_sel[2];
  __shared__ uint64_t large_above;
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const uint32_t n = a.n;
  float *logits = a.logits;
  const uint32_t p = a.dpos ? *a.dpos : 0u;

  // 1. Repetition penalty: each distinct recent token once (sampler.rs:48-64).
  if (fabsf(a.penalty - 1.0f) > 1.1920929e-7f) {
    const uint32_t n_recent = a.dpos ? p + 1 : a.n_recent;
    const uint32_t start = n_recent > kRepeatLastN ? n_recent - kRepeatLastN : 0;
    if (tid < n_recent - start) {
      const uint32_t tok = a.recent[start + tid];
      bool first = true;
      for (uint32_t j = start; j < start + tid; j++) first &= a.recent[j] != tok;
      if (first && tok < n) {
        const float l = logits[tok];
        logits[tok] = l > 0.f ? l / a.penalty : l * a.penalty;
      }
    }
    __syncthreads();
  }

  // 2. Greedy.
  if (a.temperature <= 0.f) {
    uint64_t best = 0;
    for (uint32_t i = tid; i < n; i += kSampleThreads) {
      const uint64_t k = ((uint64_t)ord_key(logits[i]) << 32) | (uint64_t)(0xffffffffu - i);
      best = best > k ? best : k;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = ((uint64_t)__shfl_xor((uint32_t)(best >> 32), off, 64) << 32) |
                         (uint64_t)__shfl_xor((uint32_t)best, off, 64);
      best = best > o ? best : o;
    }
    if (lane == 0) k16[wave] = best;
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < 16; w++) best = best > k16[w] ? best : k16[w];
      token_s = 0xffffffffu - (uint32_t)best;
    }
    __syncthreads();
  } else {
    // 3. Candidates: the kc largest logits (radix select of the kc-th).
    const uint32_t k = (a.top_k > 0 && a.top_k < n) ? a.top_k : n;
    if (k > kMaxCandidates) {
      sample_large(a, k, large_bins, u16, f16s, large_sel, &large_above, &token_s);
      goto store;
    }
    const uint32_t kc = k < kMaxCandidates ? k : kMaxCandidates;
    uint32_t prefix = 0, need = kc;  // the threshold's key bits so far, and how many of its bucket to take
    if (kc < n) {
      for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256; i += kSampleThreads) hist[i] = 0;
        __syncthreads();
        const uint32_t hi_mask = shift == 24 ? 0u : ~0u << (shift + 8);
        for (uint32_t i = tid; i < n; i += kSampleThreads) {
          const uint32_t key = ord_key(logits[i]);
          if ((key & hi_mask) == (prefix & hi_mask)) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
          uint32_t acc = 0, bin = 255;
          for (int b = 255; b >= 0; b--) {
            if (acc + hist[b] >= need) {
              bin = (uint32_t)b;
              break;
            }
            acc += hist[b];
          }
          prefix_s = prefix | (bin << shift);
          remain_s = need - acc;
        }
        __syncthreads();
        prefix = prefix_s;
        need = remain_s;
      }
    }
    // Deterministic compaction: thread t scans a contiguous range; keys above
    // the threshold all go in, ties by lowest id until kc are in.
    const uint32_t per = (n + kSampleThreads - 1) / kSampleThreads;
    const uint32_t lo = tid * per, hi = min(n, lo + per);
    uint32_t n_gt = 0, n_eq = 0;
    if (kc < n) {
      for (uint32_t i = lo; i < hi; i++) {
        const uint32_t key = ord_key(logits[i]);
        n_gt += key > prefix;
        n_eq += key == prefix;
      }
    } else {
      n_gt = hi > lo ? hi - lo : 0;
    }
    uint32_t tot_gt, tot_eq;
    const uint32_t base_gt = block_scan<uint32_t>(n_gt, u16, &tot_gt);
    const uint32_t base_eq = block_scan<uint32_t>(n_eq, u16, &tot_eq);
    {
      uint32_t g = base_gt, e = base_eq;
      for (uint32_t i = lo; i < hi; i++) {
        const float v = logits[i];
        const uint32_t key = ord_key(v);
        if (kc >= n || key > prefix) {
          cval[g] = v;
          cidx[g] = i;
          g++;
        } else if (key == prefix) {
          if (tot_gt + e < kc) {
            cval[tot_gt + e] = v;
            cidx[tot_gt + e] = i;
          }
          e++;
        }
      }
    }
    uint32_t m = kc;  // candidates, padded to a power of two for the sort
    uint32_t P = 1;
    while (P < m) P <<= 1;
    for (uint32_t i = m + tid; i < P; i += kSampleThreads) {
      cval[i] = -INFINITY;
      cidx[i] = 0xffffffffu;
    }
    __syncthreads();
    // 4a. Bitonic sort: logit descending, id ascending on ties.
    for (uint32_t size = 2; size <= P; size <<= 1) {
      for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
        for (uint32_t i = tid; i < P; i += kSampleThreads) {
          const uint32_t j = i ^ stride;
          if (j > i) {
            const bool desc = (i & size) == 0;
            const float vi = cval[i], vj = cval[j];
            const uint32_t ii = cidx[i], ij = cidx[j];
            const bool i_first = vi > vj || (vi == vj && ii < ij);
            if (desc != i_first) {
              cval[i] = vj;
              cval[j] = vi;
              cidx[i] = ij;
              cidx[j] = ii;
            }
          }
        }
        __syncthreads();
      }
    }
    // 4b. Softmax at temperature 1 (sampler.rs:82-83, 116-128).
    const float mx = cval[0];
    float sum_part = 0.f;
    for (uint32_t i = tid; i < m; i += kSampleThreads) sum_part += expf(cval[i] - mx);
    const float S = block_sum<kSampleThreads>(sum_part, f16s);
    // Each thread owns a contiguous run of candidates for the scans.
    const uint32_t cper = (m + kSampleThreads - 1) / kSampleThreads;
    const uint32_t c0 = tid * cper, c1 = min(m, c0 + cper);
    float run = 0.f;
    for (uint32_t i = c0; i < c1; i++) run += expf(cval[i] - mx) / S;
    float total;
    float cum = block_scan<float>(run, f16s, &total);
    // Top-p: the shortest prefix reaching top_p; min-p: drop below p0·min_p.
    if (tid == 0) keep_s = m;
    __syncthreads();
    for (uint32_t i = c0; i < c1; i++) {
      cum += expf(cval[i] - mx) / S;
      if (cum >= a.top_p) {
        atomicMin(&keep_s, i + 1);
        break;
      }
    }
    __syncthreads();
    const float floor_p = (1.0f / S) * a.min_p;  // the first candidate's probability times min_p
    for (uint32_t i = tid; i < keep_s; i += kSampleThreads)
      if (expf(cval[i] - mx) / S < floor_p) atomicMin(&keep_s, i);
    __syncthreads();
    const uint32_t keep = keep_s > 0 ? keep_s : 1;
    // 4c. Temperature over the kept log-probabilities, then the draw.
    const float l0 = logf(1.0f / S);
    float qs = 0.f;
    for (uint32_t i = tid; i < keep; i += kSampleThreads) qs += expf((logf(expf(cval[i] - mx) / S) - l0) / a.temperature);
    const float Sq = block_sum<kSampleThreads>(qs, f16s);
    const uint32_t q0 = tid * ((keep + kSampleThreads - 1) / kSampleThreads);
    const uint32_t q1 = min(keep, q0 + (keep + kSampleThreads - 1) / kSampleThreads);
    float qrun = 0.f;
    for (uint32_t i = q0; i < q1; i++) qrun += expf((logf(expf(cval[i] - mx) / S) - l0) / a.temperature) / Sq;
    float qtotal;
    float qcum = block_scan<float>(qrun, f16s, &qtotal);
    __shared__ float draw_s;
    if (tid == 0) {
      draw_s = next_draw(a);
      token_s = cidx[keep - 1];  // the last kept candidate when rounding leaves the draw uncovered
      keep_s = keep;             // reused below as the first index whose cumulative mass passes the draw
    }
    __syncthreads();
    const float u = draw_s;
    for (uint32_t i = q0; i < q1; i++) {
      qcum += expf((logf(expf(cval[i] - mx) / S) - l0) / a.temperature) / Sq;
      if (u < qcum) {
        atomicMin(&keep_s, i);
        break;
      }
    }
    __syncthreads();
    if (tid == 0 && keep_s < keep) token_s = cidx[keep_s];
    __syncthreads();
  }

store:
  if (tid == 0) {
    const uint32_t tok = token_s;
    if (a.dpos) {
      a.out[p + 1] = tok;
      *a.dpos = p + 1;
    } else {
      a.out[0] = tok;
    }
  }
}

void run_sample(hipStream_t s, const SampleArgs &a) { k_sample<<<1, kSampleThreads, 0, s>>>(a); }

}  // namespace bch

using namespace bch;

extern "C" int bch_sample(bch_ctx *ctx, bch_view logits, uint32_t n_vocab, bch_view recent, uint32_t n_recent,
                          const bch_sampling *settings, bch_view rng_state, bch_view out) {
  if (!settings) return fail(BCH_ERR_ARGUMENT, "sample: no settings");
  if (n_vocab == 0) return fail(BCH_ERR_ARGUMENT, "sample: an empty vocabulary");
  if (n_vocab > kSampleMaxVocab) return fail(BCH_ERR_ARGUMENT, "sample: more than 2^23 logits");
  SampleArgs a{};
  BCH_TRY(view_ptr(ctx, "sample", logits, (uint64_t)n_vocab * 4, &a.logits));
  if (n_recent) BCH_TRY(view_ptr(ctx, "sample", recent, (uint64_t)n_recent * 4, &a.recent));
  BCH_TRY(view_ptr(ctx, "sample", rng_state, 8, &a.rng));
  BCH_TRY(view_ptr(ctx, "sample", out, 4, &a.out));
  if (reinterpret_cast<uintptr_t>(a.rng) % 8) return fail(BCH_ERR_ARGUMENT, "sample: the generator state is not 8-byte aligned");
  a.n = n_vocab;
  a.n_recent = n_recent;
  a.temperature = settings->temperature;
  a.top_k = settings->top_k;
  a.top_p = settings->top_p;
  a.min_p = settings->min_p;
  a.penalty = settings->repeat_penalty;
  return launch(ctx, {"sample", 1, n_vocab, 0}, [&](hipStream_t s) { run_sample(s, a); });
}

extern "C" int bch_sample_draw(bch_ctx *ctx, bch_view logits, uint32_t n_vocab, bch_view recent, uint32_t n_recent,
                               const bch_sampling *settings, float u, bch_view out) {
  if (!settings) return fail(BCH_ERR_ARGUMENT, "sample_draw: no settings");
  if (n_vocab == 0) return fail(BCH_ERR_ARGUMENT, "sample_draw: an empty vocabulary");
  if (n_vocab > kSampleMaxVocab) return fail(BCH_ERR_ARGUMENT, "sample_draw: more than 2^23 logits");
  if (!(u >= 0.0f && u < 1.0f)) return fail(BCH_ERR_ARGUMENT, "sample_draw: the draw is outside [0, 1)");
  SampleArgs a{};
  BCH_TRY(view_ptr(ctx, "sample_draw", logits, (uint64_t)n_vocab * 4, &a.logits));
  if (n_recent) BCH_TRY(view_ptr(ctx, "sample_draw", recent, (uint64_t)n_recent * 4, &a.recent));
  BCH_TRY(view_ptr(ctx, "sample_draw", out, 4, &a.out));
  a.rng = nullptr;
  a.draw = u;
  a.n = n_vocab;
  a.n_recent = n_recent;
  a.temperature = settings->temperature;
  a.top_k = settings->top_k;
  a.top_p = settings->top_p;
  a.min_p = settings->min_p;
  a.penalty = settings->repeat_penalty;
  return launch(ctx, {"sample_draw", 1, n_vocab, 0}, [&](hipStream_t s) { run_sample(s, a); });
}
