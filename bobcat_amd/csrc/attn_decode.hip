// Decode attention with the query/key normalisation, rotation and KV-cache
// store folded in: one launch does what Recorder::rotate_and_attend records
// as norm_rope(q) + norm_rope(k -> cache) + convert_half(v -> cache) +
// attention_chunk + attention_combine (crates/bobcat/src/lfm2_metal.rs:
// 1094-1160; kernels norm.metal:43-108, attention.metal:25-120, 489-531).
//
// k_attn_decode: one workgroup per (KV head, run of HPW query heads of its
// group, split); a split covers up to kKeys consecutive positions (256 f16
// positions of a 64-wide head).  The query heads of a run share every key
// and value load, so the cache is read from HBM once per token and the
// grid at 32K positions (8 KV heads x 128 splits) fits the chip in one
// round of workgroups.  The position comes from the device counter, so the
// launch replays in a graph; splits past the last position exit at once.
// Each 256-lane workgroup
//   1. loads its query heads, the new key and value and the norm weights,
//      then issues all its key and value loads: coalesced 16-byte chunks, a
//      cache row shared by consecutive lanes, eight chunks of K and eight of
//      V per lane held in registers (memory returns in issue order, so the
//      small loads first: the work of step 2 overlaps the cache reads);
//   2. normalises and rotates (the first n_rot elements of) the query heads
//      and, if it owns the newest position, the new key, which the run's
//      first workgroup also stores with the value in the cache (no other
//      split reads them);
//   3. scores the keys for every head with a DPP reduction over each row's
//      lanes, takes each head's softmax, and accumulates P·V from the value
//      registers, reduced by lane moves within a wave and through LDS across
//      waves; waves past the last key skip both;
//   4. scales the output by the sigmoid gate of gated attention when given;
//      with several splits, writes (max, sum, output) partials through
//      device-coherent stores and counts itself in; the last split to arrive
//      combines all of the run's heads.  Data cross XCDs via sc1
//      stores/loads instead of device-scope fences, which would write back
//      the whole L2.
// k_attn_queries: the prefill form, one workgroup per (query head, split,
// query) over keys already in the cache.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "device.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kDecThreads = 256;
constexpr int kChunks = 8;       // 16-byte chunks of K (and of V) per thread
constexpr int kKeys = 1024;      // positions per split, at most
constexpr int kHd = 256;         // head size, at most
// Splits up to which the prefill form combines with one thread per element.
constexpr uint32_t kSerialCombine = 8;

// RMS-normalise one head of `hd` floats at src (scaled by w) and rotate its
// first n_rot elements NeoX-style for `position` (frequencies inv_freq),
// into dst.  Called by one whole wave; every pointer is to LDS (a load from
// global memory here would wait for all of the cache loads in flight).
__device__ __forceinline__ void norm_rope_wave(const float *src, const float *w, const float *inv_freq, uint32_t hd, uint32_t n_rot,
                               float position, float eps, float *dst) {
  const int lane = threadIdx.x % 64;
  float v[kHd / 64];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kHd / 64; j++) {
    const uint32_t i = lane + 64 * j;
    v[j] = i < hd ? src[i] : 0.f;
    ss = fmaf(v[j], v[j], ss);
  }
  ss = wave_sum(ss);
  const float scale = rsqrtf(ss / (float)hd + eps);
#pragma unroll
  for (int j = 0; j < kHd / 64; j++) {
    const uint32_t i = lane + 64 * j;
    if (i < hd) dst[i] = w[i] * (v[j] * scale);
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t half = n_rot / 2;
  float outv[kHd / 64];
#pragma unroll
  for (int j = 0; j < kHd / 64; j++) {
    const uint32_t i = lane + 64 * j;
    outv[j] = i < hd ? dst[i] : 0.f;
    if (i < n_rot) {
      const uint32_t k = i < half ? i : i - half;
      float sn, cs;
      sincosf(position * inv_freq[k], &sn, &cs);
      const float x0 = dst[k], x1 = dst[k + half];
      outv[j] = i < half ? x0 * cs - x1 * sn : x1 * cs + x0 * sn;
    }
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < kHd / 64; j++) {
    const uint32_t i = lane + 64 * j;
    if (i < hd) dst[i] = outv[j];
  }
  __builtin_amdgcn_wave_barrier();
}

// Sum over the lanes of a wave that share lane % CPR; exact in lanes < CPR.
template <int CPR>
__device__ __forceinline__ float column_sum(float v) {
  if constexpr (CPR <= 4) v += dpp<kDppRor4>(v);
  if constexpr (CPR <= 8) v += dpp<kDppRor8>(v);
  if constexpr (CPR <= 16) v += __shfl_xor(v, 16, 64);
  if constexpr (CPR <= 32) v += __shfl_xor(v, 32, 64);
  return v;
}

// Combines the (max, sum, output) partials of one head's n_splits splits
// (split sp at pp + sp·stride: m, l, o[hd]) and returns output element tid
// (tid < hd; 0 elsewhere).  The whole workgroup calls it: the split maxima
// are loaded in parallel, then THREADS / hd groups of threads each sum every
// groups-th split for all hd elements, and the groups are added through LDS,
// so the loads of different splits are in flight together instead of one
// dependent chain per element.
template <int THREADS>
__device__ float combine_partials(const float *pp, uint32_t n_splits, uint32_t stride, uint32_t hd) {
  __shared__ float o_s[THREADS], l_s[THREADS], m_w[THREADS / 64];
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  float M = -INFINITY;
  for (uint32_t sp = tid; sp < n_splits; sp += THREADS) M = fmaxf(M, coherent_load(pp + (uint64_t)sp * stride));
  M = wave_max(M);
  if (lane == 0) m_w[wave] = M;
  __syncthreads();
  M = m_w[0];
#pragma unroll
  for (int w = 1; w < THREADS / 64; w++) M = fmaxf(M, m_w[w]);
  const uint32_t groups = THREADS / hd, grp = tid / hd, e = tid % hd;
  float L = 0.f, O = 0.f;
  for (uint32_t sp = grp; sp < n_splits; sp += groups) {
    const float *p = pp + (uint64_t)sp * stride;
    const float w = expf(coherent_load(p) - M);
    L = fmaf(coherent_load(p + 1), w, L);
    O = fmaf(coherent_load(p + 2 + e), w, O);
  }
  o_s[tid] = O;
  l_s[tid] = L;
  __syncthreads();
  float out = 0.f;
  if (tid < hd) {
    float Os = 0.f, Ls = 0.f;
    for (uint32_t g = 0; g < groups; g++) {
      Os += o_s[g * hd + tid];
      Ls += l_s[g * hd + tid];
    }
    out = Os / Ls;
  }
  __syncthreads();  // o_s, l_s and m_w are reused by the next call
  return out;
}

// fmaf(a, h, c) with h one half of a packed f16 pair.  The f16 value is
// exact in f32; the compiler folds the conversion into the FMA
// (v_fma_mix_f32), one instruction instead of two.
__device__ __forceinline__ float fma_lo(float a, uint32_t pair, float c) {
  return fmaf(a, (float)__builtin_bit_cast(_Float16, (unsigned short)(pair & 0xffffu)), c);
}
__device__ __forceinline__ float fma_hi(float a, uint32_t pair, float c) {
  return fmaf(a, (float)__builtin_bit_cast(_Float16, (unsigned short)(pair >> 16)), c);
}

// acc[j] += w · (element j of a 16-byte cache chunk), j < 16 / element size.
template <bool HALF>
__device__ __forceinline__ void fma_chunk(float w, const uint4 &c4, float *acc) {
  const uint32_t d[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if constexpr (HALF) {
      acc[2 * j] = fma_lo(w, d[j], acc[2 * j]);
      acc[2 * j + 1] = fma_hi(w, d[j], acc[2 * j + 1]);
    } else {
      acc[j] = fmaf(w, __uint_as_float(d[j]), acc[j]);
    }
  }
}
// Σ_j q[j] · (element j of a 16-byte cache chunk), in element order.
template <bool HALF>
__device__ __forceinline__ float dot_chunk(const float *q, const uint4 &c4) {
  const uint32_t d[4] = {c4.x, c4.y, c4.z, c4.w};
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if constexpr (HALF) {
      part = fma_lo(q[2 * j], d[j], part);
      part = fma_hi(q[2 * j + 1], d[j], part);
    } else {
      part = fmaf(q[j], __uint_as_float(d[j]), part);
    }
  }
  return part;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
// Buffer view of the split partials for loads through the device coherence
// point (sc1), like coherent_load but 16 bytes at a time.  Buffer loads are
// instructions the compiler knows and waits for (an inline-asm load is not:
// the compiler may reuse its destination registers before the data lands).
// Word 3 is the gfx9 raw-buffer format (32-bit data); loads past `bytes`
// return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t partials_rsrc(const float *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, bytes, 0x00020000);
}
constexpr int kCachePolicySc1 = 16;  // the sc1 bit of a buffer instruction's cache policy
__device__ __forceinline__ f32x4 coherent_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, kCachePolicySc1);
}

// Chunk of 16 bytes (kEpc elements) of a cache row, as floats.
template <bool HALF>
__device__ __forceinline__ void unpack_chunk(const uint4 &w4, float *out) {
  if constexpr (HALF) {
    const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      out[2 * j] = half_bits_to_float(w[j] & 0xffffu);
      out[2 * j + 1] = half_bits_to_float(w[j] >> 16);
    }
  } else {
    out[0] = __uint_as_float(w4.x);
    out[1] = __uint_as_float(w4.y);
    out[2] = __uint_as_float(w4.z);
    out[3] = __uint_as_float(w4.w);
  }
}

// Sum over the row slots of a wave (lanes sharing lane % CPR) of kN values
// per lane, leaving each sum in one lane.  Lane moves within a 16-lane row
// (row slot bits below 4) add every value (DPP rotations); the slot bits 4
// and 5 are butterflies by permlane16/32 swaps, each of which adds two
// values of a lane pair and keeps one of them per lane, halving the values
// held.  On return, lanes with (lane % 16) < CPR hold kN / kStep sums:
// value k of such a lane is the sum of input k · kStep + sel(lane).
template <int CPR, int kN>
struct RowSlotSum {
  static constexpr bool kB4 = CPR <= 16, kB5 = CPR <= 32;
  static constexpr int kStep = (kB4 ? 2 : 1) * (kB5 ? 2 : 1);
  static constexpr int kOut = kN / kStep;
  static __device__ __forceinline__ uint32_t sel(uint32_t lane) {
    const uint32_t b4 = (lane >> 4) & 1, b5 = lane >> 5;
    return (kB4 ? b4 : 0u) + (kB5 ? (kB4 ? 2u : 1u) * b5 : 0u);
  }
  static __device__ __forceinline__ void run(float (&v)[kN], float (&out)[kOut]) {
#pragma unroll
    for (int k = 0; k < kN; k++) {
      if constexpr (CPR <= 4) v[k] += dpp<kDppRor4>(v[k]);
      if constexpr (CPR <= 8) v[k] += dpp<kDppRor8>(v[k]);
    }
    float w[kB4 ? kN / 2 : kN];
    if constexpr (kB4) {
#pragma unroll
      for (int k = 0; k < kN / 2; k++) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[2 * k]), __float_as_uint(v[2 * k + 1]),
                                                         false, false);
        w[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kN; k++) w[k] = v[k];
    }
    constexpr int kW = kB4 ? kN / 2 : kN;
    if constexpr (kB5) {
#pragma unroll
      for (int k = 0; k < kW / 2; k++) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(w[2 * k]), __float_as_uint(w[2 * k + 1]),
                                                         false, false);
        out[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kW; k++) out[k] = w[k];
    }
  }
};

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Query heads per decode workgroup at run time: HPW once the context holds
// more than a.grouped_above keys, else one (more workgroups, each with a
// shorter chain of dependent work).  The bound is where the two layouts
// measured level on one MI355X (32 x 8 heads): ~1,300 keys for 64- and
// 128-wide f16 heads and f32 caches; 256-wide f16 heads, whose splits hold
// only 64 keys, gain nothing measurable in a model's decode step below ~8K.  BCH_ATTN_GROUPED_ABOVE overrides it (0: always
// grouped; for tests).
static uint32_t grouped_above_keys(uint32_t head_dim, bool kv_half) {
  return kv_half && head_dim == 256 ? 8192u : 1280u;
}

// CPR: 16-byte chunks per cache row (head_dim * element size / 16); HPW:
// query heads per workgroup (a divisor of the group) for long contexts.
template <bool HALF, int CPR, int HPW>
__device__ __forceinline__ void attn_decode_body(const AttnDecodeArgs &a) {
  constexpr uint32_t kElem = HALF ? 2 : 4;
  constexpr uint32_t kEpc = 16 / kElem;  // elements per chunk
  constexpr uint32_t hd = CPR * kEpc;    // head size
  constexpr uint32_t kRowsPerPass = kDecThreads / CPR;
  constexpr uint32_t kps = kRowsPerPass * kChunks < (uint32_t)kKeys ? kRowsPerPass * kChunks : kKeys;
  constexpr int kWaves = kDecThreads / 64;
  static_assert(HPW <= 4, "p_s holds four heads per key");
  // f16 caches score the keys on the matrix cores: per wave kTiles tiles of
  // 16 keys, each kSteps MFMAs deep (32 head elements per step).
  constexpr uint32_t kSteps = CPR / 4, kTiles = HALF ? kChunks / kSteps : 0;
  static_assert(!HALF || kTiles * 16 * kWaves == kps, "MFMA tiles cover the split");
  // Staged inputs: HPW query heads, the new key, the new value, the query
  // and key norm weights (and, apart, the rotation frequencies).
  constexpr uint32_t kStage = (HPW + 4) * hd;
  constexpr int kSt = (kStage + kDecThreads - 1) / kDecThreads;
  constexpr uint32_t kOutMax = HPW * hd;  // output elements of a workgroup, at most
  constexpr int kOutPer = (kOutMax + kDecThreads - 1) / kDecThreads;
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid / 64, lane = tid % 64;
  const uint32_t group = a.n_heads / a.n_kv, kv_dim = a.n_kv * hd;
  const uint32_t pos = *a.dpos;
  const uint32_t n_keys = pos + 1;
  const uint32_t n_splits = (n_keys + kps - 1) / kps;
  const uint32_t hpw = HPW > 1 && n_keys > a.grouped_above ? (uint32_t)HPW : 1u;
  const uint32_t units = a.n_heads / hpw;
  const uint32_t split = blockIdx.x / units, head0 = blockIdx.x % units * hpw;
  if (split >= n_splits) return;
  const uint32_t kvh = head0 / group;
  const bool first_of_group = head0 % group == 0;
  const uint32_t n_out = hpw * hd;
  const uint32_t k0 = split * kps, len = min(k0 + kps, n_keys) - k0;
  const bool owns_new = k0 + len == n_keys;
  // Value chunk i of this thread lies in row tid / CPR + i * kRowsPerPass,
  // at column c (head elements c * kEpc ..), the same column for every
  // chunk; a wave's rows of chunk i start at wave_row0 + i * kRowsPerPass.
  // Key chunks follow the same layout for f32 caches; for f16 caches key
  // chunk t·kSteps + s holds key row wave·kps/4 + 16t + lane % 16, column
  // lane / 16 + 4s (the B operand of the MFMA).
  const uint32_t c = tid % CPR, row0 = tid / CPR, wave_row0 = wave * 64 / CPR;
  auto key_row = [&](int i) -> uint32_t {
    if constexpr (HALF) return wave * (kps / kWaves) + (i / kSteps) * 16 + lane % 16;
    else return row0 + i * kRowsPerPass;
  };
  auto key_col = [&](int i) -> uint32_t {
    if constexpr (HALF) return lane / 16 + 4 * (i % kSteps);
    else return c;
  };

  __shared__ float stage_s[kSt * kDecThreads];  // kStage used, the rest absorbs clamped duplicates
  __shared__ float freq_s[kDecThreads];
  __shared__ _Float16 qh_s[HALF ? HPW * hd : 1], ql_s[HALF ? HPW * hd : 1];
  __shared__ float4 p_s[kps];  // per key, the scores (then weights) of up to four heads
  __shared__ float red_s[kWaves][kOutMax];
  __shared__ float mw_s[kWaves][HPW], lw_s[kWaves][HPW];
  __shared__ uint32_t last_s;

  // 1. The staged inputs, then every key and value load of the split.  All
  // loads are unconditional (indices clamped into range): a load under a
  // branch makes the compiler's wait counting fall back to waiting for
  // everything, which would hold step 2 until the cache rows arrive.  The
  // new position's row is read as whatever the cache holds and replaced by
  // the staged key and value.
  float st[kSt];
#pragma unroll
  for (int j = 0; j < kSt; j++) {
    const uint32_t f = min(tid + j * kDecThreads, kStage - 1), seg = f / hd, e = f % hd;
    const float *src = seg < HPW        ? a.q + (uint64_t)min(head0 + seg, a.n_heads - 1) * a.q_head_stride + e
                       : seg == HPW     ? a.k + (uint64_t)kvh * hd + e
                       : seg == HPW + 1 ? a.v + (uint64_t)kvh * hd + e
                       : seg == HPW + 2 ? a.q_norm + e
                                        : a.k_norm + e;
    st[j] = *src;
  }
  const float fr = a.freqs.inv_freq[min(tid, 127u)];
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  uint4 kreg[kChunks], vreg[kChunks];
  const uint8_t *kc = static_cast<const uint8_t *>(a.k_cache), *vc = static_cast<const uint8_t *>(a.v_cache);
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    const uint32_t r = min(key_row(i), len - 1);
    kreg[i] = *reinterpret_cast<const uint4 *>(kc + ((uint64_t)(k0 + r) * kv_dim + (uint64_t)kvh * hd) * kElem +
                                               key_col(i) * 16);
  }
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    const uint32_t r = min(row0 + i * kRowsPerPass, len - 1);
    vreg[i] = *reinterpret_cast<const uint4 *>(vc + ((uint64_t)(k0 + r) * kv_dim + (uint64_t)kvh * hd) * kElem + c * 16);
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < kSt; j++) stage_s[tid + j * kDecThreads] = st[j];
  freq_s[tid] = fr;
  lds_barrier();

  // 2. Norm and rotation of the query heads (in place), one wave each, with
  // the f16 high and low parts of each element for the MFMA scores (q = hi
  // + lo to ~22 bits); the new key by the next wave when this split owns
  // it.  The group's first workgroup stores the new key and value in the
  // cache.
  const float position = (float)pos;
  float *const knew_s = stage_s + HPW * hd, *const vnew_s = stage_s + (HPW + 1) * hd;
  const float *const qn_s = stage_s + (HPW + 2) * hd, *const kn_s = stage_s + (HPW + 3) * hd;
  for (uint32_t it = wave; it < hpw + (owns_new ? 1u : 0u); it += kWaves) {
    if (it < hpw) {
      float *qv = stage_s + it * hd;
      norm_rope_wave(qv, qn_s, freq_s, hd, a.n_rot, position, a.eps, qv);
      if constexpr (HALF) {
        for (uint32_t i = lane; i < hd; i += 64) {
          const _Float16 hi = (_Float16)qv[i];
          qh_s[it * hd + i] = hi;
          ql_s[it * hd + i] = (_Float16)(qv[i] - (float)hi);
        }
      }
      continue;
    }
    norm_rope_wave(knew_s, kn_s, freq_s, hd, a.n_rot, position, a.eps, knew_s);
    for (uint32_t i = lane; i < hd; i += 64) {
      const uint64_t at = (uint64_t)pos * kv_dim + (uint64_t)kvh * hd + i;
      const float kv = knew_s[i], vv = vnew_s[i];
      if (HALF) {
        if (first_of_group) {
          static_cast<__half *>(a.k_cache)[at] = __float2half(kv);
          static_cast<__half *>(a.v_cache)[at] = __float2half(vv);
        }
        // Later reads of this position see the rounded values; use them now too.
        knew_s[i] = __half2float(__float2half(kv));
        vnew_s[i] = __half2float(__float2half(vv));
      } else if (first_of_group) {
        static_cast<float *>(a.k_cache)[at] = kv;
        static_cast<float *>(a.v_cache)[at] = vv;
      }
    }
  }
  lds_barrier();

  // The new position's row: its lanes take the staged key and value into
  // their chunk registers (exact: the f16 values were rounded above).
  auto pack_chunk = [&](const float *src) -> uint4 {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if constexpr (HALF)
        w[j] = (uint32_t)__half_as_ushort(__float2half(src[2 * j])) |
               ((uint32_t)__half_as_ushort(__float2half(src[2 * j + 1])) << 16);
      else
        w[j] = __float_as_uint(src[j]);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  };
  if (owns_new) {
    const uint32_t rn = pos - k0;
#pragma unroll
    for (int i = 0; i < kChunks; i++) {
      if (key_row(i) == rn) kreg[i] = pack_chunk(knew_s + key_col(i) * kEpc);
      if (row0 + i * kRowsPerPass == rn) vreg[i] = pack_chunk(vnew_s + c * kEpc);
    }
  }

  // 3. Scores of every key for the workgroup's heads, into p_s[key].
  if constexpr (HALF) {
    // Matrix cores: D[head][key] = Σ_e Q[head][e] · K[key][e] per 16-key
    // tile, with Q (rows = heads; rows past hpw zero) as its f16 high and
    // low parts, two MFMAs per step.  Lane l holds D[4(l/16) + j][l % 16],
    // so lanes 0-15 hold the four heads of key l.
    const uint32_t qrow = lane % 16;
    const bool qlive = qrow < hpw;
    const uint32_t qbase = min(qrow, hpw - 1) * hd + 8 * (lane / 16);
#pragma unroll
    for (uint32_t t = 0; t < kTiles; t++) {
      typedef float f32x4v __attribute__((ext_vector_type(4)));
      f32x4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t st2 = 0; st2 < kSteps; st2++) {
        f16x8 qh = *reinterpret_cast<const f16x8 *>(qh_s + qbase + 32 * st2);
        f16x8 ql = *reinterpret_cast<const f16x8 *>(ql_s + qbase + 32 * st2);
        if (!qlive) qh = ql = (f16x8){};
        const uint4 kv = kreg[t * kSteps + st2];
        f16x8 kb;
        __builtin_memcpy(&kb, &kv, 16);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh, kb, d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql, kb, d, 0, 0, 0);
      }
      if (lane < 16)
        p_s[wave * (kps / kWaves) + t * 16 + lane] = make_float4(d[0] * a.scale, d[1] * a.scale, d[2] * a.scale,
                                                                 d[3] * a.scale);
    }
  } else {
    // Each lane dots its chunk with every head's query; the CPR lanes of a
    // row then sum their parts.  Lane c (mod 4) writes head c's score.
    float qf[HPW][kEpc];
#pragma unroll
    for (int h = 0; h < HPW; h++)
#pragma unroll
      for (uint32_t j = 0; j < kEpc; j++) qf[h][j] = stage_s[min((uint32_t)h, hpw - 1) * hd + c * kEpc + j];
#pragma unroll
    for (int i = 0; i < kChunks; i++) {
      if (wave_row0 + i * kRowsPerPass >= len) break;
      const uint32_t r = row0 + i * kRowsPerPass;
      float sc[HPW];
#pragma unroll
      for (int h = 0; h < HPW; h++) sc[h] = group_sum<CPR>(dot_chunk<HALF>(qf[h], kreg[i])) * a.scale;
      float4 v4 = make_float4(sc[0], HPW > 1 ? sc[HPW > 1 ? 1 : 0] : 0.f, HPW > 2 ? sc[HPW > 2 ? 2 : 0] : 0.f,
                              HPW > 3 ? sc[HPW > 3 ? 3 : 0] : 0.f);
      if (c == 0) p_s[r] = v4;
    }
  }
  lds_barrier();

  // 4-5 for NH heads (the run-time head count, HPW or one): each head's
  // softmax over the split's keys by the whole workgroup, then P·V.
  auto softmax_pv = [&]<int NH>() {
    // 4. Each head's softmax over the split's keys, by the whole workgroup.
    constexpr uint32_t kPer = (kps + kDecThreads - 1) / kDecThreads;
    float e[NH][kPer];
#pragma unroll
    for (uint32_t j = 0; j < kPer; j++) {
      const uint32_t r = min(tid + kDecThreads * j, kps - 1);
      const float4 v4 = p_s[r];
      const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int h = 0; h < NH; h++) e[h][j] = tid + kDecThreads * j < len ? vv[h] : -INFINITY;
    }
#pragma unroll
    for (int h = 0; h < NH; h++) {
      float mx = -INFINITY;
#pragma unroll
      for (uint32_t j = 0; j < kPer; j++) mx = fmaxf(mx, e[h][j]);
      mx = wave_max(mx);
      if (lane == 0) mw_s[wave][h] = mx;
    }
    lds_barrier();
    float sums[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
      float mx = mw_s[0][h];
#pragma unroll
      for (int w = 1; w < kWaves; w++) mx = fmaxf(mx, mw_s[w][h]);
      sums[h] = 0.f;
#pragma unroll
      for (uint32_t j = 0; j < kPer; j++) {
        e[h][j] = expf(e[h][j] - mx);
        sums[h] += e[h][j];
      }
    }
#pragma unroll
    for (uint32_t j = 0; j < kPer; j++) {
      const uint32_t r = tid + kDecThreads * j;
      if (r < kps)
        p_s[r] = make_float4(e[0][j], NH > 1 ? e[NH > 1 ? 1 : 0][j] : 0.f, NH > 2 ? e[NH > 2 ? 2 : 0][j] : 0.f,
                             NH > 3 ? e[NH > 3 ? 3 : 0][j] : 0.f);
    }
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const float sum = wave_sum(sums[h]);
      if (lane == 0) lw_s[wave][h] = sum;
    }
    lds_barrier();
    // 5. P·V from the value chunks in registers: each lane accumulates its
    // column over its rows (weights of keys past the split's end are zero),
    // the row slots of a wave are summed by lane moves, and the waves through
    // LDS.
    constexpr int kN = NH * (int)kEpc;
    float acc[kN];
#pragma unroll
    for (int k = 0; k < kN; k++) acc[k] = 0.f;
#pragma unroll
    for (int i = 0; i < kChunks; i++) {
      if (wave_row0 + i * kRowsPerPass >= len) break;
      const float4 pw = p_s[row0 + i * kRowsPerPass];
      const float pv[4] = {pw.x, pw.y, pw.z, pw.w};
#pragma unroll
      for (int h = 0; h < NH; h++) fma_chunk<HALF>(pv[h], vreg[i], acc + h * kEpc);
    }
    using Rs = RowSlotSum<CPR, kN>;
    float red[Rs::kOut];
    Rs::run(acc, red);
    if (lane % 16 < (uint32_t)CPR) {
      const uint32_t sel = Rs::sel(lane);
#pragma unroll
      for (int k = 0; k < Rs::kOut; k++) {
        const uint32_t idx = k * Rs::kStep + sel, h = idx / kEpc, j = idx % kEpc;
        red_s[wave][h * hd + c * kEpc + j] = red[k];
      }
    }
    lds_barrier();
  };
  if constexpr (HPW == 1) {
    softmax_pv.template operator()<1>();
  } else {
    if (hpw == HPW)
      softmax_pv.template operator()<HPW>();
    else
      softmax_pv.template operator()<1>();
  }
  // Head h's maximum and sum, from the per-wave values in LDS (a register
  // array indexed by a run-time head would go to scratch memory).
  auto head_max = [&](uint32_t h) {
    float m = mw_s[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, mw_s[w][h]);
    return m;
  };
  auto head_sum = [&](uint32_t h) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) l += lw_s[w][h];
    return l;
  };

  // 6. Output, directly or through the split partials (max, sum, pad,
  // pad, output[hd]: 16-byte aligned outputs).  The output gate of gated
  // attention (qwen35.rs:422-424) applies to the combined output.  With
  // few enough splits (deferred) every split, a single one included, only
  // stores its partial: the next launch's staging combines them.
  constexpr uint32_t stride = hd + 4;
  const bool deferred = n_splits <= a.defer_splits;
  float gate[kOutPer];
#pragma unroll
  for (int j = 0; j < kOutPer; j++) {
    const uint32_t f = tid + j * kDecThreads, h = f / hd, el = f % hd;
    gate[j] = 1.0f;
    if (f < n_out) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) o += red_s[w][f];
      if (a.gate) gate[j] = 1.0f / (1.0f + expf(-a.gate[(uint64_t)(head0 + h) * a.gate_head_stride + el]));
      if (n_splits == 1 && !deferred) {
        a.out[(uint64_t)(head0 + h) * hd + el] = o / head_sum(h) * gate[j];
      } else {
        float *pp = a.partials + ((uint64_t)(head0 + h) * a.max_splits + split) * stride;
        coherent_store(pp + 4 + el, o);
        if (el == 0) {
          coherent_store(pp, head_max(h));
          coherent_store(pp + 1, head_sum(h));
        }
      }
    }
  }
  if (n_splits == 1 || deferred) return;
  // Hand-off to the last workgroup of the heads, by the hardware's ordering
  // rather than release/acquire fences (an agent-scope release writes back
  // the XCD's whole L2: 32K-context decode fell from 805 to 434 tok/s with
  // it).  The partials are agent-scope atomic stores, which gfx950 performs
  // write-through at the device coherence point (sc1); the signal fence
  // stops the compiler from sinking them below the wait, and s_waitcnt(0)
  // holds each thread until its stores are acknowledged there.  Only then
  // does the barrier let thread 0 count in with a device atomic, and the
  // last workgroup reads the partials with sc1 loads issued after that
  // atomic returned.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&a.counters[head0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_s = prev == n_splits - 1;
  }
  __syncthreads();
  if (!last_s) return;

  // Combine.  `groups` threads per quad of 4 consecutive outputs, each
  // taking every groups-th split; the groups merge through LDS.  The (max,
  // sum) headers and the output quads of a batch of splits are loaded
  // together and merged with a running maximum (the sums so far rescaled
  // when a batch raises it): one round of loads when each thread's splits
  // fit one batch of kBatchA (short contexts), else batches of kBatchB.
  const uint32_t quads = n_out / 4, groups = quads >= (uint32_t)kDecThreads ? 1u : kDecThreads / quads;
  constexpr uint32_t kBatchA = 8, kBatchB = 12;
  __shared__ f32x4 comb_s[kDecThreads];  // [group][quad]: output quads
  __shared__ float2 cml_s[kDecThreads];  // [group][quad]: (max, sum)
  const bool one_round = n_splits <= groups * kBatchA;
  if (tid < groups * quads) {
    const uint32_t qd = tid % quads, g = tid / quads, h = 4 * qd / hd, el = 4 * qd % hd;
    // One descriptor for the workgroup's heads (uniform: a per-lane
    // descriptor would make the compiler loop over its distinct values).
    const __amdgpu_buffer_rsrc_t rs =
        partials_rsrc(a.partials + (uint64_t)head0 * a.max_splits * stride, hpw * a.max_splits * stride * 4);
    const uint32_t hbase = h * a.max_splits;  // head h's first split
    float M = -INFINITY, L = 0.f;
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    if (one_round) {
      f32x4 hv[kBatchA], ov[kBatchA];
#pragma unroll
      for (uint32_t u = 0; u < kBatchA; u++) {
        const uint32_t at = (hbase + min(g + u * groups, n_splits - 1)) * stride * 4;
        hv[u] = coherent_load4(rs, at);
        ov[u] = coherent_load4(rs, at + 16 + 4 * el);
      }
#pragma unroll
      for (uint32_t u = 0; u < kBatchA; u++) M = fmaxf(M, hv[u].x);  // clamped duplicates change no maximum
#pragma unroll
      for (uint32_t u = 0; u < kBatchA; u++) {
        const float w = g + u * groups < n_splits ? expf(hv[u].x - M) : 0.f;
        L = fmaf(hv[u].y, w, L);
        O.x = fmaf(ov[u].x, w, O.x);
        O.y = fmaf(ov[u].y, w, O.y);
        O.z = fmaf(ov[u].z, w, O.z);
        O.w = fmaf(ov[u].w, w, O.w);
      }
    } else {
      for (uint32_t sp0 = g; sp0 < n_splits; sp0 += kBatchB * groups) {
        float2 mlv[kBatchB];
        f32x4 ov[kBatchB];
#pragma unroll
        for (uint32_t u = 0; u < kBatchB; u++) {
          const uint32_t at = (hbase + min(sp0 + u * groups, n_splits - 1)) * stride * 4;
          const f32x4 hv = coherent_load4(rs, at);
          mlv[u] = make_float2(hv.x, hv.y);
          ov[u] = coherent_load4(rs, at + 16 + 4 * el);
        }
        float Mn = M;
#pragma unroll
        for (uint32_t u = 0; u < kBatchB; u++) Mn = fmaxf(Mn, mlv[u].x);  // clamped duplicates change no maximum
        const float c = expf(M - Mn);  // 0 on the first batch (M = -inf)
        M = Mn;
        L *= c;
        O.x *= c, O.y *= c, O.z *= c, O.w *= c;
#pragma unroll
        for (uint32_t u = 0; u < kBatchB; u++) {
          const float w = sp0 + u * groups < n_splits ? expf(mlv[u].x - M) : 0.f;
          L = fmaf(mlv[u].y, w, L);
          O.x = fmaf(ov[u].x, w, O.x);
          O.y = fmaf(ov[u].y, w, O.y);
          O.z = fmaf(ov[u].z, w, O.z);
          O.w = fmaf(ov[u].w, w, O.w);
        }
      }
    }
    comb_s[g * quads + qd] = O;
    cml_s[g * quads + qd] = make_float2(M, L);
  }
  __syncthreads();
  const float *comb = reinterpret_cast<const float *>(comb_s);
#pragma unroll
  for (int j = 0; j < kOutPer; j++) {
    const uint32_t f = tid + j * kDecThreads, h = f / hd, qd = f / 4;
    if (f >= n_out) break;
    float M = -INFINITY;
    for (uint32_t g = 0; g < groups; g++) M = fmaxf(M, cml_s[g * quads + qd].x);
    float O = 0.f, L = 0.f;
    for (uint32_t g = 0; g < groups; g++) {
      const float2 ml = cml_s[g * quads + qd];
      const float w = expf(ml.x - M);  // 0 for a group without splits (max -inf)
      L = fmaf(ml.y, w, L);
      O = fmaf(comb[g * n_out + f], w, O);
    }
    a.out[(uint64_t)(head0 + h) * hd + f % hd] = O / L * gate[j];
  }
  if (tid == 0) coherent_store(&a.counters[head0], 0u);
}

// The kernel, in two forms: shapes whose body fits 128 registers without
// spilling are held to that (four waves per SIMD: a 32K-context grid of
// 1,024 workgroups resident at once); the others take what they need.
template <bool HALF, int CPR, int HPW>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(4))) void k_attn_decode_w4(
    AttnDecodeArgs a) {
  attn_decode_body<HALF, CPR, HPW>(a);
}
template <bool HALF, int CPR, int HPW>
__global__ __launch_bounds__(kDecThreads) void k_attn_decode(AttnDecodeArgs a) {
  attn_decode_body<HALF, CPR, HPW>(a);
}

// CPR: 16-byte chunks per cache row (head_dim * element size / 16).  Query
// z of a prefill batch sits at first_pos + z, already normalised and
// rotated, with every key already in the cache.
template <bool HALF, int CPR>
__global__ __launch_bounds__(kDecThreads) void k_attn_queries(AttnDecodeArgs a) {
  constexpr uint32_t kElem = HALF ? 2 : 4;
  constexpr uint32_t kEpc = 16 / kElem;  // elements per chunk
  constexpr uint32_t hd = CPR * kEpc;    // head size
  constexpr uint32_t kRowsPerPass = kDecThreads / CPR;
  constexpr uint32_t kps = kRowsPerPass * kChunks < (uint32_t)kKeys ? kRowsPerPass * kChunks : kKeys;
  constexpr int kWaves = kDecThreads / 64;
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid / 64, lane = tid % 64;
  const uint32_t group = a.n_heads / a.n_kv, kv_dim = a.n_kv * hd;
  const uint32_t head = blockIdx.x, split = blockIdx.y, qz = blockIdx.z;
  const uint32_t kvh = head / group;
  const uint32_t pos = a.first_pos + qz;
  const uint32_t n_keys = pos + 1;
  const uint32_t n_splits = (n_keys + kps - 1) / kps;
  if (split >= n_splits) return;
  const uint32_t k0 = split * kps, len = min(k0 + kps, n_keys) - k0;
  const uint32_t c = tid % CPR, row0 = tid / CPR, wave_row0 = wave * 64 / CPR;

  __shared__ float q_s[hd];
  __shared__ float p_s[kps];
  __shared__ float red_s[kWaves][hd];
  __shared__ float m_s, l_s;
  __shared__ uint32_t last_s;

  // Every key and value load of the split, then the query.
  uint4 kreg[kChunks], vreg[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    const uint32_t r = row0 + i * kRowsPerPass;
    kreg[i] = vreg[i] = make_uint4(0, 0, 0, 0);
    if (r < len) {
      const uint64_t at = ((uint64_t)(k0 + r) * kv_dim + (uint64_t)kvh * hd) * kElem + c * 16;
      kreg[i] = *reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(a.k_cache) + at);
      vreg[i] = *reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(a.v_cache) + at);
    }
  }
  const float *qsrc = a.q + (uint64_t)qz * a.q_stride + (uint64_t)head * a.q_head_stride;
  for (uint32_t i = tid; i < hd; i += kDecThreads) q_s[i] = qsrc[i];
  __syncthreads();

  // Scores, one row per CPR lanes.
  float qf[kEpc];
#pragma unroll
  for (uint32_t j = 0; j < kEpc; j++) qf[j] = q_s[c * kEpc + j];
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    if (wave_row0 + i * kRowsPerPass >= len) break;
    const uint32_t r = row0 + i * kRowsPerPass;
    float kv[kEpc];
    unpack_chunk<HALF>(kreg[i], kv);
    float part = 0.f;
#pragma unroll
    for (uint32_t j = 0; j < kEpc; j++) part = fmaf(qf[j], kv[j], part);
    part = group_sum<CPR>(part);
    if (c == 0 && r < len) p_s[r] = part * a.scale;
  }
  __syncthreads();

  // Softmax over the split's keys.
  constexpr uint32_t kPer = (kps + kDecThreads - 1) / kDecThreads;
  float e[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (uint32_t j = 0; j < kPer; j++) {
    const uint32_t r = tid + kDecThreads * j;
    e[j] = r < len ? p_s[r] : -INFINITY;
    mx = fmaxf(mx, e[j]);
  }
  mx = wave_max(mx);
  if (lane == 0) red_s[wave][0] = mx;
  __syncthreads();
  mx = red_s[0][0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) mx = fmaxf(mx, red_s[w][0]);
  float sum = 0.f;
#pragma unroll
  for (uint32_t j = 0; j < kPer; j++) {
    const uint32_t r = tid + kDecThreads * j;
    e[j] = expf(e[j] - mx);
    if (r < len) p_s[r] = e[j];
    sum += e[j];
  }
  sum = wave_sum(sum);
  __syncthreads();  // every wave has read red_s[*][0]
  if (lane == 0) red_s[wave][1] = sum;
  __syncthreads();
  if (tid == 0) {
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) l += red_s[w][1];
    m_s = mx;
    l_s = l;
  }

  // P·V.
  float acc[kEpc];
#pragma unroll
  for (uint32_t j = 0; j < kEpc; j++) acc[j] = 0.f;
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    if (wave_row0 + i * kRowsPerPass >= len) break;
    const uint32_t r = row0 + i * kRowsPerPass;
    if (r < len) {
      float vv[kEpc];
      unpack_chunk<HALF>(vreg[i], vv);
      const float pw = p_s[r];
#pragma unroll
      for (uint32_t j = 0; j < kEpc; j++) acc[j] = fmaf(pw, vv[j], acc[j]);
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < kEpc; j++) acc[j] = column_sum<CPR>(acc[j]);
  __syncthreads();  // red_s is reused
  if (lane < CPR)
#pragma unroll
    for (uint32_t j = 0; j < kEpc; j++) red_s[wave][c * kEpc + j] = acc[j];
  __syncthreads();

  // Output, directly or through the split partials (hand-off as in
  // k_attn_decode).
  float o = 0.f;
  if (tid < hd) {
#pragma unroll
    for (int w = 0; w < kWaves; w++) o += red_s[w][tid];
  }
  const float gate =
      (a.gate && tid < hd)
          ? 1.0f / (1.0f + expf(-a.gate[(uint64_t)qz * a.gate_query_stride + (uint64_t)head * a.gate_head_stride + tid]))
          : 1.0f;
  float *outp = a.out + (uint64_t)qz * a.out_stride + (uint64_t)head * hd;
  const uint32_t slot = qz * a.n_heads + head;  // (query, head) of the partials and counters
  if (n_splits == 1) {
    if (tid < hd) outp[tid] = o / l_s * gate;
    return;
  }
  const uint32_t stride = hd + 2;
  if (tid < hd) {
    float *pp = a.partials + ((uint64_t)slot * a.max_splits + split) * stride;
    coherent_store(pp + 2 + tid, o);
    if (tid == 0) {
      coherent_store(pp, m_s);
      coherent_store(pp + 1, l_s);
    }
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&a.counters[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_s = prev == n_splits - 1;
  }
  __syncthreads();
  if (!last_s) return;
  const float *pp = a.partials + (uint64_t)slot * a.max_splits * stride;
  if (n_splits > kSerialCombine) {
    const float o_all = combine_partials<kDecThreads>(pp, n_splits, stride, hd);
    if (tid < hd) outp[tid] = o_all * gate;
  } else if (tid < hd) {
    // A query over a short context spans a few splits: one thread per
    // element walks them.
    float M = -INFINITY;
    for (uint32_t sp = 0; sp < n_splits; sp++) M = fmaxf(M, coherent_load(pp + sp * stride));
    float L = 0.f, O = 0.f;
    for (uint32_t sp = 0; sp < n_splits; sp++) {
      const float w = expf(coherent_load(pp + sp * stride) - M);
      L = fmaf(coherent_load(pp + sp * stride + 1), w, L);
      O = fmaf(coherent_load(pp + sp * stride + 2 + tid), w, O);
    }
    outp[tid] = O / L * gate;
  }
  if (tid == 0) coherent_store(&a.counters[slot], 0u);
}

uint32_t attn_decode_keys_per_split(uint32_t head_dim, bool kv_half) {
  const uint32_t cpr = head_dim * (kv_half ? 2 : 4) / 16;
  if (head_dim > kHd || head_dim * (kv_half ? 2 : 4) % 16 || cpr < 4 || (cpr & (cpr - 1))) return 0;  // unsupported
  return std::min<uint32_t>(kKeys, kDecThreads / cpr * kChunks);
}

uint32_t attn_decode_max_splits(uint32_t n_ctx, uint32_t head_dim, bool kv_half) {
  const uint32_t kps = attn_decode_keys_per_split(head_dim, kv_half);
  return kps ? (n_ctx + kps - 1) / kps : 0;
}

RopeTable rope_table(float theta, uint32_t n_rot) {
  RopeTable f{};
  for (uint32_t i = 0; i < n_rot / 2 && i < 128; i++) f.inv_freq[i] = 1.0f / powf(theta, (float)(2 * i) / (float)n_rot);
  return f;
}

template <bool HALF, int CPR, int HPW>
static void launch_decode_cpr(hipStream_t s, const AttnDecodeArgs &a, uint32_t grid) {
  if constexpr ((HALF && CPR == 8) || (!HALF && (CPR == 8 || CPR == 16)))
    k_attn_decode_w4<HALF, CPR, HPW><<<grid, kDecThreads, 0, s>>>(a);
  else
    k_attn_decode<HALF, CPR, HPW><<<grid, kDecThreads, 0, s>>>(a);
}

template <bool HALF, int HPW>
static void launch_decode(hipStream_t s, const AttnDecodeArgs &a, uint32_t grid) {
  switch (a.head_dim * (HALF ? 2 : 4) / 16) {
    case 4: launch_decode_cpr<HALF, 4, HPW>(s, a, grid); break;
    case 8: launch_decode_cpr<HALF, 8, HPW>(s, a, grid); break;
    case 16: launch_decode_cpr<HALF, 16, HPW>(s, a, grid); break;
    case 32: launch_decode_cpr<HALF, 32, HPW>(s, a, grid); break;
    case 64:
      if constexpr (!HALF) launch_decode_cpr<HALF, 64, HPW>(s, a, grid);
      break;
    default: break;  // rejected when the driver was created
  }
}

template <bool HALF>
static void launch_queries(hipStream_t s, const AttnDecodeArgs &a, dim3 grid) {
  switch (a.head_dim * (HALF ? 2 : 4) / 16) {
    case 4: k_attn_queries<HALF, 4><<<grid, kDecThreads, 0, s>>>(a); break;
    case 8: k_attn_queries<HALF, 8><<<grid, kDecThreads, 0, s>>>(a); break;
    case 16: k_attn_queries<HALF, 16><<<grid, kDecThreads, 0, s>>>(a); break;
    case 32: k_attn_queries<HALF, 32><<<grid, kDecThreads, 0, s>>>(a); break;
    case 64: k_attn_queries<HALF, 64><<<grid, kDecThreads, 0, s>>>(a); break;
    default: break;  // rejected when the driver was created
  }
}

// Query heads per decode workgroup: four (or two, or one) heads of a group
// share its cache loads; more would hold more registers than a 256-lane
// workgroup keeps with four waves per SIMD.
static uint32_t heads_per_workgroup(uint32_t group) { return group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1; }

void run_attn_decode(hipStream_t s, const AttnDecodeArgs &args, bool kv_half) {
  AttnDecodeArgs a = args;
  const char *env = std::getenv("BCH_ATTN_GROUPED_ABOVE");
  a.grouped_above = env ? (uint32_t)std::strtoul(env, nullptr, 10) : grouped_above_keys(a.head_dim, kv_half);
  // One workgroup per (head, split) covers both layouts: with HPW heads per
  // workgroup the first 1/HPW of the grid works and the rest exits at once.
  const uint32_t hpw = heads_per_workgroup(a.n_heads / a.n_kv);
  const uint32_t grid = a.n_heads * a.max_splits;
  switch (hpw * 2 + (kv_half ? 1 : 0)) {
    case 8: launch_decode<false, 4>(s, a, grid); break;
    case 9: launch_decode<true, 4>(s, a, grid); break;
    case 4: launch_decode<false, 2>(s, a, grid); break;
    case 5: launch_decode<true, 2>(s, a, grid); break;
    case 2: launch_decode<false, 1>(s, a, grid); break;
    default: launch_decode<true, 1>(s, a, grid); break;
  }
}

// The standalone decode entry point's scratch: the position word, the
// n_heads split counters, then (16-byte aligned) the split partials.
constexpr uint64_t kDecodeScratchHeader = 512;  // floats
constexpr uint32_t kDecodeMaxHeads = 256;

__global__ void k_attn_decode_setup(uint32_t *scratch, uint32_t pos, uint32_t n_heads) {
  for (uint32_t i = threadIdx.x; i <= n_heads; i += blockDim.x) scratch[i == 0 ? 0 : 63 + i] = i == 0 ? pos : 0u;
}

void run_attn_prefill(hipStream_t s, const AttnDecodeArgs &a, bool kv_half, uint32_t n_queries) {
  dim3 grid(a.n_heads, a.max_splits, n_queries);
  if (kv_half)
    launch_queries<true>(s, a, grid);
  else
    launch_queries<false>(s, a, grid);
}

}  // namespace bch

using namespace bch;

extern "C" uint64_t bch_attention_decode_scratch_floats(uint32_t n_heads, uint32_t head_dim, uint32_t n_ctx,
                                                        int kv_half) {
  return kDecodeScratchHeader +
         (uint64_t)n_heads * attn_decode_max_splits(n_ctx, head_dim, kv_half != 0) * (head_dim + 4);
}

extern "C" int bch_attention_decode(bch_ctx *ctx, bch_view q, bch_view k, bch_view v, bch_view q_norm,
                                    bch_view k_norm, float eps, float rope_theta, uint32_t n_rot, bch_view k_cache,
                                    bch_view v_cache, int kv_half, bch_view scratch, bch_view out, uint32_t n_heads,
                                    uint32_t n_kv_heads, uint32_t head_dim, uint32_t pos, uint32_t n_ctx) {
  const bool half = kv_half != 0;
  if (n_kv_heads == 0 || n_heads % n_kv_heads || n_heads > kDecodeMaxHeads ||
      attn_decode_keys_per_split(head_dim, half) == 0 || n_rot % 2 || n_rot > head_dim || pos >= n_ctx)
    return fail(BCH_ERR_ATTENTION_LIMITS,
                "attention_decode: heads of 16-byte cache rows of 64 to 1024 bytes (a power of two, at most 256 "
                "elements), KV heads dividing at most %u query heads, an even n_rot up to the head size and a "
                "position inside the context, got %u and %u heads of %u, n_rot %u, position %u of %u",
                kDecodeMaxHeads, n_heads, n_kv_heads, head_dim, n_rot, pos, n_ctx);
  const uint64_t elem = half ? 2 : 4;
  const uint64_t cache_bytes = ((uint64_t)pos + 1) * n_kv_heads * head_dim * elem;
  const float *qp, *kp, *vp, *qnp, *knp;
  void *kcp, *vcp;
  float *sp, *op;
  BCH_TRY(view_ptr(ctx, "attention_decode", q, (uint64_t)n_heads * head_dim * 4, &qp));
  BCH_TRY(view_ptr(ctx, "attention_decode", k, (uint64_t)n_kv_heads * head_dim * 4, &kp));
  BCH_TRY(view_ptr(ctx, "attention_decode", v, (uint64_t)n_kv_heads * head_dim * 4, &vp));
  BCH_TRY(view_ptr(ctx, "attention_decode", q_norm, (uint64_t)head_dim * 4, &qnp));
  BCH_TRY(view_ptr(ctx, "attention_decode", k_norm, (uint64_t)head_dim * 4, &knp));
  BCH_TRY(view_ptr(ctx, "attention_decode", k_cache, cache_bytes, &kcp));
  BCH_TRY(view_ptr(ctx, "attention_decode", v_cache, cache_bytes, &vcp));
  BCH_TRY(view_ptr(ctx, "attention_decode", scratch,
                   bch_attention_decode_scratch_floats(n_heads, head_dim, n_ctx, kv_half) * 4, &sp));
  BCH_TRY(view_ptr(ctx, "attention_decode", out, (uint64_t)n_heads * head_dim * 4, &op));
  if (reinterpret_cast<uintptr_t>(kcp) % 16 || reinterpret_cast<uintptr_t>(vcp) % 16 ||
      reinterpret_cast<uintptr_t>(sp) % 16)
    return fail(BCH_ERR_ARGUMENT, "attention_decode: the caches and the scratch must be 16-byte aligned");
  AttnDecodeArgs a{};
  a.q = qp;
  a.k = kp;
  a.v = vp;
  a.q_norm = qnp;
  a.k_norm = knp;
  a.freqs = rope_table(rope_theta, n_rot);
  a.eps = eps;
  a.scale = 1.0f / sqrtf((float)head_dim);
  a.k_cache = kcp;
  a.v_cache = vcp;
  a.partials = sp + kDecodeScratchHeader;
  a.counters = reinterpret_cast<uint32_t *>(sp) + 64;
  a.out = op;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.head_dim = head_dim;
  a.max_splits = attn_decode_max_splits(n_ctx, head_dim, half);
  a.dpos = reinterpret_cast<const uint32_t *>(sp);
  a.q_head_stride = head_dim;
  a.n_rot = n_rot;
  return launch(ctx, {"attention_decode", 0, 0, 0}, [&](hipStream_t s) {
    k_attn_decode_setup<<<1, 256, 0, s>>>(reinterpret_cast<uint32_t *>(sp), pos, n_heads);
    run_attn_decode(s, a, half);
  });
}
