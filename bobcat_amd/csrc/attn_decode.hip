// Decode attention with the query/key normalisation, rotation and KV-cache
// store folded in: one launch does what Recorder::rotate_and_attend records
// as norm_rope(q) + norm_rope(k -> cache) + convert_half(v -> cache) +
// attention_chunk + attention_combine (crates/bobcat/src/lfm2_metal.rs:
// 1094-1160; kernels norm.metal:43-108, attention.metal:25-120, 489-531).
//
// One workgroup per (query head, split); a split covers up to kKeys consecutive
// positions (256 f16 positions of a 64-wide head, so a few splits for the
// contexts of a chat turn).  One workgroup per query head rather than per KV head spreads the
// arithmetic over four times the CUs; the heads of a group read the same
// K/V rows, mostly from L2.  The position comes from the device counter, so
// the launch replays in a graph; splits past the last position exit at once.
// Each 256-lane workgroup
//   1. issues all its key and value loads at once: coalesced 16-byte chunks,
//      a cache row shared by consecutive lanes, eight chunks of K and eight
//      of V per lane held in registers;
//   2. meanwhile normalises and rotates (the first n_rot elements of) its
//      query head into LDS and, if it owns the newest position, the new key
//      and value (the group's first head also stores them in the cache; no
//      other split reads them);
//   3. scores the keys with a DPP reduction over each row's lanes, takes the
//      softmax, and accumulates P·V from the value registers, reduced by lane
//      moves within a wave and through LDS across waves; waves past the last
//      key skip both;
//   4. scales the output by the sigmoid gate of gated attention when given;
//      with several splits, writes (max, sum, output) partials through
//      device-coherent stores and counts itself in; the last split to arrive
//      combines.  Data cross XCDs via sc1 stores/loads instead of device-scope
//      fences, which would write back the whole L2.
#include <algorithm>
#include <cmath>

#include "device.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kDecThreads = 256;  // 1024 ran 32K-context decode at 779 tok/s, 256 at 805
constexpr int kChunks = 8;       // 16-byte chunks of K (and of V) per thread
constexpr int kKeys = 1024;      // positions per split, at most
constexpr int kHd = 256;         // head size, at most
constexpr uint32_t kXcds = 8;
// Splits up to which the prefill form combines with one thread per element.
constexpr uint32_t kSerialCombine = 8;

// Workgroups of one launch: (head, split) items padded to whole runs of a
// KV group's heads on every XCD (the kernel's item mapping needs that).
static uint32_t attn_decode_grid(const AttnDecodeArgs &a) {
  const uint32_t per = kXcds * (a.n_heads / a.n_kv);
  return (a.n_heads * a.max_splits + per - 1) / per * per;
}


// RMS-normalise one head of `hd` floats at src (scaled by w) and rotate its
// first n_rot elements NeoX-style for `position`, into dst (LDS).  Called by
// one whole wave.
__device__ void norm_rope_wave(const float *src, const float *__restrict__ w, const RopeTable &freqs,
                               uint32_t hd, uint32_t n_rot, float position, float eps, float *dst) {
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
  const float scale = (float)(1.0 / sqrt((double)ss / (double)hd + (double)eps));
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
      sincosf(position * freqs.inv_freq[k], &sn, &cs);
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

// CPR: 16-byte chunks per cache row (head_dim * element size / 16).
// FUSED: one decode query at *dpos with its norm/RoPE and cache store;
// otherwise query z of a prefill batch at first_pos + z, already normalised
// and rotated, with every key already in the cache.
template <bool HALF, int CPR, bool FUSED>
__global__ __launch_bounds__(kDecThreads) void k_attn_decode(AttnDecodeArgs a) {
  constexpr uint32_t kElem = HALF ? 2 : 4;
  constexpr uint32_t kEpc = 16 / kElem;             // elements per chunk
  constexpr uint32_t hd = CPR * kEpc;               // head size
  constexpr uint32_t kRowsPerPass = kDecThreads / CPR;
  constexpr uint32_t kps = kRowsPerPass * kChunks < (uint32_t)kKeys ? kRowsPerPass * kChunks : kKeys;
  constexpr int kWaves = kDecThreads / 64;
  const uint32_t tid = threadIdx.x;
  const uint32_t wave = tid / 64, lane = tid % 64;
  const uint32_t group = a.n_heads / a.n_kv, kv_dim = a.n_kv * hd;
  // Workgroup L goes to XCD L % 8.  Item t = split · n_heads + head numbers
  // the work so that the `group` heads reading one KV head's split are
  // consecutive; runs of `group` items are dealt to the XCDs in turn, so
  // those heads run back to back on one XCD and share its L2 instead of
  // each fetching the split's keys and values from HBM.
  // (The prefill form keeps the plain grid (head, split, query): its many
  // queries fill the chip, and the padded mapping measured slower there.)
  uint32_t head = blockIdx.x, split = blockIdx.y;
  if constexpr (FUSED) {
    const uint32_t L = blockIdx.x, xcd = L % kXcds, k = L / kXcds;
    const uint32_t t = ((k / group) * kXcds + xcd) * group + k % group;
    if (t >= a.n_heads * a.max_splits) return;
    head = t % a.n_heads;
    split = t / a.n_heads;
  }
  const uint32_t kvh = head / group;
  const uint32_t qz = FUSED ? 0u : blockIdx.z;
  const uint32_t pos = FUSED ? *a.dpos : a.first_pos + qz;
  const uint32_t n_keys = pos + 1;
  const uint32_t n_splits = (n_keys + kps - 1) / kps;
  if (split >= n_splits) return;
  const uint32_t k0 = split * kps, k1 = min(k0 + kps, n_keys);
  const uint32_t len = k1 - k0;
  const bool owns_new = FUSED && k1 == n_keys;
  // Chunk i of this thread lies in row tid / CPR + i * kRowsPerPass, at
  // column c (head elements c * kEpc ..), the same column for every chunk.
  // A wave's rows of chunk i start at wave_row0 + i * kRowsPerPass.
  const uint32_t c = tid % CPR, row0 = tid / CPR, wave_row0 = wave * 64 / CPR;

  __shared__ float q_s[hd];
  __shared__ float knew_s[hd], vnew_s[hd];
  __shared__ float p_s[kps];
  __shared__ float red_s[kWaves][hd];
  __shared__ float m_s, l_s;
  __shared__ uint32_t last_s;

  // 1. Every key and value load of the split, issued before anything else.
  uint4 kreg[kChunks], vreg[kChunks];
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    const uint32_t r = row0 + i * kRowsPerPass;
    kreg[i] = vreg[i] = make_uint4(0, 0, 0, 0);
    if (r < len && !(owns_new && k0 + r == pos)) {
      const uint64_t at = ((uint64_t)(k0 + r) * kv_dim + (uint64_t)kvh * hd) * kElem + c * 16;
      kreg[i] = *reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(a.k_cache) + at);
      vreg[i] = *reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(a.v_cache) + at);
    }
  }

  // 2. The query head; the new key and value for the owning split.  Every
  // head of the group rotates the new key for itself; the group's first
  // head also stores key and value in the cache.
  const float position = (float)pos;
  if (wave == 0) {
    const float *qsrc = a.q + (uint64_t)qz * a.q_stride + (uint64_t)head * a.q_head_stride;
    if (FUSED) {
      norm_rope_wave(qsrc, a.q_norm, a.freqs, hd, a.n_rot, position, a.eps, q_s);
    } else {
      for (uint32_t i = lane; i < hd; i += 64) q_s[i] = qsrc[i];
    }
  }
  if (owns_new && wave == 1) {
    norm_rope_wave(a.k + (uint64_t)kvh * hd, a.k_norm, a.freqs, hd, a.n_rot, position, a.eps, knew_s);
    const bool store = head % group == 0;
    for (uint32_t i = lane; i < hd; i += 64) {
      const uint64_t at = (uint64_t)pos * kv_dim + (uint64_t)kvh * hd + i;
      const float kv = knew_s[i], vv = a.v[(uint64_t)kvh * hd + i];
      if (HALF) {
        if (store) {
          static_cast<__half *>(a.k_cache)[at] = __float2half(kv);
          static_cast<__half *>(a.v_cache)[at] = __float2half(vv);
        }
        // Later reads of this position see the rounded values; use them now too.
        knew_s[i] = __half2float(__float2half(kv));
        vnew_s[i] = __half2float(__float2half(vv));
      } else {
        if (store) {
          static_cast<float *>(a.k_cache)[at] = kv;
          static_cast<float *>(a.v_cache)[at] = vv;
        }
        vnew_s[i] = vv;
      }
    }
  }
  __syncthreads();

  // Unpacks a chunk (or the new position's LDS copy) to floats.
  auto unpack = [&](const uint4 &w4, const float *fresh, bool is_new, float *out) {
    if (is_new) {
#pragma unroll
      for (uint32_t j = 0; j < kEpc; j++) out[j] = fresh[c * kEpc + j];
    } else if (HALF) {
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
  };

  // 3. Scores: each lane dots its chunk with the query; the CPR lanes of a
  // row then sum their parts.  Chunks whose wave holds no key are skipped.
  float qf[kEpc];
#pragma unroll
  for (uint32_t j = 0; j < kEpc; j++) qf[j] = q_s[c * kEpc + j];
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    if (wave_row0 + i * kRowsPerPass >= len) break;
    const uint32_t r = row0 + i * kRowsPerPass;
    float kv[kEpc];
    unpack(kreg[i], knew_s, owns_new && k0 + r == pos, kv);
    float part = 0.f;
#pragma unroll
    for (uint32_t j = 0; j < kEpc; j++) part = fmaf(qf[j], kv[j], part);
    part = group_sum<CPR>(part);
    if (c == 0 && r < len) p_s[r] = part * a.scale;
  }
  __syncthreads();

  // 4. Softmax over the split's keys, by the whole workgroup.
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

  // 5. P·V from the value chunks in registers: each lane accumulates its
  // column over its rows, the lanes of one column in a wave combine by lane
  // moves, and the waves through LDS.
  float acc[kEpc];
#pragma unroll
  for (uint32_t j = 0; j < kEpc; j++) acc[j] = 0.f;
#pragma unroll
  for (int i = 0; i < kChunks; i++) {
    if (wave_row0 + i * kRowsPerPass >= len) break;
    const uint32_t r = row0 + i * kRowsPerPass;
    if (r < len) {
      float vv[kEpc];
      unpack(vreg[i], vnew_s, owns_new && k0 + r == pos, vv);
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

  // 6. Output, directly or through the split partials.
  float o = 0.f;
  if (tid < hd) {
#pragma unroll
    for (int w = 0; w < kWaves; w++) o += red_s[w][tid];
  }
  // The output gate of gated attention (qwen35.rs:422-424).
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
  // Hand-off to the last workgroup of this (query, head), by the hardware's
  // ordering rather than release/acquire fences (an agent-scope release
  // writes back the XCD's whole L2: 32K-context decode fell from 805 to 434
  // tok/s with it).  The partials are agent-scope atomic stores, which
  // gfx950 performs write-through at the device coherence point (sc1); the
  // signal fence stops the compiler from sinking them below the wait, and
  // s_waitcnt(0) holds each thread until its stores are acknowledged there.
  // Only then does the barrier let thread 0 count in with a device atomic,
  // and the last workgroup reads the partials with agent-scope atomic loads
  // (sc1, from the coherence point) issued after that atomic returned.
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
  if (FUSED || n_splits > kSerialCombine) {
    const float o_all = combine_partials<kDecThreads>(pp, n_splits, stride, hd);
    if (tid < hd) outp[tid] = o_all * gate;
  } else if (tid < hd) {
    // A prefill query over a short context spans a few splits: one thread
    // per element walks them (long contexts take the workgroup-wide combine).
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

template <bool HALF, bool FUSED>
static void launch_attn_decode(hipStream_t s, const AttnDecodeArgs &a, dim3 grid) {
  switch (a.head_dim * (HALF ? 2 : 4) / 16) {
    case 4: k_attn_decode<HALF, 4, FUSED><<<grid, kDecThreads, 0, s>>>(a); break;
    case 8: k_attn_decode<HALF, 8, FUSED><<<grid, kDecThreads, 0, s>>>(a); break;
    case 16: k_attn_decode<HALF, 16, FUSED><<<grid, kDecThreads, 0, s>>>(a); break;
    case 32: k_attn_decode<HALF, 32, FUSED><<<grid, kDecThreads, 0, s>>>(a); break;
    case 64: k_attn_decode<HALF, 64, FUSED><<<grid, kDecThreads, 0, s>>>(a); break;
    default: break;  // rejected when the driver was created
  }
}

void run_attn_decode(hipStream_t s, const AttnDecodeArgs &a, bool kv_half) {
  dim3 grid(attn_decode_grid(a));
  if (kv_half)
    launch_attn_decode<true, true>(s, a, grid);
  else
    launch_attn_decode<false, true>(s, a, grid);
}

void run_attn_prefill(hipStream_t s, const AttnDecodeArgs &a, bool kv_half, uint32_t n_queries) {
  dim3 grid(a.n_heads, a.max_splits, n_queries);
  if (kv_half)
    launch_attn_decode<true, false>(s, a, grid);
  else
    launch_attn_decode<false, false>(s, a, grid);
}

}  // namespace bch
