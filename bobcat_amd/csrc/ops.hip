// Normalisation, rotation, conversion, embedding, argmax and the gated
// short convolution: the counterparts of norm.metal and conv.metal
// (crates/bobcat-metal/src/norm.metal:7-232, conv.metal:9-108) and of their
// launchers in crates/bobcat-metal/src/backend.rs:2034-2140, 2384-2465,
// 2552-2698.
//
// Kernels whose work depends on the sequence position take it as
// `pos + (dpos ? *dpos : 0)`: the op-level API passes dpos = null, while a
// captured decode graph points dpos at a device counter so one graph serves
// every position.
#include <cmath>

#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

__device__ __forceinline__ uint32_t device_pos(uint32_t pos, const uint32_t *dpos) {
  return pos + (dpos ? *dpos : 0u);
}

// rms_norm (norm.metal:7-32): one workgroup of 256 per row.
__global__ __launch_bounds__(256) void k_rms_norm(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ out, uint32_t n, float eps) {
  __shared__ float red[4];
  const float *xr = x + (uint64_t)blockIdx.x * n;
  float *orow = out + (uint64_t)blockIdx.x * n;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
  ss = block_sum<256>(ss, red);
  const float scale = (float)(1.0 / sqrt((double)ss / (double)n + (double)eps));
  for (uint32_t i = threadIdx.x; i < n; i += 256) orow[i] = w[i] * (xr[i] * scale);
}

// norm_rope (norm.metal:43-91): one wave per (head, token); lane i holds
// elements i and i+64 .. of the head.  Per-head RMS norm scaled by `w`,
// then NeoX rotation of the first n_rot elements (i pairs with
// i + n_rot/2, frequency theta^(-2i/n_rot)).  HALF selects an f16
// destination (the KV cache).  dst_pos_stride > 0 moves the destination by
// that many elements per position unit, for a cache slot addressed from
// the device position.
template <bool HALF>
__global__ __launch_bounds__(64) void k_norm_rope(const float *src, void *dst, const float *__restrict__ w,
                                                  uint32_t head_dim, uint32_t pos, const uint32_t *dpos,
                                                  const RopeTable freqs, float eps, uint32_t src_stride,
                                                  uint32_t dst_stride, uint32_t n_rot,
                                                  uint32_t src_head_stride, uint64_t dst_pos_stride) {
  const uint32_t head = blockIdx.x, token = blockIdx.y, lane = threadIdx.x;
  const uint32_t p0 = device_pos(pos, dpos);
  const float *s = src + (uint64_t)token * src_stride + (uint64_t)head * src_head_stride;
  constexpr int kMaxPer = 4;  // head_dim <= 256
  float v[kMaxPer];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPer; j++) {
    const uint32_t i = lane + 64 * j;
    v[j] = i < head_dim ? s[i] : 0.f;
    ss = fmaf(v[j], v[j], ss);
  }
  ss = wave_sum(ss);
  const float scale = (float)(1.0 / sqrt((double)ss / (double)head_dim + (double)eps));
  __shared__ float normed[256];
#pragma unroll
  for (int j = 0; j < kMaxPer; j++) {
    const uint32_t i = lane + 64 * j;
    if (i < head_dim) normed[i] = w[i] * (v[j] * scale);
  }
  __syncthreads();
  const uint64_t base = (uint64_t)token * dst_stride + (uint64_t)head * head_dim + (uint64_t)p0 * dst_pos_stride;
  const uint32_t half_rot = n_rot / 2;
  const float position = (float)(p0 + token);
#pragma unroll
  for (int j = 0; j < kMaxPer; j++) {
    const uint32_t i = lane + 64 * j;
    if (i >= head_dim) continue;
    float out;
    bool write = true;
    if (i < half_rot) {
      const float angle = position * freqs.inv_freq[i];
      float sn, cs;
      sincosf(angle, &sn, &cs);
      const float x0 = normed[i], x1 = normed[i + half_rot];
      out = x0 * cs - x1 * sn;
      const float out2 = x1 * cs + x0 * sn;
      if (HALF) {
        static_cast<__half *>(dst)[base + i] = __float2half(out);
        static_cast<__half *>(dst)[base + i + half_rot] = __float2half(out2);
      } else {
        static_cast<float *>(dst)[base + i] = out;
        static_cast<float *>(dst)[base + i + half_rot] = out2;
      }
      write = false;
    } else if (i < n_rot) {
      write = false;  // written by its partner i - half_rot
    } else {
      out = normed[i];
    }
    if (write) {
      if (HALF)
        static_cast<__half *>(dst)[base + i] = __float2half(out);
      else
        static_cast<float *>(dst)[base + i] = out;
    }
  }
}

// convert_half (norm.metal:101-108); dst_pos_stride as in k_norm_rope.
__global__ void k_convert_half(const float *__restrict__ src, __half *__restrict__ dst, uint32_t n,
                               const uint32_t *dpos, uint64_t dst_pos_stride) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t off = dpos ? (uint64_t)(*dpos) * dst_pos_stride : 0;
  dst[off + i] = __float2half(src[i]);
}

// rows x cols floats from rows src_stride apart to rows dst_stride apart,
// as f16 (half) or f32.
template <bool HALF>
__global__ void k_copy_rows(const float *__restrict__ src, uint32_t src_stride, void *__restrict__ dst,
                            uint32_t dst_stride, uint32_t cols) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
  if (c >= cols) return;
  const float v = src[(uint64_t)r * src_stride + c];
  if (HALF)
    static_cast<__half *>(dst)[(uint64_t)r * dst_stride + c] = __float2half(v);
  else
    static_cast<float *>(dst)[(uint64_t)r * dst_stride + c] = v;
}

__global__ void k_copy(const float *__restrict__ src, float *__restrict__ dst, uint32_t n, const uint32_t *dpos,
                       uint64_t dst_pos_stride) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t off = dpos ? (uint64_t)(*dpos) * dst_pos_stride : 0;
  dst[off + i] = src[i];
}

// embed_q (norm.metal:198-232): rows tokens[t] of the matrix into out[t].
// With dpos, the token list starts at tokens[*dpos].
__global__ void k_embed(uint32_t format, const uint8_t *__restrict__ W, uint64_t row_bytes,
                        const uint32_t *__restrict__ tokens, float *__restrict__ out, uint32_t n_embd,
                        const uint32_t *dpos) {
  const uint32_t t = blockIdx.y;
  const uint32_t tok = tokens[t + (dpos ? *dpos : 0u)];
  const uint8_t *row = W + (uint64_t)tok * row_bytes;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n_embd; i += gridDim.x * blockDim.x)
    out[(uint64_t)t * n_embd + i] = dequant_elem(format, row, i);
}

// argmax (norm.metal:142-197): index of the largest of n floats, ties to
// the lowest index.  One workgroup of 1024.  With dpos, the result goes to
// out[*dpos + 1] (the next token slot) and the counter advances when
// `advance` is set.
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ x, uint32_t *out, uint32_t n,
                                                 uint32_t *dpos, int advance) {
  __shared__ float bv[16];
  __shared__ uint32_t bi[16];
  float best = -INFINITY;
  uint32_t best_i = 0;
  bool found = false;
  for (uint32_t i = threadIdx.x; i < n; i += 1024) {
    const float v = x[i];
    if (!found || v > best) {
      best = v;
      best_i = i;
      found = true;
    }
  }
  if (!found) best_i = 0xffffffffu;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const uint32_t oi = __shfl_xor(best_i, off, 64);
    if (ov > best || (ov == best && oi < best_i)) {
      best = ov;
      best_i = oi;
    }
  }
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int s = 1; s < 16; s++) {
      if (bv[s] > best || (bv[s] == best && bi[s] < best_i)) {
        best = bv[s];
        best_i = bi[s];
      }
    }
    if (best_i == 0xffffffffu) best_i = 0;
    if (dpos) {
      const uint32_t p = *dpos;
      out[p + 1] = best_i;
      if (advance) *dpos = p + 1;
    } else {
      out[0] = best_i;
    }
  }
}

// short_conv (conv.metal:9-35): one thread per channel, tokens in order.
__global__ void k_short_conv(const float *__restrict__ bcx, const float *__restrict__ taps, float *__restrict__ hist,
                             float *__restrict__ out, uint32_t n_embd, uint32_t ksize, uint32_t n_tokens) {
  const uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= n_embd) return;
  const float *t = taps + (uint64_t)ch * ksize;
  for (uint32_t tok = 0; tok < n_tokens; tok++) {
    const float *row = bcx + (uint64_t)tok * 3 * n_embd;
    const float bx = row[ch] * row[2 * n_embd + ch];
    float sum = t[ksize - 1] * bx;
    for (uint32_t k = 0; k + 1 < ksize; k++) sum = fmaf(t[k], hist[k * n_embd + ch], sum);
    for (uint32_t k = 0; k + 2 < ksize; k++) hist[k * n_embd + ch] = hist[(k + 1) * n_embd + ch];
    hist[(ksize - 2) * n_embd + ch] = bx;
    out[(uint64_t)tok * n_embd + ch] = row[n_embd + ch] * sum;
  }
}

// short_conv_batch (conv.metal:45-75): every (channel, token) at once.
__global__ void k_short_conv_batch(const float *__restrict__ bcx, const float *__restrict__ taps,
                                   const float *__restrict__ hist, float *__restrict__ out, uint32_t n_embd,
                                   uint32_t ksize, uint32_t n_tokens) {
  const uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x, tok = blockIdx.y;
  if (ch >= n_embd || tok >= n_tokens) return;
  const float *t = taps + (uint64_t)ch * ksize;
  float sum = 0.f;
  for (uint32_t k = 0; k < ksize; k++) {
    const int src = (int)tok - (int)(ksize - 1 - k);
    float bx;
    if (src >= 0) {
      const float *row = bcx + (uint64_t)src * 3 * n_embd;
      bx = row[ch] * row[2 * n_embd + ch];
    } else {
      bx = hist[(uint32_t)(src + (int)(ksize - 1)) * n_embd + ch];
    }
    sum = fmaf(t[k], bx, sum);
  }
  out[(uint64_t)tok * n_embd + ch] = bcx[(uint64_t)tok * 3 * n_embd + n_embd + ch] * sum;
}

// k_short_conv_batch, k_short_conv_history and the fp16 conversion of the
// output that the out projection's GEMM reads (k_split_hi in matmul.hip) in
// one launch.  Workgroup b takes tokens kConvTokens·b .. +kConvTokens-1
// over every channel (thread tid: channels tid + 1024·c), so it also holds
// each token's largest magnitude.  Only the first workgroup reads the
// history (the ksize-1 positions before the batch, all of them within its
// tokens), and it writes the new history after those reads.  The
// arithmetic is that of the separate kernels, operation for operation.
constexpr uint32_t kConvTokens = 2;
constexpr uint32_t kConvThreads = 1024;

template <int CPT, int KS>
__global__ __launch_bounds__(kConvThreads) void k_short_conv_split(const float *__restrict__ bcx, const float *__restrict__ taps,
                                                         float *__restrict__ hist, float *__restrict__ out,
                                                         uint32_t n_embd, uint32_t n_tokens, _Float16 *__restrict__ H,
                                                         float *__restrict__ unscale) {
  constexpr int TC = kConvTokens, NH = KS - 1, NW = TC + NH;  // window: tokens t0-NH .. t0+TC-1
  constexpr uint32_t NT = kConvThreads;
  __shared__ float red[NT / 64];
  const uint32_t tid = threadIdx.x, t0 = blockIdx.x * TC;
  float v[CPT][TC], mx[TC];
#pragma unroll
  for (int j = 0; j < TC; j++) mx[j] = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; c++) {
    const uint32_t ch = min(tid + NT * c, n_embd - 1);  // (clamped lanes compute and drop)
    // Every load of the channel first: B·X over the window (the history
    // before the batch), C of the tokens, the taps.
    float bx[NW], cv[TC], tp[KS];
#pragma unroll
    for (int i = 0; i < NW; i++) {
      const int src = (int)t0 - NH + i;
      if (src >= 0) {
        const float *r = bcx + (uint64_t)min((uint32_t)src, n_tokens - 1) * 3 * n_embd;
        bx[i] = r[ch] * r[2 * n_embd + ch];
      } else {
        bx[i] = hist[(uint32_t)(src + NH) * n_embd + ch];  // (first workgroup only)
      }
    }
#pragma unroll
    for (int j = 0; j < TC; j++) cv[j] = bcx[(uint64_t)min(t0 + j, n_tokens - 1) * 3 * n_embd + n_embd + ch];
#pragma unroll
    for (int k = 0; k < KS; k++) tp[k] = taps[(uint64_t)ch * KS + k];
#pragma unroll
    for (int j = 0; j < TC; j++) {
      float sum = 0.f;
#pragma unroll
      for (int k = 0; k < KS; k++) sum = fmaf(tp[k], bx[j + k], sum);
      v[c][j] = cv[j] * sum;
      if (tid + NT * c < n_embd && t0 + j < n_tokens) {
        out[(uint64_t)(t0 + j) * n_embd + ch] = v[c][j];
        mx[j] = fmaxf(mx[j], fabsf(v[c][j]));
      }
    }
  }
  if (blockIdx.x == 0) {
    // The new history: B·X of the batch's last NH tokens (the old history
    // where the batch is shorter), written after this workgroup's reads.
#pragma unroll
    for (int c = 0; c < CPT; c++) {
      const uint32_t ch = tid + NT * c;
      if (ch >= n_embd) continue;
      float next[NH];
#pragma unroll
      for (int k = 0; k < NH; k++) {
        const int src = (int)n_tokens - (NH - k);
        if (src >= 0) {
          const float *row = bcx + (uint64_t)src * 3 * n_embd;
          next[k] = row[ch] * row[2 * n_embd + ch];
        } else {
          next[k] = hist[(uint32_t)(src + NH) * n_embd + ch];
        }
      }
#pragma unroll
      for (int k = 0; k < NH; k++) hist[k * n_embd + ch] = next[k];
    }
  }
#pragma unroll
  for (int j = 0; j < TC; j++) {
    const uint32_t tok = t0 + j;
    const float m = block_max<NT>(mx[j], red);
    if (tok >= n_tokens) continue;  // (uniform)
    int ex = 0;
    if (m > 0.f) frexpf(m, &ex);  // m < 2^ex
    const int k2 = max(-100, min(100, 14 - ex));
    const float scale = ldexpf(1.0f, k2);
    if (tid == 0) unscale[tok] = ldexpf(1.0f, -k2);
#pragma unroll
    for (int c = 0; c < CPT; c++) {
      const uint32_t ch = tid + NT * c;
      if (ch < n_embd) H[(uint64_t)tok * n_embd + ch] = (_Float16)(v[c][j] * scale);
    }
  }
}

// short_conv_history (conv.metal:80-108).
__global__ void k_short_conv_history(const float *__restrict__ bcx, float *__restrict__ hist, uint32_t n_embd,
                                     uint32_t ksize, uint32_t n_tokens) {
  const uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= n_embd) return;
  const uint32_t nh = ksize - 1;
  float next[8];
  for (uint32_t k = 0; k < nh; k++) {
    const int src = (int)n_tokens - (int)(nh - k);
    if (src >= 0) {
      const float *row = bcx + (uint64_t)src * 3 * n_embd;
      next[k] = row[ch] * row[2 * n_embd + ch];
    } else {
      next[k] = hist[(uint32_t)(src + (int)nh) * n_embd + ch];
    }
  }
  for (uint32_t k = 0; k < nh; k++) hist[k * n_embd + ch] = next[k];
}

// Greedy selection folded into the decode graph: the logits GEMV leaves one
// (value, index) key per workgroup; these kernels produce and consume them.
__device__ __forceinline__ uint64_t max_key(uint64_t a, uint64_t b) { return a > b ? a : b; }

__global__ __launch_bounds__(1024) void k_argmax_partials(const float *__restrict__ x, uint32_t n,
                                                          uint64_t *__restrict__ partials, uint32_t n_partials) {
  __shared__ uint64_t best_s[16];
  uint64_t best = 0;
  for (uint32_t i = threadIdx.x; i < n; i += 1024) {
    const uint32_t b = __float_as_uint(x[i]) == 0x80000000u ? 0u : __float_as_uint(x[i]);  // -0 ties +0
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    best = max_key(best, ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - i));
  }
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = ((uint64_t)__shfl_xor((uint32_t)(best >> 32), off, 64) << 32) |
                       (uint64_t)__shfl_xor((uint32_t)best, off, 64);
    best = max_key(best, o);
  }
  if (threadIdx.x % 64 == 0) best_s[threadIdx.x / 64] = best;
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < n_partials; i += 1024) partials[i] = 0;
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; w++) best = max_key(best, best_s[w]);
    partials[0] = best;
  }
}

// The token the argmax keys select (generate_stream's per-step readback).
__global__ __launch_bounds__(256) void k_argmax_pick(const uint64_t *__restrict__ partials, uint32_t n_partials,
                                                     uint32_t *out) {
  __shared__ uint64_t best_s[4];
  uint64_t best = 0;
  for (uint32_t i = threadIdx.x; i < n_partials; i += 256) best = max_key(best, partials[i]);
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = ((uint64_t)__shfl_xor((uint32_t)(best >> 32), off, 64) << 32) |
                       (uint64_t)__shfl_xor((uint32_t)best, off, 64);
    best = max_key(best, o);
  }
  if (threadIdx.x % 64 == 0) best_s[threadIdx.x / 64] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++) best = max_key(best, best_s[w]);
    *out = 0xffffffffu - (uint32_t)best;
  }
}

__global__ __launch_bounds__(256) void k_embed_next(uint32_t format, const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                    uint32_t *tokens, float *__restrict__ out, uint32_t n_embd,
                                                    uint32_t *dpos, const uint64_t *__restrict__ partials,
                                                    uint32_t n_partials) {
  __shared__ uint64_t best_s[4];
  __shared__ uint32_t token_s;
  const uint32_t p = *dpos;
  // The first kP keys of each thread are loaded together (one round trip).
  constexpr int kP = 4;
  uint64_t keys[kP];
#pragma unroll
  for (int j = 0; j < kP; j++) {
    const uint32_t i = threadIdx.x + 256 * j;
    keys[j] = i < n_partials ? partials[i] : 0;
  }
  uint64_t best = 0;
#pragma unroll
  for (int j = 0; j < kP; j++) best = max_key(best, keys[j]);
  for (uint32_t i = threadIdx.x + 256 * kP; i < n_partials; i += 256) best = max_key(best, partials[i]);
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = ((uint64_t)__shfl_xor((uint32_t)(best >> 32), off, 64) << 32) |
                       (uint64_t)__shfl_xor((uint32_t)best, off, 64);
    best = max_key(best, o);
  }
  if (threadIdx.x % 64 == 0) best_s[threadIdx.x / 64] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++) best = max_key(best, best_s[w]);
    token_s = 0xffffffffu - (uint32_t)best;
  }
  __syncthreads();
  const uint32_t tok = token_s;
  const uint8_t *row = W + (uint64_t)tok * row_bytes;
  if (format == 12 && n_embd % 256 == 0 && reinterpret_cast<uintptr_t>(row) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    // Q4_K rows eight elements per thread: one 16-byte header load and one
    // 8-byte load of the eight quants (dequant_elem's arithmetic, element
    // by element, so the values are the same bits).
    for (uint32_t c0 = 8 * threadIdx.x; c0 < n_embd; c0 += 8 * 256) {
      const uint8_t *b = row + (c0 / 256) * 144;
      const uint4 h = *reinterpret_cast<const uint4 *>(b);
      const uint32_t i = c0 % 256, j = i / 32, l0 = i % 32;
      const uint2 qq = *reinterpret_cast<const uint2 *>(b + 16 + 32 * (j / 2) + l0);
      auto sbyte = [&](uint32_t k) -> uint32_t {
        const uint32_t w = k < 4 ? h.y : k < 8 ? h.z : h.w;
        return (w >> (8 * (k % 4))) & 0xffu;
      };
      const float d = half_bits_to_float(h.x & 0xffffu);
      const float dmin = half_bits_to_float(h.x >> 16);
      uint32_t sc, mn;
      if (j < 4) {
        sc = sbyte(j) & 63;
        mn = sbyte(j + 4) & 63;
      } else {
        sc = (sbyte(j + 4) & 0xf) | ((sbyte(j - 4) >> 6) << 4);
        mn = (sbyte(j + 4) >> 4) | ((sbyte(j) >> 6) << 4);
      }
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const uint32_t q = ((e < 4 ? qq.x : qq.y) >> (8 * (e % 4))) & 0xffu;
        const uint32_t nib = (j & 1) ? (q >> 4) : (q & 0xf);
        v[e] = __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)nib), __fmul_rn(dmin, (float)mn));
      }
      reinterpret_cast<float4 *>(out + c0)[0] = make_float4(v[0], v[1], v[2], v[3]);
      reinterpret_cast<float4 *>(out + c0)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (threadIdx.x == 0) {
      tokens[p + 1] = tok;
      *dpos = p + 1;  // every thread read p above, before this store
    }
    return;
  }
  if (format == 1 && n_embd % 8 == 0 && reinterpret_cast<uintptr_t>(row) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    // F16 rows eight elements (one 16-byte load) per thread.
    for (uint32_t c0 = 8 * threadIdx.x; c0 < n_embd; c0 += 8 * 256) {
      const uint4 w = *reinterpret_cast<const uint4 *>(row + 2 * (uint64_t)c0);
      reinterpret_cast<float4 *>(out + c0)[0] =
          make_float4(half_bits_to_float(w.x & 0xffffu), half_bits_to_float(w.x >> 16),
                      half_bits_to_float(w.y & 0xffffu), half_bits_to_float(w.y >> 16));
      reinterpret_cast<float4 *>(out + c0)[1] =
          make_float4(half_bits_to_float(w.z & 0xffffu), half_bits_to_float(w.z >> 16),
                      half_bits_to_float(w.w & 0xffffu), half_bits_to_float(w.w >> 16));
    }
    if (threadIdx.x == 0) {
      tokens[p + 1] = tok;
      *dpos = p + 1;  // every thread read p above, before this store
    }
    return;
  }
  // The thread's first kE elements are read before any is stored.
  constexpr int kE = 8;
  float v[kE];
#pragma unroll
  for (int j = 0; j < kE; j++) {
    const uint32_t i = threadIdx.x + 256 * j;
    v[j] = i < n_embd ? dequant_elem(format, row, i) : 0.f;
  }
#pragma unroll
  for (int j = 0; j < kE; j++) {
    const uint32_t i = threadIdx.x + 256 * j;
    if (i < n_embd) out[i] = v[j];
  }
  for (uint32_t i = threadIdx.x + 256 * kE; i < n_embd; i += 256) out[i] = dequant_elem(format, row, i);
  if (threadIdx.x == 0) {
    tokens[p + 1] = tok;
    *dpos = p + 1;  // every thread read p above, before this store
  }
}

// ------------------------------------------------------------------
// Stream-level launchers shared with the model driver.
// ------------------------------------------------------------------

void run_rms_norm(hipStream_t s, const float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps) {
  k_rms_norm<<<rows, 256, 0, s>>>(x, w, out, n, eps);
}

void run_norm_rope(hipStream_t s, const float *src, void *dst, bool half, const float *w, uint32_t n_heads,
                   uint32_t head_dim, uint32_t n_rot, uint32_t src_head_stride, uint32_t pos, const uint32_t *dpos,
                   uint32_t n_tokens, uint32_t src_stride, uint32_t dst_stride, float theta, float eps,
                   uint64_t dst_pos_stride) {
  dim3 grid(n_heads, n_tokens);
  const RopeTable f = rope_table(theta, n_rot);
  if (half)
    k_norm_rope<true><<<grid, 64, 0, s>>>(src, dst, w, head_dim, pos, dpos, f, eps, src_stride, dst_stride, n_rot,
                                          src_head_stride, dst_pos_stride);
  else
    k_norm_rope<false><<<grid, 64, 0, s>>>(src, dst, w, head_dim, pos, dpos, f, eps, src_stride, dst_stride, n_rot,
                                           src_head_stride, dst_pos_stride);
}

void run_convert_half(hipStream_t s, const float *src, void *dst, uint32_t n, const uint32_t *dpos,
                      uint64_t dst_pos_stride) {
  if (n) k_convert_half<<<div_ceil(n, 256), 256, 0, s>>>(src, static_cast<__half *>(dst), n, dpos, dst_pos_stride);
}

void run_copy_rows(hipStream_t s, const float *src, uint32_t src_stride, void *dst, uint32_t dst_stride, bool half,
                   uint32_t cols, uint32_t rows) {
  if (!cols || !rows) return;
  const dim3 grid(div_ceil(cols, 256), rows);
  if (half)
    k_copy_rows<true><<<grid, 256, 0, s>>>(src, src_stride, dst, dst_stride, cols);
  else
    k_copy_rows<false><<<grid, 256, 0, s>>>(src, src_stride, dst, dst_stride, cols);
}

void run_copy(hipStream_t s, const float *src, float *dst, uint32_t n, const uint32_t *dpos, uint64_t dst_pos_stride) {
  if (n) k_copy<<<div_ceil(n, 256), 256, 0, s>>>(src, dst, n, dpos, dst_pos_stride);
}

void run_embed(hipStream_t s, uint32_t format, const uint8_t *W, uint64_t row_bytes, const uint32_t *tokens,
               float *out, uint32_t n_embd, uint32_t n_tokens, const uint32_t *dpos) {
  dim3 grid(div_ceil(n_embd, 256), n_tokens);
  k_embed<<<grid, 256, 0, s>>>(format, W, row_bytes, tokens, out, n_embd, dpos);
}

void run_argmax(hipStream_t s, const float *x, uint32_t *out, uint32_t n, uint32_t *dpos, bool advance) {
  k_argmax<<<1, 1024, 0, s>>>(x, out, n, dpos, advance ? 1 : 0);
}

void run_argmax_pick(hipStream_t s, const uint64_t *partials, uint32_t n_partials, uint32_t *out) {
  k_argmax_pick<<<1, 256, 0, s>>>(partials, n_partials, out);
}

void run_argmax_partials(hipStream_t s, const float *logits, uint32_t n, uint64_t *partials, uint32_t n_partials) {
  k_argmax_partials<<<1, 1024, 0, s>>>(logits, n, partials, n_partials);
}

void run_embed_next(hipStream_t s, uint32_t format, const uint8_t *W, uint64_t row_bytes, uint32_t *tokens,
                    float *out, uint32_t n_embd, uint32_t *dpos, const uint64_t *partials, uint32_t n_partials) {
  k_embed_next<<<1, 256, 0, s>>>(format, W, row_bytes, tokens, out, n_embd, dpos, partials, n_partials);
}

void run_short_conv(hipStream_t s, const float *bcx, const float *taps, float *hist, float *out, uint32_t n_embd,
                    uint32_t ksize, uint32_t n_tokens) {
  k_short_conv<<<div_ceil(n_embd, 256), 256, 0, s>>>(bcx, taps, hist, out, n_embd, ksize, n_tokens);
}

bool run_short_conv_split(hipStream_t s, const float *bcx, const float *taps, float *hist, float *out,
                          uint32_t n_embd, uint32_t ksize, uint32_t n_tokens, void *scratch) {
  // LFM2's convolutions have 3 taps; other sizes take the separate kernels.
  if (!n_tokens || ksize != 3 || n_embd == 0 || n_embd > 4 * kConvThreads) return false;
  _Float16 *hx = static_cast<_Float16 *>(scratch);
  float *unscale = reinterpret_cast<float *>(hx + (uint64_t)n_tokens * n_embd);
  const uint32_t grid = div_ceil(n_tokens, kConvTokens);
  const uint32_t cpt = div_ceil(n_embd, kConvThreads);
  if (cpt <= 1)
    k_short_conv_split<1, 3><<<grid, kConvThreads, 0, s>>>(bcx, taps, hist, out, n_embd, n_tokens, hx, unscale);
  else if (cpt <= 2)
    k_short_conv_split<2, 3><<<grid, kConvThreads, 0, s>>>(bcx, taps, hist, out, n_embd, n_tokens, hx, unscale);
  else
    k_short_conv_split<4, 3><<<grid, kConvThreads, 0, s>>>(bcx, taps, hist, out, n_embd, n_tokens, hx, unscale);
  return true;
}

void run_short_conv_batch(hipStream_t s, const float *bcx, const float *taps, float *hist, float *out,
                          uint32_t n_embd, uint32_t ksize, uint32_t n_tokens) {
  dim3 grid(div_ceil(n_embd, 256), n_tokens);
  k_short_conv_batch<<<grid, 256, 0, s>>>(bcx, taps, hist, out, n_embd, ksize, n_tokens);
  k_short_conv_history<<<div_ceil(n_embd, 256), 256, 0, s>>>(bcx, hist, n_embd, ksize, n_tokens);
}

}  // namespace bch

using namespace bch;

extern "C" {

int bch_rms_norm(bch_ctx *ctx, bch_view x, bch_view weight, bch_view out, uint32_t n, uint32_t n_rows, float eps) {
  const uint64_t rows_bytes = (uint64_t)n * n_rows * 4;
  const float *xp, *wp;
  float *op;
  BCH_TRY(view_ptr(ctx, "rms_norm", x, rows_bytes, &xp));
  BCH_TRY(view_ptr(ctx, "rms_norm", weight, (uint64_t)n * 4, &wp));
  BCH_TRY(view_ptr(ctx, "rms_norm", out, rows_bytes, &op));
  if (n == 0 || n_rows == 0) return launch(ctx, {"rms_norm", 0, 0, 0}, [](hipStream_t) {});
  return launch(ctx, {"rms_norm", 0, 0, 0}, [&](hipStream_t s) { run_rms_norm(s, xp, wp, op, n, n_rows, eps); });
}

int bch_norm_rope(bch_ctx *ctx, bch_view src, bch_view dst, int dst_half, bch_view weight, uint32_t n_heads,
                  uint32_t head_dim, uint32_t n_rot, uint32_t src_head_stride, uint32_t pos, uint32_t n_tokens,
                  uint32_t src_stride, uint32_t dst_stride, float theta, float eps) {
  if (head_dim == 0 || head_dim > 256 || n_rot > head_dim || n_rot % 2)
    return fail(BCH_ERR_ARGUMENT, "norm_rope: head_dim %u (at most 256) and an even n_rot %u <= head_dim", head_dim,
                n_rot);
  auto extent = [&](uint64_t stride, uint64_t head_stride) {
    return (uint64_t)(n_tokens ? n_tokens - 1 : 0) * stride + (uint64_t)(n_heads ? n_heads - 1 : 0) * head_stride +
           head_dim;
  };
  const float *sp, *wp;
  void *dp;
  BCH_TRY(view_ptr(ctx, "norm_rope", src, extent(src_stride, src_head_stride) * 4, &sp));
  BCH_TRY(view_ptr(ctx, "norm_rope", dst, extent(dst_stride, head_dim) * (dst_half ? 2 : 4), &dp));
  BCH_TRY(view_ptr(ctx, "norm_rope", weight, (uint64_t)head_dim * 4, &wp));
  return launch(ctx, {"norm_rope", 0, 0, 0}, [&](hipStream_t s) {
    if (n_heads && n_tokens)
      run_norm_rope(s, sp, dp, dst_half != 0, wp, n_heads, head_dim, n_rot, src_head_stride, pos, nullptr, n_tokens,
                    src_stride, dst_stride, theta, eps, 0);
  });
}

int bch_convert_half(bch_ctx *ctx, bch_view src, bch_view dst, uint32_t n) {
  const float *sp;
  void *dp;
  BCH_TRY(view_ptr(ctx, "convert_half", src, (uint64_t)n * 4, &sp));
  BCH_TRY(view_ptr(ctx, "convert_half", dst, (uint64_t)n * 2, &dp));
  return launch(ctx, {"convert_half", 0, 0, 0}, [&](hipStream_t s) { run_convert_half(s, sp, dp, n, nullptr, 0); });
}

int bch_copy(bch_ctx *ctx, bch_view src, bch_view dst, uint32_t n) {
  const float *sp;
  float *dp;
  BCH_TRY(view_ptr(ctx, "copy", src, (uint64_t)n * 4, &sp));
  BCH_TRY(view_ptr(ctx, "copy", dst, (uint64_t)n * 4, &dp));
  return launch(ctx, {"copy", 0, 0, 0}, [&](hipStream_t s) { run_copy(s, sp, dp, n, nullptr, 0); });
}

int bch_embed(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_vocab, bch_view tokens, bch_view out,
              uint32_t n_embd, uint32_t n_tokens) {
  const uint64_t rb = bch_row_bytes(format, n_embd);
  if (!rb) return fail(BCH_ERR_ARGUMENT, "embed: %u columns do not tile format %u", n_embd, format);
  const uint8_t *W;
  const uint32_t *tp;
  float *op;
  BCH_TRY(view_ptr(ctx, "embed", weights, rb * n_vocab, &W));
  BCH_TRY(view_ptr(ctx, "embed", tokens, (uint64_t)n_tokens * 4, &tp));
  BCH_TRY(view_ptr(ctx, "embed", out, (uint64_t)n_tokens * n_embd * 4, &op));
  return launch(ctx, {"embed", 0, 0, 0}, [&](hipStream_t s) {
    if (n_tokens && n_embd) run_embed(s, format, W, rb, tp, op, n_embd, n_tokens, nullptr);
  });
}

int bch_argmax(bch_ctx *ctx, bch_view x, bch_view out, uint32_t n) {
  const float *xp;
  uint32_t *op;
  BCH_TRY(view_ptr(ctx, "argmax", x, (uint64_t)n * 4, &xp));
  BCH_TRY(view_ptr(ctx, "argmax", out, 4, &op));
  return launch(ctx, {"argmax", 0, 0, 0}, [&](hipStream_t s) { run_argmax(s, xp, op, n, nullptr, false); });
}

static int conv_views(bch_ctx *ctx, const char *name, bch_view bcx, bch_view taps, bch_view history, bch_view out,
                      uint32_t n_embd, uint32_t ksize, uint32_t n_tokens, const float **bp, const float **tp, float **hp,
                      float **op) {
  if (ksize < 2 || ksize > 9) return fail(BCH_ERR_ARGUMENT, "%s: 2 to 9 taps, got %u", name, ksize);
  BCH_TRY(view_ptr(ctx, name, bcx, (uint64_t)n_tokens * 3 * n_embd * 4, bp));
  BCH_TRY(view_ptr(ctx, name, taps, (uint64_t)n_embd * ksize * 4, tp));
  BCH_TRY(view_ptr(ctx, name, history, (uint64_t)n_embd * (ksize - 1) * 4, hp));
  BCH_TRY(view_ptr(ctx, name, out, (uint64_t)n_tokens * n_embd * 4, op));
  return BCH_OK;
}

int bch_short_conv(bch_ctx *ctx, bch_view bcx, bch_view taps, bch_view history, bch_view out, uint32_t n_embd,
                   uint32_t kernel_size, uint32_t n_tokens) {
  const float *bp, *tp;
  float *hp, *op;
  BCH_TRY(conv_views(ctx, "short_conv", bcx, taps, history, out, n_embd, kernel_size, n_tokens, &bp, &tp, &hp, &op));
  return launch(ctx, {"short_conv", 0, 0, 0}, [&](hipStream_t s) {
    if (n_embd && n_tokens) run_short_conv(s, bp, tp, hp, op, n_embd, kernel_size, n_tokens);
  });
}

int bch_short_conv_batch(bch_ctx *ctx, bch_view bcx, bch_view taps, bch_view history, bch_view out, uint32_t n_embd,
                         uint32_t kernel_size, uint32_t n_tokens) {
  const float *bp, *tp;
  float *hp, *op;
  BCH_TRY(conv_views(ctx, "short_conv_batch", bcx, taps, history, out, n_embd, kernel_size, n_tokens, &bp, &tp, &hp,
                     &op));
  return launch(ctx, {"short_conv_batch", 0, 0, 0}, [&](hipStream_t s) {
    if (n_embd && n_tokens) run_short_conv_batch(s, bp, tp, hp, op, n_embd, kernel_size, n_tokens);
  });
}

}  // extern "C"
