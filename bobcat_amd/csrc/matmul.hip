// Prefill GEMM: Y[t] (store) W·X[t] for a batch of tokens, on MFMA.
//
// Counterpart of Metal::matmul, Metal::matmul_experts and Metal::expand +
// matmul_f16 (crates/bobcat-metal/src/backend.rs:2470-2549,
// matmul.metal:249-504, quant.metal:276-306).  The reference expands Q4_K
// matrices to fp16 before a full 512-token batch; here each workgroup
// dequantises its weight tile straight into LDS instead, so the expanded
// matrix never touches HBM.  One kernel, k_gemm (described at its
// definition), serves dense and expert-grouped launches; accumulation is
// fp32.
#include <mutex>
#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kBK = 256;      // columns a row must be a multiple of (one Q4_K super-block)

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// Expert groups of a grouped launch (Metal::matmul_experts): the entries of
// expert e are positions offsets[e] .. offsets[e+1] of `entries`, each entry
// v = token·n_used + slot; entry v reads input row v / x_div and writes
// output row v.
struct ExpertGroups {
  const uint32_t *offsets, *entries;
  uint32_t n_experts, x_div;
};

// --- the dense prefill GEMM -------------------------------------------------
//
// Tile RB weight rows x 32·NB·NW tokens with NW waves (64·NW threads),
// wave w owning NB blocks of 32 tokens from 32·NB·w against all RB rows:
// MB·NB blocks (MB = RB/32) of v_mfma_f32_32x32x16_f16.  (NB = 2 halves
// the LDS reads per MFMA but needs more registers than two waves per SIMD
// allow; the launches use NB = 1.)  Three shapes: 128 x 256 with 8 waves (two
// per SIMD) for batches of more than 128 tokens, 128 x 128 with 4 waves,
// and 64 x 128 for matrices of at most 64 rows.  Stages of 64 columns (one
// Q4_K pair of 32-element blocks).
//
// Per stage the workgroup dequantises its RB x 64 weights once into LDS
// (each thread 32 or 16 of them, fp16 as the reference's expanded half
// tiles), and each lane loads its own token's fp16 inputs straight into
// MFMA operand registers.  The inputs are those of k_split_hi: each token
// scaled by the power of two that puts its largest magnitude in
// [2^13, 2^14) (half precision cannot overflow) and rounded to fp16 — 11
// significant bits, finer than bf16 — the scale undone in the epilogue.
// The inputs are the M operand, so the result D[token][row] has rows
// along the lanes and stores of 32 consecutive rows are contiguous.
//
// Budget per MFMA (measured on gfx950: 16 ns per 32x32x16 MFMA per SIMD,
// ~2.2 ns per wave64 VALU instruction, ~11 ns per ds_read_b128 per SIMD
// with four SIMDs reading): one LDS read of a weight fragment and, at 256
// tokens per tile, ~3 VALU instructions of dequantisation.  The VALU work
// overlaps the matrix core only if it sits between MFMAs in each wave's
// instruction stream: the next stage's dequantisation is split into parts
// placed between the MFMAs, held there by scheduling fences.
//
// Column order inside a stage.  The k-step of an MFMA sums over 16 columns
// in any order as long as both operands agree.  Lane half h (lanes 32h ..
// 32h+31) of k-step s takes the 8 columns base(s) + 16h + 0..7, base =
// {0, 8, 32, 40}: 16 contiguous bytes of the token's row and of the LDS
// weight row, and in Q4_K the low (s < 2) or high (s >= 2) nibbles of
// quant bytes 16h + 8(s%2) .. +7.
//
// Software pipeline, three stages deep: step st issues the input loads of
// stage st+2 and the raw weight loads of stage st+3, runs stage st's MFMAs
// while the lanes dequantise stage st+1 into the next LDS buffer, then one
// barrier; every load has two steps to arrive.
//
// Split K.  With few tiles (outputs of a 2048-wide residual stream) the
// column range is split over up to kMaxSplitK workgroups; each writes its
// partial product to scratch and k_gemm_reduce adds them in a fixed order
// and applies the store, so the result does not depend on timing.
constexpr int kGk = 64;             // columns per stage
constexpr int kGA = kGk + 8;        // halves per LDS weight row (padded)
constexpr uint32_t kMaxSplitK = 8;

__device__ __forceinline__ int gemm_base(int s) { return (s & 1) * 8 + (s >> 1) * 32; }

// Row t of X to fp16 with the power of two that puts max|x_t| in
// [2^13, 2^14): H[t][c] = fp16(x·s), unscale[t] = 1/s.  One workgroup per
// row.  PER > 0: each thread keeps its PER float4 (i = tid + 256·k) in
// registers, so the row is read once; PER = 0 loops, re-reading.
template <int PER>
__global__ __launch_bounds__(256) void k_split_hi(const float *__restrict__ X, uint32_t n_cols,
                                                 _Float16 *__restrict__ H, float *__restrict__ unscale) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  const float4 *x4 = reinterpret_cast<const float4 *>(X + (uint64_t)t * n_cols);
  half4_t *row = reinterpret_cast<half4_t *>(H + (uint64_t)t * n_cols);
  const uint32_t n4 = n_cols / 4;
  float4 xv[PER > 0 ? PER : 1];
  float mx = 0.f;
  auto amax = [](float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const uint32_t i = tid + 256 * k;
      xv[k] = i < n4 ? x4[i] : float4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < PER; k++) mx = fmaxf(mx, amax(xv[k]));
  } else {
    for (uint32_t i = tid; i < n4; i += 256) mx = fmaxf(mx, amax(x4[i]));
  }
  __shared__ float red[4];
  mx = block_max<256>(mx, red);
  int ex = 0;
  if (mx > 0.f) frexpf(mx, &ex);  // mx < 2^ex
  const int k2 = max(-100, min(100, 14 - ex));
  const float scale = ldexpf(1.0f, k2);
  if (tid == 0) unscale[t] = ldexpf(1.0f, -k2);
  auto put = [&](uint32_t i, float4 v) {
    half4_t o;
    o[0] = (_Float16)(v.x * scale), o[1] = (_Float16)(v.y * scale);
    o[2] = (_Float16)(v.z * scale), o[3] = (_Float16)(v.w * scale);
    row[i] = o;
  };
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++)
      if (tid + 256 * k < n4) put(tid + 256 * k, xv[k]);
  } else {
    for (uint32_t i = tid; i < n4; i += 256) put(i, x4[i]);
  }
}

// Row t of X [rows x n_cols] to fp16 with the power of two that puts
// max|x_t| in [2^13, 2^14) (k_split_hi), choosing the register form by
// row length.
static void split_hi(hipStream_t s, const float *x, uint32_t rows, uint32_t n_cols, _Float16 *h, float *unscale) {
  if (!rows) return;
  const uint32_t per = div_ceil(n_cols / 4, 256);
  if (per <= 2)
    k_split_hi<2><<<rows, 256, 0, s>>>(x, n_cols, h, unscale);
  else if (per <= 4)
    k_split_hi<4><<<rows, 256, 0, s>>>(x, n_cols, h, unscale);
  else if (per <= 12)
    k_split_hi<12><<<rows, 256, 0, s>>>(x, n_cols, h, unscale);
  else
    k_split_hi<0><<<rows, 256, 0, s>>>(x, n_cols, h, unscale);
}

// k_rms_norm (ops.hip) and k_split_hi in one pass over each row: `out`
// receives exactly k_rms_norm's values (same per-thread sums, reduction and
// scale), and H/unscale the fp16 form of those values that k_split_hi would
// make, so the GEMM that follows skips its own conversion.
//
// PER > 0: each thread keeps its PER elements (i = tid + 256·k, the order
// of k_rms_norm's sums) in registers, so the row is read once; PER = 0
// loops over rows of any length, re-reading.
//
// SUM: x first receives the column-split partial products of the GEMM
// that accumulated into it (P[split][row][i], added in split order and then
// to x, exactly as k_gemm_reduce<1> would), and the sums are written back.
template <int PER, int SPLITS>
__global__ __launch_bounds__(256) void k_rms_norm_split(float *__restrict__ x, const float *__restrict__ w,
                                                       float *__restrict__ out, uint32_t n, float eps,
                                                       _Float16 *__restrict__ H, float *__restrict__ unscale,
                                                       const float *__restrict__ P, uint32_t splits,
                                                       float *__restrict__ unscale_copy) {
  constexpr bool SUM = SPLITS > 0;
  __shared__ float red[4];
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  float *xr = x + (uint64_t)t * n;
  float *orow = out + (uint64_t)t * n;
  _Float16 *hrow = H + (uint64_t)t * n;
  const uint64_t pstride = (uint64_t)gridDim.x * n;
  const float *prow = P + (uint64_t)t * n;
  auto pending = [&](uint32_t i) {
    float v = prow[i];
    for (uint32_t sp = 1; sp < splits; sp++) v += prow[sp * pstride + i];
    return v;
  };
  // The partials of element i, all loaded before any is added (SPLITS > 0).
  auto partials = [&](uint32_t i, float *pv) __attribute__((always_inline)) {
#pragma unroll
    for (int sp = 0; sp < (SUM ? SPLITS : 1); sp++) pv[sp] = prow[sp * pstride + i];
  };
  float xv[PER > 0 ? PER : 1], wv[PER > 0 ? PER : 1];
  float ss = 0.f;
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const uint32_t i = tid + 256 * k;
      xv[k] = i < n ? xr[i] : 0.f;
      wv[k] = i < n ? w[i] : 0.f;
    }
    if constexpr (SUM) {
      float pv[PER][SUM ? SPLITS : 1];
#pragma unroll
      for (int k = 0; k < PER; k++) partials(min(tid + 256 * k, n - 1), pv[k]);
#pragma unroll
      for (int k = 0; k < PER; k++) {
        const uint32_t i = tid + 256 * k;
        float v = pv[k][0];
#pragma unroll
        for (int sp = 1; sp < SPLITS; sp++) v += pv[k][sp];
        if (i < n) {
          xv[k] += v;
          xr[i] = xv[k];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < PER; k++)
      if (tid + 256 * k < n) ss = fmaf(xv[k], xv[k], ss);
  } else {
    if constexpr (SUM)
      for (uint32_t i = tid; i < n; i += 256) xr[i] += pending(i);  // each thread re-reads only its own elements
    for (uint32_t i = tid; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
  }
  ss = block_sum<256>(ss, red);
  const float scale = (float)(1.0 / sqrt((double)ss / (double)n + (double)eps));
  float mx = 0.f;
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const uint32_t i = tid + 256 * k;
      xv[k] = wv[k] * (xv[k] * scale);
      if (i < n) {
        orow[i] = xv[k];
        mx = fmaxf(mx, fabsf(xv[k]));
      }
    }
  } else {
    for (uint32_t i = tid; i < n; i += 256) {
      const float v = w[i] * (xr[i] * scale);
      orow[i] = v;
      mx = fmaxf(mx, fabsf(v));
    }
  }
  mx = block_max<256>(mx, red);
  int ex = 0;
  if (mx > 0.f) frexpf(mx, &ex);  // mx < 2^ex
  const int k2 = max(-100, min(100, 14 - ex));
  const float s2 = ldexpf(1.0f, k2);
  if (tid == 0) {
    unscale[t] = ldexpf(1.0f, -k2);
    if (unscale_copy) unscale_copy[t] = ldexpf(1.0f, -k2);
  }
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++)
      if (tid + 256 * k < n) hrow[tid + 256 * k] = (_Float16)(xv[k] * s2);
  } else {
    for (uint32_t i = tid; i < n; i += 256) hrow[i] = (_Float16)(orow[i] * s2);
  }
}

template <int STORE>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ P, uint32_t splits, uint64_t n,
                                                     float *__restrict__ Y);

void finish_pending_sum(hipStream_t s, PendingSum &p, float *y) {
  if (p.splits > 1) {
    const dim3 g((uint32_t)((p.n + 255) / 256));
    k_gemm_reduce<1><<<g, 256, 0, s>>>(p.part, p.splits, p.n, y);
  }
  p = PendingSum{};
}

void run_rms_norm_split(hipStream_t s, float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps,
                        void *scratch, PendingSum *pending, float *unscale_copy) {
  if (!rows) return;
  _Float16 *hx = static_cast<_Float16 *>(scratch);
  float *unscale = reinterpret_cast<float *>(hx + (uint64_t)rows * n);
  bool sum = pending && pending->splits > 1;
  const uint32_t ps = sum ? pending->splits : 0;
  if (sum && (pending->n != (uint64_t)rows * n || (ps != 2 && ps != 4 && ps != 8) ||
              reinterpret_cast<const uint8_t *>(pending->part) < reinterpret_cast<uint8_t *>(unscale + rows))) {
    // Not this norm's rows, or the fp16 inputs written here would cover the
    // partials: add them first.
    finish_pending_sum(s, *pending, x);
    sum = false;
  }
  const float *P = sum ? pending->part : nullptr;
  const uint32_t splits = sum ? pending->splits : 0;
  auto go = [&](auto per) {
    constexpr int PER = decltype(per)::value;
    if (!sum)
      k_rms_norm_split<PER, 0><<<rows, 256, 0, s>>>(x, w, out, n, eps, hx, unscale, P, splits, unscale_copy);
    else if (splits == 2)
      k_rms_norm_split<PER, 2><<<rows, 256, 0, s>>>(x, w, out, n, eps, hx, unscale, P, splits, unscale_copy);
    else if (splits == 4)
      k_rms_norm_split<PER, 4><<<rows, 256, 0, s>>>(x, w, out, n, eps, hx, unscale, P, splits, unscale_copy);
    else
      k_rms_norm_split<PER, 8><<<rows, 256, 0, s>>>(x, w, out, n, eps, hx, unscale, P, splits, unscale_copy);
  };
  if (n <= 1024)
    go(std::integral_constant<int, 4>{});
  else if (n <= 2048)
    go(std::integral_constant<int, 8>{});
  else if (n <= 4096)
    go(std::integral_constant<int, 16>{});
  else
    go(std::integral_constant<int, 0>{});
  if (pending) *pending = PendingSum{};
}

struct HiInputs {
  const _Float16 *h;
  const float *unscale;
};

// (Clang vector types rather than uint4: copies of uint4 become memcpy
// calls that kept these registers in scratch memory.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw bytes of one thread's weights of a stage: for Q4_K the super-block
// header and the quant bytes of its columns (16 or 8 bytes).
struct GemmRaw {
  u32x4 h, q;
};

// Thread's weights of stage k0 for row `row`: with WPT = 32, columns
// 16c .. 16c+15 and 32+16c .. 32+16c+15 (c = 0, 1); with WPT = 16, columns
// 8c .. 8c+7 and 32+8c .. 32+8c+7 (c = 0..3) — in Q4_K the low and high
// nibbles of quant bytes [WPT/2·c, WPT/2·(c+1)) of the pair.
template <uint32_t FMT, int WPT>
__device__ __forceinline__ void gemm_fetch(const uint8_t *__restrict__ row, uint32_t k0, int c, GemmRaw &r) {
  if constexpr (FMT == 12) {
    const uint8_t *blk = row + (k0 / 256) * 144;
    r.h = *reinterpret_cast<const u32x4 *>(blk);
    const uint8_t *q = blk + 16 + 32 * ((k0 & 255u) / 64) + (WPT / 2) * c;
    if constexpr (WPT == 32) {
      r.q = *reinterpret_cast<const u32x4 *>(q);
    } else {
      const uint2 v = *reinterpret_cast<const uint2 *>(q);
      r.q = u32x4{v.x, v.y, 0u, 0u};
    }
  }
}

// The thread's weights of stage k0 for the formats other than Q4_K, read
// and converted directly (F16, F32, and the block formats through
// dequant_elem).
template <uint32_t FMT, int WPT>
__device__ __forceinline__ void gemm_dequant_direct(const uint8_t *__restrict__ row, uint32_t k0, int c, bool valid,
                                                    _Float16 *__restrict__ dst) {
  constexpr int H = WPT / 2;  // weights per nibble half
  _Float16 *lo = dst + H * c, *hi = dst + 32 + H * c;
  const uint32_t kl = k0 + H * c, kh = k0 + 32 + H * c;
#pragma unroll
  for (int w = 0; w < H / 4; w++) {
    half4_t l4, h4;
    if constexpr (FMT == 1) {
      const _Float16 *f = reinterpret_cast<const _Float16 *>(row);
      l4 = *reinterpret_cast<const half4_t *>(f + kl + 4 * w);
      h4 = *reinterpret_cast<const half4_t *>(f + kh + 4 * w);
    } else if constexpr (FMT == 0) {
      const float *f = reinterpret_cast<const float *>(row);
      const float4 u = *reinterpret_cast<const float4 *>(f + kl + 4 * w);
      const float4 v = *reinterpret_cast<const float4 *>(f + kh + 4 * w);
      l4[0] = (_Float16)u.x, l4[1] = (_Float16)u.y, l4[2] = (_Float16)u.z, l4[3] = (_Float16)u.w;
      h4[0] = (_Float16)v.x, h4[1] = (_Float16)v.y, h4[2] = (_Float16)v.z, h4[3] = (_Float16)v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        l4[i] = (_Float16)dequant_elem(FMT, row, kl + 4 * w + i);
        h4[i] = (_Float16)dequant_elem(FMT, row, kh + 4 * w + i);
      }
    }
    if (!valid) l4 = half4_t{}, h4 = half4_t{};
    *reinterpret_cast<half4_t *>(lo + 4 * w) = l4;
    *reinterpret_cast<half4_t *>(hi + 4 * w) = h4;
  }
}

// Q4_K dequantisation of a thread's stage in parts, so that the parts can
// be interleaved with MFMAs: q4k_scales once, then part J per call — eight
// weights of one nibble half from two quant dwords, (d·sc)·q − dmin·m each
// rounded to fp16, stored as one 16-byte LDS write.  (Parts of four low and
// four high weights stored as two 8-byte writes put four lanes of a wave on
// each pair of banks, a 2-way conflict on every write; 16-byte writes of
// eight consecutive weights spread a wave's rows over all banks.)
struct Q4kScales {
  float a_lo, b_lo, a_hi, b_hi;
};

// (valid false: all four zero, so the part writes zeros.)
__device__ __forceinline__ Q4kScales q4k_scales(const GemmRaw &r, uint32_t k0, bool valid) {
  const uint32_t sc = q4k_pair_scales(r.h.y, r.h.z, r.h.w, (int)((k0 & 255u) / 64));
  const float d = valid ? half_bits_to_float(r.h.x & 0xffffu) : 0.f;
  const float dmin = valid ? half_bits_to_float(r.h.x >> 16) : 0.f;
  return {d * ubyte0(sc), dmin * ubyte2(sc), d * ubyte1(sc), dmin * ubyte3(sc)};
}

template <int WPT, int J>
__device__ __forceinline__ void q4k_part(const GemmRaw &r, const Q4kScales &f, int c, _Float16 *__restrict__ dst) {
  constexpr int H = WPT / 2;                      // weights of each nibble half per thread
  constexpr int HALVES = H / 8;                   // parts per nibble half (1 or 2)
  constexpr bool HI = J >= HALVES;                // which nibble half
  constexpr int P = HI ? J - HALVES : J;          // eight weights P of that half
  const uint32_t v0 = P == 0 ? r.q.x : r.q.z, v1 = P == 0 ? r.q.y : r.q.w;
  const uint32_t q0 = HI ? (v0 >> 4) & 0x0f0f0f0fu : v0 & 0x0f0f0f0fu;
  const uint32_t q1 = HI ? (v1 >> 4) & 0x0f0f0f0fu : v1 & 0x0f0f0f0fu;
  const float a = HI ? f.a_hi : f.a_lo, b = HI ? f.b_hi : f.b_lo;
  half8_t w;
  w[0] = (_Float16)(a * ubyte0(q0) - b);
  w[1] = (_Float16)(a * ubyte1(q0) - b);
  w[2] = (_Float16)(a * ubyte2(q0) - b);
  w[3] = (_Float16)(a * ubyte3(q0) - b);
  w[4] = (_Float16)(a * ubyte0(q1) - b);
  w[5] = (_Float16)(a * ubyte1(q1) - b);
  w[6] = (_Float16)(a * ubyte2(q1) - b);
  w[7] = (_Float16)(a * ubyte3(q1) - b);
  *reinterpret_cast<half8_t *>(dst + (HI ? 32 : 0) + H * c + 8 * P) = w;
}

template <uint32_t FMT, int WPT>
__device__ __forceinline__ void gemm_dequant_all(const uint8_t *__restrict__ row, uint32_t k0, int c,
                                                 const GemmRaw &r, _Float16 *__restrict__ dst) {
  if constexpr (FMT == 12) {
    const Q4kScales f = q4k_scales(r, k0, true);
    q4k_part<WPT, 0>(r, f, c, dst);
    q4k_part<WPT, 1>(r, f, c, dst);
    if constexpr (WPT == 32) {
      q4k_part<WPT, 2>(r, f, c, dst);
      q4k_part<WPT, 3>(r, f, c, dst);
    }
  } else {
    gemm_dequant_direct<FMT, WPT>(row, k0, c, true, dst);
  }
}

// Y (store) or partials: D[token][row] of the launch.  Splits > 1 write
// partial products to P[split] (k_gemm_reduce applies the store).  STORE 3
// is the SwiGLU pair (Metal::matmul_experts's paired tile,
// matmul.metal:249-395, for dense matrices): the tile's first RB/2 rows
// are rows of W (gate projections), the other RB/2 the same rows of W2
// (up projections), and Y receives silu(gate)·up for RB/2 output rows, so
// the gate products never go through memory and each token's inputs are
// loaded once for both matrices.
//
// GROUPED: the expert-grouped launch (Metal::matmul_experts, matmul.metal:
// 462-504).  W (and W2) stack n_experts matrices; the entries of expert e
// are positions offsets[e] .. offsets[e+1] of `entries`, entry v =
// token·n_used + slot reading input row v / x_div and writing output row
// v.  blockIdx.x is the row tile, blockIdx.y numbers the token tiles of
// all experts one after the other (the grid is an upper bound).
template <uint32_t FMT, int STORE, int RB, int NW, int NB, bool GROUPED = false>
__global__ __launch_bounds__(64 * NW) void k_gemm(const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2,
                                                  uint64_t row_bytes, HiInputs X, float *__restrict__ Y,
                                                  float *__restrict__ P, uint32_t n_rows, uint32_t n_cols,
                                                  uint32_t n_tokens, uint32_t splits, ExpertGroups groups) {
  static_assert(!GROUPED || STORE == 0 || STORE == 3, "grouped launches overwrite");
  constexpr bool PAIR = STORE == 3;
  constexpr int OR = PAIR ? RB / 2 : RB;  // output rows per tile
  constexpr int NT = 64 * NW;          // threads
  constexpr int MB = RB / 32;          // row blocks
  constexpr int BT = 32 * NB * NW;     // tokens per tile
  // Weights a thread dequantises per stage (16 or 32): the first DT threads
  // dequantise (all of them unless RB x 64 does not divide evenly, as for
  // 192-row tiles, where the last waves only run MFMAs).
  constexpr int WPT = RB * kGk / NT > 16 ? 32 : 16;
  constexpr int TPR = kGk / WPT;       // threads per weight row
  constexpr int DT = RB * TPR;         // dequantising threads
  static_assert(DT <= NT && DT % 64 == 0 && RB * kGk / NT <= 32, "dequantisation roles");
  constexpr int PARTS = WPT / 8;       // Q4_K dequantisation parts per stage (4 or 2)
  constexpr int MFMAS = MB * NB * 4;   // MFMAs per wave per stage
  constexpr int GAP = MFMAS / PARTS;   // MFMAs between dequantisation parts
  __shared__ __align__(16) _Float16 A[3][RB * kGA];
  __shared__ float us_s[BT];           // the tile's token scales
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, h = lane / 32;
  __shared__ uint32_t ent_s[GROUPED ? BT : 1];  // grouped: the tile's entries
  uint32_t rt, sp = 0, tok0, tok_end = n_tokens;  // tokens [tok0, tok_end) of this tile's group
  if constexpr (GROUPED) {
    // Find this tile's expert: the offsets go to LDS, one thread walks them.
    __shared__ uint32_t off_s[kMoeMaxExperts + 1];
    __shared__ uint32_t pick[3];
    for (uint32_t e = tid; e <= groups.n_experts; e += NT) off_s[e] = groups.offsets[e];
    __syncthreads();
    if (tid == 0) {
      uint32_t t = blockIdx.y, e = 0;
      for (; e < groups.n_experts; e++) {
        const uint32_t tiles = (off_s[e + 1] - off_s[e] + BT - 1) / BT;
        if (t < tiles) break;
        t -= tiles;
      }
      pick[0] = e;
      pick[1] = e < groups.n_experts ? off_s[e] + t * BT : 0;
      pick[2] = e < groups.n_experts ? off_s[e + 1] : 0;
    }
    __syncthreads();
    if (pick[0] >= groups.n_experts) return;  // past the last tile (uniform)
    W += (uint64_t)pick[0] * n_rows * row_bytes;
    if (PAIR) W2 += (uint64_t)pick[0] * n_rows * row_bytes;
    tok0 = pick[1];
    tok_end = pick[2];
    rt = blockIdx.x;
    if (tid < BT) ent_s[tid] = groups.entries[min(tok0 + tid, tok_end - 1)];
  } else {
    const uint32_t n_rt = (n_rows + OR - 1) / OR, n_tt = (n_tokens + BT - 1) / BT;
    const uint32_t total = n_rt * n_tt * splits;
    // XCD-aware order: workgroup L runs on XCD L % 8, so logical tile
    // (L % 8)·⌈total/8⌉ + L/8 hands each XCD a contiguous run, split-major
    // then token-tile-major: the row tiles sharing a token tile's inputs
    // share that XCD's L2.
    const uint32_t per = (total + 7) / 8, logical = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (logical >= total) return;
    rt = logical % n_rt;
    sp = logical / (n_rt * n_tt);
    tok0 = ((logical / n_rt) % n_tt) * BT;
  }
  const uint32_t row0 = rt * OR;
  const uint32_t n_stages = n_cols / kGk;
  // 32-bit: at most kMaxSplitK splits of at most 2^26 stages.
  const uint32_t st0 = sp * n_stages / splits;
  const uint32_t st1 = (sp + 1) * n_stages / splits;
  const uint32_t last = st1 - 1;

  // Dequantising role: weight row ar, part ac.  (Rows past the end are
  // clamped; their outputs are never stored.)
  const bool dq = tid < DT;  // (wave-uniform)
  const int ar = dq ? tid / TPR : 0, ac = tid % TPR;
  const uint8_t *wrow = PAIR && ar >= OR ? W2 + (uint64_t)min(row0 + ar - OR, n_rows - 1) * row_bytes
                                         : W + (uint64_t)min(row0 + ar, n_rows - 1) * row_bytes;
  // MFMA role: tokens tok0 + 32·NB·wave + 32j + lane%32 (clamped), lane half h.
  // (Grouped: entry p reads input row entries[p] / x_div.)
  auto x_index = [&](uint32_t p) -> uint32_t {
    if constexpr (GROUPED)
      return groups.entries[min(p, tok_end - 1)] / groups.x_div;
    else
      return min(p, n_tokens - 1);
  };
  const u32x4 *xrow[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
    xrow[j] = reinterpret_cast<const u32x4 *>(X.h + (uint64_t)x_index(tok0 + 32 * NB * wave + 32 * j + lane % 32) *
                                                        n_cols + 16 * h);
  static_assert(BT <= NT, "one thread per token scale");
  // Grouped: a wave whose tokens all lie past its expert's entries (an
  // expert's last tile is often partly empty) skips its MFMAs; it still
  // takes its share of the dequantisation.
  const bool live = __builtin_amdgcn_readfirstlane(tok0 + 32 * NB * wave < tok_end ? 1 : 0) != 0;
  if (tid < BT) us_s[tid] = X.unscale[x_index(tok0 + tid)];

  // The lane's inputs of a stage: token block j, k-step s at v[4j + s].
  struct BRegs {
    u32x4 v[4 * NB];
  };
  auto load_b = [&](uint32_t st, BRegs &b) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int s = 0; s < 4; s++) b.v[4 * j + s] = xrow[j][(st * kGk + gemm_base(s)) / 8];
  };

  float16_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // Three sets of everything, stage x in set (x - st0) % 3: raw weights
  // r, inputs b, LDS weight buffer A.  Step st (set q) waits for the loads
  // of step st-2 only, issues the inputs of stage st+2 (set q+2) and the
  // raw weights of stage st+3 (set q), dequantises stage st+1 (set q+1)
  // into LDS between the MFMAs of stage st (set q), then one barrier.
  // Loads thus have two steps to arrive.  The loop runs whole triples of
  // steps; stages past the split's last are dummies whose loads re-read
  // the last stage and whose weights dequantise to zeros, adding nothing.
  GemmRaw r0{}, r1{}, r2{};
  BRegs b0{}, b1{}, b2{};
  constexpr int NL = (FMT == 12 ? 2 : 0) + 4 * NB;  // loads a step issues
  if (dq) gemm_fetch<FMT, WPT>(wrow, st0 * kGk, ac, r0);
  load_b(st0, b0);
  if (dq) {
    gemm_fetch<FMT, WPT>(wrow, min(st0 + 1, last) * kGk, ac, r1);
    gemm_dequant_all<FMT, WPT>(wrow, st0 * kGk, ac, r0, &A[0][ar * kGA]);
    gemm_fetch<FMT, WPT>(wrow, min(st0 + 2, last) * kGk, ac, r2);
  }
  load_b(min(st0 + 1, last), b1);
  __syncthreads();

  auto step = [&](uint32_t st, GemmRaw &rq, const GemmRaw &rn, BRegs &b2n, const BRegs &bq, const _Float16 *ab,
                  _Float16 *anext) __attribute__((always_inline)) {
    // Wait for the loads of step st-2 (the most recent NL, of step st-1,
    // may stay in flight).  (Left to itself the compiler counts loads
    // across the loop's back edge conservatively and stalls the MFMAs on
    // loads issued just above them.)
    __builtin_amdgcn_s_waitcnt((NL & 15) | ((NL >> 4) << 14) | 0x0f70);  // vmcnt(NL)
    load_b(min(st + 2, last), b2n);
    if (DT == NT || dq) gemm_fetch<FMT, WPT>(wrow, min(st + 3, last) * kGk, ac, rq);
    const bool valid = st + 1 <= last;
    const uint32_t kn = min(st + 1, last) * kGk;
    Q4kScales f{};
    if constexpr (FMT == 12)
      f = q4k_scales(rn, kn, valid);
    else
      if (DT == NT || dq) gemm_dequant_direct<FMT, WPT>(wrow, kn, ac, valid, anext);
    // MFMAs k-step by k-step, each k-step's weight fragments read from LDS
    // one k-step ahead, a part of the next stage's dequantisation after
    // every GAP MFMAs, fenced so the scheduler keeps that order.
    const _Float16 *ap = ab + (lane % 32) * kGA + 16 * h;
    half8_t wf[2][MB];
#pragma unroll
    for (int i = 0; i < MB; i++) wf[0][i] = *reinterpret_cast<const half8_t *>(ap + 32 * i * kGA + gemm_base(0));
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if (s < 3) {
#pragma unroll
        for (int i = 0; i < MB; i++)
          wf[(s + 1) & 1][i] = *reinterpret_cast<const half8_t *>(ap + 32 * i * kGA + gemm_base(s + 1));
      }
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++) {
          if (!GROUPED || live)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, bq.v[4 * j + s]),
                                                               wf[s & 1][i], acc[i][j], 0, 0, 0);
          if constexpr (FMT == 12) {
            const int m = (s * MB + i) * NB + j;  // MFMA index in the stage
            if (m % GAP == GAP - 1 && (DT == NT || dq)) {
              switch (m / GAP) {
                case 0: q4k_part<WPT, 0>(rn, f, ac, anext); break;
                case 1: q4k_part<WPT, 1>(rn, f, ac, anext); break;
                case 2: if constexpr (PARTS > 2) q4k_part<WPT, 2>(rn, f, ac, anext); break;
                case 3: if constexpr (PARTS > 3) q4k_part<WPT, 3>(rn, f, ac, anext); break;
              }
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
    }
    __syncthreads();
  };
  _Float16 *a0 = &A[0][ar * kGA], *a1 = &A[1][ar * kGA], *a2 = &A[2][ar * kGA];
  for (uint32_t st = st0; st <= last; st += 3) {
    step(st, r0, r1, b2, b0, A[0], a1);
    step(st + 1, r1, r2, b0, b1, A[1], a2);
    step(st + 2, r2, r0, b1, b2, A[2], a0);
  }

  // acc[i][j][e]: token 32·NB·wave + 32j + 8(e/4) + 4h + e%4 of the tile,
  // row 32i + lane%32.  The epilogue's loads (prior outputs, with clamped
  // addresses) are unconditional so that they issue together; only the
  // stores test bounds.
#pragma unroll
  for (int i = 0; i < OR / 32; i++) {
    const uint32_t row = row0 + 32 * i + lane % 32;
    const uint32_t rowc = min(row, n_rows - 1);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int tw = 32 * NB * wave + 32 * j;  // first token of the block in the tile
      const uint32_t tb = tok0 + tw;
      float v[16], prior[16];
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int tl = tw + 8 * (e / 4) + 4 * h + e % 4;
        v[e] = acc[i][j][e] * us_s[tl];
        if (PAIR) prior[e] = acc[i + OR / 32][j][e] * us_s[tl];  // the up product
        else if (STORE != 0 && splits == 1) prior[e] = Y[(uint64_t)min(tok0 + tl, n_tokens - 1) * n_rows + rowc];
      }
      // Output row of tile token tl: the token itself, or (grouped) its entry.
      auto y_row = [&](int tl) -> uint64_t {
        if constexpr (GROUPED)
          return ent_s[tl];
        else
          return tok0 + tl;
      };
#pragma unroll
      for (int e = 0; e < 16; e++) {
        if (PAIR)
          v[e] = silu_f(v[e]) * prior[e];
        else if (splits > 1)
          ;
        else if (STORE == 1)
          v[e] += prior[e];
        else if (STORE == 2)
          v[e] *= silu_f(prior[e]);
      }
      float *dst = splits > 1 ? P + (uint64_t)sp * n_tokens * n_rows : Y;
      if (row >= n_rows) continue;
      if (tb + 32 <= tok_end) {
#pragma unroll
        for (int e = 0; e < 16; e++) dst[y_row(tw + 8 * (e / 4) + 4 * h + e % 4) * n_rows + row] = v[e];
      } else {
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int tl = tw + 8 * (e / 4) + 4 * h + e % 4;
          if (tok0 + tl < tok_end) dst[y_row(tl) * n_rows + row] = v[e];
        }
      }
    }
  }
}

// Y (store) Σ_split P[split], the splits added in order.
template <int STORE>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ P, uint32_t splits, uint64_t n,
                                                     float *__restrict__ Y) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v = P[i];
  for (uint32_t sp = 1; sp < splits; sp++) v += P[sp * n + i];
  if (STORE == 0)
    Y[i] = v;
  else if (STORE == 1)
    Y[i] += v;
  else
    Y[i] = silu_f(Y[i]) * v;
}

template <uint32_t FMT, int RB, int NW, int NB>
static void gemm_launch(hipStream_t s, const uint8_t *W, const uint8_t *W2, uint64_t rb, const HiInputs &x, float *y,
                        float *part, uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens, uint32_t store,
                        uint32_t splits, PendingSum *defer) {
  const uint32_t out_rows = store == 3 ? RB / 2 : RB;
  const uint32_t total = div_ceil(n_rows, out_rows) * div_ceil(n_tokens, 32 * NB * NW) * splits;
  const dim3 grid(8 * div_ceil(total, 8));
  const dim3 block(64 * NW);
  if (store == 3) {
    // (Paired tiles hold whole 32-row blocks of both matrices.)
    if constexpr (RB % 64 == 0)
      k_gemm<FMT, 3, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, 1,
                                                        ExpertGroups{});
  } else if (splits > 1 || store == 0)
    k_gemm<FMT, 0, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, splits, ExpertGroups{});
  else if (store == 1)
    k_gemm<FMT, 1, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, splits, ExpertGroups{});
  else
    k_gemm<FMT, 2, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, splits, ExpertGroups{});
  if (splits > 1 && store == 1 && defer) {
    // The next kernel (k_rms_norm_split) adds the partials.
    *defer = PendingSum{part, splits, (uint64_t)n_tokens * n_rows};
    return;
  }
  if (splits > 1 && store != 3) {
    const uint64_t n = (uint64_t)n_tokens * n_rows;
    const dim3 g((uint32_t)((n + 255) / 256));
    if (store == 0)
      k_gemm_reduce<0><<<g, 256, 0, s>>>(part, splits, n, y);
    else if (store == 1)
      k_gemm_reduce<1><<<g, 256, 0, s>>>(part, splits, n, y);
    else
      k_gemm_reduce<2><<<g, 256, 0, s>>>(part, splits, n, y);
  }
}

// Tile and column split of a launch, from measurements at 512 tokens: the
// largest tile that still gives most CUs a workgroup, unsplit — 128 x 256
// for 10752 x 2048 (168 tiles, 52 us), 128 x 128 for 6144 x 2048 (192
// tiles, 35 us); long rows split K on the large tile — 2048 x 10752 with
// 8 splits (49 us; 221 unsplit); the rest take 64 x 128 tiles, splitting
// while the workgroups fit the CUs — 2048 x 2048 with 2 (23 us), 512 x 2048
// with 4 (14 us).  Partials must fit `part_floats`.
struct GemmShape {
  // cfg 0: 128 rows x 256 tokens, 8 waves; 1: 128 x 128, 4 waves; 2: 64 x 128, 4 waves; 3: 96 x 128, 4 waves
  uint32_t cfg, splits;
};

static GemmShape gemm_shape(uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens, uint64_t part_floats, uint32_t cus) {
  auto tiles = [&](uint32_t br, uint32_t bt) { return (uint64_t)div_ceil(n_rows, br) * div_ceil(n_tokens, bt); };
  const uint64_t enough = (uint64_t)cus * 3 / 5;
  const uint32_t n_stages = n_cols / kGk;
  auto fits = [&](uint32_t splits) {
    return splits <= kMaxSplitK && n_stages / splits >= 8 && (uint64_t)splits * n_tokens * n_rows <= part_floats;
  };
  if (n_tokens > 128 && n_rows > 64 && tiles(128, 256) >= enough) return {0, 1};
  if (n_tokens > 128 && n_rows > 64 && n_cols >= 8192) {
    uint32_t splits = 1;
    while (tiles(128, 256) * splits < cus && fits(2 * splits)) splits *= 2;
    return {0, splits};
  }
  if (n_rows > 64 && tiles(128, 128) >= enough) {
    // 96-row tiles when they cover the CUs in fewer rounds of less work
    // (6144 x 2048 at 512 tokens: 256 workgroups instead of 192).
    auto rounds = [&](uint32_t br) { return (tiles(br, 128) + cus - 1) / cus; };
    if (rounds(96) * 96 < rounds(128) * 128) return {3, 1};
    return {1, 1};
  }
  uint32_t splits = 1;
  while (tiles(64, 128) * splits * 2 <= cus && fits(2 * splits)) splits *= 2;
  return {2, splits};
}

template <uint32_t FMT>
static void gemm_fmt(hipStream_t s, const uint8_t *W, const uint8_t *W2, uint64_t rb, const HiInputs &x, float *y,
                     float *part, uint64_t part_floats, uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens,
                     uint32_t store, uint32_t cus, PendingSum *defer) {
  GemmShape g = gemm_shape(store == 3 ? 2 * n_rows : n_rows, n_cols, n_tokens, part_floats, cus);
  if (store == 3) {
    // The pair needs 128- or 192-row tiles (64 or 96 output rows) and no
    // column split.  With 256-token tiles it takes 192 rows when that needs
    // fewer rounds of workgroups over the CUs per row of work: at 512
    // tokens a 10752-row pair is 224 tiles of 96 rows (one round) instead
    // of 336 of 64 (two rounds, 80 CUs running a second tile).
    g.splits = 1;
    if (g.cfg == 2 || g.cfg == 3) g.cfg = 1;
    const uint64_t tt = div_ceil(n_tokens, 256), c = cus ? cus : 256;
    auto rounds = [&](uint32_t out_rows) { return (div_ceil(n_rows, out_rows) * tt + c - 1) / c; };
    if (g.cfg == 0 && rounds(96) * 192 < rounds(64) * 128) {
      const uint32_t total = div_ceil(n_rows, 96) * (uint32_t)tt;
      k_gemm<FMT, 3, 192, 8, 1><<<dim3(8 * div_ceil(total, 8)), dim3(512), 0, s>>>(
          W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, 1, ExpertGroups{});
      return;
    }
  }
  if (g.cfg == 3 && store != 3)
    gemm_launch<FMT, 96, 4, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits, defer);
  else if (g.cfg == 0)
    gemm_launch<FMT, 128, 8, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits, defer);
  else if (g.cfg == 1)
    gemm_launch<FMT, 128, 4, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits, defer);
  else
    gemm_launch<FMT, 64, 4, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits, defer);
}


// The fp16 inputs (2 bytes a column) and one f32 unscale per row of inputs.
uint64_t matmul_split_bytes(uint32_t n_rows, uint32_t n_cols) { return (uint64_t)n_rows * (2ull * n_cols + 4); }

uint64_t matmul_scratch_bytes(uint32_t n_tokens, uint32_t n_cols, uint32_t n_rows) {
  return (matmul_split_bytes(n_tokens, n_cols) + 255) / 256 * 256 + 4ull * kMaxSplitK * n_tokens * n_rows;
}

static uint32_t device_cus() {
  static uint32_t cus = 0;
  if (!cus) {
    int dev = 0;
    hipDeviceProp_t prop;
    cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
              ? (uint32_t)prop.multiProcessorCount
              : 256u;
  }
  return cus;
}

void run_matmul(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *xf,
                float *y, uint32_t n_tokens, uint32_t store, void *scratch, uint64_t scratch_bytes, bool split_ready,
                const uint8_t *W2, PendingSum *defer) {
  if (defer) *defer = PendingSum{};
  if (!n_tokens) return;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  // The fp16 inputs and their scales (n_tokens·(2·n_cols + 4) bytes, within
  // matmul_split_bytes), then the split-K partials.  With split_ready the
  // previous launch on this scratch converted the same inputs.
  _Float16 *hx = static_cast<_Float16 *>(scratch);
  float *unscale = reinterpret_cast<float *>(hx + (uint64_t)n_tokens * n_cols);
  if (!split_ready) split_hi(s, xf, n_tokens, n_cols, hx, unscale);
  const HiInputs x{hx, unscale};
  const uint64_t used = (matmul_split_bytes(n_tokens, n_cols) + 255) / 256 * 256;
  float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(scratch) + used);
  const uint64_t part_floats = scratch_bytes > used ? (scratch_bytes - used) / 4 : 0;
  const uint32_t cus = device_cus();
  switch (format) {
    case 12: gemm_fmt<12>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
    case 1: gemm_fmt<1>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
    case 14: gemm_fmt<14>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
    case 13: gemm_fmt<13>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
    case 8: gemm_fmt<8>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
    case 2: gemm_fmt<2>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
    default: gemm_fmt<0>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus, defer); break;
  }
}

static bool matmul_format(uint32_t f) {
  return f == 12 || f == 1 || f == 0 || f == 13 || f == 14 || f == 8 || f == 2;
}

void run_matmul_experts(hipStream_t s, uint32_t format, const uint8_t *W, const uint8_t *up, uint32_t n_rows,
                        uint32_t n_cols, uint32_t n_experts, const float *xf, bool shared_input,
                        const uint32_t *offsets, const uint32_t *entries, uint32_t n_used, float *y,
                        uint32_t n_tokens, void *split, bool split_ready) {
  if (!n_tokens) return;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint32_t input_rows = shared_input ? n_tokens : n_used * n_tokens;
  _Float16 *hx = static_cast<_Float16 *>(split);
  float *unscale = reinterpret_cast<float *>(hx + (uint64_t)input_rows * n_cols);
  if (!(split_ready && shared_input)) split_hi(s, xf, input_rows, n_cols, hx, unscale);
  const HiInputs x{hx, unscale};
  const ExpertGroups g{offsets, entries, n_experts, shared_input ? n_used : 1u};
  // 128 x 128 tiles (4 waves): an expert's tokens are few.  With `up` the
  // gate and up matrices run as one paired launch (64 output rows a tile).
  const uint32_t n_entries = n_used * n_tokens;
  const uint32_t out_rows = up ? 64 : 128;
  const dim3 grid(div_ceil(n_rows, out_rows), div_ceil(n_entries, 128) + n_experts);
  auto go = [&](auto fmt) {
    constexpr uint32_t F = decltype(fmt)::value;
    if (up)
      k_gemm<F, 3, 128, 4, 1, true><<<grid, 256, 0, s>>>(W, up, rb, x, y, nullptr, n_rows, n_cols, n_entries, 1, g);
    else
      k_gemm<F, 0, 128, 4, 1, true><<<grid, 256, 0, s>>>(W, W, rb, x, y, nullptr, n_rows, n_cols, n_entries, 1, g);
  };
  if (format == 12)
    go(std::integral_constant<uint32_t, 12>{});
  else if (format == 1)
    go(std::integral_constant<uint32_t, 1>{});
  else
    go(std::integral_constant<uint32_t, 0>{});
}

// --- bch_matmul_noalloc: the split inputs in a static device array ---------
//
// For callers that cannot allocate (code under graph capture, serving loops
// that forbid hipMalloc): the per-launch input split lives in `scratch`, a
// file-scope device array that every GPU the library runs on holds until the
// process ends.  Its device address on each GPU comes from
// hipGetSymbolAddress, once per device, when bch_open runs there; host code
// never passes the array's name itself to a kernel.  All calls on one GPU
// share the array: calls that overlap on one GPU (two streams, two threads)
// race on it.  Nothing in it needs clearing (each launch writes every byte it
// reads).

constexpr uint64_t kNoAllocScratchBytes = 16ull << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices] = {};

int matmul_noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(BCH_ERR_NO_DEVICE, "device %d beyond %d", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return BCH_OK;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(BCH_ERR_EXECUTION, "cannot find the no-allocation scratch on device %d: %s", device,
                hipGetErrorString(e));
  g_scratch_ptr[device] = p;
  return BCH_OK;
}

static void *noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_ptr[device];
}

}  // namespace bch

using namespace bch;

extern "C" uint64_t bch_matmul_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int bch_matmul_noalloc(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows, uint32_t n_cols,
                                  bch_view x, bch_view y, uint32_t n_tokens, uint32_t store) {
  if (!matmul_format(format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "format %u matrices have no matrix-matrix kernel", format);
  if (store > 2) return fail(BCH_ERR_ARGUMENT, "matmul_noalloc: unknown store mode %u", store);
  if (n_rows == 0 || n_cols == 0 || n_cols % kBK)
    return fail(BCH_ERR_ARGUMENT, "matmul_noalloc: %u x %u needs columns in multiples of %d", n_rows, n_cols, kBK);
  // The inputs plus the partials of the column split bch_matmul picks for
  // this shape: when they fit, the launch below picks the same split (its
  // smaller budget still holds it), so the results equal bch_matmul's bit
  // for bit.
  const GemmShape g = gemm_shape(n_rows, n_cols, n_tokens, (uint64_t)kMaxSplitK * n_tokens * n_rows, device_cus());
  const uint64_t need = (matmul_split_bytes(n_tokens, n_cols) + 255) / 256 * 256 +
                        (g.splits > 1 ? 4ull * g.splits * n_tokens * n_rows : 0);
  if (need > kNoAllocScratchBytes)
    return fail(BCH_ERR_ARGUMENT,
                "matmul_noalloc: %u tokens of %u x %u need %llu bytes of scratch, more than its %llu "
                "(use bch_matmul)",
                n_tokens, n_rows, n_cols, (unsigned long long)need, (unsigned long long)kNoAllocScratchBytes);
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint8_t *W;
  const float *xp;
  float *yp;
  BCH_TRY(view_ptr(ctx, "matmul_noalloc", weights, rb * n_rows, &W));
  BCH_TRY(view_ptr(ctx, "matmul_noalloc", x, (uint64_t)n_tokens * n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matmul_noalloc", y, (uint64_t)n_tokens * n_rows * 4, &yp));
  if (reinterpret_cast<uintptr_t>(W) % 16 || reinterpret_cast<uintptr_t>(xp) % 16)
    return fail(BCH_ERR_ARGUMENT, "matmul_noalloc: weights and inputs must be 16-byte aligned");
  void *split = noalloc_scratch(ctx->device);
  if (!split) return fail(BCH_ERR_NO_DEVICE, "matmul_noalloc: the scratch of device %d is not set up", ctx->device);
  if (!ctx->recording && !ctx->capturing) return fail(BCH_ERR_NOT_RECORDING, "no recording is open");
  // No profiling events here (creating them allocates): the launch only.
  if (n_tokens) run_matmul(ctx->stream, format, W, n_rows, n_cols, xp, yp, n_tokens, store, split, kNoAllocScratchBytes);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(BCH_ERR_EXECUTION, "matmul_noalloc launch: %s", hipGetErrorString(e));
  return BCH_OK;
}

extern "C" int bch_matmul(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows, uint32_t n_cols,
                          bch_view x, bch_view y, uint32_t n_tokens, uint32_t store) {
  if (!matmul_format(format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "format %u matrices have no matrix-matrix kernel", format);
  if (store > 2) return fail(BCH_ERR_ARGUMENT, "matmul: unknown store mode %u", store);
  if (n_rows == 0 || n_cols == 0 || n_cols % kBK)
    return fail(BCH_ERR_ARGUMENT, "matmul: %u x %u needs columns in multiples of %d", n_rows, n_cols, kBK);
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint8_t *W;
  const float *xp;
  float *yp;
  BCH_TRY(view_ptr(ctx, "matmul", weights, rb * n_rows, &W));
  BCH_TRY(view_ptr(ctx, "matmul", x, (uint64_t)n_tokens * n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matmul", y, (uint64_t)n_tokens * n_rows * 4, &yp));
  if (reinterpret_cast<uintptr_t>(W) % 16 || reinterpret_cast<uintptr_t>(xp) % 16)
    return fail(BCH_ERR_ARGUMENT, "matmul: weights and inputs must be 16-byte aligned");
  const char *name = format == 12 ? "matmul_q4k"
                     : format == 14 ? "matmul_q6k"
                     : format == 13 ? "matmul_q5k"
                     : format == 8  ? "matmul_q8_0"
                     : format == 2  ? "matmul_q4_0"
                     : format == 1  ? "matmul_f16"
                                    : "matmul_f32";
  void *split = nullptr;
  const uint64_t scratch_bytes = matmul_scratch_bytes(n_tokens, n_cols, n_rows);
  BCH_TRY(ctx_scratch(ctx, scratch_bytes, &split));
  return launch(ctx, {name, n_rows, n_cols, rb * n_rows}, [&](hipStream_t s) {
    if (n_tokens) run_matmul(s, format, W, n_rows, n_cols, xp, yp, n_tokens, store, split, scratch_bytes);
  });
}

namespace bch {

// ---------------------------------------------------------------------
// Expanded fp16 weights and the SwiGLU hand-off of the library GEMM pair
// ---------------------------------------------------------------------

// out[r][c] = the fp16 weight k_gemm dequantises into LDS for row r,
// column c (the same fetch and conversion code, so the same bits).  Two
// threads per 64-column stage of a row, each 32 weights.
template <uint32_t FMT>
__global__ __launch_bounds__(256) void k_expand_f16(const uint8_t *__restrict__ W, uint64_t row_bytes, uint32_t n_rows,
                                                    uint32_t n_cols, _Float16 *__restrict__ out) {
  const uint32_t stages = n_cols / kGk;
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)n_rows * stages * 2) return;
  const int c = (int)(i & 1);
  const uint64_t rs = i >> 1;
  const uint32_t row = (uint32_t)(rs / stages), k0 = (uint32_t)(rs % stages) * kGk;
  const uint8_t *wr = W + (uint64_t)row * row_bytes;
  GemmRaw r{};
  gemm_fetch<FMT, 32>(wr, k0, c, r);
  gemm_dequant_all<FMT, 32>(wr, k0, c, r, out + (uint64_t)row * n_cols + k0);
}

bool expand_f16_supported(uint32_t format, uint32_t n_cols) {
  return n_cols % kGk == 0 && (format == 12 || format == 1 || format == 0 || format == 13 || format == 14 ||
                               format == 8 || format == 2);
}

void run_expand_f16(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                    _Float16 *out) {
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint64_t threads = (uint64_t)n_rows * (n_cols / kGk) * 2;
  const dim3 grid((uint32_t)div_ceil(threads, 256));
  switch (format) {
    case 12: k_expand_f16<12><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
    case 1: k_expand_f16<1><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
    case 14: k_expand_f16<14><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
    case 13: k_expand_f16<13><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
    case 8: k_expand_f16<8><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
    case 2: k_expand_f16<2><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
    default: k_expand_f16<0><<<grid, 256, 0, s>>>(W, rb, n_rows, n_cols, out); break;
  }
}

// Token t of the pair product D [n_tokens][2 n_ff] (gate rows, then up
// rows, of inputs scaled by 1/us[t]): ffn = silu(g·us)·(u·us), as k_gemm's
// paired epilogue computes it, then the fp16 inputs of the down projection
// exactly as k_split_hi makes them from ffn (H [n_tokens][n_ff], then
// unscale [n_tokens]).  F32 (optional) receives ffn itself.  PER > 0: each
// thread keeps its PER float4 of ffn in registers; PER = 0 recomputes.
template <int PER>
__global__ __launch_bounds__(256) void k_swiglu_split(const float *__restrict__ D, uint32_t n_ff,
                                                      const float *__restrict__ us, float *__restrict__ F32,
                                                      _Float16 *__restrict__ H, float *__restrict__ unscale) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x, n4 = n_ff / 4;
  const float4 *g4 = reinterpret_cast<const float4 *>(D + (uint64_t)t * 2 * n_ff);
  const float4 *u4 = g4 + n4;
  const float s = us[t];
  auto act = [&](uint32_t i) {
    const float4 g = g4[i], u = u4[i];
    return float4{silu_f(g.x * s) * (u.x * s), silu_f(g.y * s) * (u.y * s), silu_f(g.z * s) * (u.z * s),
                  silu_f(g.w * s) * (u.w * s)};
  };
  auto amax = [](float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
  float4 xv[PER > 0 ? PER : 1];
  float mx = 0.f;
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const uint32_t i = tid + 256 * k;
      xv[k] = i < n4 ? act(i) : float4{0.f, 0.f, 0.f, 0.f};
      mx = fmaxf(mx, amax(xv[k]));
    }
  } else {
    for (uint32_t i = tid; i < n4; i += 256) mx = fmaxf(mx, amax(act(i)));
  }
  __shared__ float red[4];
  mx = block_max<256>(mx, red);
  int ex = 0;
  if (mx > 0.f) frexpf(mx, &ex);
  const int k2 = max(-100, min(100, 14 - ex));
  const float scale = ldexpf(1.0f, k2);
  if (tid == 0) unscale[t] = ldexpf(1.0f, -k2);
  half4_t *row = reinterpret_cast<half4_t *>(H + (uint64_t)t * n_ff);
  float4 *f4 = F32 ? reinterpret_cast<float4 *>(F32 + (uint64_t)t * n_ff) : nullptr;
  auto put = [&](uint32_t i, float4 v) {
    half4_t o;
    o[0] = (_Float16)(v.x * scale), o[1] = (_Float16)(v.y * scale);
    o[2] = (_Float16)(v.z * scale), o[3] = (_Float16)(v.w * scale);
    row[i] = o;
    if (f4) f4[i] = v;
  };
  if constexpr (PER > 0) {
#pragma unroll
    for (int k = 0; k < PER; k++)
      if (tid + 256 * k < n4) put(tid + 256 * k, xv[k]);
  } else {
    for (uint32_t i = tid; i < n4; i += 256) put(i, act(i));
  }
}

void run_swiglu_split(hipStream_t s, const float *D, uint32_t n_ff, uint32_t n_tokens, const float *us, float *f32,
                      void *scratch) {
  _Float16 *H = static_cast<_Float16 *>(scratch);
  float *unscale = reinterpret_cast<float *>(H + (uint64_t)n_tokens * n_ff);
  const uint32_t n4 = n_ff / 4;
  if (n4 <= 4 * 256)
    k_swiglu_split<4><<<n_tokens, 256, 0, s>>>(D, n_ff, us, f32, H, unscale);
  else if (n4 <= 8 * 256)
    k_swiglu_split<8><<<n_tokens, 256, 0, s>>>(D, n_ff, us, f32, H, unscale);
  else if (n4 <= 12 * 256)
    k_swiglu_split<12><<<n_tokens, 256, 0, s>>>(D, n_ff, us, f32, H, unscale);
  else
    k_swiglu_split<0><<<n_tokens, 256, 0, s>>>(D, n_ff, us, f32, H, unscale);
}

}  // namespace bch
