// Prefill GEMM: Y[t] (store) W·X[t] for a batch of tokens, on MFMA.
//
// Counterpart of Metal::matmul and Metal::expand + matmul_f16
// (crates/bobcat-metal/src/backend.rs:2470-2549, matmul.metal:249-438,
// quant.metal:276-306).  The reference expands Q4_K matrices to fp16 before
// a full 512-token batch; here each workgroup dequantises its weight tile
// straight into LDS instead, so the expanded matrix never touches HBM.
//
// Two kernels: k_gemm for dense matrices (described at its definition
// below) and k_matmul for the expert-grouped launches of the MoE layers.
// k_matmul's tile is 128 weight rows x 64 tokens in pipeline steps of 128
// columns; before it, k_split_rows scales each token's inputs by a power of
// two into fp16 range and splits them into an fp16 high part and an fp16
// residual, and both are multiplied, so those inputs keep ~22 bits.
// Weights go to LDS as fp16 (the reference's expanded half tiles);
// accumulation is fp32.
#include <mutex>
#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kBM = 128;      // weight rows of the larger tile
constexpr int kBN = 64;       // tokens per tile
constexpr int kBK = 256;      // columns a row must be a multiple of (one Q4_K super-block)
constexpr int kStep = 128;    // columns per pipeline step (half a super-block)
constexpr int kPad = 8;       // halves of padding per LDS row (bank spread, 16-byte rows)
constexpr int kLds = kStep + kPad;

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// The raw bytes of 64 consecutive weights of a row (one Q4_K unit: the
// super-block header and the pair's 32 quant bytes), for prefetching.
struct RawUnit {
  uint4 h, q0, q1;
};

__device__ __forceinline__ RawUnit fetch_q4k(const uint8_t *__restrict__ row, uint32_t k256, int p) {
  const uint8_t *blk = row + (k256 / 256) * 144;
  const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * p);
  return RawUnit{*reinterpret_cast<const uint4 *>(blk), qp[0], qp[1]};
}

// Q4_K unit p of a super-block to 64 halves: (d·sc)·q − dmin·m per element.
__device__ __forceinline__ void expand_q4k(const RawUnit &u, int p, _Float16 *dst) {
  const uint32_t qw[8] = {u.q0.x, u.q0.y, u.q0.z, u.q0.w, u.q1.x, u.q1.y, u.q1.z, u.q1.w};
  const uint32_t sc = q4k_pair_scales(u.h.y, u.h.z, u.h.w, p);
  const float d = half_bits_to_float(u.h.x & 0xffffu), dmin = half_bits_to_float(u.h.x >> 16);
  const float a_lo = d * ubyte0(sc), a_hi = d * ubyte1(sc);
  const float b_lo = dmin * ubyte2(sc), b_hi = dmin * ubyte3(sc);
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const uint32_t lo = qw[k] & 0x0f0f0f0fu, hi = (qw[k] >> 4) & 0x0f0f0f0fu;
    half4_t l4, h4;
    l4[0] = (_Float16)(a_lo * ubyte0(lo) - b_lo);
    l4[1] = (_Float16)(a_lo * ubyte1(lo) - b_lo);
    l4[2] = (_Float16)(a_lo * ubyte2(lo) - b_lo);
    l4[3] = (_Float16)(a_lo * ubyte3(lo) - b_lo);
    h4[0] = (_Float16)(a_hi * ubyte0(hi) - b_hi);
    h4[1] = (_Float16)(a_hi * ubyte1(hi) - b_hi);
    h4[2] = (_Float16)(a_hi * ubyte2(hi) - b_hi);
    h4[3] = (_Float16)(a_hi * ubyte3(hi) - b_hi);
    *reinterpret_cast<half4_t *>(dst + 4 * k) = l4;
    *reinterpret_cast<half4_t *>(dst + 32 + 4 * k) = h4;
  }
}

// F16/F32 rows: 64 consecutive weights from column k to halves.
template <uint32_t FMT>
__device__ __forceinline__ void expand_float(const uint8_t *__restrict__ row, uint32_t k, _Float16 *dst) {
  if constexpr (FMT == 1) {
    const uint4 *src = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(row) + k);
    uint4 *o = reinterpret_cast<uint4 *>(dst);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = src[i];
  } else {
    const float4 *src = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(row) + k);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 v = src[i];
      half4_t h;
      h[0] = (_Float16)v.x;
      h[1] = (_Float16)v.y;
      h[2] = (_Float16)v.z;
      h[3] = (_Float16)v.w;
      *reinterpret_cast<half4_t *>(dst + 4 * i) = h;
    }
  }
}

// Q8_0 / Q4_0 / Q5_K / Q6_K rows: 64 consecutive weights from column k, each
// dequantised exactly as the scalar path does (formats.h dequant_elem), then
// rounded to half.  (These formats appear in a few tensors of real Q4_K_M
// files; the byte-wise reads are not tuned.)
template <uint32_t FMT>
__device__ __forceinline__ void expand_generic(const uint8_t *__restrict__ row, uint32_t k, _Float16 *dst) {
#pragma unroll 8
  for (int i = 0; i < 64; i += 4) {
    half4_t h;
#pragma unroll
    for (int j = 0; j < 4; j++) h[j] = (_Float16)dequant_elem(FMT, row, k + i + j);
    *reinterpret_cast<half4_t *>(dst + i) = h;
  }
}

// Row t of X [n_rows x n_cols] f32 to fp16 high and low parts: with s the
// power of two that puts max|x_t| in [2^13, 2^14) (half precision cannot
// overflow in the MFMA operands), hi = fp16(x·s), lo = fp16(x·s − hi), and
// unscale[t] = 1/s.  Each group of 8 columns is stored as its 8 high halves
// then its 8 low halves (32 bytes), so a GEMM thread's 32 columns of a step
// are 128 contiguous bytes.  One workgroup per row.
__global__ __launch_bounds__(256) void k_split_rows(const float *__restrict__ X, uint32_t n_cols,
                                                   _Float16 *__restrict__ HL, float *__restrict__ unscale) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  const float4 *x4 = reinterpret_cast<const float4 *>(X + (uint64_t)t * n_cols);
  const uint32_t n4 = n_cols / 4;
  float mx = 0.f;
  for (uint32_t i = tid; i < n4; i += 256) {
    const float4 v = x4[i];
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  __shared__ float red[4];
  mx = wave_max(mx);
  if (tid % 64 == 0) red[tid / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int ex = 0;
  if (mx > 0.f) frexpf(mx, &ex);  // mx < 2^ex
  const int k = max(-100, min(100, 14 - ex));
  const float scale = ldexpf(1.0f, k);
  if (tid == 0) unscale[t] = ldexpf(1.0f, -k);
  _Float16 *row = HL + (uint64_t)t * 2 * n_cols;
  for (uint32_t i = tid; i < n4; i += 256) {
    const float4 v4 = x4[i];
    const float v[4] = {v4.x * scale, v4.y * scale, v4.z * scale, v4.w * scale};
    half4_t h, l;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      h[j] = (_Float16)v[j];
      l[j] = (_Float16)(v[j] - (float)h[j]);
    }
    _Float16 *g = row + (i / 2) * 16 + (i % 2) * 4;
    *reinterpret_cast<half4_t *>(g) = h;
    *reinterpret_cast<half4_t *>(g + 8) = l;
  }
}

// The split inputs of a launch: rows of 2·n_cols halves (groups of 8 high
// then 8 low) and the per-row unscale, carved from one scratch region.
struct SplitInputs {
  const _Float16 *hl;
  const float *unscale;
};

static SplitInputs split_inputs(hipStream_t s, const float *x, uint32_t n_rows, uint32_t n_cols, void *scratch) {
  _Float16 *hl = static_cast<_Float16 *>(scratch);
  float *u = reinterpret_cast<float *>(hl + (uint64_t)n_rows * 2 * n_cols);
  if (n_rows) k_split_rows<<<n_rows, 256, 0, s>>>(x, n_cols, hl, u);
  return SplitInputs{hl, u};
}

// Tile 128 weight rows x 64 tokens; 256 threads = 4 waves in a 2x2
// arrangement, each wave owning 64 rows x 32 tokens as two 32x32 MFMA
// blocks.  A pipeline step covers 128 columns: thread t expands weight row
// t/2, unit t%2, and splits 32 inputs of token t/4.  The next step's weight
// and input loads are issued into registers before this step's MFMAs.
// Expert groups of a grouped launch (Metal::matmul_experts): the entries of
// expert e are positions offsets[e] .. offsets[e+1] of `entries`, each entry
// v = token·n_used + slot; entry v reads input row v / x_div and writes
// output row v.  The token tiles of all experts are numbered one after the
// other along blockIdx.y.
struct ExpertGroups {
  const uint32_t *offsets, *entries;
  uint32_t n_experts, x_div;
};

template <uint32_t FMT, int STORE, int MB, bool GROUPED>
__global__ __launch_bounds__(256) void k_matmul(const uint8_t *__restrict__ W, uint64_t row_bytes, SplitInputs X,
                                                float *__restrict__ Y, uint32_t n_rows, uint32_t n_cols,
                                                uint32_t n_tokens, ExpertGroups groups) {
  constexpr int BM = 64 * MB;           // weight rows of this tile (MB 32-row blocks per wave)
  extern __shared__ _Float16 lds[];
  _Float16 *A = lds;                    // [BM][kLds]
  _Float16 *Bh = A + BM * kLds;         // [kBN][kLds]
  _Float16 *Bl = Bh + kBN * kLds;       // [kBN][kLds]
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  // Dense launches are one-dimensional and XCD-aware: workgroup L runs on
  // XCD L % 8 (round-robin dispatch), so logical tile (L % 8)·⌈total/8⌉ + L/8
  // gives each XCD a contiguous run of tiles in token-tile-major order — the
  // row tiles sharing a token tile's inputs then share that XCD's L2 instead
  // of every XCD reading every input tile.
  uint32_t row_tile = blockIdx.x, tok_tile = blockIdx.y;
  if constexpr (!GROUPED) {
    const uint32_t n_rt = (n_rows + BM - 1) / BM, total = n_rt * ((n_tokens + kBN - 1) / kBN);
    const uint32_t per = (total + 7) / 8, logical = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (logical >= total) return;
    row_tile = logical % n_rt;
    tok_tile = logical / n_rt;
  }
  const uint32_t row0 = row_tile * BM;
  uint32_t tok0 = tok_tile * kBN, tok_end = n_tokens;  // positions [tok0, tok_end) of this tile's group
  const int wm = wave / 2, wn = wave % 2;
  if constexpr (GROUPED) {
    // Find this tile's expert: the offsets go to LDS, one thread walks them.
    __shared__ uint32_t off_s[kMoeMaxExperts + 1];
    __shared__ uint32_t pick[3];
    for (uint32_t e = tid; e <= groups.n_experts; e += 256) off_s[e] = groups.offsets[e];
    __syncthreads();
    if (tid == 0) {
      uint32_t t = blockIdx.y, e = 0;
      for (; e < groups.n_experts; e++) {
        const uint32_t tiles = (off_s[e + 1] - off_s[e] + kBN - 1) / kBN;
        if (t < tiles) break;
        t -= tiles;
      }
      pick[0] = e;
      pick[1] = e < groups.n_experts ? off_s[e] + t * kBN : 0;
      pick[2] = e < groups.n_experts ? off_s[e + 1] : 0;
    }
    __syncthreads();
    if (pick[0] >= groups.n_experts) return;  // past the last tile (the grid is an upper bound)
    W += (uint64_t)pick[0] * n_rows * row_bytes;
    tok0 = pick[1];
    tok_end = pick[2];
  }
  // Input and output rows of tile position p.
  auto x_row = [&](uint32_t p) { return GROUPED ? groups.entries[p] / groups.x_div : p; };
  auto y_row = [&](uint32_t p) { return GROUPED ? groups.entries[p] : p; };

  // This thread's weight row and unit (threads past 2·BM stage no weights),
  // and token and quarter.
  const bool a_thread = tid < 2 * BM;
  const int ar = a_thread ? tid / 2 : 0, aq = tid % 2;
  const uint8_t *wrow = W + (uint64_t)min(row0 + ar, n_rows - 1) * row_bytes;
  const int bt = tid / 4, bq = tid % 4;
  // (Tokens past the tile's end stage a copy of the last row; their output
  // columns are never stored.)
  // This thread's 32 columns of a step: 4 groups of (8 high, 8 low) halves.
  const uint4 *xrow = reinterpret_cast<const uint4 *>(X.hl + (uint64_t)x_row(min(tok0 + bt, tok_end - 1)) * 2 * n_cols +
                                                      2 * 32 * bq);

  // Loads of a step, issued a step ahead.  (Plain locals rather than an
  // array captured by a lambda: the compiler kept such an array in scratch
  // memory, which waited on each load.)
  RawUnit ra{};
  uint4 x0, x1, x2, x3, x4, x5, x6, x7;
#define BCH_PREFETCH(k0)                                                                     \
  do {                                                                                       \
    if constexpr (FMT == 12)                                                                 \
      if (a_thread) ra = fetch_q4k(wrow, (k0) & ~255u, (int)(((k0) & 255u) / 64) + aq);       \
    const uint4 *src_ = xrow + (k0) / 4;                                                     \
    x0 = src_[0], x1 = src_[1], x2 = src_[2], x3 = src_[3];                                  \
    x4 = src_[4], x5 = src_[5], x6 = src_[6], x7 = src_[7];                                  \
  } while (0)

  float16_t total[MB];
#pragma unroll
  for (int b = 0; b < MB; b++)
#pragma unroll
    for (int i = 0; i < 16; i++) total[b][i] = 0.f;

  BCH_PREFETCH(0u);
  for (uint32_t k0 = 0; k0 < n_cols; k0 += kStep) {
    // Stage this step: weights to halves, inputs scaled and split.
    if (a_thread) {
      if constexpr (FMT == 12)
        expand_q4k(ra, (int)((k0 & 255u) / 64) + aq, A + ar * kLds + 64 * aq);
      else if constexpr (FMT == 2 || FMT == 8 || FMT == 13 || FMT == 14)
        expand_generic<FMT>(wrow, k0 + 64 * aq, A + ar * kLds + 64 * aq);
      else
        expand_float<FMT>(wrow, k0 + 64 * aq, A + ar * kLds + 64 * aq);
    }
    {
      uint4 *dh = reinterpret_cast<uint4 *>(Bh + bt * kLds + 32 * bq);
      uint4 *dl = reinterpret_cast<uint4 *>(Bl + bt * kLds + 32 * bq);
      dh[0] = x0, dl[0] = x1, dh[1] = x2, dl[1] = x3;
      dh[2] = x4, dl[2] = x5, dh[3] = x6, dl[3] = x7;
    }
    __syncthreads();
    if (k0 + kStep < n_cols) BCH_PREFETCH(k0 + kStep);
    // 8 k-steps of 16 (gfx950's 32x32x16 f16 MFMA): lane supplies
    // A[row = lane%32][k + 8*(lane/32) .. +8] and B[k + 8*(lane/32) .. +8][col = lane%32].
    const _Float16 *arow0 = A + (wm * 32 * MB + lane % 32) * kLds + 8 * (lane / 32);
    const _Float16 *bhrow = Bh + (wn * 32 + lane % 32) * kLds + 8 * (lane / 32);
    const _Float16 *blrow = Bl + (wn * 32 + lane % 32) * kLds + 8 * (lane / 32);
#pragma unroll 4
    for (int kk = 0; kk < kStep; kk += 16) {
      const half8_t bh = *reinterpret_cast<const half8_t *>(bhrow + kk);
      const half8_t bl = *reinterpret_cast<const half8_t *>(blrow + kk);
      half8_t a[MB];
#pragma unroll
      for (int b = 0; b < MB; b++) a[b] = *reinterpret_cast<const half8_t *>(arow0 + 32 * b * kLds + kk);
#pragma unroll
      for (int b = 0; b < MB; b++) total[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[b], bh, total[b], 0, 0, 0);
#pragma unroll
      for (int b = 0; b < MB; b++) total[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[b], bl, total[b], 0, 0, 0);
    }
    __syncthreads();
  }
  // total[b][r] holds D[row = 32b + 8*(r/4) + 4*(lane/32) + r%4][token = lane%32].
  const uint32_t tok = tok0 + wn * 32 + lane % 32;
  if (tok >= tok_end) return;
  const uint64_t yr = y_row(tok);
  const float us = X.unscale[x_row(tok)];  // undoes the token's input scaling
#pragma unroll
  for (int b = 0; b < MB; b++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t row = row0 + wm * 32 * MB + 32 * b + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
      if (row < n_rows) {
        float *y = Y + yr * n_rows + row;
        const float v = total[b][r] * us;
        if (STORE == 0)
          *y = v;
        else if (STORE == 1)
          *y += v;
        else
          *y = silu_f(*y) * v;
      }
    }
}

#undef BCH_PREFETCH

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
// row.
__global__ __launch_bounds__(256) void k_split_hi(const float *__restrict__ X, uint32_t n_cols,
                                                 _Float16 *__restrict__ H, float *__restrict__ unscale) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  const float4 *x4 = reinterpret_cast<const float4 *>(X + (uint64_t)t * n_cols);
  const uint32_t n4 = n_cols / 4;
  float mx = 0.f;
  for (uint32_t i = tid; i < n4; i += 256) {
    const float4 v = x4[i];
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  __shared__ float red[4];
  mx = wave_max(mx);
  if (tid % 64 == 0) red[tid / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int ex = 0;
  if (mx > 0.f) frexpf(mx, &ex);  // mx < 2^ex
  const int k = max(-100, min(100, 14 - ex));
  const float scale = ldexpf(1.0f, k);
  if (tid == 0) unscale[t] = ldexpf(1.0f, -k);
  half4_t *row = reinterpret_cast<half4_t *>(H + (uint64_t)t * n_cols);
  for (uint32_t i = tid; i < n4; i += 256) {
    const float4 v = x4[i];
    half4_t o;
    o[0] = (_Float16)(v.x * scale), o[1] = (_Float16)(v.y * scale);
    o[2] = (_Float16)(v.z * scale), o[3] = (_Float16)(v.w * scale);
    row[i] = o;
  }
}

// k_rms_norm (ops.hip) and k_split_hi in one pass over each row: `out`
// receives exactly k_rms_norm's values (same per-thread sums, reduction and
// scale), and H/unscale the fp16 form of those values that k_split_hi would
// make, so the GEMM that follows skips its own conversion.
__global__ __launch_bounds__(256) void k_rms_norm_split(const float *__restrict__ x, const float *__restrict__ w,
                                                       float *__restrict__ out, uint32_t n, float eps,
                                                       _Float16 *__restrict__ H, float *__restrict__ unscale) {
  __shared__ float red[4];
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  const float *xr = x + (uint64_t)t * n;
  float *orow = out + (uint64_t)t * n;
  float ss = 0.f;
  for (uint32_t i = tid; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
  ss = block_sum<256>(ss, red);
  const float scale = (float)(1.0 / sqrt((double)ss / (double)n + (double)eps));
  float mx = 0.f;
  for (uint32_t i = tid; i < n; i += 256) {
    const float v = w[i] * (xr[i] * scale);
    orow[i] = v;
    mx = fmaxf(mx, fabsf(v));
  }
  mx = block_max<256>(mx, red);
  int ex = 0;
  if (mx > 0.f) frexpf(mx, &ex);  // mx < 2^ex
  const int k = max(-100, min(100, 14 - ex));
  const float s2 = ldexpf(1.0f, k);
  if (tid == 0) unscale[t] = ldexpf(1.0f, -k);
  _Float16 *hrow = H + (uint64_t)t * n;
  for (uint32_t i = tid; i < n; i += 256) hrow[i] = (_Float16)(orow[i] * s2);
}

void run_rms_norm_split(hipStream_t s, const float *x, const float *w, float *out, uint32_t n, uint32_t rows,
                        float eps, void *scratch) {
  if (!rows) return;
  _Float16 *hx = static_cast<_Float16 *>(scratch);
  float *unscale = reinterpret_cast<float *>(hx + (uint64_t)rows * n);
  k_rms_norm_split<<<rows, 256, 0, s>>>(x, w, out, n, eps, hx, unscale);
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
// be interleaved with MFMAs: q4k_scales once, then part J (one quant dword:
// 4 low-nibble and 4 high-nibble weights, (d·sc)·q − dmin·m each, rounded
// to fp16) per call.
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
  constexpr int H = WPT / 2;
  const uint32_t v = J == 0 ? r.q.x : J == 1 ? r.q.y : J == 2 ? r.q.z : r.q.w;
  const uint32_t ql = v & 0x0f0f0f0fu, qh = (v >> 4) & 0x0f0f0f0fu;
  half4_t l4, h4;
  l4[0] = (_Float16)(f.a_lo * ubyte0(ql) - f.b_lo);
  l4[1] = (_Float16)(f.a_lo * ubyte1(ql) - f.b_lo);
  l4[2] = (_Float16)(f.a_lo * ubyte2(ql) - f.b_lo);
  l4[3] = (_Float16)(f.a_lo * ubyte3(ql) - f.b_lo);
  h4[0] = (_Float16)(f.a_hi * ubyte0(qh) - f.b_hi);
  h4[1] = (_Float16)(f.a_hi * ubyte1(qh) - f.b_hi);
  h4[2] = (_Float16)(f.a_hi * ubyte2(qh) - f.b_hi);
  h4[3] = (_Float16)(f.a_hi * ubyte3(qh) - f.b_hi);
  *reinterpret_cast<half4_t *>(dst + H * c + 4 * J) = l4;
  *reinterpret_cast<half4_t *>(dst + 32 + H * c + 4 * J) = h4;
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
template <uint32_t FMT, int STORE, int RB, int NW, int NB>
__global__ __launch_bounds__(64 * NW) void k_gemm(const uint8_t *__restrict__ W, const uint8_t *__restrict__ W2,
                                                  uint64_t row_bytes, HiInputs X, float *__restrict__ Y,
                                                  float *__restrict__ P, uint32_t n_rows, uint32_t n_cols,
                                                  uint32_t n_tokens, uint32_t splits) {
  constexpr bool PAIR = STORE == 3;
  constexpr int OR = PAIR ? RB / 2 : RB;  // output rows per tile
  constexpr int NT = 64 * NW;          // threads
  constexpr int MB = RB / 32;          // row blocks
  constexpr int BT = 32 * NB * NW;     // tokens per tile
  constexpr int WPT = RB * kGk / NT;   // weights a thread dequantises per stage (32 or 16)
  constexpr int TPR = NT / RB;         // threads per weight row
  static_assert(WPT == 32 || WPT == 16, "a thread dequantises 16 or 32 weights per stage");
  constexpr int PARTS = WPT / 8;       // Q4_K dequantisation parts per stage (4 or 2)
  constexpr int MFMAS = MB * NB * 4;   // MFMAs per wave per stage
  constexpr int GAP = MFMAS / PARTS;   // MFMAs between dequantisation parts
  __shared__ __align__(16) _Float16 A[3][RB * kGA];
  __shared__ float us_s[BT];           // the tile's token scales
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, h = lane / 32;
  const uint32_t n_rt = (n_rows + OR - 1) / OR, n_tt = (n_tokens + BT - 1) / BT;
  const uint32_t total = n_rt * n_tt * splits;
  // XCD-aware order: workgroup L runs on XCD L % 8, so logical tile
  // (L % 8)·⌈total/8⌉ + L/8 hands each XCD a contiguous run, split-major
  // then token-tile-major: the row tiles sharing a token tile's inputs share
  // that XCD's L2.
  const uint32_t per = (total + 7) / 8, logical = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (logical >= total) return;
  const uint32_t rt = logical % n_rt, tt = (logical / n_rt) % n_tt, sp = logical / (n_rt * n_tt);
  const uint32_t row0 = rt * OR, tok0 = tt * BT;
  const uint32_t n_stages = n_cols / kGk;
  const uint32_t st0 = (uint32_t)((uint64_t)sp * n_stages / splits);
  const uint32_t st1 = (uint32_t)((uint64_t)(sp + 1) * n_stages / splits);
  const uint32_t last = st1 - 1;

  // Dequantising role: weight row ar, part ac.  (Rows past the end are
  // clamped; their outputs are never stored.)
  const int ar = tid / TPR, ac = tid % TPR;
  const uint8_t *wrow = PAIR && ar >= OR ? W2 + (uint64_t)min(row0 + ar - OR, n_rows - 1) * row_bytes
                                         : W + (uint64_t)min(row0 + ar, n_rows - 1) * row_bytes;
  // MFMA role: tokens tok0 + 32·NB·wave + 32j + lane%32 (clamped), lane half h.
  const u32x4 *xrow[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
    xrow[j] = reinterpret_cast<const u32x4 *>(
        X.h + (uint64_t)min(tok0 + 32 * NB * wave + 32 * j + lane % 32, n_tokens - 1) * n_cols + 16 * h);
  static_assert(BT <= NT, "one thread per token scale");
  if (tid < BT) us_s[tid] = X.unscale[min(tok0 + tid, n_tokens - 1)];

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
  gemm_fetch<FMT, WPT>(wrow, st0 * kGk, ac, r0);
  load_b(st0, b0);
  gemm_fetch<FMT, WPT>(wrow, min(st0 + 1, last) * kGk, ac, r1);
  gemm_dequant_all<FMT, WPT>(wrow, st0 * kGk, ac, r0, &A[0][ar * kGA]);
  gemm_fetch<FMT, WPT>(wrow, min(st0 + 2, last) * kGk, ac, r2);
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
    gemm_fetch<FMT, WPT>(wrow, min(st + 3, last) * kGk, ac, rq);
    const bool valid = st + 1 <= last;
    const uint32_t kn = min(st + 1, last) * kGk;
    Q4kScales f{};
    if constexpr (FMT == 12)
      f = q4k_scales(rn, kn, valid);
    else
      gemm_dequant_direct<FMT, WPT>(wrow, kn, ac, valid, anext);
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
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, bq.v[4 * j + s]),
                                                             wf[s & 1][i], acc[i][j], 0, 0, 0);
          if constexpr (FMT == 12) {
            const int m = (s * MB + i) * NB + j;  // MFMA index in the stage
            if (m % GAP == GAP - 1) {
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
      if (tb + 32 <= n_tokens) {
#pragma unroll
        for (int e = 0; e < 16; e++) dst[(uint64_t)(tb + 8 * (e / 4) + 4 * h + e % 4) * n_rows + row] = v[e];
      } else {
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const uint32_t tok = tb + 8 * (e / 4) + 4 * h + e % 4;
          if (tok < n_tokens) dst[(uint64_t)tok * n_rows + row] = v[e];
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
                        uint32_t splits) {
  const uint32_t out_rows = store == 3 ? RB / 2 : RB;
  const uint32_t total = div_ceil(n_rows, out_rows) * div_ceil(n_tokens, 32 * NB * NW) * splits;
  const dim3 grid(8 * div_ceil(total, 8));
  const dim3 block(64 * NW);
  if (store == 3)
    k_gemm<FMT, 3, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, 1);
  else if (splits > 1 || store == 0)
    k_gemm<FMT, 0, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, splits);
  else if (store == 1)
    k_gemm<FMT, 1, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, splits);
  else
    k_gemm<FMT, 2, RB, NW, NB><<<grid, block, 0, s>>>(W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, splits);
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
  uint32_t cfg, splits;  // cfg 0: 128 rows x 256 tokens, 8 waves; 1: 128 x 128, 4 waves; 2: 64 x 128, 4 waves
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
  if (n_rows > 64 && tiles(128, 128) >= enough) return {1, 1};
  uint32_t splits = 1;
  while (tiles(64, 128) * splits * 2 <= cus && fits(2 * splits)) splits *= 2;
  return {2, splits};
}

template <uint32_t FMT>
static void gemm_fmt(hipStream_t s, const uint8_t *W, const uint8_t *W2, uint64_t rb, const HiInputs &x, float *y,
                     float *part, uint64_t part_floats, uint32_t n_rows, uint32_t n_cols, uint32_t n_tokens,
                     uint32_t store, uint32_t cus) {
  GemmShape g = gemm_shape(store == 3 ? 2 * n_rows : n_rows, n_cols, n_tokens, part_floats, cus);
  if (store == 3) {
    // The pair needs 128-row tiles (64 output rows) and no column split.
    g.splits = 1;
    if (g.cfg == 2) g.cfg = 1;
  }
  if (g.cfg == 0)
    gemm_launch<FMT, 128, 8, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits);
  else if (g.cfg == 1)
    gemm_launch<FMT, 128, 4, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits);
  else
    gemm_launch<FMT, 64, 4, 1>(s, W, W2, rb, x, y, part, n_rows, n_cols, n_tokens, store, g.splits);
}

template <uint32_t FMT, int MB>
static void matmul_tile(hipStream_t s, const uint8_t *W, uint64_t rb, const SplitInputs &x, float *y, uint32_t n_rows,
                        uint32_t n_cols, uint32_t n_tokens, uint32_t store) {
  const uint32_t total = div_ceil(n_rows, 64 * MB) * div_ceil(n_tokens, kBN);
  const dim3 grid(8 * div_ceil(total, 8));  // XCD-aware tile order (see k_matmul)
  const size_t lds = (size_t)(64 * MB + 2 * kBN) * kLds * sizeof(_Float16);
  const ExpertGroups none{};
  if (store == 0)
    k_matmul<FMT, 0, MB, false><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_tokens, none);
  else if (store == 1)
    k_matmul<FMT, 1, MB, false><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_tokens, none);
  else
    k_matmul<FMT, 2, MB, false><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_tokens, none);
}

// Grouped launch over n_entries entries (64-row tiles; an expert's tiles
// are few).  Store 0 overwrites, 2 applies SiLU(y)·product.
template <uint32_t FMT>
static void matmul_experts_fmt(hipStream_t s, const uint8_t *W, uint64_t rb, const SplitInputs &x, float *y,
                               uint32_t n_rows, uint32_t n_cols, uint32_t n_entries, uint32_t store,
                               const ExpertGroups &g) {
  dim3 grid(div_ceil(n_rows, 64), div_ceil(n_entries, kBN) + g.n_experts);
  const size_t lds = (size_t)(64 + 2 * kBN) * kLds * sizeof(_Float16);
  if (store == 2)
    k_matmul<FMT, 2, 1, true><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_entries, g);
  else
    k_matmul<FMT, 0, 1, true><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_entries, g);
}

// 128-row tiles when they give the chip at least two workgroups per CU,
// 64-row tiles (twice the workgroups) otherwise.
template <uint32_t FMT>
static void matmul_fmt(hipStream_t s, const uint8_t *W, uint64_t rb, const SplitInputs &x, float *y, uint32_t n_rows,
                       uint32_t n_cols, uint32_t n_tokens, uint32_t store) {
  const uint64_t big_tiles = (uint64_t)div_ceil(n_rows, 128) * div_ceil(n_tokens, kBN);
  if (big_tiles >= 512)
    matmul_tile<FMT, 2>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else
    matmul_tile<FMT, 1>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
}

static void set_lds_limits();

uint64_t matmul_split_bytes(uint32_t n_rows, uint32_t n_cols) { return (uint64_t)n_rows * (4ull * n_cols + 4); }

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
                const uint8_t *W2) {
  if (!n_tokens) return;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  // The fp16 inputs and their scales (n_tokens·(2·n_cols + 4) bytes, within
  // matmul_split_bytes), then the split-K partials.  With split_ready the
  // previous launch on this scratch converted the same inputs.
  _Float16 *hx = static_cast<_Float16 *>(scratch);
  float *unscale = reinterpret_cast<float *>(hx + (uint64_t)n_tokens * n_cols);
  if (!split_ready) k_split_hi<<<n_tokens, 256, 0, s>>>(xf, n_cols, hx, unscale);
  const HiInputs x{hx, unscale};
  const uint64_t used = (matmul_split_bytes(n_tokens, n_cols) + 255) / 256 * 256;
  float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(scratch) + used);
  const uint64_t part_floats = scratch_bytes > used ? (scratch_bytes - used) / 4 : 0;
  const uint32_t cus = device_cus();
  switch (format) {
    case 12: gemm_fmt<12>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
    case 1: gemm_fmt<1>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
    case 14: gemm_fmt<14>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
    case 13: gemm_fmt<13>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
    case 8: gemm_fmt<8>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
    case 2: gemm_fmt<2>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
    default: gemm_fmt<0>(s, W, W2, rb, x, y, part, part_floats, n_rows, n_cols, n_tokens, store, cus); break;
  }
}

static bool matmul_format(uint32_t f) {
  return f == 12 || f == 1 || f == 0 || f == 13 || f == 14 || f == 8 || f == 2;
}

void run_matmul_experts(hipStream_t s, uint32_t format, const uint8_t *W, const uint8_t *up, uint32_t n_rows,
                        uint32_t n_cols, uint32_t n_experts, const float *xf, bool shared_input,
                        const uint32_t *offsets, const uint32_t *entries, uint32_t n_used, float *y,
                        uint32_t n_tokens, void *split) {
  set_lds_limits();
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const SplitInputs x = split_inputs(s, xf, shared_input ? n_tokens : n_used * n_tokens, n_cols, split);
  const ExpertGroups g{offsets, entries, n_experts, shared_input ? n_used : 1u};
  const uint32_t n_entries = n_used * n_tokens;
  auto one = [&](const uint8_t *w, uint32_t store) {
    if (format == 12)
      matmul_experts_fmt<12>(s, w, rb, x, y, n_rows, n_cols, n_entries, store, g);
    else if (format == 1)
      matmul_experts_fmt<1>(s, w, rb, x, y, n_rows, n_cols, n_entries, store, g);
    else
      matmul_experts_fmt<0>(s, w, rb, x, y, n_rows, n_cols, n_entries, store, g);
  };
  one(W, 0);
  if (up) one(up, 2);  // SwiGLU: the up products times SiLU of the gate products
}

static void set_lds_limits() {
  static bool done = false;
  if (done) return;
  done = true;
  const int lds = (kBM + 2 * kBN) * kLds * sizeof(_Float16);
#define BCH_SET(F, S)                                                                                          \
  hipFuncSetAttribute((const void *)k_matmul<F, S, 2, false>, hipFuncAttributeMaxDynamicSharedMemorySize, lds); \
  hipFuncSetAttribute((const void *)k_matmul<F, S, 1, false>, hipFuncAttributeMaxDynamicSharedMemorySize, lds)
  BCH_SET(12, 0); BCH_SET(12, 1); BCH_SET(12, 2);
  BCH_SET(1, 0); BCH_SET(1, 1); BCH_SET(1, 2);
  BCH_SET(0, 0); BCH_SET(0, 1); BCH_SET(0, 2);
  BCH_SET(14, 0); BCH_SET(14, 1); BCH_SET(14, 2);
  BCH_SET(13, 0); BCH_SET(13, 1); BCH_SET(13, 2);
  BCH_SET(8, 0); BCH_SET(8, 1); BCH_SET(8, 2);
  BCH_SET(2, 0); BCH_SET(2, 1); BCH_SET(2, 2);
#undef BCH_SET
#define BCH_SET(F, S) \
  hipFuncSetAttribute((const void *)k_matmul<F, S, 1, true>, hipFuncAttributeMaxDynamicSharedMemorySize, lds)
  BCH_SET(12, 0); BCH_SET(12, 2); BCH_SET(1, 0); BCH_SET(1, 2); BCH_SET(0, 0); BCH_SET(0, 2);
#undef BCH_SET
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
  const uint64_t need = matmul_split_bytes(n_tokens, n_cols);
  if (need > kNoAllocScratchBytes)
    return fail(BCH_ERR_ARGUMENT,
                "matmul_noalloc: %u tokens of %u columns need %llu bytes of scratch, more than its %llu "
                "(use bch_matmul)",
                n_tokens, n_cols, (unsigned long long)need, (unsigned long long)kNoAllocScratchBytes);
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
  set_lds_limits();
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
  set_lds_limits();
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
