// Prefill GEMM: Y[t] (store) W·X[t] for a batch of tokens, on MFMA.
//
// Counterpart of Metal::matmul and Metal::expand + matmul_f16
// (crates/bobcat-metal/src/backend.rs:2470-2549, matmul.metal:249-438,
// quant.metal:276-306).  The reference expands Q4_K matrices to fp16 before
// a full 512-token batch; here each workgroup dequantises its weight tile
// straight into LDS instead, so the expanded matrix never touches HBM.
//
// Tile: 128 weight rows x 64 tokens, in pipeline steps of 128 columns;
// v_mfma_f32_32x32x16_f16 on LDS tiles.  Weights go to LDS as fp16 (the
// reference's expanded half tiles).  Before the GEMM, k_split_rows scales
// each token's inputs by a power of two into fp16 range and splits them into
// an fp16 high part and an fp16 residual (once per launch, not once per
// weight tile); both are multiplied, so the inputs keep ~22 bits whatever
// their magnitude.  Accumulation is fp32.
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

void run_matmul(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *xf,
                float *y, uint32_t n_tokens, uint32_t store, void *split) {
  set_lds_limits();
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const SplitInputs x = split_inputs(s, xf, n_tokens, n_cols, split);
  if (format == 12)
    matmul_fmt<12>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else if (format == 1)
    matmul_fmt<1>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else if (format == 14)
    matmul_fmt<14>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else if (format == 13)
    matmul_fmt<13>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else if (format == 8)
    matmul_fmt<8>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else if (format == 2)
    matmul_fmt<2>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else
    matmul_fmt<0>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
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
  if (n_tokens) run_matmul(ctx->stream, format, W, n_rows, n_cols, xp, yp, n_tokens, store, split);
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
  BCH_TRY(ctx_scratch(ctx, matmul_split_bytes(n_tokens, n_cols), &split));
  return launch(ctx, {name, n_rows, n_cols, rb * n_rows}, [&](hipStream_t s) {
    if (n_tokens) run_matmul(s, format, W, n_rows, n_cols, xp, yp, n_tokens, store, split);
  });
}
