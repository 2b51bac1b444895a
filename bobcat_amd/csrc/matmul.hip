// Prefill GEMM: Y[t] (store) W·X[t] for a batch of tokens, on MFMA.
//
// Counterpart of Metal::matmul and Metal::expand + matmul_f16
// (crates/bobcat-metal/src/backend.rs:2470-2549, matmul.metal:249-438,
// quant.metal:276-306).  The reference expands Q4_K matrices to fp16 before
// a full 512-token batch; here each workgroup dequantises its weight tile
// straight into LDS instead, so the expanded matrix never touches HBM.
//
// Tile: 64 weight rows x 64 tokens x 256 columns (one Q4_K super-block per
// row).  256 threads = 4 waves in a 2x2 arrangement, each wave owning a
// 32x32 output block computed with v_mfma_f32_32x32x8_f16.  Weights go to
// LDS as fp16 (the reference's expanded half tiles); each token's inputs
// are scaled by a power of two into fp16 range and split into an fp16 high
// part and an fp16 residual, both multiplied, so the inputs keep ~22 bits
// whatever their magnitude.  Accumulation is fp32.
#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kBM = 64;       // weight rows per tile
constexpr int kBN = 64;       // tokens per tile
constexpr int kBK = 256;      // columns per step
constexpr int kPad = 8;       // halves of padding per LDS row (bank spread, 16-byte rows)
constexpr int kLds = kBK + kPad;

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float silu_f(float v) { return v / (1.0f + expf(-v)); }

// Dequantise 64 consecutive weights of row `row` starting at column k0+64p
// into fp16 at dst (64 halves).
template <uint32_t FMT>
__device__ __forceinline__ void dequant64(const uint8_t *__restrict__ row, uint32_t k0, int p, _Float16 *dst) {
  if constexpr (FMT == 12) {
    const uint8_t *blk = row + (k0 / 256) * 144;
    const uint4 h = *reinterpret_cast<const uint4 *>(blk);
    const uint4 *qp = reinterpret_cast<const uint4 *>(blk + 16 + 32 * p);
    const uint4 q0 = qp[0], q1 = qp[1];
    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const uint32_t sc = q4k_pair_scales(h.y, h.z, h.w, p);
    const float d = half_bits_to_float(h.x & 0xffffu), dmin = half_bits_to_float(h.x >> 16);
    const float a_lo = d * ubyte0(sc), a_hi = d * ubyte1(sc);
    const float b_lo = dmin * ubyte2(sc), b_hi = dmin * ubyte3(sc);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t lo = qw[k] & 0x0f0f0f0fu, hi = (qw[k] >> 4) & 0x0f0f0f0fu;
      dst[4 * k + 0] = (_Float16)(a_lo * ubyte0(lo) - b_lo);
      dst[4 * k + 1] = (_Float16)(a_lo * ubyte1(lo) - b_lo);
      dst[4 * k + 2] = (_Float16)(a_lo * ubyte2(lo) - b_lo);
      dst[4 * k + 3] = (_Float16)(a_lo * ubyte3(lo) - b_lo);
      dst[32 + 4 * k + 0] = (_Float16)(a_hi * ubyte0(hi) - b_hi);
      dst[32 + 4 * k + 1] = (_Float16)(a_hi * ubyte1(hi) - b_hi);
      dst[32 + 4 * k + 2] = (_Float16)(a_hi * ubyte2(hi) - b_hi);
      dst[32 + 4 * k + 3] = (_Float16)(a_hi * ubyte3(hi) - b_hi);
    }
  } else if constexpr (FMT == 1) {
    const uint4 *src = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(row) + k0 + 64 * p);
    uint4 *o = reinterpret_cast<uint4 *>(dst);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = src[i];
  } else {  // F32
    const float4 *src = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(row) + k0 + 64 * p);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 v = src[i];
      dst[4 * i + 0] = (_Float16)v.x;
      dst[4 * i + 1] = (_Float16)v.y;
      dst[4 * i + 2] = (_Float16)v.z;
      dst[4 * i + 3] = (_Float16)v.w;
    }
  }
}

template <uint32_t FMT, int STORE>
__global__ __launch_bounds__(256) void k_matmul(const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                const float *__restrict__ X, float *__restrict__ Y, uint32_t n_rows,
                                                uint32_t n_cols, uint32_t n_tokens) {
  extern __shared__ _Float16 lds[];
  _Float16 *A = lds;                    // [kBM][kLds]
  _Float16 *Bh = A + kBM * kLds;        // [kBN][kLds]
  _Float16 *Bl = Bh + kBN * kLds;       // [kBN][kLds]
  __shared__ float unscale[kBN];        // 2^-k that undoes each token's input scaling
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const uint32_t row0 = blockIdx.x * kBM, tok0 = blockIdx.y * kBN;
  const int wm = wave / 2, wn = wave % 2;

  float16_t total;
#pragma unroll
  for (int i = 0; i < 16; i++) total[i] = 0.f;

  for (uint32_t k0 = 0; k0 < n_cols; k0 += kBK) {
    // Weights: thread -> (row, quarter of the 256 columns).
    {
      const int r = tid / 4, p = tid % 4;
      const uint32_t grow = min(row0 + r, n_rows - 1);
      dequant64<FMT>(W + (uint64_t)grow * row_bytes, k0, p, A + r * kLds + 64 * p);
    }
    // Inputs: thread -> (token, quarter).  Each token's 256 inputs are
    // scaled by a power of two that brings their largest magnitude just
    // under 2^14 (so half precision cannot overflow), then split into an
    // fp16 high part and an fp16 residual.  The scaling is exact and is
    // undone on the tile's products below.
    {
      const int t = tid / 4, p = tid % 4;
      const uint32_t gt = tok0 + t;
      _Float16 *dh = Bh + t * kLds + 64 * p, *dl = Bl + t * kLds + 64 * p;
      float v[64];
      if (gt < n_tokens) {
        const float4 *src = reinterpret_cast<const float4 *>(X + (uint64_t)gt * n_cols + k0 + 64 * p);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const float4 q = src[i];
          v[4 * i] = q.x;
          v[4 * i + 1] = q.y;
          v[4 * i + 2] = q.z;
          v[4 * i + 3] = q.w;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = 0.f;
      }
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < 64; i++) mx = fmaxf(mx, fabsf(v[i]));
      mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
      int ex = 0;
      if (mx > 0.f) frexpf(mx, &ex);          // mx < 2^ex
      const int k = max(-100, min(100, 14 - ex));
      const float scale = ldexpf(1.0f, k);
      if (p == 0) unscale[t] = ldexpf(1.0f, -k);
#pragma unroll
      for (int i = 0; i < 64; i++) {
        const float sv = v[i] * scale;
        const _Float16 h = (_Float16)sv;
        dh[i] = h;
        dl[i] = (_Float16)(sv - (float)h);
      }
    }
    __syncthreads();
    // 32 k-steps of 8: lane supplies A[row = lane%32][k + 4*(lane/32) .. +4].
    const _Float16 *arow = A + (wm * 32 + lane % 32) * kLds + 4 * (lane / 32);
    const _Float16 *bhrow = Bh + (wn * 32 + lane % 32) * kLds + 4 * (lane / 32);
    const _Float16 *blrow = Bl + (wn * 32 + lane % 32) * kLds + 4 * (lane / 32);
    float16_t acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
#pragma unroll 8
    for (int kk = 0; kk < kBK; kk += 8) {
      const half4_t a = *reinterpret_cast<const half4_t *>(arow + kk);
      const half4_t bh = *reinterpret_cast<const half4_t *>(bhrow + kk);
      const half4_t bl = *reinterpret_cast<const half4_t *>(blrow + kk);
      acc = __builtin_amdgcn_mfma_f32_32x32x8f16(a, bh, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x8f16(a, bl, acc, 0, 0, 0);
    }
    // Every accumulator of a lane belongs to token column lane%32.
    const float us = unscale[wn * 32 + lane % 32];
#pragma unroll
    for (int i = 0; i < 16; i++) total[i] = fmaf(acc[i], us, total[i]);
    __syncthreads();
  }
  // total[r] holds D[row = 8*(r/4) + 4*(lane/32) + r%4][token = lane%32].
  const uint32_t tok = tok0 + wn * 32 + lane % 32;
  if (tok >= n_tokens) return;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const uint32_t row = row0 + wm * 32 + 8 * (r / 4) + 4 * (lane / 32) + (r % 4);
    if (row < n_rows) {
      float *y = Y + (uint64_t)tok * n_rows + row;
      if (STORE == 0)
        *y = total[r];
      else if (STORE == 1)
        *y += total[r];
      else
        *y = silu_f(*y) * total[r];
    }
  }
}

template <uint32_t FMT>
static void matmul_fmt(hipStream_t s, const uint8_t *W, uint64_t rb, const float *x, float *y, uint32_t n_rows,
                       uint32_t n_cols, uint32_t n_tokens, uint32_t store) {
  dim3 grid(div_ceil(n_rows, kBM), div_ceil(n_tokens, kBN));
  const size_t lds = (size_t)(kBM + 2 * kBN) * kLds * sizeof(_Float16);
  if (store == 0)
    k_matmul<FMT, 0><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_tokens);
  else if (store == 1)
    k_matmul<FMT, 1><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_tokens);
  else
    k_matmul<FMT, 2><<<grid, 256, lds, s>>>(W, rb, x, y, n_rows, n_cols, n_tokens);
}

static void set_lds_limits();

void run_matmul(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                float *y, uint32_t n_tokens, uint32_t store) {
  set_lds_limits();
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (format == 12)
    matmul_fmt<12>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else if (format == 1)
    matmul_fmt<1>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
  else
    matmul_fmt<0>(s, W, rb, x, y, n_rows, n_cols, n_tokens, store);
}

static bool matmul_format(uint32_t f) { return f == 12 || f == 1 || f == 0; }

static void set_lds_limits() {
  static bool done = false;
  if (done) return;
  done = true;
  const int lds = (kBM + 2 * kBN) * kLds * sizeof(_Float16);
#define BCH_SET(F, S) hipFuncSetAttribute((const void *)k_matmul<F, S>, hipFuncAttributeMaxDynamicSharedMemorySize, lds)
  BCH_SET(12, 0); BCH_SET(12, 1); BCH_SET(12, 2);
  BCH_SET(1, 0); BCH_SET(1, 1); BCH_SET(1, 2);
  BCH_SET(0, 0); BCH_SET(0, 1); BCH_SET(0, 2);
#undef BCH_SET
}

}  // namespace bch

using namespace bch;

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
  const char *name = format == 12 ? "matmul_q4k" : format == 1 ? "matmul_f16" : "matmul_f32";
  return launch(ctx, {name, n_rows, n_cols, rb * n_rows}, [&](hipStream_t s) {
    if (n_tokens) run_matmul(s, format, W, n_rows, n_cols, xp, yp, n_tokens, store);
  });
}
