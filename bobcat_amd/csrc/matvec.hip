// Matrix-vector kernels for decode: y (=|+=) W·x with the RMS norm of x
// optionally fused in, the SwiGLU pair, and the gated short-convolution
// input projection.  Counterparts of matvec_k / matvec_k_swiglu /
// matvec_conv (crates/bobcat-metal/src/matvec.metal:298-576) and their
// launchers Metal::matvec / matvec_swiglu / matvec_conv
// (crates/bobcat-metal/src/backend.rs:1344-1417, 2329-2377).
//
// Layout on gfx950: a workgroup is 4 waves of 64 lanes.  A wave splits into
// 64/LPR groups of LPR lanes; each group computes R consecutive rows.  Lane
// i of a group walks units i, i+LPR, ... of the row (formats.h), loads the
// unit's inputs once and streams the R rows' weights against them with
// 16-byte loads.  Group partial sums reduce with cross-lane shuffles.  LPR
// and R are picked per shape so that every lane has whole units and the
// grid holds enough waves to cover all 256 CUs.
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "formats.h"
#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// 1/sqrt(mean(x²) + eps) over the n floats at x, computed by the whole
// workgroup (precise::rsqrt in matvec.metal:349-364; the scale is rounded
// from double like scalar.rs:239-249).
__device__ __forceinline__ float norm_scale(const float *__restrict__ x, uint32_t n, float eps) {
  __shared__ float red[kWaves];
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) ss = fmaf(x[i], x[i], ss);
  ss = block_sum<kThreads>(ss, red);
  return (float)(1.0 / sqrt((double)ss / (double)n + (double)eps));
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

template <class F, int LPR, int R, bool NORM, bool ACC>
__global__ __launch_bounds__(kThreads) void k_matvec(const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                     const float *__restrict__ x, float *__restrict__ y,
                                                     uint32_t n_rows, uint32_t n_units,
                                                     const float *__restrict__ nw, float eps,
                                                     uint32_t n_cols) {
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / LPR, li = lane % LPR;
  const uint32_t first = ((blockIdx.x * kWaves + wave) * G + g) * R;
  float scale = 1.f;
  if (NORM) scale = norm_scale(x, n_cols, eps);
  if (first < n_rows) {
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) rows[r] = W + (uint64_t)min(first + r, n_rows - 1) * row_bytes;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (uint32_t u = li; u < n_units; u += LPR) {
      typename F::Frag f;
      F::template load<NORM>(x, nw, u, f);
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] += F::dot(rows[r], u, f);
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
    if (li == 0) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (first + r < n_rows) {
          const float t = acc[r] * scale;
          y[first + r] = ACC ? y[first + r] + t : t;
        }
      }
    }
  }
}

// Rows of three matrices that share one input, as one launch: row r of the
// stacked matrix comes from W0 (r < r0), W1 (r < r0 + r1) or W2, and goes
// to the matching output.  Used for an attention layer's q, k and v.
template <class F, int LPR, int R, bool NORM>
__global__ __launch_bounds__(kThreads) void k_matvec3(const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
                                                      const uint8_t *__restrict__ W2, uint32_t r0, uint32_t r1,
                                                      uint64_t row_bytes, const float *__restrict__ x,
                                                      float *__restrict__ y0, float *__restrict__ y1,
                                                      float *__restrict__ y2, uint32_t n_rows, uint32_t n_units,
                                                      const float *__restrict__ nw, float eps, uint32_t n_cols) {
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / LPR, li = lane % LPR;
  const uint32_t first = ((blockIdx.x * kWaves + wave) * G + g) * R;
  float scale = 1.f;
  if (NORM) scale = norm_scale(x, n_cols, eps);
  if (first < n_rows) {
    const uint8_t *rows[R];
    float *outs[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = min(first + r, n_rows - 1);
      if (row < r0) {
        rows[r] = W0 + (uint64_t)row * row_bytes;
        outs[r] = y0 + row;
      } else if (row < r0 + r1) {
        rows[r] = W1 + (uint64_t)(row - r0) * row_bytes;
        outs[r] = y1 + (row - r0);
      } else {
        rows[r] = W2 + (uint64_t)(row - r0 - r1) * row_bytes;
        outs[r] = y2 + (row - r0 - r1);
      }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (uint32_t u = li; u < n_units; u += LPR) {
      typename F::Frag f;
      F::template load<NORM>(x, nw, u, f);
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] += F::dot(rows[r], u, f);
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = group_sum<LPR>(acc[r]);
    if (li == 0) {
#pragma unroll
      for (int r = 0; r < R; r++)
        if (first + r < n_rows) *outs[r] = acc[r] * scale;
    }
  }
}

template <class F, int LPR, int R>
__global__ __launch_bounds__(kThreads) void k_matvec_swiglu(const uint8_t *__restrict__ Wg,
                                                            const uint8_t *__restrict__ Wu, uint64_t row_bytes,
                                                            const float *__restrict__ x, float *__restrict__ y,
                                                            uint32_t n_rows, uint32_t n_units,
                                                            const float *__restrict__ nw, float eps,
                                                            uint32_t n_cols) {
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / LPR, li = lane % LPR;
  const uint32_t first = ((blockIdx.x * kWaves + wave) * G + g) * R;
  const float scale = norm_scale(x, n_cols, eps);
  if (first < n_rows) {
    const uint8_t *gr[R], *ur[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint64_t off = (uint64_t)min(first + r, n_rows - 1) * row_bytes;
      gr[r] = Wg + off;
      ur[r] = Wu + off;
    }
    float ag[R], au[R];
#pragma unroll
    for (int r = 0; r < R; r++) ag[r] = au[r] = 0.f;
    for (uint32_t u = li; u < n_units; u += LPR) {
      typename F::Frag f;
      F::template load<true>(x, nw, u, f);
#pragma unroll
      for (int r = 0; r < R; r++) {
        ag[r] += F::dot(gr[r], u, f);
        au[r] += F::dot(ur[r], u, f);
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      ag[r] = group_sum<LPR>(ag[r]);
      au[r] = group_sum<LPR>(au[r]);
    }
    if (li == 0) {
#pragma unroll
      for (int r = 0; r < R; r++)
        if (first + r < n_rows) y[first + r] = silu(ag[r] * scale) * (au[r] * scale);
    }
  }
}

// One group per channel: rows ch, n_embd+ch and 2·n_embd+ch give B, C and
// X; the group's first lane then runs the channel's convolution as
// matvec_conv does (matvec.metal:386-454).
template <class F, int LPR, bool NORM>
__global__ __launch_bounds__(kThreads) void k_matvec_conv(const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                          const float *__restrict__ x, uint32_t n_units,
                                                          const float *__restrict__ nw, float eps,
                                                          uint32_t n_cols, const float *__restrict__ taps,
                                                          float *__restrict__ history, float *__restrict__ out,
                                                          uint32_t n_embd, uint32_t ksize) {
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / LPR, li = lane % LPR;
  const uint32_t ch = (blockIdx.x * kWaves + wave) * G + g;
  float scale = 1.f;
  if (NORM) scale = norm_scale(x, n_cols, eps);
  if (ch < n_embd) {
    const uint8_t *rows[3];
#pragma unroll
    for (int r = 0; r < 3; r++) rows[r] = W + (uint64_t)(r * n_embd + ch) * row_bytes;
    float acc[3] = {0.f, 0.f, 0.f};
    for (uint32_t u = li; u < n_units; u += LPR) {
      typename F::Frag f;
      F::template load<NORM>(x, nw, u, f);
#pragma unroll
      for (int r = 0; r < 3; r++) acc[r] += F::dot(rows[r], u, f);
    }
#pragma unroll
    for (int r = 0; r < 3; r++) acc[r] = group_sum<LPR>(acc[r]);
    if (li == 0) {
      const float b = acc[0] * scale, c = acc[1] * scale, xin = acc[2] * scale;
      const float *t = taps + (uint64_t)ch * ksize;
      const float bx = b * xin;
      float sum = t[ksize - 1] * bx;
      for (uint32_t k = 0; k + 1 < ksize; k++) sum = fmaf(t[k], history[k * n_embd + ch], sum);
      for (uint32_t k = 0; k + 2 < ksize; k++) history[k * n_embd + ch] = history[(k + 1) * n_embd + ch];
      history[(ksize - 2) * n_embd + ch] = bx;
      out[ch] = c * sum;
    }
  }
}

// Dequantise rows of any format into floats, one thread per element.
__global__ void k_dequantize(uint32_t format, const uint8_t *__restrict__ W, uint64_t row_bytes,
                             float *__restrict__ out, uint32_t n_rows, uint32_t n_cols) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (uint64_t)n_rows * n_cols) return;
  const uint32_t r = (uint32_t)(i / n_cols), c = (uint32_t)(i % n_cols);
  out[i] = dequant_elem(format, W + r * row_bytes, c);
}

// ---------------------------------------------------------------------
// Host side: shape → (LPR, R) and the instantiation tables.
// ---------------------------------------------------------------------

struct Geometry {
  int lpr;
  int r;
};

// Pick lanes per row and rows per group: every lane should own the same
// number of units (no idle tail), and the grid should hold at least
// ~8 waves per CU; among equals prefer more rows per group, which loads
// each input once for more rows.
static Geometry choose(uint32_t n_rows, uint32_t n_units, uint32_t n_cus, int max_r) {
  Geometry best{64, 1};
  double best_score = -1.0;
  const double want_waves = (double)(n_cus ? n_cus : 256) * 8.0;
  for (int lpr : {64, 32, 16, 8, 4}) {
    const uint32_t iters = (n_units + lpr - 1) / lpr;
    const double util = (double)n_units / ((double)lpr * iters);
    for (int r : {8, 4, 2, 1}) {
      if (r > max_r) continue;
      const double rows_per_wave = (double)(kWave / lpr) * r;
      const double waves = std::ceil(n_rows / rows_per_wave);
      const double occ = std::min(1.0, waves / want_waves);
      const double score = util * occ * (1.0 + 0.02 * r) * (1.0 + 0.01 * lpr / 64.0);
      if (score > best_score) {
        best_score = score;
        best = {lpr, r};
      }
    }
  }
  return best;
}

static uint32_t grid_for(uint32_t n_rows, Geometry g) {
  const uint32_t rows_per_block = kWaves * (kWave / g.lpr) * g.r;
  return div_ceil(n_rows, rows_per_block);
}

// Call f.template operator()<LPR, R>() for the runtime geometry.
template <class Fn>
static void dispatch_geometry(Geometry g, Fn &&f) {
#define BCH_R_CASES(L)                                       \
  switch (g.r) {                                             \
    case 8: f.template operator()<L, 8>(); break;            \
    case 4: f.template operator()<L, 4>(); break;            \
    case 2: f.template operator()<L, 2>(); break;            \
    default: f.template operator()<L, 1>(); break;           \
  }
  switch (g.lpr) {
    case 64: BCH_R_CASES(64) break;
    case 32: BCH_R_CASES(32) break;
    case 16: BCH_R_CASES(16) break;
    case 8: BCH_R_CASES(8) break;
    default: BCH_R_CASES(4) break;
  }
#undef BCH_R_CASES
}

template <class F>
static void matvec_f(hipStream_t s, Geometry g, const uint8_t *W, uint64_t rb, const float *x, float *y,
                     uint32_t n_rows, uint32_t n_units, const float *nw, float eps, uint32_t n_cols, bool norm,
                     bool acc) {
  const uint32_t grid = grid_for(n_rows, g);
  dispatch_geometry(g, [&]<int L, int R>() {
    if (norm && acc)
      k_matvec<F, L, R, true, true><<<grid, kThreads, 0, s>>>(W, rb, x, y, n_rows, n_units, nw, eps, n_cols);
    else if (norm)
      k_matvec<F, L, R, true, false><<<grid, kThreads, 0, s>>>(W, rb, x, y, n_rows, n_units, nw, eps, n_cols);
    else if (acc)
      k_matvec<F, L, R, false, true><<<grid, kThreads, 0, s>>>(W, rb, x, y, n_rows, n_units, nw, eps, n_cols);
    else
      k_matvec<F, L, R, false, false><<<grid, kThreads, 0, s>>>(W, rb, x, y, n_rows, n_units, nw, eps, n_cols);
  });
}

template <class F>
static void matvec3_f(hipStream_t s, Geometry g, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2,
                      uint32_t r0, uint32_t r1, uint64_t rb, const float *x, float *y0, float *y1, float *y2,
                      uint32_t n_rows, uint32_t n_units, const float *nw, float eps, uint32_t n_cols) {
  const uint32_t grid = grid_for(n_rows, g);
  dispatch_geometry(g, [&]<int L, int R>() {
    if (nw)
      k_matvec3<F, L, R, true><<<grid, kThreads, 0, s>>>(W0, W1, W2, r0, r1, rb, x, y0, y1, y2, n_rows, n_units, nw,
                                                         eps, n_cols);
    else
      k_matvec3<F, L, R, false><<<grid, kThreads, 0, s>>>(W0, W1, W2, r0, r1, rb, x, y0, y1, y2, n_rows, n_units, nw,
                                                          eps, n_cols);
  });
}

template <class F>
static void swiglu_f(hipStream_t s, Geometry g, const uint8_t *Wg, const uint8_t *Wu, uint64_t rb, const float *x,
                     float *y, uint32_t n_rows, uint32_t n_units, const float *nw, float eps, uint32_t n_cols) {
  const uint32_t grid = grid_for(n_rows, g);
  dispatch_geometry(g, [&]<int L, int R>() {
    k_matvec_swiglu<F, L, R><<<grid, kThreads, 0, s>>>(Wg, Wu, rb, x, y, n_rows, n_units, nw, eps, n_cols);
  });
}

static bool is_gemv_format(uint32_t f) {
  return f == Q4K::kFormat || f == F16::kFormat || f == F32::kFormat || f == Q6K::kFormat || f == Q5K::kFormat ||
         f == Q8_0::kFormat || f == Q4_0::kFormat;
}

// Weights per unit (formats.h).
static uint32_t unit_of(uint32_t f) {
  if (f == Q4K::kFormat || f == Q5K::kFormat || f == Q6K::kFormat || f == Q8_0::kFormat || f == Q4_0::kFormat) return 64;
  return f == F16::kFormat ? F16::kUnit : F32::kUnit;
}

// Columns a row of format f must be a multiple of (whole super-blocks).
static uint32_t cols_of(uint32_t f) {
  return f == Q4K::kFormat || f == Q5K::kFormat || f == Q6K::kFormat ? 256 : unit_of(f);
}

static const char *format_name(uint32_t f) {
  switch (f) {
    case 12: return "q4k";
    case 14: return "q6k";
    case 13: return "q5k";
    case 8: return "q8_0";
    case 2: return "q4_0";
    case 1: return "f16";
    default: return "f32";
  }
}

// Call f.template operator()<Format>() for a runtime format id.
template <class Fn>
static void dispatch_format(uint32_t format, Fn &&f) {
  if (format == Q4K::kFormat)
    f.template operator()<Q4K>();
  else if (format == F16::kFormat)
    f.template operator()<F16>();
  else if (format == Q6K::kFormat)
    f.template operator()<Q6K>();
  else if (format == Q5K::kFormat)
    f.template operator()<Q5K>();
  else if (format == Q8_0::kFormat)
    f.template operator()<Q8_0>();
  else if (format == Q4_0::kFormat)
    f.template operator()<Q4_0>();
  else
    f.template operator()<F32>();
}

void run_matvec(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                float *y, const float *norm_w, float eps, bool accumulate, uint32_t n_cus) {
  if (fast_matvec(s, format, W, n_rows, n_cols, x, y, norm_w, eps, accumulate, n_cus)) return;
  const uint32_t n_units = n_cols / unit_of(format);
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const Geometry g = choose(n_rows, n_units, n_cus, 8);
  dispatch_format(format, [&]<class F>() {
    matvec_f<F>(s, g, W, rb, x, y, n_rows, n_units, norm_w, eps, n_cols, norm_w != nullptr, accumulate);
  });
}

void run_matvec3(hipStream_t s, uint32_t format, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2, uint32_t r0,
                 uint32_t r1, uint32_t r2, uint32_t n_cols, const float *x, float *y0, float *y1, float *y2,
                 const float *norm_w, float eps, uint32_t n_cus) {
  if (fast_matvec3(s, format, W0, W1, W2, r0, r1, r2, n_cols, x, y0, y1, y2, norm_w, eps, n_cus))
    return;
  const uint32_t n_units = n_cols / unit_of(format);
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint32_t n_rows = r0 + r1 + r2;
  const Geometry g = choose(n_rows, n_units, n_cus, 8);
  dispatch_format(format, [&]<class F>() {
    matvec3_f<F>(s, g, W0, W1, W2, r0, r1, rb, x, y0, y1, y2, n_rows, n_units, norm_w, eps, n_cols);
  });
}

void run_matvec_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_rows,
                       uint32_t n_cols, const float *x, float *y, const float *norm_w, float eps, uint32_t n_cus) {
  if (fast_matvec_swiglu(s, format, Wg, Wu, n_rows, n_cols, x, y, norm_w, eps, n_cus))
    return;
  const uint32_t n_units = n_cols / unit_of(format);
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const Geometry g = choose(n_rows, n_units, n_cus, 4);
  dispatch_format(format, [&]<class F>() { swiglu_f<F>(s, g, Wg, Wu, rb, x, y, n_rows, n_units, norm_w, eps, n_cols); });
}

void run_matvec_conv(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_cols, const float *x,
                     const float *norm_w, float eps, const float *taps, float *history, float *out, uint32_t n_embd,
                     uint32_t ksize, uint32_t n_cus) {
  if (fast_matvec_conv(s, format, W, n_cols, x, norm_w, eps, taps, history, out, n_embd, ksize, n_cus))
    return;
  const uint32_t n_units = n_cols / Q4K::kUnit;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const Geometry g = choose(n_embd, n_units, n_cus, 1);
  const uint32_t grid = div_ceil(n_embd, kWaves * (kWave / g.lpr));
  dispatch_geometry(Geometry{g.lpr, 1}, [&]<int L, int R>() {
    if (norm_w)
      k_matvec_conv<Q4K, L, true><<<grid, kThreads, 0, s>>>(W, rb, x, n_units, norm_w, eps, n_cols, taps, history, out,
                                                            n_embd, ksize);
    else
      k_matvec_conv<Q4K, L, false><<<grid, kThreads, 0, s>>>(W, rb, x, n_units, norm_w, eps, n_cols, taps, history,
                                                             out, n_embd, ksize);
  });
}

static int check_shape(const char *name, uint32_t format, uint32_t n_rows, uint32_t n_cols) {
  if (!is_gemv_format(format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "%s: format %u has no matrix-vector kernel", name, format);
  if (n_rows == 0 || n_cols == 0 || n_cols % cols_of(format))
    return fail(BCH_ERR_ARGUMENT, "%s: %u x %u does not tile format %u", name, n_rows, n_cols, format);
  return BCH_OK;
}

static int check_align(const char *name, const void *p, uintptr_t a) {
  if (reinterpret_cast<uintptr_t>(p) % a)
    return fail(BCH_ERR_ARGUMENT, "%s: operand is not %zu-byte aligned", name, (size_t)a);
  return BCH_OK;
}

}  // namespace bch

using namespace bch;

extern "C" {

int bch_dequantize(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows, uint32_t n_cols,
                   bch_view out) {
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (!rb) return fail(BCH_ERR_ARGUMENT, "dequantize: %u columns do not tile format %u", n_cols, format);
  const uint8_t *W;
  float *o;
  BCH_TRY(view_ptr(ctx, "dequantize", weights, rb * n_rows, &W));
  BCH_TRY(view_ptr(ctx, "dequantize", out, (uint64_t)n_rows * n_cols * 4, &o));
  const uint64_t n = (uint64_t)n_rows * n_cols;
  return launch(ctx, {"dequantize", n_rows, n_cols, rb * n_rows}, [&](hipStream_t s) {
    if (n) k_dequantize<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(format, W, rb, o, n_rows, n_cols);
  });
}

int bch_matvec(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows, uint32_t n_cols, bch_view x,
               bch_view y, const bch_norm *norm, int accumulate) {
  BCH_TRY(check_shape("matvec", format, n_rows, n_cols));
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint8_t *W;
  const float *xp, *nw = nullptr;
  float *yp;
  BCH_TRY(view_ptr(ctx, "matvec", weights, rb * n_rows, &W));
  BCH_TRY(view_ptr(ctx, "matvec", x, (uint64_t)n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matvec", y, (uint64_t)n_rows * 4, &yp));
  if (norm) BCH_TRY(view_ptr(ctx, "matvec", norm->weight, (uint64_t)n_cols * 4, &nw));
  BCH_TRY(check_align("matvec", W, 16));
  BCH_TRY(check_align("matvec", xp, 16));
  if (nw) BCH_TRY(check_align("matvec", nw, 16));
  const float eps = norm ? norm->eps : 0.f;
  char name[32];
  snprintf(name, sizeof name, "matvec_%s", format_name(format));
  return launch(ctx, {name, n_rows, n_cols, rb * n_rows}, [&](hipStream_t s) {
    run_matvec(s, format, W, n_rows, n_cols, xp, yp, nw, eps, accumulate != 0, ctx->n_cus);
  });
}

int bch_matvec_swiglu(bch_ctx *ctx, uint32_t format, bch_view gate, bch_view up, uint32_t n_rows, uint32_t n_cols,
                      bch_view x, bch_norm norm, bch_view y) {
  BCH_TRY(check_shape("matvec_swiglu", format, n_rows, n_cols));
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint8_t *Wg, *Wu;
  const float *xp, *nw;
  float *yp;
  BCH_TRY(view_ptr(ctx, "matvec_swiglu", gate, rb * n_rows, &Wg));
  BCH_TRY(view_ptr(ctx, "matvec_swiglu", up, rb * n_rows, &Wu));
  BCH_TRY(view_ptr(ctx, "matvec_swiglu", x, (uint64_t)n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matvec_swiglu", y, (uint64_t)n_rows * 4, &yp));
  BCH_TRY(view_ptr(ctx, "matvec_swiglu", norm.weight, (uint64_t)n_cols * 4, &nw));
  BCH_TRY(check_align("matvec_swiglu", Wg, 16));
  BCH_TRY(check_align("matvec_swiglu", Wu, 16));
  BCH_TRY(check_align("matvec_swiglu", xp, 16));
  BCH_TRY(check_align("matvec_swiglu", nw, 16));
  char name[32];
  snprintf(name, sizeof name, "matvec_swiglu_%s", format_name(format));
  return launch(ctx, {name, n_rows, n_cols, 2 * rb * n_rows}, [&](hipStream_t s) {
    run_matvec_swiglu(s, format, Wg, Wu, n_rows, n_cols, xp, yp, nw, norm.eps, ctx->n_cus);
  });
}

int bch_matvec_conv(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_cols, bch_view x,
                    const bch_norm *norm, bch_view taps, bch_view history, bch_view out, uint32_t n_embd,
                    uint32_t kernel_size) {
  if (format != Q4K::kFormat)
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "format %u matrices have no fused short convolution kernel", format);
  if (kernel_size < 2 || kernel_size > 9)
    return fail(BCH_ERR_ARGUMENT, "a short convolution needs 2 to 9 taps, got %u", kernel_size);
  const uint32_t n_rows = 3 * n_embd;
  BCH_TRY(check_shape("matvec_conv", format, n_rows, n_cols));
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const uint8_t *W;
  const float *xp, *tp, *nw = nullptr;
  float *hp, *op;
  BCH_TRY(view_ptr(ctx, "matvec_conv", weights, rb * n_rows, &W));
  BCH_TRY(view_ptr(ctx, "matvec_conv", x, (uint64_t)n_cols * 4, &xp));
  BCH_TRY(view_ptr(ctx, "matvec_conv", taps, (uint64_t)n_embd * kernel_size * 4, &tp));
  BCH_TRY(view_ptr(ctx, "matvec_conv", history, (uint64_t)n_embd * (kernel_size - 1) * 4, &hp));
  BCH_TRY(view_ptr(ctx, "matvec_conv", out, (uint64_t)n_embd * 4, &op));
  if (norm) BCH_TRY(view_ptr(ctx, "matvec_conv", norm->weight, (uint64_t)n_cols * 4, &nw));
  BCH_TRY(check_align("matvec_conv", W, 16));
  BCH_TRY(check_align("matvec_conv", xp, 16));
  if (nw) BCH_TRY(check_align("matvec_conv", nw, 16));
  const float eps = norm ? norm->eps : 0.f;
  return launch(ctx, {"matvec_conv_q4k", n_rows, n_cols, rb * n_rows}, [&](hipStream_t s) {
    run_matvec_conv(s, format, W, n_cols, xp, nw, eps, tp, hp, op, n_embd, kernel_size, ctx->n_cus);
  });
}

}  // extern "C"
