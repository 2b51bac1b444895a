// Entry points of the slab GEMV (gemv_slab.h) for Q4_K rows: integer
// activations (Q4K8) for rows of up to 4096 columns, float activations for
// the wide rows of the down projections.  Each returns false, launching
// nothing, when the shape is not one it is built for, and the caller then
// takes the x-stationary kernel of gemv.h.
#include <cstdlib>

#include "gemv_slab.h"

namespace bch {

namespace {

// BCH_NO_SLAB=1 turns the slab path off (for measuring it against the
// x-stationary kernel).  Results are the same either way.
bool slab_enabled() {
  static const bool on = [] {
    const char *v = std::getenv("BCH_NO_SLAB");
    return !(v && v[0] == '1');
  }();
  return on;
}

template <class F, int LPR, bool NORM, class P, class In>
bool slab_maxi_switch(hipStream_t s, uint32_t maxi, uint32_t grid, const P &p, const float *x, const float *nw,
                      float eps, uint32_t n_items, uint32_t n_units, uint32_t n_cols, const In &in) {
  switch (maxi) {
    case 1: launch_slab<F, LPR, 1, NORM>(s, grid, p, x, nw, eps, n_items, n_units, n_cols, in); return true;
    case 2: launch_slab<F, LPR, 2, NORM>(s, grid, p, x, nw, eps, n_items, n_units, n_cols, in); return true;
    case 3: launch_slab<F, LPR, 3, NORM>(s, grid, p, x, nw, eps, n_items, n_units, n_cols, in); return true;
    case 4: launch_slab<F, LPR, 4, NORM>(s, grid, p, x, nw, eps, n_items, n_units, n_cols, in); return true;
    default: return false;
  }
}

template <class F, int LPR, bool NORM, class P, class In = PlainIn>
bool slab_lpr(hipStream_t s, const P &p, const float *x, const float *nw, float eps, uint32_t n_items,
              uint32_t n_units, uint32_t n_cols, uint32_t n_cus, const In &in = In{}) {
  constexpr uint32_t G = LPR <= 64 ? 256 / LPR : 1;
  const uint32_t grid = slab_grid(n_items, G, n_cus);
  const uint32_t maxi = slab_maxi(n_items, G, grid);
  return slab_maxi_switch<F, LPR, NORM>(s, maxi, grid, p, x, nw, eps, n_items, n_units, n_cols, in);
}

// Rows of up to 4096 columns (16, 32 or 64 units of 64 weights).
template <bool NORM, class P, class In = PlainIn>
bool slab_narrow(hipStream_t s, const P &p, const float *x, const float *nw, float eps, uint32_t n_items,
                 uint32_t n_cols, uint32_t n_cus, const In &in = In{}) {
  const uint32_t n_units = n_cols / 64;
  switch (lanes_for(n_units)) {
    case 16: return slab_lpr<Q4K8, 16, NORM>(s, p, x, nw, eps, n_items, n_units, n_cols, n_cus, in);
    case 32: return slab_lpr<Q4K8, 32, NORM>(s, p, x, nw, eps, n_items, n_units, n_cols, n_cus, in);
    case 64: return slab_lpr<Q4K8, 64, NORM>(s, p, x, nw, eps, n_items, n_units, n_cols, n_cus, in);
    default: return false;
  }
}

// Wide rows (4097 to 16384 columns): one row per 128-, 192- or 256-lane group.
template <class P>
bool slab_wide(hipStream_t s, const P &p, const float *x, uint32_t n_items, uint32_t n_cols, uint32_t n_cus) {
  const uint32_t n_units = n_cols / 64;
  switch (lanes_for(n_units)) {
    case 128: return slab_lpr<Q4K, 128, false>(s, p, x, nullptr, 0.f, n_items, n_units, n_cols, n_cus);
    case 192: return slab_lpr<Q4K, 192, false>(s, p, x, nullptr, 0.f, n_items, n_units, n_cols, n_cus);
    case 256: return slab_lpr<Q4K, 256, false>(s, p, x, nullptr, 0.f, n_items, n_units, n_cols, n_cus);
    default: return false;
  }
}

bool slab_format_ok(uint32_t format, uint32_t n_cols) {
  return slab_enabled() && format == Q4K::kFormat && n_cols % 256 == 0 && n_cols > 0;
}

}  // namespace

bool slab_matvec(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                 float *y, const float *nw, float eps, bool accumulate, uint32_t n_cus) {
  if (!slab_format_ok(format, n_cols)) return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (n_cols <= 4096) {
    if (accumulate)
      return nw ? slab_narrow<true>(s, PlainItems<true>{W, rb, y}, x, nw, eps, n_rows, n_cols, n_cus)
                : slab_narrow<false>(s, PlainItems<true>{W, rb, y}, x, nw, eps, n_rows, n_cols, n_cus);
    return nw ? slab_narrow<true>(s, PlainItems<false>{W, rb, y}, x, nw, eps, n_rows, n_cols, n_cus)
              : slab_narrow<false>(s, PlainItems<false>{W, rb, y}, x, nw, eps, n_rows, n_cols, n_cus);
  }
  if (nw) return false;
  return accumulate ? slab_wide(s, PlainItems<true>{W, rb, y}, x, n_rows, n_cols, n_cus)
                    : slab_wide(s, PlainItems<false>{W, rb, y}, x, n_rows, n_cols, n_cus);
}

bool slab_split_supported(uint32_t format, uint32_t n_cols) {
  const int lanes = lanes_for(n_cols / 64);  // the widths slab_narrow serves
  return slab_format_ok(format, n_cols) && n_cols <= 4096 && (lanes == 16 || lanes == 32 || lanes == 64);
}

bool slab_matvec_split(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                       const SplitOut &in, float *y, uint32_t n_cus) {
  if (!slab_split_supported(format, n_cols) || in.head_dim % 4 || in.defer > kDeferSplits || in.max_splits == 0 ||
      in.kps == 0)
    return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  const PlainItems<true> p{W, rb, y};
  if (in.gate) return slab_narrow<false>(s, p, in.out, nullptr, 0.f, n_rows, n_cols, n_cus, SplitIn<true>{in});
  return slab_narrow<false>(s, p, in.out, nullptr, 0.f, n_rows, n_cols, n_cus, SplitIn<false>{in});
}

bool slab_matvec3(hipStream_t s, uint32_t format, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2, uint32_t r0,
                  uint32_t r1, uint32_t r2, uint32_t n_cols, const float *x, float *y0, float *y1, float *y2,
                  const float *nw, float eps, uint32_t n_cus) {
  if (!slab_format_ok(format, n_cols) || n_cols > 4096 || !nw) return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return slab_narrow<true>(s, ThreeItems{W0, W1, W2, r0, r1, rb, y0, y1, y2}, x, nw, eps, r0 + r1 + r2, n_cols,
                           n_cus);
}

bool slab_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_rows,
                 uint32_t n_cols, const float *x, float *y, const float *nw, float eps, uint32_t n_cus) {
  if (!slab_format_ok(format, n_cols) || n_cols > 4096 || !nw) return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return slab_narrow<true>(s, SwigluItems{Wg, Wu, rb, y}, x, nw, eps, n_rows, n_cols, n_cus);
}

bool slab_experts_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_ff,
                         uint32_t n_cols, const uint32_t *ids, uint32_t n_used, const float *x, float *y,
                         uint32_t n_cus) {
  if (!slab_format_ok(format, n_cols) || n_cols > 4096) return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return slab_narrow<false>(s, ExpertSwigluItems{Wg, Wu, rb, ids, n_ff, y}, x, nullptr, 0.f, n_used * n_ff, n_cols,
                            n_cus);
}

bool slab_conv(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_cols, const float *x, const float *nw,
               float eps, const float *taps, float *history, float *out, uint32_t n_embd, uint32_t ksize,
               uint32_t n_cus) {
  if (!slab_format_ok(format, n_cols) || n_cols > 4096 || !nw || ksize > ConvItems::kMaxTaps || ksize < 2)
    return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return slab_narrow<true>(s, ConvItems{W, rb, n_embd, ksize, taps, history, out}, x, nw, eps, n_embd, n_cols, n_cus);
}

bool slab_gdn_in(hipStream_t s, uint32_t format, const uint8_t *Wqkv, const uint8_t *Wz, const uint8_t *Wb,
                 const uint8_t *Wa, uint32_t conv_dim, uint32_t value_dim, uint32_t n_v, uint32_t n_cols,
                 const float *x, const float *nw, float eps, const float *taps, float *hist, uint32_t ksize,
                 float *conv_out, float *z, float *beta, float *alpha, uint32_t n_cus) {
  if (!slab_format_ok(format, n_cols) || n_cols > 4096 || !nw) return false;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return slab_narrow<true>(s,
                           GdnInItems{Wqkv, Wz, Wb, Wa, conv_dim, value_dim, n_v, rb, taps, hist, ksize, conv_out, z,
                                      beta, alpha},
                           x, nw, eps, conv_dim + value_dim + 2 * n_v, n_cols, n_cus);
}

}  // namespace bch
