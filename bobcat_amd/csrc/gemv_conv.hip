// Entry points of the x-stationary GEMV (gemv.h) for one family of item policies;
// the families sit in separate files so they compile in parallel.
#include "gemv.h"

namespace bch {

bool fast_matvec_gdn_in(hipStream_t s, uint32_t format, const uint8_t *Wqkv, const uint8_t *Wz, const uint8_t *Wb,
                        const uint8_t *Wa, uint32_t conv_dim, uint32_t value_dim, uint32_t n_v, uint32_t n_cols,
                        const float *x, const float *nw, float eps, const float *taps, float *hist, uint32_t ksize,
                        float *conv_out, float *z, float *beta, float *alpha, uint32_t n_cus) {
  if (slab_gdn_in(s, format, Wqkv, Wz, Wb, Wa, conv_dim, value_dim, n_v, n_cols, x, nw, eps, taps, hist, ksize, conv_out, z, beta, alpha, n_cus)) return true;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return gemv_any(s, format,
                  GdnInItems{Wqkv, Wz, Wb, Wa, conv_dim, value_dim, n_v, rb, taps, hist, ksize, conv_out, z, beta, alpha},
                  x, nw, eps, conv_dim + value_dim + 2 * n_v, n_cols, n_cus);
}

bool fast_matvec_conv(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_cols, const float *x,
                      const float *nw, float eps, const float *taps, float *history, float *out, uint32_t n_embd,
                      uint32_t ksize, uint32_t n_cus) {
  if (slab_conv(s, format, W, n_cols, x, nw, eps, taps, history, out, n_embd, ksize, n_cus)) return true;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return gemv_any(s, format, ConvItems{W, rb, n_embd, ksize, taps, history, out}, x, nw, eps, n_embd, n_cols, n_cus);
}

}  // namespace bch
