// Entry points of the x-stationary GEMV (gemv.h) for one family of item policies;
// the families sit in separate files so they compile in parallel.
#include "gemv.h"

namespace bch {

bool fast_matvec(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                 float *y, const float *nw, float eps, bool accumulate, uint32_t n_cus) {
  if (slab_matvec(s, format, W, n_rows, n_cols, x, y, nw, eps, accumulate, n_cus)) return true;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  if (accumulate) return gemv_any(s, format, PlainItems<true>{W, rb, y}, x, nw, eps, n_rows, n_cols, n_cus);
  return gemv_any(s, format, PlainItems<false>{W, rb, y}, x, nw, eps, n_rows, n_cols, n_cus);
}

bool fast_matvec3(hipStream_t s, uint32_t format, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2, uint32_t r0,
                  uint32_t r1, uint32_t r2, uint32_t n_cols, const float *x, float *y0, float *y1, float *y2,
                  const float *nw, float eps, uint32_t n_cus) {
  if (slab_matvec3(s, format, W0, W1, W2, r0, r1, r2, n_cols, x, y0, y1, y2, nw, eps, n_cus)) return true;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return gemv_any(s, format, ThreeItems{W0, W1, W2, r0, r1, rb, y0, y1, y2}, x, nw, eps, r0 + r1 + r2, n_cols,
                  n_cus);
}

}  // namespace bch
