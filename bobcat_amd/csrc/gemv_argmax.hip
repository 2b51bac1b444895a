// Entry points of the x-stationary GEMV (gemv.h) for one family of item policies;
// the families sit in separate files so they compile in parallel.
#include "gemv.h"

namespace bch {

bool fast_matvec_argmax(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                        const float *x, float *y, const float *nw, float eps, uint64_t *partials, uint32_t n_cus) {
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return gemv_any(s, format, ArgmaxItems{W, rb, y, partials}, x, nw, eps, n_rows, n_cols, n_cus);
}

}  // namespace bch
