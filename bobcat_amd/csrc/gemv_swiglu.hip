// Entry points of the x-stationary GEMV (gemv.h) for one family of item policies;
// the families sit in separate files so they compile in parallel.
#include "gemv.h"

namespace bch {

bool fast_matvec_experts_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_ff,
                                uint32_t n_cols, const uint32_t *ids, uint32_t n_used, const float *x, float *y,
                                uint32_t n_cus) {
  if (slab_experts_swiglu(s, format, Wg, Wu, n_ff, n_cols, ids, n_used, x, y, n_cus)) return true;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return gemv_any(s, format, ExpertSwigluItems{Wg, Wu, rb, ids, n_ff, y}, x, nullptr, 0.f, n_used * n_ff, n_cols,
                  n_cus);
}

bool fast_matvec_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_rows,
                        uint32_t n_cols, const float *x, float *y, const float *nw, float eps, uint32_t n_cus) {
  if (slab_swiglu(s, format, Wg, Wu, n_rows, n_cols, x, y, nw, eps, n_cus)) return true;
  const uint64_t rb = bch_row_bytes(format, n_cols);
  return gemv_any(s, format, SwigluItems{Wg, Wu, rb, y}, x, nw, eps, n_rows, n_cols, n_cus);
}

}  // namespace bch
