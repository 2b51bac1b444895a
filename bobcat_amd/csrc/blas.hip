// The library GEMM of the prefill SwiGLU pair: hipBLASLt on expanded fp16
// weights.  At 512 tokens the gate|up product of LFM2-2.6B (21504 x 2048)
// runs at ~950 TFLOP/s in hipBLASLt against ~600 for the fused Q4_K tile,
// whose dequantisation per MFMA cannot shrink at that batch; the weights'
// fp16 copy costs 2 bytes a weight of HBM, which the 288 GB part has to
// spare.  The product's inputs are the fp16 inputs k_rms_norm_split leaves
// (each token scaled by a power of two), so the result is the same sum of
// the same fp16 products as the fused tile's, in another order.
#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

#include "kernels.h"
#include "runtime.h"

namespace bch {
namespace {

struct Blas {
  hipblasLtHandle_t handle = nullptr;
  hipblasLtMatmulDesc_t desc = nullptr;
  std::map<std::tuple<uint32_t, uint32_t, uint32_t>, hipblasLtMatmulAlgo_t> algos;
  bool broken = false;
};

std::mutex g_blas_mu;
std::map<int, Blas> g_blas;  // per device

int blas_fail(const char *what, int st) {
  return fail(BCH_ERR_EXECUTION, "hipBLASLt %s failed (status %d)", what, st);
}

// The device's handle and matmul description (f32 compute and
// scale, D = W^T-view · H: transA = T, transB = N), created on first use.
int blas_get(Blas **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(BCH_ERR_EXECUTION, "hipGetDevice failed");
  Blas &b = g_blas[dev];
  if (b.broken) return fail(BCH_ERR_EXECUTION, "hipBLASLt unavailable on device %d", dev);
  if (!b.handle) {
    int st;
    if ((st = hipblasLtCreate(&b.handle)) != HIPBLAS_STATUS_SUCCESS) {
      b.broken = true;
      return blas_fail("create", st);
    }
    if ((st = hipblasLtMatmulDescCreate(&b.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F)) != HIPBLAS_STATUS_SUCCESS) {
      b.broken = true;
      return blas_fail("matmul description", st);
    }
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(b.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    hipblasLtMatmulDescSetAttribute(b.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  }
  *out = &b;
  return BCH_OK;
}

struct Layouts {
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  ~Layouts() {
    if (a) hipblasLtMatrixLayoutDestroy(a);
    if (b) hipblasLtMatrixLayoutDestroy(b);
    if (d) hipblasLtMatrixLayoutDestroy(d);
  }
};

}  // namespace

int blas_prepare() {
  std::lock_guard<std::mutex> lk(g_blas_mu);
  Blas *b;
  return blas_get(&b);
}

// D [n_tokens][n_rows] (f32, row-major) = H [n_tokens][n_cols] (fp16) ·
// W16 [n_rows][n_cols]^T.  In hipBLASLt's column-major terms D^T (n_rows x
// n_tokens, ld n_rows) = op_T(W16 as n_cols x n_rows) · H^T (n_cols x
// n_tokens).
int run_blas_gemm_f16(hipStream_t s, const _Float16 *W16, uint32_t n_rows, uint32_t n_cols, const _Float16 *H,
                      uint32_t n_tokens, float *D) {
  std::lock_guard<std::mutex> lk(g_blas_mu);
  Blas *b;
  BCH_TRY(blas_get(&b));
  Layouts L;
  int st;
  if ((st = hipblasLtMatrixLayoutCreate(&L.a, HIP_R_16F, n_cols, n_rows, n_cols)) ||
      (st = hipblasLtMatrixLayoutCreate(&L.b, HIP_R_16F, n_cols, n_tokens, n_cols)) ||
      (st = hipblasLtMatrixLayoutCreate(&L.d, HIP_R_32F, n_rows, n_tokens, n_rows)))
    return blas_fail("matrix layout", st);
  const auto key = std::make_tuple(n_rows, n_cols, n_tokens);
  auto it = b->algos.find(key);
  if (it == b->algos.end()) {
    hipblasLtMatmulPreference_t pref;
    if ((st = hipblasLtMatmulPreferenceCreate(&pref))) return blas_fail("preference", st);
    // Algorithms without a workspace only: nothing is shared between calls.
    const uint64_t ws = 0;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    st = hipblasLtMatmulAlgoGetHeuristic(b->handle, b->desc, L.a, L.b, L.d, L.d, pref, 1, res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st || found < 1) return blas_fail("heuristic", st ? st : -1);
    it = b->algos.emplace(key, res[0].algo).first;
  }
  const float alpha = 1.0f, beta = 0.0f;
  if ((st = hipblasLtMatmul(b->handle, b->desc, &alpha, W16, L.a, H, L.b, &beta, D, L.d, D, L.d, &it->second,
                            nullptr, 0, s)))
    return blas_fail("matmul", st);
  return BCH_OK;
}

// The SwiGLU pair of a prefill batch on the library GEMM: `split` holds the
// batch's fp16 inputs (k_rms_norm_split's), pair_us their token scales,
// gate_up16 the expanded [2 n_ff][n_cols] weights.  False (with the error
// printed) when hipBLASLt fails, so the caller runs the Q4_K tile instead.
bool run_blas_pair(hipStream_t s, const _Float16 *gate_up16, uint32_t n_ff, uint32_t n_cols, uint32_t n_tokens,
                   void *split, float *pair_out, const float *pair_us, float *ffn) {
  if (run_blas_gemm_f16(s, gate_up16, 2 * n_ff, n_cols, static_cast<const _Float16 *>(split), n_tokens, pair_out) !=
      BCH_OK) {
    fprintf(stderr, "bobcat_hip: %s; the SwiGLU pair runs on the Q4_K tile\n", bch_last_error());
    return false;
  }
  run_swiglu_split(s, pair_out, n_ff, n_tokens, pair_us, ffn, split);
  return true;
}

}  // namespace bch
