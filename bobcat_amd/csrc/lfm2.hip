// The LFM2 driver: the MI355X counterpart of Lfm2Metal
// (crates/bobcat/src/lfm2_metal.rs:125-1548).
//
// * Weights are copied once into one HBM allocation, each tensor 256-byte
//   aligned (the reference wraps the mmap'd file; MI355X has no unified
//   memory).
// * A decode step is the launch sequence of Recorder::record_step
//   (lfm2_metal.rs:1162-1242) with three fusions: q/k/v projections in one
//   launch, split-K attention with its combine in one launch, and the conv
//   input projection fused with the convolution (as the reference does).
// * Every kernel of a step reads the sequence position from a device
//   counter, so the step is captured once as a HIP graph and replayed.
//   generate() replays "argmax of the logits into the next token slot,
//   advance the counter, run the step" with no host round trip per token
//   (the reference keeps 3 command buffers in flight for the same reason,
//   lfm2_metal.rs:29-31, 564-655).
// * Prefill runs in batches of up to 512 tokens through the MFMA GEMM
//   (Recorder::record_batch, lfm2_metal.rs:1455-1548).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "driver.h"

namespace bch {

constexpr uint32_t kAttnQueryBatch = 64;

struct Layer {
  bool attention = false;
  uint32_t cache_index = 0;
  const float *attn_norm = nullptr, *ffn_norm = nullptr;
  const float *taps = nullptr;
  DevMatrix in_proj, out_proj, wq, wk, wv, wo, gate, up, down;
  const float *q_norm = nullptr, *k_norm = nullptr;
  // Rows of wq, wk and wv together when the three lie back to back in
  // device memory in one format (one prefill GEMM), else 0.
  uint32_t qkv_rows = 0;
  // Mixture of experts (lfm2.rs:128-142): the F32 router, the routing bias
  // and the stacked expert matrices.
  bool moe = false;
  DevMatrix router, gate_exps, up_exps, down_exps;
  const float *expert_bias = nullptr;
  // Dense SwiGLU: the gate rows then the up rows as fp16 [2 n_ff][n_embd]
  // for the library GEMM of prefill batches (expanded once at creation).
  _Float16 *gate_up16 = nullptr;
};


}  // namespace bch

using namespace bch;

struct bch_lfm2 : bch::Sequence {
  // Hyperparameters (lfm2.rs:17-49).
  uint32_t n_ff, n_heads, n_kv_heads, head_dim, conv_kernel;
  uint32_t n_experts = 0, n_used = 0, n_ff_expert = 0;
  float rope_theta, norm_eps;
  uint32_t n_attn = 0, n_conv = 0;
  uint32_t q_dim, kv_dim;
  std::vector<Layer> layers;
  DevMatrix token_embd, output;
  const float *output_norm = nullptr;
  // Device memory.
  void *k_cache = nullptr, *v_cache = nullptr;
  float *conv_state = nullptr, *hidden = nullptr, *normed = nullptr, *bcx = nullptr, *conv_out = nullptr;
  float *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *ffn = nullptr;
  float *qkv = nullptr;  // prefill: q | k | v of each token from one GEMM (Layer::qkv_rows)
  float *partials = nullptr;
  uint64_t partial_floats = 0;  // floats of `partials`
  uint32_t *counters = nullptr;
  uint32_t *route = nullptr;  // expert routes of a batch (route_bytes(n_used, batch))
  float *route_scores = nullptr;  // router scores of a batch [batch][n_experts]
  uint32_t *route_counters = nullptr;  // [batch], zeroed
  // Batched experts: the batch's entries grouped by expert, each entry's
  // SwiGLU activations and down projection (Recorder::grouped_moe).
  uint32_t *moe_offsets = nullptr, *moe_entries = nullptr;
  float *expert_ffn = nullptr, *expert_out = nullptr;
  void *split = nullptr;  // prefill GEMM scratch: split inputs and split-K partials (matmul_scratch_bytes)
  uint64_t split_bytes = 0;
  bool kv_half = true;

  uint64_t cache_elems_per_layer() const { return (uint64_t)n_ctx * kv_dim; }
  void *cache_layer(void *base, uint32_t ci) const {
    return static_cast<char *>(base) + cache_elems_per_layer() * ci * (kv_half ? 2 : 4);
  }
  void *cache_slot(void *base, uint32_t ci, uint32_t pos) const {
    return static_cast<char *>(cache_layer(base, ci)) + (uint64_t)pos * kv_dim * (kv_half ? 2 : 4);
  }

  void record_step(hipStream_t st, bool greedy_input, bool trace, bool short_ctx) override;
  void record_batch(hipStream_t st, uint32_t pos, uint32_t count, bool want_logits, bool trace) override;
  std::vector<std::pair<void *, uint64_t>> state_regions() const override {
    return {{conv_state, (uint64_t)n_conv * (conv_kernel - 1) * n_embd * 4}};
  }
};

namespace bch {

// ---------------------------------------------------------------------
// Recording
// ---------------------------------------------------------------------

// The mixture of experts of one token (Recorder::moe with n = 1,
// lfm2_metal.rs:1251-1313): route `x` (RMS-normalised into `normed` when
// `norm` is given, else `x` is already normalised), the SwiGLU rows of the
// picked experts into m->ffn, then their weighted down projections added
// to `residual`.
static void record_moe_token(bch_lfm2 *m, hipStream_t s, const Layer &L, const float *x, const float *norm,
                             float *normed, uint32_t *route, float *residual) {
  const uint32_t n = m->n_embd, cus = m->ctx->n_cus;
  if (norm)
    run_moe_route(s, x, norm, m->norm_eps, normed, reinterpret_cast<const float *>(L.router.data), L.expert_bias,
                  route, n, m->n_experts, m->n_used, 1, m->route_scores, m->route_counters);
  const float *in = norm ? normed : x;
  fast_matvec_experts_swiglu(s, L.gate_exps.format, L.gate_exps.data, L.up_exps.data, m->n_ff_expert, n, route,
                             m->n_used, in, m->ffn, cus);
  run_experts_down(s, L.down_exps.format, L.down_exps.data, n, m->n_ff_expert, m->ffn, route, m->n_used, residual,
                   cus);
}

// One decode step at the position *m->dpos (Recorder::record_step).  With
// `greedy_input`, the step first takes the greedy token of the previous
// logits (from m->argmax_partials), stores it at tokens[*dpos + 1] and
// advances *dpos.  The logits leave their argmax partials behind for the
// next such step.  With `trace`, activations are copied into m->trace:
// embedding, each layer's output, final norm.
static void lfm2_step(bch_lfm2 *m, hipStream_t s, bool greedy_input, bool trace, bool short_ctx) {
  const uint32_t n = m->n_embd, cus = m->ctx->n_cus;
  uint32_t *dp = m->dpos;
  const uint64_t tstride = (uint64_t)m->trace_rows * n;  // floats per traced activation
  const uint64_t embd_rb = bch_row_bytes(m->token_embd.format, n);
  if (greedy_input)
    run_embed_next(s, m->token_embd.format, m->token_embd.data, embd_rb, m->tokens, m->hidden, n, dp,
                   m->argmax_partials, kArgmaxPartials);
  else
    run_embed(s, m->token_embd.format, m->token_embd.data, embd_rb, m->tokens, m->hidden, n, 1, dp);
  if (trace) run_copy(s, m->hidden, m->trace, n, nullptr, 0);
  for (uint32_t il = 0; il < m->n_layers; il++) {
    const Layer &L = m->layers[il];
    if (!L.attention) {
      float *hist = m->conv_state + (uint64_t)L.cache_index * (m->conv_kernel - 1) * n;
      run_matvec_conv(s, L.in_proj.format, L.in_proj.data, n, m->hidden, L.attn_norm, m->norm_eps, L.taps, hist,
                      m->conv_out, n, m->conv_kernel, cus);
      run_matvec(s, L.out_proj.format, L.out_proj.data, n, n, m->conv_out, m->hidden, nullptr, 0.f, true, cus);
    } else {
      const uint32_t ci = L.cache_index;
      if (L.wq.format == L.wk.format && L.wq.format == L.wv.format) {
        run_matvec3(s, L.wq.format, L.wq.data, L.wk.data, L.wv.data, m->q_dim, m->kv_dim, m->kv_dim, n, m->hidden,
                    m->q, m->k, m->v, L.attn_norm, m->norm_eps, cus);
      } else {  // mixed formats (Q4_K_M files keep attn_v in Q6_K): one launch each
        run_matvec(s, L.wq.format, L.wq.data, m->q_dim, n, m->hidden, m->q, L.attn_norm, m->norm_eps, false, cus);
        run_matvec(s, L.wk.format, L.wk.data, m->kv_dim, n, m->hidden, m->k, L.attn_norm, m->norm_eps, false, cus);
        run_matvec(s, L.wv.format, L.wv.data, m->kv_dim, n, m->hidden, m->v, L.attn_norm, m->norm_eps, false, cus);
      }
      AttnDecodeArgs ad{};
      ad.q = m->q;
      ad.k = m->k;
      ad.v = m->v;
      ad.q_norm = L.q_norm;
      ad.k_norm = L.k_norm;
      ad.freqs = rope_table(m->rope_theta, m->head_dim);
      ad.eps = m->norm_eps;
      ad.scale = 1.0f / sqrtf((float)m->head_dim);
      ad.k_cache = m->cache_layer(m->k_cache, ci);
      ad.v_cache = m->cache_layer(m->v_cache, ci);
      ad.partials = m->partials;
      ad.counters = m->counters;
      ad.out = m->attn;
      ad.n_heads = m->n_heads;
      ad.n_kv = m->n_kv_heads;
      ad.head_dim = m->head_dim;
      ad.max_splits = attn_decode_max_splits(m->n_ctx, m->head_dim, m->kv_half);
      ad.dpos = dp;
      ad.q_head_stride = m->head_dim;
      ad.n_rot = m->head_dim;
      ad.gate = nullptr;
      ad.gate_head_stride = 0;
      // Short contexts leave the splits' combine to wo's input staging.
      const bool defer = short_ctx && slab_split_supported(L.wo.format, m->q_dim);
      ad.defer_splits = defer ? kDeferSplits : 0;
      run_attn_decode(s, ad, m->kv_half);
      const SplitOut so{m->partials, m->attn, nullptr, dp, attn_decode_keys_per_split(m->head_dim, m->kv_half),
                        ad.max_splits, m->head_dim, 0, ad.defer_splits};
      if (!defer || !slab_matvec_split(s, L.wo.format, L.wo.data, n, m->q_dim, so, m->hidden, cus))
        run_matvec(s, L.wo.format, L.wo.data, n, m->q_dim, m->attn, m->hidden, nullptr, 0.f, true, cus);
    }
    if (L.moe) {
      record_moe_token(m, s, L, m->hidden, L.ffn_norm, m->normed, m->route, m->hidden);
    } else {
      run_matvec_swiglu(s, L.gate.format, L.gate.data, L.up.data, m->n_ff, n, m->hidden, m->ffn, L.ffn_norm,
                        m->norm_eps, cus);
      run_matvec(s, L.down.format, L.down.data, n, m->n_ff, m->ffn, m->hidden, nullptr, 0.f, true, cus);
    }
    if (trace) run_copy(s, m->hidden, m->trace + (1 + il) * tstride, n, nullptr, 0);
  }
  if (trace) run_rms_norm(s, m->hidden, m->output_norm, m->trace + (1 + m->n_layers) * tstride, n, 1, m->norm_eps);
  if (!fast_matvec_argmax(s, m->output.format, m->output.data, m->n_vocab, n, m->hidden, m->logits, m->output_norm,
                          m->norm_eps, m->argmax_partials, cus)) {
    run_matvec(s, m->output.format, m->output.data, m->n_vocab, n, m->hidden, m->logits, m->output_norm, m->norm_eps,
               false, cus);
    run_argmax_partials(s, m->logits, m->n_vocab, m->argmax_partials, kArgmaxPartials);
  }
}

// With BCH_LFM2_CHECK=1 in the environment, record_batch synchronises after
// each launch and reports on stderr the first one that leaves a non-finite
// value in its output (a diagnostics mode, like the reference's per-launch
// profiling in backend.rs:1285-1340).
static bool check_mode() {
  static const bool on = getenv("BCH_LFM2_CHECK") && atoi(getenv("BCH_LFM2_CHECK")) != 0;
  return on;
}

static void check_finite(hipStream_t s, const char *what, uint32_t layer, const float *p, uint64_t count) {
  if (!check_mode()) return;
  static bool reported = false;
  if (reported) return;
  hipStreamSynchronize(s);
  std::vector<float> h(count);
  hipMemcpy(h.data(), p, count * 4, hipMemcpyDeviceToHost);
  for (uint64_t i = 0; i < count; i++) {
    if (!std::isfinite(h[i])) {
      fprintf(stderr, "bch_lfm2: first non-finite value after %s of layer %u (element %llu of %llu)\n", what, layer,
              (unsigned long long)i, (unsigned long long)count);
      reported = true;
      return;
    }
  }
}

// A prefill batch of `count` tokens at positions pos.. (record_batch).
static void lfm2_batch(bch_lfm2 *m, hipStream_t s, uint32_t pos, uint32_t count, bool want_logits, bool trace) {
  const uint32_t n = m->n_embd, cus = m->ctx->n_cus;
  const uint64_t tstride = (uint64_t)m->trace_rows * n;
  run_embed(s, m->token_embd.format, m->token_embd.data, bch_row_bytes(m->token_embd.format, n), m->tokens + pos,
            m->hidden, n, count, nullptr);
  if (trace) run_copy(s, m->hidden, m->trace, count * n, nullptr, 0);
  // A column-split sum into the residual stream (out_proj, wo, down) is left
  // to the norm that reads the residual next, unless something else reads
  // it first (the trace copy, the diagnostics checks).
  PendingSum pend;
  PendingSum *const defer = trace || check_mode() ? nullptr : &pend;
  for (uint32_t il = 0; il < m->n_layers; il++) {
    const Layer &L = m->layers[il];
    // The norm also writes the fp16 inputs of the projection that follows.
    run_rms_norm_split(s, m->hidden, L.attn_norm, m->normed, n, count, m->norm_eps, m->split, &pend);
    check_finite(s, "attn_norm", il, m->normed, (uint64_t)count * n);
    if (!L.attention) {
      float *hist = m->conv_state + (uint64_t)L.cache_index * (m->conv_kernel - 1) * n;
      run_matmul(s, L.in_proj.format, L.in_proj.data, 3 * n, n, m->normed, m->bcx, count, 0, m->split, m->split_bytes,
                 true);
      check_finite(s, "in_proj", il, m->bcx, (uint64_t)count * 3 * n);
      // The convolution also writes the fp16 inputs of the out projection.
      const bool split = run_short_conv_split(s, m->bcx, L.taps, hist, m->conv_out, n, m->conv_kernel, count, m->split);
      if (!split) run_short_conv_batch(s, m->bcx, L.taps, hist, m->conv_out, n, m->conv_kernel, count);
      check_finite(s, "short_conv", il, m->conv_out, (uint64_t)count * n);
      run_matmul(s, L.out_proj.format, L.out_proj.data, n, n, m->conv_out, m->hidden, count, 1, m->split, m->split_bytes,
                 split, nullptr, defer);
      check_finite(s, "out_proj", il, m->hidden, (uint64_t)count * n);
    } else {
      const uint32_t ci = L.cache_index;
      // q, k and v (which read the fp16 inputs the norm wrote): one GEMM
      // when the three matrices lie back to back, each token's row then
      // q | k | v.
      const float *qs = m->q, *ks = m->k, *vs = m->v;
      uint32_t qkv_stride = m->q_dim, kv_stride = m->kv_dim;
      if (L.qkv_rows) {
        run_matmul(s, L.wq.format, L.wq.data, L.qkv_rows, n, m->normed, m->qkv, count, 0, m->split, m->split_bytes,
                   true);
        qs = m->qkv, ks = m->qkv + m->q_dim, vs = m->qkv + m->q_dim + m->kv_dim;
        qkv_stride = kv_stride = L.qkv_rows;
      } else {
        run_matmul(s, L.wq.format, L.wq.data, m->q_dim, n, m->normed, m->q, count, 0, m->split, m->split_bytes, true);
        run_matmul(s, L.wk.format, L.wk.data, m->kv_dim, n, m->normed, m->k, count, 0, m->split, m->split_bytes, true);
        run_matmul(s, L.wv.format, L.wv.data, m->kv_dim, n, m->normed, m->v, count, 0, m->split, m->split_bytes, true);
      }
      check_finite(s, "q", il, qs, (uint64_t)count * qkv_stride);
      run_norm_rope(s, qs, m->q, false, L.q_norm, m->n_heads, m->head_dim, m->head_dim, m->head_dim, pos, nullptr,
                    count, qkv_stride, m->q_dim, m->rope_theta, m->norm_eps, 0);
      run_norm_rope(s, ks, m->cache_slot(m->k_cache, ci, pos), m->kv_half, L.k_norm, m->n_kv_heads, m->head_dim,
                    m->head_dim, m->head_dim, pos, nullptr, count, kv_stride, m->kv_dim, m->rope_theta, m->norm_eps,
                    0);
      run_copy_rows(s, vs, kv_stride, m->cache_slot(m->v_cache, ci, pos), m->kv_dim, m->kv_half, m->kv_dim, count);
      if (attn_prefill_mfma_supported(m->n_heads, m->n_kv_heads, m->head_dim, m->kv_half))
        run_attn_prefill_mfma(s, m->q, m->cache_layer(m->k_cache, ci), m->cache_layer(m->v_cache, ci), m->attn,
                              m->n_heads, m->n_kv_heads, m->head_dim, pos, count, m->q_dim, m->q_dim,
                              1.0f / sqrtf((float)m->head_dim), m->partials, m->partial_floats);
      else
      for (uint32_t q0 = 0; q0 < count; q0 += kAttnQueryBatch) {
        const uint32_t nq = std::min(kAttnQueryBatch, count - q0);
        AttnDecodeArgs ad{};
        ad.q = m->q + (uint64_t)q0 * m->q_dim;
        ad.q_stride = m->q_dim;
        ad.q_head_stride = m->head_dim;
        ad.scale = 1.0f / sqrtf((float)m->head_dim);
        ad.k_cache = m->cache_layer(m->k_cache, ci);
        ad.v_cache = m->cache_layer(m->v_cache, ci);
        ad.partials = m->partials;
        ad.counters = m->counters;
        ad.out = m->attn + (uint64_t)q0 * m->q_dim;
        ad.out_stride = m->q_dim;
        ad.n_heads = m->n_heads;
        ad.n_kv = m->n_kv_heads;
        ad.head_dim = m->head_dim;
        ad.first_pos = pos + q0;
        ad.max_splits = attn_decode_max_splits(pos + q0 + nq, m->head_dim, m->kv_half);
        run_attn_prefill(s, ad, m->kv_half, nq);
      }
      check_finite(s, "attention", il, m->attn, (uint64_t)count * m->q_dim);
      run_matmul(s, L.wo.format, L.wo.data, n, m->q_dim, m->attn, m->hidden, count, 1, m->split, m->split_bytes, false,
                 nullptr, defer);
      check_finite(s, "attn_output", il, m->hidden, (uint64_t)count * n);
    }
    // (The MoE experts' shared input is this norm's output too.)
    const bool pair_ok = L.gate_up16 && count > kBlasPairMinTokens;
    run_rms_norm_split(s, m->hidden, L.ffn_norm, m->normed, n, count, m->norm_eps, m->split, &pend,
                       pair_ok ? m->pair_us : nullptr);
    check_finite(s, "ffn_norm", il, m->normed, (uint64_t)count * n);
    if (L.moe) {
      // Route the whole batch in one launch, then each token's experts.
      run_moe_route(s, m->normed, nullptr, 0.f, nullptr, reinterpret_cast<const float *>(L.router.data),
                    L.expert_bias, m->route, n, m->n_experts, m->n_used, count, m->route_scores, m->route_counters);
      const bool grouped = count > 1 && n % 256 == 0 && m->n_ff_expert % 256 == 0 &&
                           L.gate_exps.format == L.up_exps.format;
      if (grouped) {
        // lfm2_metal.rs:1317-1380: group the entries by expert, one MFMA
        // GEMM per stacked matrix over all experts, then the weighted sum.
        run_moe_group(s, m->route, m->moe_offsets, m->moe_entries, m->n_experts, m->n_used, count);
        run_matmul_experts(s, L.gate_exps.format, L.gate_exps.data, L.up_exps.data, m->n_ff_expert, n,
                           m->n_experts, m->normed, true, m->moe_offsets, m->moe_entries, m->n_used, m->expert_ffn,
                           count, m->split, true);
        run_matmul_experts(s, L.down_exps.format, L.down_exps.data, nullptr, n, m->n_ff_expert, m->n_experts,
                           m->expert_ffn, false, m->moe_offsets, m->moe_entries, m->n_used, m->expert_out, count,
                           m->split);
        run_moe_combine(s, m->expert_out, m->route, m->hidden, n, m->n_used, count);
      } else {
        for (uint32_t t = 0; t < count; t++)
          record_moe_token(m, s, L, m->normed + (uint64_t)t * n, nullptr, nullptr,
                           m->route + (uint64_t)t * 2 * m->n_used, m->hidden + (uint64_t)t * n);
      }
      check_finite(s, "moe", il, m->hidden, (uint64_t)count * n);
    } else {
      // The pair through the library GEMM on the expanded weights when the
      // model has them; its SwiGLU also writes the down projection's inputs.
      const bool blas_pair = pair_ok && run_blas_pair(s, L.gate_up16, m->n_ff, n, count, m->split, m->pair_out,
                                                      m->pair_us, check_mode() ? m->ffn : nullptr);
      if (!blas_pair && L.gate.format == L.up.format) {
        // Gate and up in one paired launch: ffn = silu(gate·x) ⊙ (up·x).
        run_matmul(s, L.gate.format, L.gate.data, m->n_ff, n, m->normed, m->ffn, count, 3, m->split, m->split_bytes,
                   true, L.up.data);
      } else if (!blas_pair) {
        run_matmul(s, L.gate.format, L.gate.data, m->n_ff, n, m->normed, m->ffn, count, 0, m->split, m->split_bytes,
                   true);
        check_finite(s, "gate", il, m->ffn, (uint64_t)count * m->n_ff);
        run_matmul(s, L.up.format, L.up.data, m->n_ff, n, m->normed, m->ffn, count, 2, m->split, m->split_bytes, true);
      }
      check_finite(s, "swiglu", il, m->ffn, (uint64_t)count * m->n_ff);
      run_matmul(s, L.down.format, L.down.data, n, m->n_ff, m->ffn, m->hidden, count, 1, m->split, m->split_bytes,
                 blas_pair, nullptr, defer);
      check_finite(s, "down", il, m->hidden, (uint64_t)count * n);
    }
    if (trace) run_copy(s, m->hidden, m->trace + (1 + il) * tstride, count * n, nullptr, 0);
  }
  finish_pending_sum(s, pend, m->hidden);
  if (trace) run_rms_norm(s, m->hidden, m->output_norm, m->trace + (1 + m->n_layers) * tstride, n, count, m->norm_eps);
  if (want_logits)
    run_matvec(s, m->output.format, m->output.data, m->n_vocab, n, m->hidden + (uint64_t)(count - 1) * n, m->logits,
               m->output_norm, m->norm_eps, false, cus);
}

}  // namespace bch

void bch_lfm2::record_step(hipStream_t st, bool greedy_input, bool trace, bool short_ctx) {
  lfm2_step(this, st, greedy_input, trace, short_ctx);
}
void bch_lfm2::record_batch(hipStream_t st, uint32_t pos, uint32_t count, bool want_logits, bool trace) {
  lfm2_batch(this, st, pos, count, want_logits, trace);
}

namespace bch {
}  // namespace bch

extern "C" {

int bch_lfm2_new(bch_ctx *ctx, const bch_lfm2_model *md, uint32_t n_ctx, int kv_half, bch_lfm2 **out) {
  *out = nullptr;
  if (n_ctx == 0) return fail(BCH_ERR_ARGUMENT, "the context must hold a token");
  if (!md->layers || md->n_layers == 0 || md->n_embd == 0 || md->n_heads == 0)
    return fail(BCH_ERR_ARGUMENT, "the model has no layers");
  const uint32_t n = md->n_embd, hd = md->head_dim;
  if (md->conv_kernel < 2 || md->conv_kernel > 9)
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "a convolution of 2 to 9 taps, got %u", md->conv_kernel);
  bool any_attn = false, any_moe = false;
  for (uint32_t il = 0; il < md->n_layers; il++) {
    any_moe |= md->layers[il].is_moe != 0;
    any_attn |= md->layers[il].is_attention != 0;
  }
  if (any_moe) {
    // check_experts (lfm2_metal.rs:842-866) and this build's kernel limits.
    if (md->n_experts > kMoeMaxExperts || md->n_experts_used > kMoeMaxUsed || md->n_experts_used == 0 ||
        md->n_experts_used > md->n_experts)
      return fail(BCH_ERR_EXPERT_LIMITS, "at most %u of %u experts per token, got %u of %u", kMoeMaxUsed,
                  kMoeMaxExperts, md->n_experts_used, md->n_experts);
    if (n % 4 || n > 16384 || md->n_ff_expert == 0 || md->n_ff_expert > 4096 || md->n_ff_expert % 256)
      return fail(BCH_ERR_UNSUPPORTED_FORMAT, "expert shapes %u x %u are outside the expert kernels", md->n_ff_expert,
                  n);
  }
  if (any_attn) {
    const uint32_t group = md->n_kv_heads ? md->n_heads / md->n_kv_heads : 0;
    if (!md->n_kv_heads || md->n_heads % md->n_kv_heads || group > 4 || hd < 32 || hd > 256 || (hd & (hd - 1)))
      return fail(BCH_ERR_ATTENTION_LIMITS,
                  "a head size of 32, 64, 128 or 256 and at most 4 query heads per KV head, got %u and %u",
                  hd, group);
  }
  auto *m = new bch_lfm2();
  m->ctx = ctx;
  m->s = ctx->stream;
  m->n_layers = md->n_layers;
  m->n_embd = n;
  m->n_ff = md->n_ff;
  m->n_heads = md->n_heads;
  m->n_kv_heads = md->n_kv_heads;
  m->head_dim = hd;
  m->n_vocab = md->n_vocab;
  m->conv_kernel = md->conv_kernel;
  m->n_experts = any_moe ? md->n_experts : 0;
  m->n_used = any_moe ? md->n_experts_used : 0;
  m->n_ff_expert = any_moe ? md->n_ff_expert : 0;
  m->rope_theta = md->rope_theta;
  m->norm_eps = md->norm_eps;
  m->q_dim = md->n_heads * hd;
  m->kv_dim = md->n_kv_heads * hd;
  m->n_ctx = n_ctx;
  m->kv_half = kv_half != 0;
  m->batch = std::min(n_ctx, kPrefillBatch);
  auto cleanup = [&](int rc) {
    bch_lfm2_free(m);
    return rc;
  };

  // Validate and plan the weight upload.
  Uploader up;
  m->layers.resize(md->n_layers);
  auto vec = [&](const float *p, uint64_t count, const float **field, const char *name) {
    return up.vec(p, count, field, name);
  };
  auto mat = [&](const bch_matrix &src, uint32_t rows, uint32_t cols, DevMatrix *dst, const char *name) {
    return up.mat(src, rows, cols, dst, name);
  };
  for (uint32_t il = 0; il < md->n_layers; il++) {
    const bch_lfm2_layer &S = md->layers[il];
    Layer &L = m->layers[il];
    int rc;
    if ((rc = vec(S.attn_norm, n, &L.attn_norm, "attn_norm")) || (rc = vec(S.ffn_norm, n, &L.ffn_norm, "ffn_norm")))
      return cleanup(rc);
    L.attention = S.is_attention != 0;
    if (L.attention) {
      L.cache_index = m->n_attn++;
      if ((rc = mat(S.wq, m->q_dim, n, &L.wq, "attn_q")) || (rc = mat(S.wk, m->kv_dim, n, &L.wk, "attn_k")) ||
          (rc = mat(S.wv, m->kv_dim, n, &L.wv, "attn_v")) || (rc = mat(S.wo, n, m->q_dim, &L.wo, "attn_output")) ||
          (rc = vec(S.q_norm, hd, &L.q_norm, "attn_q_norm")) || (rc = vec(S.k_norm, hd, &L.k_norm, "attn_k_norm")))
        return cleanup(rc);
    } else {
      L.cache_index = m->n_conv++;
      if ((rc = mat(S.in_proj, 3 * n, n, &L.in_proj, "shortconv.in_proj")) ||
          (rc = mat(S.out_proj, n, n, &L.out_proj, "shortconv.out_proj")) ||
          (rc = vec(S.conv_taps, (uint64_t)n * md->conv_kernel, &L.taps, "shortconv.conv")))
        return cleanup(rc);
      // The fused conv projection takes every GEMV format up to 16384 columns
      // (the x-stationary kernel); wider rows only as Q4_K.
      if (S.in_proj.format != BCH_Q4K && n > 16384)
        return cleanup(fail(BCH_ERR_UNSUPPORTED_FORMAT, "layer %u: the fused conv projection needs Q4_K", il));
    }
    L.moe = S.is_moe != 0;
    if (L.moe) {
      const uint32_t ne = md->n_experts, nff = md->n_ff_expert;
      if ((rc = mat(S.router, ne, n, &L.router, "ffn_gate_inp")) ||
          (rc = vec(S.expert_bias, ne, &L.expert_bias, "exp_probs_b")) ||
          (rc = mat(S.gate_exps, ne * nff, n, &L.gate_exps, "ffn_gate_exps")) ||
          (rc = mat(S.up_exps, ne * nff, n, &L.up_exps, "ffn_up_exps")) ||
          (rc = mat(S.down_exps, ne * n, nff, &L.down_exps, "ffn_down_exps")))
        return cleanup(rc);
      if (S.router.format != BCH_F32)
        return cleanup(fail(BCH_ERR_UNSUPPORTED_FORMAT, "layer %u: the router must be F32, got format %u", il,
                            S.router.format));
      if (S.gate_exps.format != S.up_exps.format || (S.gate_exps.format != BCH_Q4K && S.gate_exps.format != BCH_F16 &&
                                                     S.gate_exps.format != BCH_F32) ||
          (S.down_exps.format != BCH_Q4K && S.down_exps.format != BCH_F16 && S.down_exps.format != BCH_F32))
        return cleanup(fail(BCH_ERR_UNSUPPORTED_FORMAT, "layer %u: experts in Q4_K, F16 or F32", il));
    } else {
      if ((rc = mat(S.gate, md->n_ff, n, &L.gate, "ffn_gate")) || (rc = mat(S.up, md->n_ff, n, &L.up, "ffn_up")) ||
          (rc = mat(S.down, n, md->n_ff, &L.down, "ffn_down")))
        return cleanup(rc);
      if (S.gate.format != S.up.format)
        return cleanup(fail(BCH_ERR_UNSUPPORTED_FORMAT, "layer %u: gate and up matrices of one format", il));
    }
  }
  {
    int rc;
    if ((rc = mat(md->token_embd, md->n_vocab, n, &m->token_embd, "token_embd")) ||
        (rc = mat(md->output, md->n_vocab, n, &m->output, "output")) ||
        (rc = vec(md->output_norm, n, &m->output_norm, "token_embd_norm")))
      return cleanup(rc);
  }
  if (int rc = m->upload(up)) return cleanup(rc);
  bool any_qkv = false;
  for (Layer &L : m->layers) {
    if (!L.attention || L.wq.format != L.wk.format || L.wq.format != L.wv.format) continue;
    const uint64_t rb = bch_row_bytes(L.wq.format, n);
    if (L.wk.data == L.wq.data + rb * m->q_dim && L.wv.data == L.wk.data + rb * m->kv_dim) {
      L.qkv_rows = m->q_dim + 2 * m->kv_dim;
      any_qkv = true;
    }
  }
  // Buffers (Lfm2Metal::new, lfm2_metal.rs:153-203).
  {
    const uint64_t rows = m->batch;
    const uint64_t cache = (uint64_t)m->n_attn * n_ctx * m->kv_dim * (m->kv_half ? 2 : 4);
    uint64_t partial_floats = attention_partial_floats(std::min<uint32_t>(m->batch, kAttnQueryBatch), m->n_heads,
                                                            hd, attn_decode_max_splits(n_ctx, hd, m->kv_half));
    // The MFMA prefill attention splits the keys of a batch up to 4 ways.
    if (attn_prefill_mfma_supported(m->n_heads, m->n_kv_heads, hd, m->kv_half))
      partial_floats = std::max(partial_floats, attn_prefill_partial_floats(m->batch, m->n_heads, hd, 4));
    m->partial_floats = partial_floats;
    const uint32_t widest = std::max({n, m->q_dim, m->n_ff});
    const uint64_t split_bytes = m->split_bytes =
        std::max(matmul_scratch_bytes((uint32_t)rows, widest, n),
                 matmul_split_bytes((uint32_t)(std::max(1u, m->n_used) * rows), std::max(1u, m->n_ff_expert)));
    int rc = 0;
    (void)((rc = m->alloc(cache, &m->k_cache)) || (rc = m->alloc(cache, &m->v_cache)) ||
           (rc = m->alloc_t((uint64_t)m->n_conv * (m->conv_kernel - 1) * n, &m->conv_state)) ||
           (rc = m->alloc_t(rows * n, &m->hidden)) || (rc = m->alloc_t(rows * n, &m->normed)) ||
           (rc = m->alloc_t(rows * 3 * n, &m->bcx)) || (rc = m->alloc_t(rows * n, &m->conv_out)) ||
           (rc = m->alloc_t(rows * m->q_dim + 4, &m->q)) || (rc = m->alloc_t(rows * m->kv_dim + 4, &m->k)) ||
           (rc = m->alloc_t(rows * m->kv_dim + 4, &m->v)) || (rc = m->alloc_t(rows * m->q_dim + 4, &m->attn)) ||
           (any_qkv && (rc = m->alloc_t(rows * (m->q_dim + 2 * m->kv_dim), &m->qkv))) ||
           (rc = m->alloc_t(std::max<uint64_t>(rows * m->n_ff, (uint64_t)m->n_used * m->n_ff_expert), &m->ffn)) ||
           (rc = m->alloc_t(partial_floats + 4, &m->partials)) ||
           (rc = m->alloc_t((uint64_t)kAttnQueryBatch * std::max(1u, m->n_heads), &m->counters)) ||
           (rc = m->alloc_t(2 * (uint64_t)std::max(1u, m->n_used) * rows, &m->route)) ||
           (rc = m->alloc_t((uint64_t)std::max(1u, m->n_experts) * rows, &m->route_scores)) ||
           (rc = m->alloc_t(rows, &m->route_counters)) ||
           (rc = m->alloc_t((uint64_t)m->n_experts + 1, &m->moe_offsets)) ||
           (rc = m->alloc_t(std::max(1u, m->n_used) * rows, &m->moe_entries)) ||
           (rc = m->alloc_t(std::max<uint64_t>(1, (uint64_t)m->n_used * rows * m->n_ff_expert), &m->expert_ffn)) ||
           (rc = m->alloc_t(std::max<uint64_t>(1, (uint64_t)m->n_used * rows * n), &m->expert_out)) ||
           (rc = m->alloc(split_bytes, &m->split)) ||
           (rc = m->alloc_common()));
    if (rc) return cleanup(rc);
  }
  // The dense layers' SwiGLU pairs expanded for the library GEMM of prefill.
  for (Layer &L : m->layers)
    if (!L.moe)
      if (int rc = m->expand_pair(L.gate, L.up, m->n_ff, &L.gate_up16)) return cleanup(rc);
  if (int rc = m->finish_pairs(m->n_ff)) return cleanup(rc);
  // Decode steps at positions with at most kDeferSplits attention splits
  // take the deferred-combine form.
  m->short_below = deferred_combine_below(m->head_dim, m->kv_half);
  *out = m;
  return BCH_OK;
}

void bch_lfm2_free(bch_lfm2 *m) { delete m; }

uint32_t bch_lfm2_n_past(const bch_lfm2 *m) { return m->n_past; }
double bch_lfm2_last_gpu_seconds(const bch_lfm2 *m) { return m->last_gpu_seconds; }
int bch_lfm2_reset(bch_lfm2 *m) { return m->reset(); }

int bch_lfm2_step(bch_lfm2 *m, uint32_t token, float *logits, float *trace_embedding, float *trace_layers,
                  float *trace_final) {
  return m->step(token, logits, trace_embedding, trace_layers, trace_final);
}

int bch_lfm2_prefill(bch_lfm2 *m, const uint32_t *tokens, uint32_t n_tokens, float *logits, float *trace_embedding,
                     float *trace_layers, float *trace_final) {
  return m->prefill(tokens, n_tokens, logits, trace_embedding, trace_layers, trace_final);
}

int bch_lfm2_greedy_token(bch_lfm2 *m, uint32_t *token) { return m->greedy_token(token); }
int bch_lfm2_generate(bch_lfm2 *m, uint32_t *out, uint32_t n) { return m->generate(out, n); }
int bch_lfm2_generate_next(bch_lfm2 *m, uint32_t *out, uint32_t n) { return m->generate_next(out, n); }
int bch_lfm2_generate_stream(bch_lfm2 *m, uint32_t max_tokens, bch_emit_fn emit, void *user, uint32_t *gained,
                             uint32_t *n_gained) {
  return m->generate_stream(max_tokens, emit, user, gained, n_gained);
}
int bch_lfm2_generate_sampled(bch_lfm2 *m, uint32_t *out, uint32_t n, const bch_sampling *settings, uint64_t seed) {
  return m->generate_sampled(out, n, settings, seed);
}

// The checkpoint carries resets, n_past, the convolution state and the logits.
uint64_t bch_lfm2_checkpoint_bytes(const bch_lfm2 *m) { return m->checkpoint_bytes(); }
int bch_lfm2_checkpoint(bch_lfm2 *m, void *blob, uint64_t bytes) { return m->checkpoint(blob, bytes); }
int bch_lfm2_restore(bch_lfm2 *m, const void *blob, uint64_t bytes) { return m->restore(blob, bytes); }

}  // extern "C"
