// The Qwen3.5 driver: the MI355X counterpart of Qwen35Metal
// (crates/bobcat/src/qwen35_metal.rs), on the shared sequence protocol of
// driver.h.
//
// Decode step, per layer:
// * Gated DeltaNet: one launch projects the normalised token to the q/k/v
//   channels (with the causal convolution, SiLU and history update fused
//   into the rows' stores), the output gate z, beta and alpha; one launch
//   runs the gated delta rule (gates and q/k L2 norms fused in); one applies
//   the gated output norm; the output projection adds to the residual.
// * Gated attention: one launch projects the query/gate blocks, keys and
//   values; the fused decode attention normalises and rotates the first
//   n_rot elements of the query and the new key, stores the new position,
//   attends, and multiplies by the sigmoid gate; the output projection adds
//   to the residual.
// * The SwiGLU block as in LFM2.
// Prefill batches run the projections through the MFMA GEMM, the
// convolution per channel over the batch, and the recurrence with each
// state column resident in one wave for the whole batch.
#include <cmath>
#include <cstring>
#include <vector>

#include "driver.h"

namespace bch {

constexpr uint32_t kQwenAttnQueryBatch = 64;

struct QwenLayer {
  bool attention = false;
  uint32_t cache_index = 0;
  const float *attn_norm = nullptr, *ffn_norm = nullptr;
  DevMatrix wq, wk, wv, wo;
  const float *q_norm = nullptr, *k_norm = nullptr;
  DevMatrix qkv, z, beta, alpha, out;
  const float *taps = nullptr, *dt_bias = nullptr, *a = nullptr, *ssm_norm = nullptr;
  DevMatrix gate, up, down;
  // The SwiGLU pair as fp16 [gate rows; up rows] for the library GEMM of
  // prefill batches (Sequence::expand_pair), or nullptr.
  _Float16 *gate_up16 = nullptr;
  // Prefill: rows of wq | wk | wv (attention) or qkv | z | beta | alpha
  // (DeltaNet) when they lie back to back in device memory in one format
  // (one GEMM), else 0.
  uint32_t fused_rows = 0;
};

}  // namespace bch

using namespace bch;

struct bch_qwen35 : bch::Sequence {
  // Hyperparameters (qwen35.rs:31-67).
  uint32_t n_ff, n_heads, n_kv_heads, head_dim, n_rot, conv_kernel, n_k, n_v, k_dim, v_dim;
  float rope_theta, norm_eps;
  uint32_t q_dim, kv_dim, key_dim, value_dim, conv_dim;
  uint32_t n_attn = 0, n_delta = 0;
  std::vector<QwenLayer> layers;
  DevMatrix token_embd, output;
  const float *output_norm = nullptr;
  bool kv_half = true;
  uint32_t prefill_splits = 1;
  // Device memory.
  void *k_cache = nullptr, *v_cache = nullptr;
  void *split = nullptr;  // prefill GEMM scratch: split inputs and split-K partials (matmul_scratch_bytes)
  uint64_t split_bytes = 0;
  float *conv_state = nullptr, *delta_state = nullptr;
  float *hidden = nullptr, *normed = nullptr, *q_gate = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
        *attn = nullptr, *proj = nullptr, *conv_out = nullptr, *z = nullptr, *beta = nullptr, *alpha = nullptr,
        *delta_out = nullptr, *ffn = nullptr, *partials = nullptr;
  float *fused = nullptr;  // prefill: the output rows of a QwenLayer::fused_rows GEMM
  uint64_t partial_floats = 0;  // floats of `partials`
  float *chunk_scratch = nullptr;  // the chunked DeltaNet form's per-chunk matrices (prefill)
  uint32_t *counters = nullptr;

  void *cache_layer(void *base, uint32_t ci) const {
    return static_cast<char *>(base) + (uint64_t)n_ctx * kv_dim * ci * (kv_half ? 2 : 4);
  }
  void *cache_slot(void *base, uint32_t ci, uint32_t pos) const {
    return static_cast<char *>(cache_layer(base, ci)) + (uint64_t)pos * kv_dim * (kv_half ? 2 : 4);
  }
  float *conv_layer(uint32_t di) const { return conv_state + (uint64_t)di * conv_dim * (conv_kernel - 1); }
  float *state_layer(uint32_t di) const { return delta_state + (uint64_t)di * n_v * k_dim * v_dim; }

  void record_step(hipStream_t st, bool greedy_input, bool trace, bool short_ctx) override;
  void record_batch(hipStream_t st, uint32_t pos, uint32_t count, bool want_logits, bool trace) override;
  std::vector<std::pair<void *, uint64_t>> state_regions() const override {
    return {{conv_state, (uint64_t)n_delta * conv_dim * (conv_kernel - 1) * 4},
            {delta_state, (uint64_t)n_delta * n_v * k_dim * v_dim * 4}};
  }
};

void bch_qwen35::record_step(hipStream_t st, bool greedy_input, bool trace, bool short_ctx) {
  const uint32_t n = n_embd, cus = ctx->n_cus;
  uint32_t *dp = dpos;
  const uint64_t tstride = (uint64_t)trace_rows * n;
  const uint64_t embd_rb = bch_row_bytes(token_embd.format, n);
  if (greedy_input)
    run_embed_next(st, token_embd.format, token_embd.data, embd_rb, tokens, hidden, n, dp, argmax_partials,
                   kArgmaxPartials);
  else
    run_embed(st, token_embd.format, token_embd.data, embd_rb, tokens, hidden, n, 1, dp);
  if (trace) run_copy(st, hidden, this->trace, n, nullptr, 0);
  for (uint32_t il = 0; il < n_layers; il++) {
    const QwenLayer &L = layers[il];
    if (L.attention) {
      const uint32_t ci = L.cache_index;
      if (L.wq.format == L.wk.format && L.wq.format == L.wv.format) {
        run_matvec3(st, L.wq.format, L.wq.data, L.wk.data, L.wv.data, 2 * q_dim, kv_dim, kv_dim, n, hidden, q_gate, k,
                    v, L.attn_norm, norm_eps, cus);
      } else {  // mixed formats: one launch each
        run_matvec(st, L.wq.format, L.wq.data, 2 * q_dim, n, hidden, q_gate, L.attn_norm, norm_eps, false, cus);
        run_matvec(st, L.wk.format, L.wk.data, kv_dim, n, hidden, k, L.attn_norm, norm_eps, false, cus);
        run_matvec(st, L.wv.format, L.wv.data, kv_dim, n, hidden, v, L.attn_norm, norm_eps, false, cus);
      }
      AttnDecodeArgs ad{};
      ad.q = q_gate;
      ad.k = k;
      ad.v = v;
      ad.q_norm = L.q_norm;
      ad.k_norm = L.k_norm;
      ad.freqs = rope_table(rope_theta, n_rot);
      ad.eps = norm_eps;
      ad.scale = 1.0f / sqrtf((float)head_dim);
      ad.k_cache = cache_layer(k_cache, ci);
      ad.v_cache = cache_layer(v_cache, ci);
      ad.partials = partials;
      ad.counters = counters;
      ad.out = attn;
      ad.n_heads = n_heads;
      ad.n_kv = n_kv_heads;
      ad.head_dim = head_dim;
      ad.max_splits = attn_decode_max_splits(n_ctx, head_dim, kv_half);
      ad.dpos = dp;
      ad.q_head_stride = 2 * head_dim;
      ad.n_rot = n_rot;
      ad.gate = q_gate + head_dim;
      ad.gate_head_stride = 2 * head_dim;
      // Short contexts leave the splits' combine (and the gate) to wo's
      // input staging.
      const bool defer = short_ctx && slab_split_supported(L.wo.format, q_dim);
      ad.defer_splits = defer ? kDeferSplits : 0;
      run_attn_decode(st, ad, kv_half);
      const SplitOut so{partials, attn, q_gate + head_dim, dp, attn_decode_keys_per_split(head_dim, kv_half),
                        ad.max_splits, head_dim, 2 * head_dim, ad.defer_splits};
      if (!defer || !slab_matvec_split(st, L.wo.format, L.wo.data, n, q_dim, so, hidden, cus))
        run_matvec(st, L.wo.format, L.wo.data, n, q_dim, attn, hidden, nullptr, 0.f, true, cus);
    } else {
      const uint32_t di = L.cache_index;
      fast_matvec_gdn_in(st, L.qkv.format, L.qkv.data, L.z.data, L.beta.data, L.alpha.data, conv_dim, value_dim, n_v,
                         n, hidden, L.attn_norm, norm_eps, L.taps, conv_layer(di), conv_kernel, conv_out, z, beta,
                         alpha, cus);
      GdnArgs g{};
      g.y = conv_out;
      g.beta = beta;
      g.alpha = alpha;
      g.a = L.a;
      g.dt_bias = L.dt_bias;
      g.state = state_layer(di);
      g.out = delta_out;
      g.n_k = n_k;
      g.n_v = n_v;
      g.k_dim = k_dim;
      g.v_dim = v_dim;
      g.n_tokens = 1;
      g.q_scale = 1.0f / sqrtf((float)k_dim);
      g.raw_gates = true;
      const bool fused = gdn_step_supported(g);
      if (fused) {
        g.norm_w = L.ssm_norm;
        g.gate_z = z;
        g.norm_eps = norm_eps;
      }
      run_gdn_recurrence(st, g);
      if (!fused) run_gdn_gated_norm(st, delta_out, L.ssm_norm, z, v_dim, n_v, norm_eps);
      run_matvec(st, L.out.format, L.out.data, n, value_dim, delta_out, hidden, nullptr, 0.f, true, cus);
    }
    run_matvec_swiglu(st, L.gate.format, L.gate.data, L.up.data, n_ff, n, hidden, ffn, L.ffn_norm, norm_eps, cus);
    run_matvec(st, L.down.format, L.down.data, n, n_ff, ffn, hidden, nullptr, 0.f, true, cus);
    if (trace) run_copy(st, hidden, this->trace + (1 + il) * tstride, n, nullptr, 0);
  }
  if (trace) run_rms_norm(st, hidden, output_norm, this->trace + (1 + n_layers) * tstride, n, 1, norm_eps);
  if (!fast_matvec_argmax(st, output.format, output.data, n_vocab, n, hidden, logits, output_norm, norm_eps,
                          argmax_partials, cus)) {
    run_matvec(st, output.format, output.data, n_vocab, n, hidden, logits, output_norm, norm_eps, false, cus);
    run_argmax_partials(st, logits, n_vocab, argmax_partials, kArgmaxPartials);
  }
}

void bch_qwen35::record_batch(hipStream_t st, uint32_t pos, uint32_t count, bool want_logits, bool trace) {
  const uint32_t n = n_embd, cus = ctx->n_cus;
  const uint64_t tstride = (uint64_t)trace_rows * n;
  run_embed(st, token_embd.format, token_embd.data, bch_row_bytes(token_embd.format, n), tokens + pos, hidden, n,
            count, nullptr);
  if (trace) run_copy(st, hidden, this->trace, count * n, nullptr, 0);
  // A column-split sum into the residual stream (wo, out, down) is left to
  // the norm that reads the residual next (not when tracing copies it).
  PendingSum pend;
  PendingSum *const defer = trace ? nullptr : &pend;
  for (uint32_t il = 0; il < n_layers; il++) {
    const QwenLayer &L = layers[il];
    // The norm also writes the fp16 inputs of the projections that follow.
    run_rms_norm_split(st, hidden, L.attn_norm, normed, n, count, norm_eps, split, &pend);
    if (L.attention) {
      const uint32_t ci = L.cache_index;
      // The interleaved query/gate projection, k and v: one GEMM when the
      // matrices lie back to back (each token's row then q/gate | k | v).
      const float *qg = q_gate, *ks = k, *vs = v;
      uint32_t qg_stride = 2 * q_dim, kv_stride = kv_dim;
      if (L.fused_rows) {
        run_matmul(st, L.wq.format, L.wq.data, L.fused_rows, n, normed, fused, count, 0, split, split_bytes, true);
        qg = fused, ks = fused + 2 * q_dim, vs = fused + 2 * q_dim + kv_dim;
        qg_stride = kv_stride = L.fused_rows;
      } else {
        run_matmul(st, L.wq.format, L.wq.data, 2 * q_dim, n, normed, q_gate, count, 0, split, split_bytes, true);
        run_matmul(st, L.wk.format, L.wk.data, kv_dim, n, normed, k, count, 0, split, split_bytes, true);
        run_matmul(st, L.wv.format, L.wv.data, kv_dim, n, normed, v, count, 0, split, split_bytes, true);
      }
      // The queries come out of the interleaved query/gate projection.
      run_norm_rope(st, qg, q, false, L.q_norm, n_heads, head_dim, n_rot, 2 * head_dim, pos, nullptr, count,
                    qg_stride, q_dim, rope_theta, norm_eps, 0);
      run_norm_rope(st, ks, cache_slot(k_cache, ci, pos), kv_half, L.k_norm, n_kv_heads, head_dim, n_rot, head_dim,
                    pos, nullptr, count, kv_stride, kv_dim, rope_theta, norm_eps, 0);
      run_copy_rows(st, vs, kv_stride, cache_slot(v_cache, ci, pos), kv_dim, kv_half, kv_dim, count);
      // Attention with the output gate of each head applied in the same launch.
      if (attn_prefill_mfma_supported(n_heads, n_kv_heads, head_dim, kv_half))
        run_attn_prefill_mfma(st, q, cache_layer(k_cache, ci), cache_layer(v_cache, ci), attn, n_heads, n_kv_heads,
                              head_dim, pos, count, q_dim, q_dim, 1.0f / sqrtf((float)head_dim), partials,
                              partial_floats, qg + head_dim, 2 * head_dim, qg_stride);
      else
      for (uint32_t q0 = 0; q0 < count; q0 += kQwenAttnQueryBatch) {
        const uint32_t nq = std::min(kQwenAttnQueryBatch, count - q0);
        AttnDecodeArgs ad{};
        ad.q = q + (uint64_t)q0 * q_dim;
        ad.q_stride = q_dim;
        ad.q_head_stride = head_dim;
        ad.scale = 1.0f / sqrtf((float)head_dim);
        ad.k_cache = cache_layer(k_cache, ci);
        ad.v_cache = cache_layer(v_cache, ci);
        ad.partials = partials;
        ad.counters = counters;
        ad.out = attn + (uint64_t)q0 * q_dim;
        ad.out_stride = q_dim;
        ad.gate = qg + (uint64_t)q0 * qg_stride + head_dim;
        ad.gate_head_stride = 2 * head_dim;
        ad.gate_query_stride = qg_stride;
        ad.n_heads = n_heads;
        ad.n_kv = n_kv_heads;
        ad.head_dim = head_dim;
        ad.first_pos = pos + q0;
        ad.max_splits = attn_decode_max_splits(pos + q0 + nq, head_dim, kv_half);
        run_attn_prefill(st, ad, kv_half, nq);
      }
      run_matmul(st, L.wo.format, L.wo.data, n, q_dim, attn, hidden, count, 1, split, split_bytes, false, nullptr, defer);
    } else {
      const uint32_t di = L.cache_index;
      // qkv, z, beta and alpha: one GEMM when the matrices lie back to back
      // (each token's row then qkv | z | beta | alpha).
      const float *ps = proj, *zs = z, *bs = beta, *as = alpha;
      uint32_t stride = 0;
      if (L.fused_rows) {
        run_matmul(st, L.qkv.format, L.qkv.data, L.fused_rows, n, normed, fused, count, 0, split, split_bytes, true);
        ps = fused, zs = fused + conv_dim, bs = zs + value_dim, as = bs + n_v;
        stride = L.fused_rows;
      } else {
        run_matmul(st, L.qkv.format, L.qkv.data, conv_dim, n, normed, proj, count, 0, split, split_bytes, true);
        run_matmul(st, L.z.format, L.z.data, value_dim, n, normed, z, count, 0, split, split_bytes, true);
        run_matmul(st, L.beta.format, L.beta.data, n_v, n, normed, beta, count, 0, split, split_bytes, true);
        run_matmul(st, L.alpha.format, L.alpha.data, n_v, n, normed, alpha, count, 0, split, split_bytes, true);
      }
      run_gdn_conv(st, ps, L.taps, conv_layer(di), conv_out, conv_dim, conv_kernel, count, stride);
      GdnArgs g{};
      g.y = conv_out;
      g.beta = bs;
      g.alpha = as;
      g.gate_stride = stride;
      g.a = L.a;
      g.dt_bias = L.dt_bias;
      g.state = state_layer(di);
      g.out = delta_out;
      g.n_k = n_k;
      g.n_v = n_v;
      g.k_dim = k_dim;
      g.v_dim = v_dim;
      g.n_tokens = count;
      g.q_scale = 1.0f / sqrtf((float)k_dim);
      g.raw_gates = true;
      // Batches of more than one token take the chunked (WY) form.
      if (count == 1 || !chunk_scratch || !run_gdn_chunked(st, g, chunk_scratch)) run_gdn_recurrence(st, g);
      run_gdn_gated_norm(st, delta_out, L.ssm_norm, zs, v_dim, count * n_v, norm_eps, n_v, stride);
      run_matmul(st, L.out.format, L.out.data, n, value_dim, delta_out, hidden, count, 1, split, split_bytes, false,
                 nullptr, defer);
    }
    const bool pair_ok = L.gate_up16 && count > kBlasPairMinTokens;
    run_rms_norm_split(st, hidden, L.ffn_norm, normed, n, count, norm_eps, split, &pend, pair_ok ? pair_us : nullptr);
    // The pair through the library GEMM on the expanded weights when the
    // model has them; its SwiGLU also writes the down projection's inputs.
    const bool blas_pair = pair_ok && run_blas_pair(st, L.gate_up16, n_ff, n, count, split, pair_out, pair_us, nullptr);
    if (!blas_pair && L.gate.format == L.up.format) {
      // Gate and up in one paired launch: ffn = silu(gate·x) ⊙ (up·x).
      run_matmul(st, L.gate.format, L.gate.data, n_ff, n, normed, ffn, count, 3, split, split_bytes, true,
                 L.up.data);
    } else if (!blas_pair) {
      run_matmul(st, L.gate.format, L.gate.data, n_ff, n, normed, ffn, count, 0, split, split_bytes, true);
      run_matmul(st, L.up.format, L.up.data, n_ff, n, normed, ffn, count, 2, split, split_bytes, true);
    }
    run_matmul(st, L.down.format, L.down.data, n, n_ff, ffn, hidden, count, 1, split, split_bytes, blas_pair, nullptr,
               defer);
    if (trace) run_copy(st, hidden, this->trace + (1 + il) * tstride, count * n, nullptr, 0);
  }
  finish_pending_sum(st, pend, hidden);
  if (trace) run_rms_norm(st, hidden, output_norm, this->trace + (1 + n_layers) * tstride, n, count, norm_eps);
  if (want_logits)
    run_matvec(st, output.format, output.data, n_vocab, n, hidden + (uint64_t)(count - 1) * n, logits, output_norm,
               norm_eps, false, cus);
}

extern "C" {

int bch_qwen35_new(bch_ctx *ctx, const bch_qwen35_model *md, uint32_t n_ctx, int kv_half, bch_qwen35 **out) {
  *out = nullptr;
  if (n_ctx == 0) return fail(BCH_ERR_ARGUMENT, "the context must hold a token");
  if (!md->layers || md->n_layers == 0 || md->n_embd == 0) return fail(BCH_ERR_ARGUMENT, "the model has no layers");
  const uint32_t n = md->n_embd, hd = md->head_dim;
  bool any_attn = false, any_delta = false;
  for (uint32_t il = 0; il < md->n_layers; il++) {
    any_attn |= md->layers[il].is_attention != 0;
    any_delta |= md->layers[il].is_attention == 0;
  }
  if (any_attn) {
    const uint32_t group = md->n_kv_heads ? md->n_heads / md->n_kv_heads : 0;
    if (!md->n_kv_heads || md->n_heads % md->n_kv_heads || group > 4 || hd < 32 || hd > 256 || (hd & (hd - 1)) ||
        md->n_rot == 0 || md->n_rot > hd || md->n_rot % 2)
      return fail(BCH_ERR_ATTENTION_LIMITS,
                  "a head size of 32, 64, 128 or 256, at most 4 query heads per KV head and an even rotation of at "
                  "most the head size, got %u, %u and %u", hd, group, md->n_rot);
  }
  if (any_delta) {
    // DeltaNetLimits (backend.rs:1899-1911) and this build's kernels.
    if (md->conv_kernel < 2 || md->conv_kernel > kGdnMaxKernel || md->n_k_heads == 0 ||
        md->n_v_heads % md->n_k_heads || (md->k_head_dim != 64 && md->k_head_dim != 128) || md->v_head_dim == 0 ||
        md->v_head_dim % 4 || md->v_head_dim > 1024)
      return fail(BCH_ERR_DELTANET_LIMITS,
                  "DeltaNet: 2 to %u taps, key heads of 64 or 128, value heads a multiple of the key heads and of 4 "
                  "(got %u taps, %u/%u heads of %u/%u)", kGdnMaxKernel, md->conv_kernel, md->n_k_heads,
                  md->n_v_heads, md->k_head_dim, md->v_head_dim);
  }
  auto *m = new bch_qwen35();
  m->ctx = ctx;
  m->s = ctx->stream;
  m->n_layers = md->n_layers;
  m->n_embd = n;
  m->n_vocab = md->n_vocab;
  m->n_ff = md->n_ff;
  m->n_heads = md->n_heads;
  m->n_kv_heads = md->n_kv_heads;
  m->head_dim = hd;
  m->n_rot = md->n_rot;
  m->conv_kernel = md->conv_kernel;
  m->n_k = md->n_k_heads;
  m->n_v = md->n_v_heads;
  m->k_dim = md->k_head_dim;
  m->v_dim = md->v_head_dim;
  m->rope_theta = md->rope_theta;
  m->norm_eps = md->norm_eps;
  m->q_dim = md->n_heads * hd;
  m->kv_dim = md->n_kv_heads * hd;
  m->key_dim = m->n_k * m->k_dim;
  m->value_dim = m->n_v * m->v_dim;
  m->conv_dim = 2 * m->key_dim + m->value_dim;
  m->n_ctx = n_ctx;
  m->kv_half = kv_half != 0;
  m->batch = std::min(n_ctx, kPrefillBatch);
  auto cleanup = [&](int rc) {
    delete m;
    return rc;
  };

  Uploader up;
  m->layers.resize(md->n_layers);
  for (uint32_t il = 0; il < md->n_layers; il++) {
    const bch_qwen35_layer &S = md->layers[il];
    QwenLayer &L = m->layers[il];
    int rc;
    if ((rc = up.vec(S.attn_norm, n, &L.attn_norm, "attn_norm")) ||
        (rc = up.vec(S.ffn_norm, n, &L.ffn_norm, "post_attention_norm")))
      return cleanup(rc);
    L.attention = S.is_attention != 0;
    if (L.attention) {
      L.cache_index = m->n_attn++;
      if ((rc = up.mat(S.wq, 2 * m->q_dim, n, &L.wq, "attn_q")) || (rc = up.mat(S.wk, m->kv_dim, n, &L.wk, "attn_k")) ||
          (rc = up.mat(S.wv, m->kv_dim, n, &L.wv, "attn_v")) || (rc = up.mat(S.wo, n, m->q_dim, &L.wo, "attn_output")) ||
          (rc = up.vec(S.q_norm, hd, &L.q_norm, "attn_q_norm")) || (rc = up.vec(S.k_norm, hd, &L.k_norm, "attn_k_norm")))
        return cleanup(rc);
    } else {
      L.cache_index = m->n_delta++;
      if ((rc = up.mat(S.qkv, m->conv_dim, n, &L.qkv, "attn_qkv")) ||
          (rc = up.mat(S.z, m->value_dim, n, &L.z, "attn_gate")) || (rc = up.mat(S.beta, m->n_v, n, &L.beta, "ssm_beta")) ||
          (rc = up.mat(S.alpha, m->n_v, n, &L.alpha, "ssm_alpha")) ||
          (rc = up.mat(S.out, n, m->value_dim, &L.out, "ssm_out")) ||
          (rc = up.vec(S.conv_taps, (uint64_t)m->conv_dim * m->conv_kernel, &L.taps, "ssm_conv1d")) ||
          (rc = up.vec(S.dt_bias, m->n_v, &L.dt_bias, "ssm_dt")) || (rc = up.vec(S.a, m->n_v, &L.a, "ssm_a")) ||
          (rc = up.vec(S.ssm_norm, m->v_dim, &L.ssm_norm, "ssm_norm")))
        return cleanup(rc);
      if (S.qkv.format != S.z.format || S.qkv.format != S.beta.format || S.qkv.format != S.alpha.format)
        return cleanup(fail(BCH_ERR_UNSUPPORTED_FORMAT, "layer %u: DeltaNet input projections of one format", il));
    }
    if ((rc = up.mat(S.gate, md->n_ff, n, &L.gate, "ffn_gate")) || (rc = up.mat(S.up, md->n_ff, n, &L.up, "ffn_up")) ||
        (rc = up.mat(S.down, n, md->n_ff, &L.down, "ffn_down")))
      return cleanup(rc);
    if (S.gate.format != S.up.format)
      return cleanup(fail(BCH_ERR_UNSUPPORTED_FORMAT, "layer %u: gate and up matrices of one format", il));
  }
  {
    int rc;
    if ((rc = up.mat(md->token_embd, md->n_vocab, n, &m->token_embd, "token_embd")) ||
        (rc = up.mat(md->output, md->n_vocab, n, &m->output, "output")) ||
        (rc = up.vec(md->output_norm, n, &m->output_norm, "output_norm")))
      return cleanup(rc);
  }
  if (int rc = m->upload(up)) return cleanup(rc);
  uint32_t fused_widest = 0;
  for (QwenLayer &L : m->layers) {
    // Matrices the uploader placed back to back (in the order they were added).
    auto follows = [&](const DevMatrix &a, const DevMatrix &b) {
      return a.format == b.format && b.data == a.data + bch_row_bytes(a.format, n) * a.n_rows;
    };
    if (L.attention ? follows(L.wq, L.wk) && follows(L.wk, L.wv)
                    : follows(L.qkv, L.z) && follows(L.z, L.beta) && follows(L.beta, L.alpha))
      L.fused_rows = L.attention ? L.wq.n_rows + L.wk.n_rows + L.wv.n_rows
                                 : L.qkv.n_rows + L.z.n_rows + L.beta.n_rows + L.alpha.n_rows;
    fused_widest = std::max(fused_widest, L.fused_rows);
  }
  {
    const uint64_t rows = m->batch;
    const uint64_t cache = (uint64_t)m->n_attn * n_ctx * m->kv_dim * (m->kv_half ? 2 : 4);
    m->prefill_splits = attention_splits(n_ctx, std::max(1u, m->n_kv_heads), ctx->n_cus);
    uint64_t partial_floats = attention_partial_floats(std::min<uint32_t>(m->batch, kQwenAttnQueryBatch),
                                                            m->n_heads, hd, attn_decode_max_splits(n_ctx, hd, m->kv_half));
    // The MFMA prefill attention splits the keys of a batch up to 4 ways.
    if (attn_prefill_mfma_supported(m->n_heads, m->n_kv_heads, hd, m->kv_half))
      partial_floats = std::max(partial_floats, attn_prefill_partial_floats(m->batch, m->n_heads, hd, 4));
    m->partial_floats = partial_floats;
    int rc = 0;
    (void)((rc = m->alloc(cache, &m->k_cache)) || (rc = m->alloc(cache, &m->v_cache)) ||
           (rc = m->alloc_t((uint64_t)m->n_delta * m->conv_dim * (m->conv_kernel - 1), &m->conv_state)) ||
           (rc = m->alloc_t((uint64_t)m->n_delta * m->n_v * m->k_dim * m->v_dim, &m->delta_state)) ||
           (rc = m->alloc_t(rows * n, &m->hidden)) || (rc = m->alloc_t(rows * n, &m->normed)) ||
           (rc = m->alloc_t(rows * 2 * m->q_dim + 4, &m->q_gate)) ||
           (fused_widest && (rc = m->alloc_t(rows * fused_widest, &m->fused))) || (rc = m->alloc_t(rows * m->q_dim + 4, &m->q)) ||
           (rc = m->alloc_t(rows * m->kv_dim + 4, &m->k)) || (rc = m->alloc_t(rows * m->kv_dim + 4, &m->v)) ||
           (rc = m->alloc_t(rows * m->q_dim + 4, &m->attn)) || (rc = m->alloc_t(rows * m->conv_dim + 4, &m->proj)) ||
           (rc = m->alloc_t(rows * m->conv_dim + 4, &m->conv_out)) ||
           (rc = m->alloc_t(rows * m->value_dim + 4, &m->z)) || (rc = m->alloc_t(rows * m->n_v + 4, &m->beta)) ||
           (rc = m->alloc_t(rows * m->n_v + 4, &m->alpha)) || (rc = m->alloc_t(rows * m->value_dim + 4, &m->delta_out)) ||
           (rc = m->alloc_t(rows * m->n_ff, &m->ffn)) ||
           (rc = m->alloc(m->split_bytes = matmul_scratch_bytes((uint32_t)rows,
                                                                std::max({n, m->q_dim, m->value_dim, m->n_ff}), n),
                          &m->split)) || (rc = m->alloc_t(partial_floats + 4, &m->partials)) ||
           (rc = m->alloc_t((uint64_t)kQwenAttnQueryBatch * std::max(1u, m->n_heads), &m->counters)) ||
           (rc = m->alloc_t(gdn_chunk_scratch_floats(m->n_v, m->k_dim, m->v_dim, (uint32_t)rows), &m->chunk_scratch)) ||
           (rc = m->alloc_common()));
    if (rc) return cleanup(rc);
  }
  // The SwiGLU pairs expanded for the library GEMM of prefill.
  for (QwenLayer &L : m->layers)
    if (int rc = m->expand_pair(L.gate, L.up, m->n_ff, &L.gate_up16)) return cleanup(rc);
  if (int rc = m->finish_pairs(m->n_ff)) return cleanup(rc);
  // Decode steps at positions with at most kDeferSplits attention splits
  // take the deferred-combine form.
  m->short_below = deferred_combine_below(m->head_dim, m->kv_half);
  *out = m;
  return BCH_OK;
}

void bch_qwen35_free(bch_qwen35 *m) { delete m; }
uint32_t bch_qwen35_n_past(const bch_qwen35 *m) { return m->n_past; }
double bch_qwen35_last_gpu_seconds(const bch_qwen35 *m) { return m->last_gpu_seconds; }
int bch_qwen35_reset(bch_qwen35 *m) { return m->reset(); }

int bch_qwen35_step(bch_qwen35 *m, uint32_t token, float *logits, float *trace_embedding, float *trace_layers,
                    float *trace_final) {
  return m->step(token, logits, trace_embedding, trace_layers, trace_final);
}

int bch_qwen35_prefill(bch_qwen35 *m, const uint32_t *tokens, uint32_t n_tokens, float *logits, float *trace_embedding,
                       float *trace_layers, float *trace_final) {
  return m->prefill(tokens, n_tokens, logits, trace_embedding, trace_layers, trace_final);
}

// Gpu::hidden (crates/bobcat-cli/src/backend.rs:150-160): reset, then
// Qwen35Metal::prefill with only its final-norm output.
int bch_qwen35_hidden(bch_qwen35 *m, const uint32_t *tokens, uint32_t n_tokens, float *hidden) {
  if (!hidden) return fail(BCH_ERR_ARGUMENT, "hidden: no output rows");
  BCH_TRY(m->reset());
  return m->prefill(tokens, n_tokens, nullptr, nullptr, nullptr, hidden);
}

int bch_qwen35_greedy_token(bch_qwen35 *m, uint32_t *token) { return m->greedy_token(token); }
int bch_qwen35_generate(bch_qwen35 *m, uint32_t *out, uint32_t n) { return m->generate(out, n); }
int bch_qwen35_generate_next(bch_qwen35 *m, uint32_t *out, uint32_t n) { return m->generate_next(out, n); }
int bch_qwen35_generate_stream(bch_qwen35 *m, uint32_t max_tokens, bch_emit_fn emit, void *user, uint32_t *gained,
                               uint32_t *n_gained) {
  return m->generate_stream(max_tokens, emit, user, gained, n_gained);
}
int bch_qwen35_generate_sampled(bch_qwen35 *m, uint32_t *out, uint32_t n, const bch_sampling *settings, uint64_t seed) {
  return m->generate_sampled(out, n, settings, seed);
}

// The checkpoint carries resets, n_past, the convolution histories, the
// DeltaNet states and the logits.
uint64_t bch_qwen35_checkpoint_bytes(const bch_qwen35 *m) { return m->checkpoint_bytes(); }
int bch_qwen35_checkpoint(bch_qwen35 *m, void *blob, uint64_t bytes) { return m->checkpoint(blob, bytes); }
int bch_qwen35_restore(bch_qwen35 *m, const void *blob, uint64_t bytes) { return m->restore(blob, bytes); }

}  // extern "C"
