// Stream-level launchers of every kernel, shared by the C-ABI op functions
// and the model drivers.  They check nothing: callers validate shapes and
// views first.  `dpos`, where present, points at a device position counter
// (see ops.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bch {

// Inverse RoPE frequencies 1/theta^(2i/n_rot), computed on the host with the
// host's powf (as scalar::rope_neox does, crates/bobcat/src/scalar.rs:257-260)
// so device angles equal the CPU path's bit for bit; passed by value.
struct RopeTable {
  float inv_freq[128];
};
RopeTable rope_table(float theta, uint32_t n_rot);

// attn_decode.hip: decode attention of one query at position *dpos with the
// q/k RMS norm + RoPE and the KV-cache store of the new position folded in.
struct AttnDecodeArgs {
  const float *q, *k, *v;          // raw projections of the token
  const float *q_norm, *k_norm;    // [head_dim]
  RopeTable freqs;
  float eps, scale;
  void *k_cache, *v_cache;         // this layer's caches, [pos][n_kv][head_dim]
  float *partials;                 // n_heads * max_splits * (head_dim + 4), 16-byte aligned
  uint32_t *counters;              // n_heads zeroed (left zeroed on exit)
  float *out;                      // [n_heads * head_dim]
  uint32_t n_heads, n_kv, head_dim, max_splits;
  const uint32_t *dpos;
  uint32_t q_head_stride;          // floats from one query head to the next in q
  uint32_t n_rot;                  // leading elements of a head that RoPE rotates
  const float *gate;               // nullable: out[h] *= sigmoid(gate[h·gate_head_stride ..])
  uint32_t gate_head_stride;
  // Prefill (run_attn_prefill): query z sits at first_pos + z, its query at
  // q + z·q_stride, its output at out + z·out_stride, its gate at
  // gate + z·gate_query_stride; partials and counters hold n_queries·n_heads slots.
  uint32_t first_pos, q_stride, out_stride, gate_query_stride;
  // Decode: one query head per workgroup while the context holds at most this
  // many keys, else a group's heads share each workgroup (set by
  // run_attn_decode).
  uint32_t grouped_above;
  // Decode: while the context has at most this many splits (0: never, at
  // most kDeferSplits), every split only stores its partial (including the
  // single split of a short context) and the out projection's input staging
  // combines them (slab_matvec_split); no counters, no combining workgroup,
  // and the output gate is left to that staging too.  Past it the launch
  // combines as usual into `out`, gated.
  uint32_t defer_splits;
};
constexpr uint32_t kDeferSplits = 4;
uint32_t attn_decode_keys_per_split(uint32_t head_dim, bool kv_half);
uint32_t attn_decode_max_splits(uint32_t n_ctx, uint32_t head_dim, bool kv_half);
void run_attn_decode(hipStream_t s, const AttnDecodeArgs &a, bool kv_half);
// Attention of n_queries prefill queries with normalised, rotated queries and
// every key already in the cache; max_splits must cover first_pos + n_queries.
void run_attn_prefill(hipStream_t s, const AttnDecodeArgs &a, bool kv_half, uint32_t n_queries);

// matvec.hip
void run_matvec(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                float *y, const float *norm_w, float eps, bool accumulate, uint32_t n_cus);
void run_matvec_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_rows,
                       uint32_t n_cols, const float *x, float *y, const float *norm_w, float eps, uint32_t n_cus);
void run_matvec_conv(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_cols, const float *x,
                     const float *norm_w, float eps, const float *taps, float *history, float *out, uint32_t n_embd,
                     uint32_t ksize, uint32_t n_cus);
// Three projections of one input (q, k, v of an attention layer) in one
// launch: rows [0, r0) from W0 into y0, [r0, r0+r1) from W1 into y1, the
// rest from W2 into y2.
void run_matvec3(hipStream_t s, uint32_t format, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2, uint32_t r0,
                 uint32_t r1, uint32_t r2, uint32_t n_cols, const float *x, float *y0, float *y1, float *y2,
                 const float *norm_w, float eps, uint32_t n_cus);

// gemv.hip: x-stationary variants of the four above for rows of at most
// 256 units; they return false (launching nothing) for wider rows.
bool fast_matvec(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                 float *y, const float *norm_w, float eps, bool accumulate, uint32_t n_cus);
bool fast_matvec_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_rows,
                        uint32_t n_cols, const float *x, float *y, const float *norm_w, float eps, uint32_t n_cus);
bool fast_matvec3(hipStream_t s, uint32_t format, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2, uint32_t r0,
                  uint32_t r1, uint32_t r2, uint32_t n_cols, const float *x, float *y0, float *y1, float *y2,
                  const float *norm_w, float eps, uint32_t n_cus);
bool fast_matvec_conv(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_cols, const float *x,
                      const float *norm_w, float eps, const float *taps, float *history, float *out, uint32_t n_embd,
                      uint32_t ksize, uint32_t n_cus);

// gemv_slab.hip: the slab GEMV (every weight load of a workgroup issued
// before its input is staged) for Q4_K rows; the fast_* functions above try
// these first.  Each returns false, launching nothing, for shapes it does not
// serve.
bool slab_matvec(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                 float *y, const float *nw, float eps, bool accumulate, uint32_t n_cus);
bool slab_matvec3(hipStream_t s, uint32_t format, const uint8_t *W0, const uint8_t *W1, const uint8_t *W2, uint32_t r0,
                  uint32_t r1, uint32_t r2, uint32_t n_cols, const float *x, float *y0, float *y1, float *y2,
                  const float *nw, float eps, uint32_t n_cus);
bool slab_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_rows,
                 uint32_t n_cols, const float *x, float *y, const float *nw, float eps, uint32_t n_cus);
bool slab_experts_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_ff,
                         uint32_t n_cols, const uint32_t *ids, uint32_t n_used, const float *x, float *y,
                         uint32_t n_cus);
bool slab_conv(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_cols, const float *x, const float *nw,
               float eps, const float *taps, float *history, float *out, uint32_t n_embd, uint32_t ksize,
               uint32_t n_cus);
// The decode attention's output as the out projection reads it: while the
// context has at most `defer` splits (of `kps` keys, counted from *dpos),
// the split partials (max, sum, pad, pad, output[head_dim] per head and
// split; max_splits per head) combined here, times sigmoid(gate) when
// gated; past it the combined, gated `out`.
struct SplitOut {
  const float *partials;
  const float *out;
  const float *gate;  // nullable: gate[h·gate_head_stride + e]
  const uint32_t *dpos;
  uint32_t kps, max_splits, head_dim, gate_head_stride, defer;
};
// The out projection y += W · attention output on the slab kernel, the
// deferred splits combined while its input is staged; false (launching
// nothing) for shapes it does not serve, which slab_split_supported tells
// beforehand.
bool slab_split_supported(uint32_t format, uint32_t n_cols);
bool slab_matvec_split(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                       const SplitOut &in, float *y, uint32_t n_cus);
bool slab_gdn_in(hipStream_t s, uint32_t format, const uint8_t *Wqkv, const uint8_t *Wz, const uint8_t *Wb,
                 const uint8_t *Wa, uint32_t conv_dim, uint32_t value_dim, uint32_t n_v, uint32_t n_cols,
                 const float *x, const float *nw, float eps, const float *taps, float *hist, uint32_t ksize,
                 float *conv_out, float *z, float *beta, float *alpha, uint32_t n_cus);

// The logits GEMV with a per-workgroup argmax partial (at most
// kArgmaxPartials); false when the shape has no fast path.
constexpr uint32_t kArgmaxPartials = 1024;
bool fast_matvec_argmax(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                        const float *x, float *y, const float *norm_w, float eps, uint64_t *partials, uint32_t n_cus);

// moe.hip + gemv.hip: mixture of experts.  A route holds, per token, the
// n_used expert ids the router picked and then their n_used weights as
// float bits (route_bytes = 2 * n_used * n_tokens * 4).
constexpr uint32_t kMoeMaxExperts = 128;  // MOE_MAX_EXPERTS
constexpr uint32_t kMoeMaxUsed = 8;       // MOE_MAX_USED
// Route n_tokens tokens of x; with norm_w, RMS-normalise each token first
// and store it at `normed`.
// Batched experts (prefill): grouping, grouped GEMM, weighted combine.
void run_moe_group(hipStream_t s, const uint32_t *route, uint32_t *offsets, uint32_t *entries, uint32_t n_experts,
                   uint32_t n_used, uint32_t n_tokens);
// split_ready (shared_input only): `split` already holds x's fp16 inputs
// (run_rms_norm_split wrote them), so they are not converted again.
void run_matmul_experts(hipStream_t s, uint32_t format, const uint8_t *W, const uint8_t *up, uint32_t n_rows,
                        uint32_t n_cols, uint32_t n_experts, const float *x, bool shared_input,
                        const uint32_t *offsets, const uint32_t *entries, uint32_t n_used, float *y,
                        uint32_t n_tokens, void *split, bool split_ready = false);
void run_moe_combine(hipStream_t s, const float *x, const uint32_t *route, float *y, uint32_t n_embd,
                     uint32_t n_used, uint32_t n_tokens);
// With `scores` (n_tokens · n_experts floats of scratch) and `counters`
// (n_tokens zeroed u32, left zeroed) the scores are spread over (token,
// 4-expert) workgroups and the last of a token's picks its route; without,
// one workgroup per token does both.
void run_moe_route(hipStream_t s, const float *x, const float *norm_w, float eps, float *normed, const float *router,
                   const float *bias, uint32_t *route, uint32_t n_cols, uint32_t n_experts, uint32_t n_used,
                   uint32_t n_tokens, float *scores, uint32_t *counters);
// y[slot][r] = silu(G_e·x)[r] · (U_e·x)[r] for the n_used experts e of `ids`.
bool fast_matvec_experts_swiglu(hipStream_t s, uint32_t format, const uint8_t *Wg, const uint8_t *Wu, uint32_t n_ff,
                                uint32_t n_cols, const uint32_t *ids, uint32_t n_used, const float *x, float *y,
                                uint32_t n_cus);
// y[r] += Σ_slot weight_slot · (D_e · x[slot])[r] for one token's route;
// false when the shape or format has no kernel.
bool run_experts_down(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                      const float *x, const uint32_t *route, uint32_t n_used, float *y, uint32_t n_cus);

// gdn.hip + gemv.hip: Gated DeltaNet (qwen35.rs:430-516).  A DeltaNet token
// holds conv_dim = 2·n_k·k_dim + n_v·v_dim floats after its projection: the
// query heads, the key heads, the value heads; value head j reads key head
// j % n_k.  States are [head][k_dim rows][v_dim columns] (qwen35.rs:570-576).
constexpr uint32_t kGdnMaxKernel = 8;  // GDN_MAX_KERNEL
bool fast_matvec_gdn_in(hipStream_t s, uint32_t format, const uint8_t *Wqkv, const uint8_t *Wz, const uint8_t *Wb,
                        const uint8_t *Wa, uint32_t conv_dim, uint32_t value_dim, uint32_t n_v, uint32_t n_cols,
                        const float *x, const float *nw, float eps, const float *taps, float *hist, uint32_t ksize,
                        float *conv_out, float *z, float *beta, float *alpha, uint32_t n_cus);
struct GdnArgs {
  const float *y;                 // [n_tokens][conv_dim], after the convolution
  const float *beta, *alpha;      // [n_tokens][n_v] (rows gate_stride apart): raw projections (raw_gates) or gated
  const float *a, *dt_bias;       // [n_v], for raw gates
  float *state;                   // [n_v][k_dim][v_dim]
  float *out;                     // [n_tokens][n_v·v_dim]
  uint32_t n_k, n_v, k_dim, v_dim, n_tokens;
  float q_scale;
  bool raw_gates;
  // Decode only (gdn_step_supported): with norm_w, out of each value head
  // becomes norm_w ⊙ rmsnorm(out) ⊙ silu(gate_z[head]) in the same launch.
  const float *norm_w, *gate_z;
  float norm_eps;
  uint32_t gate_stride;  // floats between the tokens' beta (and alpha) rows; 0: n_v
};
// Whether a one-token recurrence runs k_gdn_step (which fuses the gated norm).
bool gdn_step_supported(const GdnArgs &a);
// false when k_dim is not 64 or 128 (or v_dim not a multiple of the columns per workgroup).
bool run_gdn_recurrence(hipStream_t s, const GdnArgs &a);
// The chunked (WY) form of the same recurrence for prefill batches, in 64-token
// chunks; `scratch` holds gdn_chunk_scratch_floats() floats (16-byte aligned).
bool gdn_chunked_supported(const GdnArgs &a);
uint64_t gdn_chunk_scratch_floats(uint32_t n_v, uint32_t k_dim, uint32_t v_dim, uint32_t n_tokens);
bool run_gdn_chunked(hipStream_t s, const GdnArgs &a, float *scratch);
// x_stride: floats between the tokens' input rows (0: channels).
void run_gdn_conv(hipStream_t s, const float *x, const float *taps, float *hist, float *y, uint32_t channels,
                  uint32_t ksize, uint32_t n_tokens, uint32_t x_stride = 0);
void run_gdn_gates(hipStream_t s, float *beta, float *alpha, const float *a, const float *dt_bias, uint32_t n_v,
                   uint32_t n);
// x[r] (v_dim floats per row) = w ⊙ rmsnorm(x[r]) ⊙ silu(z[r]), in place.
// z_stride: floats between the tokens' gate rows, each n_v heads of v_dim
// (0: the rows are contiguous).
void run_gdn_gated_norm(hipStream_t s, float *x, const float *w, const float *z, uint32_t v_dim, uint32_t n_rows,
                        float eps, uint32_t n_v = 1, uint32_t z_stride = 0);
// attn[t][h·hd + d] *= sigmoid(q_gate[t][(2h + 1)·hd + d]).
void run_attention_gate(hipStream_t s, float *attn, const float *q_gate, uint32_t head_dim, uint32_t q_dim,
                        uint32_t n_tokens);

// sample.hip: Sampler::sample on the GPU.  With dpos, the recent tokens
// are recent[0..*dpos] and the token goes to out[*dpos + 1], advancing
// *dpos; otherwise recent holds n_recent tokens and the token goes to out[0].
constexpr uint32_t kMaxCandidates = 4096;  // candidates kept after top-k, at most
struct SampleArgs {
  float *logits;  // penalised in place
  uint32_t n;
  const uint32_t *recent;
  uint32_t n_recent;
  uint32_t *dpos;
  uint32_t *out;
  uint64_t *rng;  // wyrand state; null: the draw is `draw`
  float draw;
  float temperature, top_p, min_p, penalty;
  uint32_t top_k;
};
void run_sample(hipStream_t s, const SampleArgs &a);

// ops.hip
// argmax of n logits as partials[0] (an argmax key), with partials[1..n_partials) zeroed.
void run_argmax_partials(hipStream_t s, const float *logits, uint32_t n, uint64_t *partials, uint32_t n_partials);
// The token the argmax keys select, stored at *out.
void run_argmax_pick(hipStream_t s, const uint64_t *partials, uint32_t n_partials, uint32_t *out);
// The next decode step's first launch: reduce the argmax partials to the
// greedy token, store it at tokens[*dpos + 1], advance *dpos, and embed it.
void run_embed_next(hipStream_t s, uint32_t format, const uint8_t *W, uint64_t row_bytes, uint32_t *tokens,
                    float *out, uint32_t n_embd, uint32_t *dpos, const uint64_t *partials, uint32_t n_partials);
void run_rms_norm(hipStream_t s, const float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps);
void run_norm_rope(hipStream_t s, const float *src, void *dst, bool half, const float *w, uint32_t n_heads,
                   uint32_t head_dim, uint32_t n_rot, uint32_t src_head_stride, uint32_t pos, const uint32_t *dpos,
                   uint32_t n_tokens, uint32_t src_stride, uint32_t dst_stride, float theta, float eps,
                   uint64_t dst_pos_stride);
void run_convert_half(hipStream_t s, const float *src, void *dst, uint32_t n, const uint32_t *dpos,
                      uint64_t dst_pos_stride);
void run_copy(hipStream_t s, const float *src, float *dst, uint32_t n, const uint32_t *dpos, uint64_t dst_pos_stride);
// rows x cols floats, rows src_stride apart, to rows dst_stride apart (f16
// when half).
void run_copy_rows(hipStream_t s, const float *src, uint32_t src_stride, void *dst, uint32_t dst_stride, bool half,
                   uint32_t cols, uint32_t rows);
void run_embed(hipStream_t s, uint32_t format, const uint8_t *W, uint64_t row_bytes, const uint32_t *tokens,
               float *out, uint32_t n_embd, uint32_t n_tokens, const uint32_t *dpos);
void run_argmax(hipStream_t s, const float *x, uint32_t *out, uint32_t n, uint32_t *dpos, bool advance);
void run_short_conv(hipStream_t s, const float *bcx, const float *taps, float *hist, float *out, uint32_t n_embd,
                    uint32_t ksize, uint32_t n_tokens);
void run_short_conv_batch(hipStream_t s, const float *bcx, const float *taps, float *hist, float *out,
                          uint32_t n_embd, uint32_t ksize, uint32_t n_tokens);
// run_short_conv_batch plus, in scratch, the fp16 inputs of the output
// (as run_rms_norm_split leaves them) for a following run_matmul(..., x =
// out, n_tokens, n_cols = n_embd, scratch, ..., split_ready = true), in one
// launch.  False (nothing launched) for shapes it does not take: ksize
// other than 3, or more than 4096 channels.
bool run_short_conv_split(hipStream_t s, const float *bcx, const float *taps, float *hist, float *out,
                          uint32_t n_embd, uint32_t ksize, uint32_t n_tokens, void *scratch);

// attention.hip.  Causal GQA attention of n_queries queries at positions
// first_pos + dpos.. over a cache of [pos][n_kv][head_dim] (f16 when
// kv_half).  `partials` holds attention_partial_floats() floats and
// `counters` n_queries * n_kv_heads zeroed u32 (left zeroed on exit).
uint32_t attention_splits(uint32_t n_keys_max, uint32_t n_kv_heads, uint32_t n_cus);
uint64_t attention_partial_floats(uint32_t n_queries, uint32_t n_heads, uint32_t head_dim, uint32_t splits);
void run_attention(hipStream_t s, const float *q, const void *k_cache, const void *v_cache, bool kv_half,
                   float *partials, uint32_t *counters, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                   uint32_t head_dim, uint32_t first_pos, const uint32_t *dpos, uint32_t n_queries, uint32_t splits);

// attn_prefill.hip: causal GQA attention of n_queries queries at positions
// first_pos.. over the f16 cache (their keys already stored), on MFMA.  q and
// out rows are q_stride / out_stride floats apart, head h at h·head_dim.
// `partials` (nullable) is scratch for key splits.  `gate` (nullable): the
// output of (query z, head h) is scaled element-wise by sigmoid of the gate
// at gate + z·gate_query_stride + h·gate_head_stride (gated attention).
bool attn_prefill_mfma_supported(uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, bool kv_half);
void run_attn_prefill_mfma(hipStream_t s, const float *q, const void *k_cache, const void *v_cache, float *out,
                           uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t first_pos,
                           uint32_t n_queries, uint32_t q_stride, uint32_t out_stride, float scale,
                           float *partials, uint64_t partial_floats, const float *gate = nullptr,
                           uint32_t gate_head_stride = 0, uint32_t gate_query_stride = 0);
// Key splits run_attn_prefill_mfma uses for a batch (1 without scratch):
// the keys are split so the launch fills the chip, each split's
// (max, sum, output) partials going to `partials` (partial_floats floats).
uint32_t attn_prefill_splits(uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t first_pos,
                             uint32_t n_queries, uint64_t partial_floats);
// Floats of the partials of n_queries queries in `splits` key splits.
uint64_t attn_prefill_partial_floats(uint32_t n_queries, uint32_t n_heads, uint32_t head_dim, uint32_t splits);

// matmul.hip.  Y[t] (store) W·X[t] for n_tokens rows; store 0 overwrite,
// 1 accumulate, 2 swiglu (y = silu(y) * product).
// `scratch` holds the inputs split into fp16 high and low parts
// (matmul_split_bytes(n_tokens, n_cols) bytes) and, after them, the
// split-K partial products: scratch_bytes bounds how many column splits a
// launch may use (matmul_scratch_bytes(n_tokens, n_cols, n_rows) allows
// all; matmul_split_bytes alone allows none).
uint64_t matmul_split_bytes(uint32_t n_rows, uint32_t n_cols);
uint64_t matmul_scratch_bytes(uint32_t n_tokens, uint32_t n_cols, uint32_t n_rows);
// A column-split sum an accumulating run_matmul left for the next kernel:
// y += Σ_split part[split] (n floats each), in split order.
struct PendingSum {
  const float *part = nullptr;
  uint32_t splits = 0;
  uint64_t n = 0;
};
// Adds a pending sum into y (its run_matmul's y) and clears it.
void finish_pending_sum(hipStream_t s, PendingSum &p, float *y);
// run_rms_norm's output for `rows` rows of n, and in `scratch` the fp16
// inputs a following run_matmul(..., x = out, n_tokens = rows, n_cols = n,
// scratch, ..., split_ready = true) reads.  With `pending` (left by the
// run_matmul that accumulated into x, on the same scratch) x first
// receives that sum, written back to x; the pending sum is then cleared.
// unscale_copy (optional, [rows]): a second copy of the token scales,
// outside the scratch (run_blas_pair's).
void run_rms_norm_split(hipStream_t s, float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps,
                        void *scratch, PendingSum *pending = nullptr, float *unscale_copy = nullptr);
// store 3: y = silu(W·x) ⊙ (W2·x), W and W2 the gate and up matrices of
// a SwiGLU (same format and shape).  split_ready: the previous run_matmul
// on this scratch had the same x, n_tokens and n_cols, so its fp16 inputs
// are reused instead of converted again.
// defer (store 1 only): when the launch splits the columns, the partial sums
// are left in scratch and described in *defer instead of added to y; the
// caller passes *defer to the run_rms_norm_split that reads y next, or to
// finish_pending_sum.  (*defer is cleared when nothing is left pending.)
void run_matmul(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols, const float *x,
                float *y, uint32_t n_tokens, uint32_t store, void *scratch, uint64_t scratch_bytes,
                bool split_ready = false, const uint8_t *W2 = nullptr, PendingSum *defer = nullptr);

// Expanded fp16 copy of a weight matrix ([n_rows][n_cols], the values
// k_gemm dequantises) for the library GEMM; n_cols a multiple of 64.
bool expand_f16_supported(uint32_t format, uint32_t n_cols);
void run_expand_f16(hipStream_t s, uint32_t format, const uint8_t *W, uint32_t n_rows, uint32_t n_cols,
                    _Float16 *out);
// blas.hip.  D [n_tokens][n_rows] f32 = H [n_tokens][n_cols] fp16 · W16^T
// through hipBLASLt (the device's handle and workspace made on first use,
// or by blas_prepare).
int blas_prepare();
int run_blas_gemm_f16(hipStream_t s, const _Float16 *W16, uint32_t n_rows, uint32_t n_cols, const _Float16 *H,
                      uint32_t n_tokens, float *D);
// The SwiGLU of a library pair product D [n_tokens][2 n_ff] whose inputs
// had the token scales us (1/us applied to each token's fp16 inputs): the
// down projection's fp16 inputs go to `scratch` as run_matmul's
// split_ready expects them, and ffn to f32 when given.
void run_swiglu_split(hipStream_t s, const float *D, uint32_t n_ff, uint32_t n_tokens, const float *us, float *f32,
                      void *scratch);
// The SwiGLU pair of a prefill batch on the library GEMM (run_blas_gemm_f16
// then run_swiglu_split): the inputs in `split` as run_rms_norm_split
// leaves them, their token scales also in pair_us (its unscale_copy: the
// SwiGLU overwrites the ones in `split`), pair_out [n_tokens][2 n_ff] its
// own buffer, ffn (optional) the f32 activations.  False when the library
// call fails (printed); nothing was then written.
bool run_blas_pair(hipStream_t s, const _Float16 *gate_up16, uint32_t n_ff, uint32_t n_cols, uint32_t n_tokens,
                   void *split, float *pair_out, const float *pair_us, float *ffn);
// Prefill batches of more than this many tokens take the library pair.
constexpr uint32_t kBlasPairMinTokens = 128;
// Pairs of fewer weights (gate and up together) keep the Q4_K tile.
constexpr uint64_t kBlasPairMinWeights = 1ull << 24;

}  // namespace bch
