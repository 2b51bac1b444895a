/* bobcat_hip.h — C ABI of the MI355X (gfx950) backend for bobcat's per-token
 * language-model loop.
 *
 * The op set mirrors the concrete `bobcat_metal::Metal` API that bobcat's
 * drivers call today (crates/bobcat-metal/src/backend.rs:1027-2699,
 * re-exported at crates/bobcat-metal/src/lib.rs:13-17).  Every launcher takes
 * views (buffer, byte offset) as the reference does (backend.rs:300-341),
 * checks each view against its buffer's length before launching
 * (backend.rs:1297-1314, 2771-2790), and returns a status code; the message of
 * the last failure on the calling thread comes from bch_last_error().
 *
 * Work goes onto one in-order HIP stream per context, so the reference's
 * barriers (backend.rs:1255) order nothing extra here and cost nothing.
 * bch_commit() returns a monotonically increasing ticket and bch_wait(t)
 * drains every ticket up to t (crates/bobcat-metal/src/commands.rs:293-338).
 *
 * Sizes are u32 as in the reference; byte offsets and lengths are u64.
 * No HIP or torch type appears in any signature.
 */
#ifndef BOBCAT_HIP_H
#define BOBCAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* Status codes: one per variant of bobcat_metal::Error                */
/* (crates/bobcat-metal/src/backend.rs:162-298) that can arise here.   */
/* ------------------------------------------------------------------ */
typedef enum bch_status {
  BCH_OK = 0,
  BCH_ERR_NO_DEVICE = 1,        /* Error::NoDevice */
  BCH_ERR_ALLOCATION = 2,       /* Error::Allocation */
  BCH_ERR_NOT_RECORDING = 3,    /* Error::NotRecording */
  BCH_ERR_ALREADY_RECORDING = 4,/* Error::AlreadyRecording */
  BCH_ERR_OUT_OF_BOUNDS = 5,    /* Error::OutOfBounds */
  BCH_ERR_FOREIGN_BUFFER = 6,   /* Error::ForeignBuffer */
  BCH_ERR_BUSY = 7,             /* Error::Busy */
  BCH_ERR_ACCESS = 8,           /* Error::Access */
  BCH_ERR_ATTENTION_LIMITS = 9, /* Error::AttentionLimits */
  BCH_ERR_UNSUPPORTED_FORMAT = 10, /* Error::NoFusedConv / NoExpansion / NoExperts */
  BCH_ERR_DELTANET_LIMITS = 11, /* Error::DeltaNetLimits */
  BCH_ERR_EXPERT_LIMITS = 12,   /* Error::ExpertLimits */
  BCH_ERR_EXECUTION = 13,       /* Error::Execution */
  BCH_ERR_ARGUMENT = 14,        /* bobcat::Error::Argument (crates/bobcat/src/error.rs) */
  BCH_ERR_CONTEXT_FULL = 15,    /* bobcat::Error::ContextFull */
  BCH_ERR_TOKEN = 16,           /* bobcat::Error::Token */
  BCH_ERR_GATE_SHAPE = 17,      /* Error::GateShape */
  BCH_ERR_GGUF = 18,            /* bobcat_gguf::Error (crates/bobcat-gguf/src/lib.rs:27-95) */
  BCH_ERR_MODEL = 19,           /* bobcat::Error::{Metadata, Architecture, Hyperparameters, MissingTensor,
                                   TensorShape, TensorType, KvHeads, OddHeadDim} of a model file */
} bch_status;

/* Return the message of the last failed call on this thread ("" if none). */
const char *bch_last_error(void);

/* ------------------------------------------------------------------ */
/* Weight formats.  Values are ggml type ids, as TensorType::id        */
/* (crates/bobcat-gguf/src/lib.rs:137-148); the block layouts match    */
/* ggml's (scalar.rs:56-202).                                          */
/* ------------------------------------------------------------------ */
typedef enum bch_format {
  BCH_F32 = 0,
  BCH_F16 = 1,
  BCH_Q4_0 = 2,
  BCH_Q8_0 = 8,
  BCH_Q4K = 12,
  BCH_Q5K = 13,
  BCH_Q6K = 14,
  BCH_BF16 = 30,
} bch_format;

/* Bytes of one row of n_cols elements of `format` (scalar.rs:28-31), or 0
 * when n_cols fills no whole number of blocks or the format is unknown. */
uint64_t bch_row_bytes(uint32_t format, uint32_t n_cols);

/* ------------------------------------------------------------------ */
/* Device, buffers, views (backend.rs:1083-1230)                        */
/* ------------------------------------------------------------------ */
typedef struct bch_ctx bch_ctx;
typedef struct bch_buffer bch_buffer;

/* A position inside a buffer, as bobcat_metal::View (backend.rs:337-341). */
typedef struct bch_view {
  bch_buffer *buffer;
  uint64_t offset;
} bch_view;

/* An RMS normalization a matrix-vector launch applies to its input first
 * (bobcat_metal::Norm, backend.rs:344-350). */
typedef struct bch_norm {
  bch_view weight;
  float eps;
} bch_norm;

/* Metal::open (backend.rs:1083).  Opens device 0 and one stream. */
int bch_open(bch_ctx **out);
void bch_close(bch_ctx *ctx);
/* Name of the device and its compute-unit count, for reports. */
int bch_device_info(bch_ctx *ctx, char *name, size_t name_len, uint32_t *n_cus);

/* Metal::new_buffer (backend.rs:1124): `len` zeroed bytes of HBM. */
int bch_buffer_new(bch_ctx *ctx, uint64_t len, bch_buffer **out);
/* Metal::wrap_mapping (backend.rs:1145): the weights of a file.  MI355X has
 * no unified memory, so the bytes are copied to HBM once. */
int bch_buffer_from_host(bch_ctx *ctx, const void *data, uint64_t len, bch_buffer **out);
void bch_buffer_free(bch_buffer *buffer);
uint64_t bch_buffer_len(const bch_buffer *buffer);
/* The device address of the buffer's first byte, for interop. */
void *bch_buffer_device_ptr(const bch_buffer *buffer);

/* Metal::write / Metal::read (backend.rs:1180-1230).  Fail with BCH_ERR_BUSY
 * while committed work is in flight and with BCH_ERR_ACCESS past the end. */
int bch_write(bch_ctx *ctx, bch_view view, const void *data, uint64_t bytes);
int bch_read(bch_ctx *ctx, bch_view view, void *out, uint64_t bytes);

/* ------------------------------------------------------------------ */
/* Recording (backend.rs:1244-1295, commands.rs:207-411)               */
/* ------------------------------------------------------------------ */
int bch_begin(bch_ctx *ctx);
void bch_discard(bch_ctx *ctx);
/* Launches on one in-order stream are ordered already; kept for parity. */
void bch_barrier(bch_ctx *ctx);
int bch_commit(bch_ctx *ctx, uint64_t *ticket);
/* Wait for `ticket` and every earlier one; *gpu_seconds (nullable) receives
 * the device time between the commit's begin and its end. */
int bch_wait(bch_ctx *ctx, uint64_t ticket, double *gpu_seconds);
/* commit + wait (Metal::end, backend.rs:1276). */
int bch_end(bch_ctx *ctx, double *gpu_seconds);

/* Metal::set_profiling / profile (backend.rs:1285-1295, 376-391). */
typedef struct bch_profile_entry {
  char name[48];
  uint32_t n_rows;
  uint32_t n_cols;
  uint64_t calls;
  double seconds;
  uint64_t bytes;
} bch_profile_entry;
void bch_set_profiling(bch_ctx *ctx, int enabled);
uint32_t bch_profile_count(const bch_ctx *ctx);
int bch_profile_get(const bch_ctx *ctx, uint32_t index, bch_profile_entry *out);

/* ------------------------------------------------------------------ */
/* Ops.  Each records one or more launches on the context's stream.    */
/* ------------------------------------------------------------------ */

/* Dequantize n_rows rows of n_cols weights of `format` into floats at
 * `out` (scalar::dequantize, scalar.rs:59-79; bit-exact). */
int bch_dequantize(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows,
                   uint32_t n_cols, bch_view out);

/* Metal::matvec (backend.rs:1344-1380): y (=|+=) W·x, optionally with the
 * RMS norm of x fused in (norm may be NULL). */
int bch_matvec(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows,
               uint32_t n_cols, bch_view x, bch_view y, const bch_norm *norm,
               int accumulate);

/* Metal::matvec_swiglu (backend.rs:1385-1417): y = silu(G·n(x)) ⊙ (U·n(x)). */
int bch_matvec_swiglu(bch_ctx *ctx, uint32_t format, bch_view gate, bch_view up,
                      uint32_t n_rows, uint32_t n_cols, bch_view x, bch_norm norm,
                      bch_view y);

/* Metal::matvec_conv (backend.rs:2329-2377): the 3·n_embd-row input
 * projection of a gated short convolution followed by the convolution of
 * one token; updates `history` ((kernel_size-1)·n_embd floats). */
int bch_matvec_conv(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_cols,
                    bch_view x, const bch_norm *norm, bch_view taps, bch_view history,
                    bch_view out, uint32_t n_embd, uint32_t kernel_size);

/* Metal::short_conv / short_conv_batch (backend.rs:2384-2465): the gated
 * short convolution of n_tokens tokens whose rows of 3·n_embd floats at
 * `bcx` hold B, C and X. */
int bch_short_conv(bch_ctx *ctx, bch_view bcx, bch_view taps, bch_view history,
                   bch_view out, uint32_t n_embd, uint32_t kernel_size, uint32_t n_tokens);
int bch_short_conv_batch(bch_ctx *ctx, bch_view bcx, bch_view taps, bch_view history,
                         bch_view out, uint32_t n_embd, uint32_t kernel_size, uint32_t n_tokens);

/* Metal::rms_norm (backend.rs:2034-2059). */
int bch_rms_norm(bch_ctx *ctx, bch_view x, bch_view weight, bch_view out, uint32_t n,
                 uint32_t n_rows, float eps);

/* Metal::norm_rope (backend.rs:2070-2123). */
int bch_norm_rope(bch_ctx *ctx, bch_view src, bch_view dst, int dst_half, bch_view weight,
                  uint32_t n_heads, uint32_t head_dim, uint32_t n_rot,
                  uint32_t src_head_stride, uint32_t pos, uint32_t n_tokens,
                  uint32_t src_stride, uint32_t dst_stride, float theta, float eps);

/* Metal::convert_half / copy (backend.rs:2126, 2552). */
int bch_convert_half(bch_ctx *ctx, bch_view src, bch_view dst, uint32_t n);
int bch_copy(bch_ctx *ctx, bch_view src, bch_view dst, uint32_t n);

/* Metal::embed (backend.rs:2570-2608): dequantize rows tokens[t] of the
 * n_vocab-row matrix into `out`, for n_tokens u32 token ids. */
int bch_embed(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_vocab,
              bch_view tokens, bch_view out, uint32_t n_embd, uint32_t n_tokens);

/* Metal::attention (backend.rs:2150-2320): causal GQA attention of
 * n_queries queries at positions first_pos.. over an f16 or f32 cache laid
 * out [pos][kv_head][head_dim].  `scratch` holds
 * bch_attention_scratch_floats(...) floats. */
int bch_attention(bch_ctx *ctx, bch_view q, bch_view k_cache, bch_view v_cache, int kv_half,
                  bch_view scratch, bch_view out, uint32_t n_heads, uint32_t n_kv_heads,
                  uint32_t head_dim, uint32_t first_pos, uint32_t n_queries, uint32_t n_ctx);
/* MI355X addition (no counterpart in the reference): the prefill form of
 * Metal::attention (backend.rs:2150-2320, attention_flash attention.metal:
 * 289-480) on MFMA, for an f16 cache, head_dim 64, 128 or 256 and at most 4 query
 * heads per KV head (else BCH_ERR_ATTENTION_LIMITS).  Queries and
 * probabilities enter the products as f16 high + low parts (~22 bits), so
 * results agree with bch_attention to ~1e-6 of the outputs' scale, not
 * bit for bit.  No scratch. */
int bch_attention_prefill(bch_ctx *ctx, bch_view q, bch_view k_cache, bch_view v_cache, bch_view out,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t first_pos,
                          uint32_t n_queries, uint32_t n_ctx);
/* attention_scratch_floats (backend.rs:2739-2748). */
uint64_t bch_attention_scratch_floats(uint32_t n_heads, uint32_t head_dim, uint32_t n_ctx,
                                      uint32_t n_queries);
/* MI355X addition (no counterpart in the reference as one call): the
 * decode step of an LFM2 attention layer after its projections
 * (lfm2.rs:515-555) as the model drivers run it: each query head and key
 * head RMS-normalised with q_norm / k_norm [head_dim] (eps), its first
 * n_rot elements rotated NeoX-style for position `pos` (rope_theta), the
 * key and value stored in the caches at `pos` (rounded to f16 when
 * kv_half), then softmax(q·k/√head_dim)·v over positions 0..pos into `out`.
 * q: [n_heads][head_dim], k and v: [n_kv_heads][head_dim], f32; caches
 * [pos][kv_head][head_dim].  Head sizes whose cache rows are 64 to 1024
 * bytes in powers of two, up to 256 elements; at most 256 query heads.
 * `scratch` holds bch_attention_decode_scratch_floats(...) floats,
 * 16-byte aligned (the MFMA-scored f16 path agrees with bch_attention to
 * ~1e-6 of the outputs' scale). */
int bch_attention_decode(bch_ctx *ctx, bch_view q, bch_view k, bch_view v, bch_view q_norm, bch_view k_norm,
                         float eps, float rope_theta, uint32_t n_rot, bch_view k_cache, bch_view v_cache,
                         int kv_half, bch_view scratch, bch_view out, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t pos, uint32_t n_ctx);
uint64_t bch_attention_decode_scratch_floats(uint32_t n_heads, uint32_t head_dim, uint32_t n_ctx, int kv_half);

/* bch_matmul without any allocation: the same kernels, column split and
 * results (bit for bit) as bch_matmul, with the launch's scratch — its fp16
 * inputs, n_tokens·(2·n_cols + 4) bytes, and the partial sums of the column
 * split bch_matmul picks for the shape, 4·splits·n_tokens·n_rows bytes when
 * it splits — in a static device array of bch_matmul_noalloc_max_bytes()
 * (16 MiB) that each GPU holds for the life of the process, instead of
 * context scratch that may grow with hipMalloc.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid allocation).  Launches needing more
 * fail with BCH_ERR_ARGUMENT.  All calls on one GPU share the array, so
 * calls that overlap on one GPU (other streams or threads) race. */
int bch_matmul_noalloc(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows, uint32_t n_cols,
                       bch_view x, bch_view y, uint32_t n_tokens, uint32_t store);
uint64_t bch_matmul_noalloc_max_bytes(void);
/* Metal::matmul (backend.rs:2470-2516): Y[t] (store) W·X[t] for n_tokens
 * rows of n_cols floats at x; store as bobcat_metal::Store
 * (backend.rs:360-370). */
typedef enum bch_store { BCH_STORE_OVERWRITE = 0, BCH_STORE_ACCUMULATE = 1, BCH_STORE_SWIGLU = 2 } bch_store;
int bch_matmul(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows,
               uint32_t n_cols, bch_view x, bch_view y, uint32_t n_tokens, uint32_t store);

/* Metal::argmax (backend.rs:2612): index of the largest of n floats, ties
 * to the lowest index, as a u32 at `out`. */
int bch_argmax(bch_ctx *ctx, bch_view x, bch_view out, uint32_t n);

/* read_sum (crates/bobcat-metal/src/bandwidth.rs:20-34): n_threads threads
 * (a multiple of 256) each sum the float4 values of `src` at a stride of
 * the grid into out[thread].  The streaming-read bandwidth probe. */
int bch_read_sum(bch_ctx *ctx, bch_view src, uint64_t n_vectors, bch_view out, uint32_t n_threads);

/* ------------------------------------------------------------------ */
/* Mixture of experts.  A route holds, per token, the n_used expert ids */
/* the router picked, then their n_used weights as float bits          */
/* (moe.metal:1-6).  Limits: n_experts <= 128, 1 <= n_used <= 8        */
/* (backend.rs:2728-2734).  Expert matrices stack the experts by rows. */
/* ------------------------------------------------------------------ */

/* route_bytes (backend.rs:2724-2726): 2 * n_used * n_tokens * 4. */
uint64_t bch_route_bytes(uint32_t n_used, uint32_t n_tokens);
/* Metal::moe_route (backend.rs:1428-1479): sigmoid scores of the F32
 * router [n_experts x n_cols], top n_used by score + bias (ties to the
 * lower expert), weights = score / (sum of picked scores + 1e-6).  With
 * `norm` (nullable), each token is first RMS-normalised into `normed`. */
int bch_moe_route(bch_ctx *ctx, bch_view x, const bch_norm *norm, bch_view normed, bch_view router,
                  bch_view bias, bch_view route, uint32_t n_cols, uint32_t n_experts, uint32_t n_used,
                  uint32_t n_tokens);
/* Metal::matvec_experts_swiglu (backend.rs:1481-1536): row n_used·t + s of
 * y [n_rows floats] = silu(G_e·x_t) ⊙ U_e·x_t for the expert e in slot s. */
int bch_matvec_experts_swiglu(bch_ctx *ctx, uint32_t format, bch_view gate, bch_view up, uint32_t n_rows,
                              uint32_t n_cols, uint32_t n_experts, bch_view x, bch_view route, uint32_t n_used,
                              bch_view y, uint32_t n_tokens);
/* Metal::matvec_experts_down (backend.rs:1538-1597): y_t += Σ_s w_s ·
 * D_e·x_{n_used·t+s}, the experts added in route order. */
int bch_matvec_experts_down(bch_ctx *ctx, uint32_t format, bch_view weights, uint32_t n_rows, uint32_t n_cols,
                            uint32_t n_experts, bch_view x, bch_view route, uint32_t n_used, bch_view y,
                            uint32_t n_tokens);
/* Metal::moe_group (backend.rs:1599-1628): the n_used·n_tokens entries
 * v = n_used·t + s grouped by expert; expert e's entries are
 * entries[offsets[e] .. offsets[e+1]) in token order, offsets[n_experts]
 * the total.  offsets: n_experts + 1 u32, entries: n_used·n_tokens u32. */
int bch_moe_group(bch_ctx *ctx, bch_view route, bch_view offsets, bch_view entries, uint32_t n_experts,
                  uint32_t n_used, uint32_t n_tokens);
/* Metal::matmul_experts (backend.rs:1630-1703): each expert of the stack
 * times the inputs grouped to it, on MFMA.  Entry v reads row v of x, or
 * row v / n_used with shared_input, and overwrites row v of y; with `up`
 * (may be NULL) y = silu(W_e·x) ⊙ Up_e·x.  Columns a multiple of 256. */
int bch_matmul_experts(bch_ctx *ctx, uint32_t format, bch_view weights, const bch_view *up, uint32_t n_rows,
                       uint32_t n_cols, uint32_t n_experts, bch_view x, int shared_input, bch_view offsets,
                       bch_view entries, uint32_t n_used, bch_view y, uint32_t n_tokens);
/* Metal::moe_combine (backend.rs:1705-1731): y_t += Σ_s w_s · x_{n_used·t+s},
 * the slots summed in route order before the add. */
int bch_moe_combine(bch_ctx *ctx, bch_view x, bch_view route, bch_view y, uint32_t n_embd, uint32_t n_used,
                    uint32_t n_tokens);

/* ------------------------------------------------------------------ */
/* Sampling                                                            */
/* ------------------------------------------------------------------ */

/* bobcat::Sampling (crates/bobcat/src/lfm2.rs:53-64). */
typedef struct bch_sampling {
  float temperature;    /* <= 0 picks the most likely token */
  uint32_t top_k;       /* 0 keeps every token */
  float top_p;
  float min_p;
  float repeat_penalty; /* 1 turns the penalty off */
} bch_sampling;

/* The per-token callback of generate_stream (the `emit` closure of
 * lfm2_metal.rs:425-431): return nonzero to keep generating. */
typedef int (*bch_emit_fn)(uint32_t token, void *user);

/* Sampler::sample (crates/bobcat-cli/src/sampler.rs:45-112) on the GPU:
 * penalty over the distinct tokens of the last 64 of `recent` (applied to
 * `logits` in place), top-k, top-p, min-p, temperature, then a draw from the
 * wyrand generator whose 8-byte state is at `rng_state` (advanced by one
 * draw).  The token goes to `out` (4 bytes).  Every candidate of the
 * vocabulary takes part: top_k = 0 (or top_k >= n_vocab) keeps them all, and
 * any top_k up to n_vocab is honoured exactly. */
int bch_sample(bch_ctx *ctx, bch_view logits, uint32_t n_vocab, bch_view recent, uint32_t n_recent,
               const bch_sampling *settings, bch_view rng_state, bch_view out);

/* bch_sample with the draw given: `u` in [0, 1) takes the place of the
 * generator's f32 (sampler.rs:102-109 walks the kept candidates with it).
 * No counterpart in the reference, whose Sampler owns its generator; for
 * callers that keep their own random stream.  Fails with BCH_ERR_ARGUMENT
 * for u outside [0, 1). */
int bch_sample_draw(bch_ctx *ctx, bch_view logits, uint32_t n_vocab, bch_view recent, uint32_t n_recent,
                    const bch_sampling *settings, float u, bch_view out);

/* ------------------------------------------------------------------ */
/* Gated DeltaNet and gated attention (Qwen3.5)                        */
/* A DeltaNet token holds conv_dim = 2·n_k·k_dim + n_v·v_dim floats:    */
/* the query heads, the key heads, the value heads; value head j reads  */
/* key head j % n_k (gdn.metal:1-6).  States are [n_v][k_dim][v_dim].   */
/* ------------------------------------------------------------------ */

/* DeltaShape (backend.rs, gdn_recurrence's shape argument). */
typedef struct bch_delta_shape {
  uint32_t n_k_heads;
  uint32_t n_v_heads;
  uint32_t k_dim;
  uint32_t v_dim;
} bch_delta_shape;

/* Metal::gdn_conv (gdn.metal:8-42): causal convolution of n_tokens tokens
 * of `channels` floats with kernel_size (2..8) taps per channel, the oldest
 * first, SiLU of each result into y; `history` [channels][kernel_size-1]
 * moves forward. */
int bch_gdn_conv(bch_ctx *ctx, bch_view x, bch_view taps, bch_view history, bch_view y, uint32_t channels,
                 uint32_t kernel_size, uint32_t n_tokens);
/* Metal::gdn_gates (gdn.metal:125-149): beta <- sigmoid(beta), alpha <-
 * exp(a·softplus(alpha + dt_bias)) for n values, n_v_heads per token. */
int bch_gdn_gates(bch_ctx *ctx, bch_view beta, bch_view alpha, bch_view a, bch_view dt_bias, uint32_t n_v_heads,
                  uint32_t n);
/* Metal::gdn_recurrence (gdn.metal:204-290): the gated delta rule over
 * n_tokens tokens of y (after gdn_conv) with the gated beta and decay;
 * queries and keys are L2-normalised here (eps 1e-6), queries times q_scale.
 * Key heads of 64 or 128. */
int bch_gdn_recurrence(bch_ctx *ctx, bch_view y, bch_view beta, bch_view decay, bch_view state, bch_view out,
                       const bch_delta_shape *shape, uint32_t n_tokens, float q_scale);
/* The recurrence of bch_gdn_recurrence in its chunked (WY) form, for
 * prefill: 64-token chunks, each chunk's deltas from a triangular solve
 * (I + A) D = diag(beta)(V - diag(gamma) K S0) and the state carried from
 * chunk to chunk; same arguments and result (to rounding) as
 * bch_gdn_recurrence, whose reference form is gdn.metal:204-290 and
 * qwen35.rs:430-516 (the reference has no chunked form).  `scratch` holds
 * bch_gdn_chunk_scratch_floats(shape, n_tokens) floats.  Value heads of at
 * most 256, a multiple of 8. */
uint64_t bch_gdn_chunk_scratch_floats(const bch_delta_shape *shape, uint32_t n_tokens);
int bch_gdn_recurrence_chunked(bch_ctx *ctx, bch_view y, bch_view beta, bch_view decay, bch_view state,
                               bch_view out, const bch_delta_shape *shape, uint32_t n_tokens, float q_scale,
                               bch_view scratch);
/* Metal::gdn_gated_norm (gdn.metal:100-123): each row of v_dim floats of x
 * <- weight ⊙ rmsnorm(row) ⊙ silu(z row), in place. */
int bch_gdn_gated_norm(bch_ctx *ctx, bch_view x, bch_view weight, bch_view z, uint32_t v_dim, uint32_t n_rows,
                       float eps);
/* Metal::attention_gate (gdn.metal:300-322): attn [n_tokens][q_dim] *=
 * sigmoid of the gate half of each head's block in q_gate
 * [n_tokens][2·q_dim]. */
int bch_attention_gate(bch_ctx *ctx, bch_view attn, bch_view q_gate, uint32_t head_dim, uint32_t q_dim,
                       uint32_t n_tokens);

/* ------------------------------------------------------------------ */
/* LFM2 driver (crates/bobcat/src/lfm2_metal.rs:125-779)               */
/* ------------------------------------------------------------------ */

/* A matrix of the model: n_rows rows of n_cols elements of `format` at
 * host address `data` (ggml's ne[1], ne[0]; lfm2.rs:66-71). */
typedef struct bch_matrix {
  uint32_t format;
  uint32_t n_rows;
  uint32_t n_cols;
  const void *data;
} bch_matrix;

/* One LFM2 layer (lfm2.rs:150-170).  `is_attention` picks the mixer;
 * `is_moe` picks the feed-forward block.  Unused members stay zero. */
typedef struct bch_lfm2_layer {
  uint32_t is_attention;
  uint32_t is_moe;
  const float *attn_norm;   /* [n_embd] */
  const float *ffn_norm;    /* [n_embd] */
  /* convolution mixer */
  const float *conv_taps;   /* [n_embd][conv_kernel] */
  bch_matrix in_proj;       /* 3·n_embd × n_embd */
  bch_matrix out_proj;      /* n_embd × n_embd */
  /* attention mixer */
  bch_matrix wq, wk, wv, wo;
  const float *q_norm;      /* [head_dim] */
  const float *k_norm;      /* [head_dim] */
  /* dense feed-forward */
  bch_matrix gate, up, down;
  /* mixture of experts: experts stacked by rows (lfm2.rs:128-142) */
  bch_matrix router;        /* n_experts × n_embd, F32 */
  const float *expert_bias; /* [n_experts] */
  bch_matrix gate_exps, up_exps, down_exps;
} bch_lfm2_layer;

/* lfm2::Hyperparameters (lfm2.rs:17-49) plus the tensors. */
typedef struct bch_lfm2_model {
  uint32_t n_layers;
  uint32_t n_embd;
  uint32_t n_ff;
  uint32_t n_experts;
  uint32_t n_experts_used;
  uint32_t n_ff_expert;
  uint32_t n_heads;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  uint32_t n_vocab;
  uint32_t conv_kernel;
  float rope_theta;
  float norm_eps;
  const bch_lfm2_layer *layers;
  bch_matrix token_embd;    /* n_vocab × n_embd */
  bch_matrix output;        /* n_vocab × n_embd (tied: same data as token_embd) */
  const float *output_norm; /* [n_embd] */
} bch_lfm2_model;

typedef struct bch_lfm2 bch_lfm2;

/* Lfm2Metal::new (lfm2_metal.rs:125-220): copies the weights to HBM and
 * allocates the caches for sequences of up to n_ctx tokens. */
int bch_lfm2_new(bch_ctx *ctx, const bch_lfm2_model *model, uint32_t n_ctx, int kv_half,
                 bch_lfm2 **out);
void bch_lfm2_free(bch_lfm2 *lfm2);
uint32_t bch_lfm2_n_past(const bch_lfm2 *lfm2);
/* Lfm2Metal::reset (lfm2_metal.rs:237-247). */
int bch_lfm2_reset(bch_lfm2 *lfm2);
/* Lfm2Metal::step (lfm2_metal.rs:308-365); logits (nullable) receives
 * n_vocab floats; trace arrays (nullable) receive the embedding, every
 * layer's output and the final norm of the token. */
int bch_lfm2_step(bch_lfm2 *lfm2, uint32_t token, float *logits, float *trace_embedding,
                  float *trace_layers, float *trace_final);
/* Lfm2Metal::prefill (lfm2_metal.rs:662-762), in batches of up to 512
 * tokens; logits (nullable) receives the last token's.  The trace arrays
 * (nullable) receive every token's activations: trace_embedding and
 * trace_final n_tokens·n_embd floats, trace_layers layer by layer, each
 * layer's n_tokens rows together (lfm2.rs:630-675). */
int bch_lfm2_prefill(bch_lfm2 *lfm2, const uint32_t *tokens, uint32_t n_tokens, float *logits,
                     float *trace_embedding, float *trace_layers, float *trace_final);
/* Lfm2Metal::greedy_token (lfm2_metal.rs:372-398). */
int bch_lfm2_greedy_token(bch_lfm2 *lfm2, uint32_t *token);
/* Lfm2Metal::generate (lfm2_metal.rs:408-411): n greedy tokens, the first
 * the argmax of the current logits; each step runs on the GPU with no host
 * round trip (a captured HIP graph replayed per token). */
int bch_lfm2_generate(bch_lfm2 *lfm2, uint32_t *out, uint32_t n);
/* Lfm2Metal::generate_next (lfm2_metal.rs:413-420): consume the current
 * greedy selection (greedy_token) and n - 1 more, storing the selection after
 * each of the n steps; the last stays unconsumed.  n = 0 changes nothing. */
int bch_lfm2_generate_next(bch_lfm2 *lfm2, uint32_t *out, uint32_t n);
/* Lfm2Metal::generate_stream (lfm2_metal.rs:425-560; called by enum Gpu,
 * crates/bobcat-cli/src/backend.rs:128-137).  Emits the argmax of the
 * current logits, then runs up to max_tokens - 1 greedy steps (bounded by the
 * free context), passing each selected token to emit(token, user) as soon as
 * its step finishes; up to three steps are queued ahead of the host.  When
 * emit returns 0 no further step is queued (queued steps still run).
 * `gained` (room for max_tokens) receives the tokens the sequence consumed,
 * *n_gained of them: every emitted token but the last, possibly followed by
 * tokens selected after the last emitted one — the Vec the reference
 * returns. */
int bch_lfm2_generate_stream(bch_lfm2 *lfm2, uint32_t max_tokens, bch_emit_fn emit, void *user, uint32_t *gained,
                             uint32_t *n_gained);
/* Lfm2Metal::checkpoint / restore (lfm2_metal.rs:250-288).  The blob holds
 * the reset count, n_past, the convolution history and the logits;
 * bch_lfm2_checkpoint_bytes gives its size. */
/* generate with Sampler::sample instead of argmax (engine.rs:615-630 runs
 * the sampler on the CPU; here it runs inside the replayed graph): n tokens,
 * the generator seeded with `seed`; the recent tokens of the penalty are
 * the sequence's own. */
int bch_lfm2_generate_sampled(bch_lfm2 *lfm2, uint32_t *out, uint32_t n, const bch_sampling *settings,
                              uint64_t seed);
uint64_t bch_lfm2_checkpoint_bytes(const bch_lfm2 *lfm2);
int bch_lfm2_checkpoint(bch_lfm2 *lfm2, void *blob, uint64_t bytes);
int bch_lfm2_restore(bch_lfm2 *lfm2, const void *blob, uint64_t bytes);
/* Last call's host-side recording time and device time (lfm2_metal.rs:222-230). */
double bch_lfm2_last_gpu_seconds(const bch_lfm2 *lfm2);

/* ------------------------------------------------------------------ */
/* Qwen3.5 (crates/bobcat/src/qwen35.rs, qwen35_metal.rs)              */
/* ------------------------------------------------------------------ */

/* One Qwen3.5 layer (qwen35.rs:86-145): a gated attention mixer or a Gated
 * DeltaNet mixer, then a SwiGLU block.  Norm weights are as the GGUF stores
 * them (the +1 of the zero-centred norms baked in); `a` is -exp(A_log). */
typedef struct bch_qwen35_layer {
  uint32_t is_attention;
  const float *attn_norm;   /* [n_embd] */
  const float *ffn_norm;    /* [n_embd] (post_attention_norm) */
  /* gated attention */
  bch_matrix wq;            /* 2·n_heads·head_dim × n_embd: per head its queries, then its gate */
  bch_matrix wk, wv;        /* n_kv_heads·head_dim × n_embd */
  bch_matrix wo;            /* n_embd × n_heads·head_dim */
  const float *q_norm;      /* [head_dim] */
  const float *k_norm;      /* [head_dim] */
  /* Gated DeltaNet */
  bch_matrix qkv;           /* conv_dim × n_embd: queries, keys, values */
  bch_matrix z;             /* value_dim × n_embd: the gate of the output norm */
  bch_matrix beta;          /* n_v_heads × n_embd */
  bch_matrix alpha;         /* n_v_heads × n_embd */
  const float *conv_taps;   /* [conv_dim][conv_kernel], the oldest first */
  const float *dt_bias;     /* [n_v_heads] */
  const float *a;           /* [n_v_heads], -exp(A_log) */
  const float *ssm_norm;    /* [v_head_dim] */
  bch_matrix out;           /* n_embd × value_dim */
  /* feed-forward */
  bch_matrix gate, up, down;
} bch_qwen35_layer;

/* qwen35::Hyperparameters (qwen35.rs:31-67) plus the tensors. */
typedef struct bch_qwen35_model {
  uint32_t n_layers;
  uint32_t n_embd;
  uint32_t n_ff;
  uint32_t n_vocab;
  uint32_t n_heads;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  uint32_t n_rot;           /* leading elements of a head that RoPE rotates */
  float rope_theta;
  float norm_eps;
  uint32_t conv_kernel;
  uint32_t n_k_heads;       /* DeltaNet query/key heads */
  uint32_t n_v_heads;       /* DeltaNet value heads, a multiple of n_k_heads */
  uint32_t k_head_dim;
  uint32_t v_head_dim;
  const bch_qwen35_layer *layers;
  bch_matrix token_embd;
  bch_matrix output;        /* tied: same data as token_embd */
  const float *output_norm;
} bch_qwen35_model;

typedef struct bch_qwen35 bch_qwen35;

/* Qwen35Metal::new: copies the weights to HBM and allocates the KV caches,
 * convolution histories and DeltaNet states for sequences of up to n_ctx
 * tokens.  Limits: attention as LFM2 plus an even n_rot <= head_dim;
 * DeltaNet 2..8 taps, key heads of 64 or 128 (DeltaNetLimits). */
int bch_qwen35_new(bch_ctx *ctx, const bch_qwen35_model *model, uint32_t n_ctx, int kv_half, bch_qwen35 **out);
void bch_qwen35_free(bch_qwen35 *qwen);
uint32_t bch_qwen35_n_past(const bch_qwen35 *qwen);
/* Qwen35Metal::reset: zero histories and states, n_past = 0. */
int bch_qwen35_reset(bch_qwen35 *qwen);
/* Qwen35Metal::step / prefill / greedy_token / generate, with the same
 * arguments and traces as the bch_lfm2_ functions. */
int bch_qwen35_step(bch_qwen35 *qwen, uint32_t token, float *logits, float *trace_embedding, float *trace_layers,
                    float *trace_final);
int bch_qwen35_prefill(bch_qwen35 *qwen, const uint32_t *tokens, uint32_t n_tokens, float *logits,
                       float *trace_embedding, float *trace_layers, float *trace_final);
/* Gpu::hidden (crates/bobcat-cli/src/backend.rs:150-160): start a new
 * sequence (reset) and prefill `tokens`, writing each token's normalised
 * last hidden state — the final RMSNorm's output, the input of the output
 * projection — to `hidden`, n_tokens rows of n_embd floats; no logits.  As
 * Qwen35Metal::prefill(tokens, None, Some(final_norm), None)
 * (qwen35_metal.rs:557-600), for the decision head. */
int bch_qwen35_hidden(bch_qwen35 *qwen, const uint32_t *tokens, uint32_t n_tokens, float *hidden);
int bch_qwen35_greedy_token(bch_qwen35 *qwen, uint32_t *token);
int bch_qwen35_generate(bch_qwen35 *qwen, uint32_t *out, uint32_t n);
/* Qwen35Metal's generate_next (same protocol as bch_lfm2_generate_next). */
int bch_qwen35_generate_next(bch_qwen35 *qwen, uint32_t *out, uint32_t n);
/* Qwen35Metal's generate_stream (qwen35_metal.rs, same protocol as
 * bch_lfm2_generate_stream). */
int bch_qwen35_generate_stream(bch_qwen35 *qwen, uint32_t max_tokens, bch_emit_fn emit, void *user,
                               uint32_t *gained, uint32_t *n_gained);
int bch_qwen35_generate_sampled(bch_qwen35 *qwen, uint32_t *out, uint32_t n, const bch_sampling *settings,
                                uint64_t seed);
/* Qwen35Metal::checkpoint / restore (qwen35::Checkpoint): resets, n_past,
 * the convolution histories, the DeltaNet states and the logits. */
uint64_t bch_qwen35_checkpoint_bytes(const bch_qwen35 *qwen);
int bch_qwen35_checkpoint(bch_qwen35 *qwen, void *blob, uint64_t bytes);
int bch_qwen35_restore(bch_qwen35 *qwen, const void *blob, uint64_t bytes);
double bch_qwen35_last_gpu_seconds(const bch_qwen35 *qwen);

/* ------------------------------------------------------------------ */
/* GGUF files (crates/bobcat-gguf/src/lib.rs) and model loading         */
/* ------------------------------------------------------------------ */

typedef struct bch_gguf bch_gguf;

/* One tensor of a GGUF file (bobcat_gguf::Tensor, lib.rs:265-296). */
typedef struct bch_gguf_tensor_info {
  const char *name;    /* valid while the file is open */
  uint32_t n_dims;
  uint64_t ne[4];      /* innermost first; 1 past n_dims */
  uint32_t type;       /* ggml type id = bch_format */
  const void *data;    /* the tensor's bytes in the file */
  uint64_t offset;     /* of the data from the file's start */
  uint64_t bytes;
} bch_gguf_tensor_info;

/* Gguf::parse (lib.rs:310-345): parse `size` bytes the caller keeps alive
 * until bch_gguf_free.  Every read is checked against the end and every size
 * against overflow; a malformed file fails with BCH_ERR_GGUF and the
 * reference's message (bch_last_error). */
int bch_gguf_parse(const void *bytes, uint64_t size, bch_gguf **out);
/* The same over a read-only mapping of the file at `path` (Storage::open). */
int bch_gguf_open(const char *path, bch_gguf **out);
void bch_gguf_free(bch_gguf *gguf);
/* Gguf::bytes (lib.rs:348-351). */
const void *bch_gguf_bytes(const bch_gguf *gguf, uint64_t *size);
/* Gguf::u32 / f32 / bool / string / array_len / array_u32 / string_array
 * (lib.rs:358-455): BCH_ERR_ARGUMENT when the key is absent or of another
 * type (u32: any integer that fits; f32: F32 or F64). */
int bch_gguf_u32(const bch_gguf *gguf, const char *key, uint32_t *out);
int bch_gguf_f32(const bch_gguf *gguf, const char *key, float *out);
int bch_gguf_bool(const bch_gguf *gguf, const char *key, int *out);
int bch_gguf_string(const bch_gguf *gguf, const char *key, const char **ptr, uint64_t *len);
int bch_gguf_array_len(const bch_gguf *gguf, const char *key, uint64_t *count);
int bch_gguf_array_u32(const bch_gguf *gguf, const char *key, uint64_t index, uint32_t *out);
int bch_gguf_array_string(const bch_gguf *gguf, const char *key, uint64_t index, const char **ptr, uint64_t *len);
/* Gguf::tensor / tensor_data (lib.rs:458-466), and the tensors in file order. */
int bch_gguf_tensor(const bch_gguf *gguf, const char *name, bch_gguf_tensor_info *out);
uint64_t bch_gguf_n_tensors(const bch_gguf *gguf);
int bch_gguf_tensor_at(const bch_gguf *gguf, uint64_t index, bch_gguf_tensor_info *out);

/* lfm2::Model::load (lfm2.rs:186-232, 737-1004) for "lfm2" and "lfm2moe"
 * files: fills `model` and layers[0..n_layers) (room for max_layers) with
 * the hyperparameters and pointers into the file, ready for bch_lfm2_new;
 * the file stays open while they are used.  Errors: BCH_ERR_MODEL. */
int bch_lfm2_model_from_gguf(const bch_gguf *gguf, bch_lfm2_model *model, bch_lfm2_layer *layers,
                             uint32_t max_layers);
/* qwen35::Model::load (qwen35.rs:186-230, 630-745) for "qwen35" files. */
int bch_qwen35_model_from_gguf(const bch_gguf *gguf, bch_qwen35_model *model, bch_qwen35_layer *layers,
                               uint32_t max_layers);

#ifdef __cplusplus
}
#endif
#endif
