// The part of the model drivers that does not depend on the architecture: a
// sequence on the GPU (Lfm2Metal / Qwen35Metal share the same protocol,
// crates/bobcat/src/lfm2_metal.rs:125-779, qwen35_metal.rs).
//
// A Sequence owns one HBM allocation of weights, the token ring and the
// device position counter that every decode kernel reads (so a decode step
// is captured once as a HIP graph and replayed), the logits with their
// argmax keys, the sampler state and the trace buffer.  The model supplies
// the launches of one decode step and of one prefill batch, and the device
// regions of its recurrent state (convolution histories, DeltaNet states)
// that reset clears and checkpoints carry.
#pragma once
#include <cstdint>
#include <utility>
#include <vector>

#include "kernels.h"
#include "runtime.h"

namespace bch {

constexpr uint32_t kPrefillBatch = 512;  // PREFILL_BATCH (lfm2_metal.rs:33-34)

struct DevMatrix {
  uint32_t format = 0, n_rows = 0, n_cols = 0;
  const uint8_t *data = nullptr;
};

// Host tensors -> one device allocation.  add() plans a copy (tied tensors
// share one); the owner fixes up device pointers once the copy is made.
struct Uploader {
  std::vector<std::pair<const void *, uint64_t>> items;  // host pointer, bytes
  std::vector<uint64_t> offsets;
  std::vector<std::pair<const void **, size_t>> fixups;  // device pointer field -> item
  uint64_t total = 0;
  size_t add(const void *p, uint64_t bytes);
  int vec(const float *p, uint64_t count, const float **field, const char *name);
  int mat(const bch_matrix &src, uint32_t rows, uint32_t cols, DevMatrix *dst, const char *name);
};

bool gemv_format(uint32_t f);
int check_matrix(const bch_matrix &mat, uint32_t rows, uint32_t cols, const char *name);
int check_hip(hipError_t e, const char *what);

// Decode steps replay a captured HIP graph unless BCH_LFM2_NO_GRAPH=1, which
// issues the same launches on the stream one by one (for tools that do not
// follow graph launches, such as per-kernel tracing).
bool use_graphs();
// Positions below which decode attention leaves its splits' combine to the
// out projection (kDeferSplits splits of the head size's split length);
// BCH_NO_DEFER=1 makes it 0 (never), for measuring the two forms.
uint32_t deferred_combine_below(uint32_t head_dim, bool kv_half);

struct Sequence {
  virtual ~Sequence();

  bch_ctx *ctx = nullptr;
  hipStream_t s = nullptr;
  uint32_t n_layers = 0, n_embd = 0, n_vocab = 0;
  uint32_t n_ctx = 0, n_past = 0, batch = 0;
  uint64_t resets = 0;
  bool have_logits = false;
  // Device memory.
  std::vector<void *> allocations;
  uint8_t *weights = nullptr;
  float *logits = nullptr, *trace = nullptr;
  uint32_t trace_rows = 0;  // tokens each traced activation holds (lfm2_metal.rs:764-779)
  uint32_t *tokens = nullptr, *dpos = nullptr, *greedy = nullptr;
  uint64_t *argmax_partials = nullptr;  // kArgmaxPartials argmax keys of the logits
  uint64_t *rng = nullptr;              // sampler state
  // Graphs and timing.
  // Each in two forms: [1] for steps at positions below short_below (the
  // model's short-context form), [0] for the others.
  hipGraphExec_t step_graph[2] = {}, gen_graph[2] = {}, sample_graph[2] = {};
  bch_sampling sample_settings[2] = {};  // the settings sample_graph[i] was captured with
  uint32_t short_below = 0;  // set by the model: steps below it take its short-context form
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double last_gpu_seconds = 0.0;
  // Host staging of the small asynchronous uploads (they must outlive the call).
  uint32_t dpos_host = 0, token_host = 0;
  uint64_t rng_host = 0;
  // generate_stream: the token each in-flight step selected, per slot, on
  // the device and in pinned host memory, with the event of its copy.
  static constexpr int kStreamInFlight = 3;  // GENERATE_IN_FLIGHT (lfm2_metal.rs:36)
  uint32_t *stream_dev = nullptr, *stream_host = nullptr;
  hipEvent_t stream_ev[kStreamInFlight] = {};

  // --- the model's part ------------------------------------------------
  // One decode step at position *dpos.  With greedy_input the step first
  // takes the argmax of the previous logits (from argmax_partials) as its
  // token; it leaves logits and their argmax partials for the next one.
  // With trace, it copies the activations into `trace`.  short_ctx: the
  // step runs at a position below short_below.
  virtual void record_step(hipStream_t st, bool greedy_input, bool trace, bool short_ctx) = 0;
  // A prefill batch of `count` tokens at positions pos.. (tokens already in
  // the ring); the logits of its last token when want_logits.
  virtual void record_batch(hipStream_t st, uint32_t pos, uint32_t count, bool want_logits, bool trace) = 0;
  // Device regions of the recurrent state, which reset() zeroes and
  // checkpoints save (the caches need neither: positions are rewritten).
  virtual std::vector<std::pair<void *, uint64_t>> state_regions() const = 0;

  // --- shared ------------------------------------------------------------
  int alloc(uint64_t bytes, void **out);
  template <class T>
  int alloc_t(uint64_t count, T **out) {
    void *p;
    BCH_TRY(alloc(count * sizeof(T), &p));
    *out = static_cast<T *>(p);
    return BCH_OK;
  }
  // Copy the planned weights to HBM and fix up the device pointers.
  int upload(Uploader &up);
  // The buffers every sequence has; called by the model's constructor.
  int alloc_common();
  // The library SwiGLU pair of prefill batches (run_blas_pair): when it is
  // enabled for this model (BCH_NO_BLAS unset, batches larger than
  // kBlasPairMinTokens, at least kBlasPairMinWeights in the pair or
  // BCH_BLAS_PAIR=1, n_ff a multiple of 4) and the format expands,
  // *out receives the fp16 [gate rows; up rows] copy, else nullptr.
  int expand_pair(const DevMatrix &gate, const DevMatrix &up, uint32_t n_ff, _Float16 **out);
  // After the expansions: the pair's product and scale buffers (when any
  // layer expanded), the library handle, and the expansions finished.
  int finish_pairs(uint32_t n_ff);
  bool blas_wanted(uint32_t format, uint64_t weights, uint64_t min_weights) const;
  float *pair_out = nullptr, *pair_us = nullptr;  // pair product; a copy of the batch's token scales
  bool any_pair = false;

  int reset();
  int step(uint32_t token, float *logits, float *trace_embedding, float *trace_layers, float *trace_final);
  int prefill(const uint32_t *toks, uint32_t n, float *logits, float *trace_embedding, float *trace_layers,
              float *trace_final);
  int greedy_token(uint32_t *token);
  int generate(uint32_t *out, uint32_t n);
  int generate_sampled(uint32_t *out, uint32_t n, const bch_sampling *settings, uint64_t seed);
  int generate_next(uint32_t *out, uint32_t n);
  int generate_stream(uint32_t max_tokens, bch_emit_fn emit, void *user, uint32_t *gained, uint32_t *n_gained);
  uint64_t checkpoint_bytes() const;
  int checkpoint(void *blob, uint64_t bytes);
  int restore(const void *blob, uint64_t bytes);

 protected:
  int busy_check() const;
  int set_dpos(uint32_t value);
  int finish();
  int ensure_trace_rows(uint32_t rows);
  int capture(bool greedy_input, const SampleArgs *sampler, bool short_ctx, hipGraphExec_t *out);
  // Whether the step at position pos takes the short-context form.
  bool short_at(uint32_t pos) const { return pos < short_below; }
  int launch_gen_step(uint32_t pos);
};

}  // namespace bch
