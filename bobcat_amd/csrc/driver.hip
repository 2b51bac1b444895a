// The architecture-independent part of the model drivers (driver.h): weight
// upload, the shared buffers, and the sequence protocol of Lfm2Metal /
// Qwen35Metal (crates/bobcat/src/lfm2_metal.rs:237-779): reset, step,
// prefill in batches, greedy and sampled generation from replayed graphs,
// checkpoint and restore.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "driver.h"

namespace bch {

static uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

size_t Uploader::add(const void *p, uint64_t bytes) {
  for (size_t i = 0; i < items.size(); i++)
    if (items[i].first == p && items[i].second == bytes) return i;  // tied tensors share a copy
  items.push_back({p, bytes});
  offsets.push_back(total);
  total = align256(total + bytes);
  return items.size() - 1;
}

int Uploader::vec(const float *p, uint64_t count, const float **field, const char *name) {
  if (!p) return fail(BCH_ERR_ARGUMENT, "missing tensor %s", name);
  fixups.push_back({reinterpret_cast<const void **>(field), add(p, count * 4)});
  return BCH_OK;
}

int Uploader::mat(const bch_matrix &src, uint32_t rows, uint32_t cols, DevMatrix *dst, const char *name) {
  BCH_TRY(check_matrix(src, rows, cols, name));
  dst->format = src.format;
  dst->n_rows = rows;
  dst->n_cols = cols;
  fixups.push_back({reinterpret_cast<const void **>(&dst->data), add(src.data, bch_row_bytes(src.format, cols) * rows)});
  return BCH_OK;
}

bool gemv_format(uint32_t f) {
  return f == BCH_Q4K || f == BCH_F16 || f == BCH_F32 || f == BCH_Q5K || f == BCH_Q6K || f == BCH_Q8_0 || f == BCH_Q4_0;
}

int check_matrix(const bch_matrix &mat, uint32_t rows, uint32_t cols, const char *name) {
  if (!mat.data) return fail(BCH_ERR_ARGUMENT, "missing tensor %s", name);
  if (mat.n_rows != rows || mat.n_cols != cols)
    return fail(BCH_ERR_ARGUMENT, "tensor %s is %u x %u, expected %u x %u", name, mat.n_rows, mat.n_cols, rows, cols);
  if (!gemv_format(mat.format))
    return fail(BCH_ERR_UNSUPPORTED_FORMAT, "tensor %s: format %u is not supported (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F16 or F32)",
                name, mat.format);
  if ((mat.format == BCH_Q4K || mat.format == BCH_Q5K || mat.format == BCH_Q6K) && cols % 256)
    return fail(BCH_ERR_ARGUMENT, "tensor %s: columns not a multiple of 256", name);
  if ((mat.format == BCH_Q8_0 || mat.format == BCH_Q4_0) && cols % 64)
    return fail(BCH_ERR_ARGUMENT, "tensor %s: columns not a multiple of 64", name);
  return BCH_OK;
}

int check_hip(hipError_t e, const char *what) {
  if (e != hipSuccess) return fail(BCH_ERR_EXECUTION, "%s: %s", what, hipGetErrorString(e));
  return BCH_OK;
}

bool use_graphs() {
  static const bool on = !(getenv("BCH_LFM2_NO_GRAPH") && atoi(getenv("BCH_LFM2_NO_GRAPH")) != 0);
  return on;
}

uint32_t deferred_combine_below(uint32_t head_dim, bool kv_half) {
  static const bool off = getenv("BCH_NO_DEFER") && atoi(getenv("BCH_NO_DEFER")) != 0;
  return off ? 0u : kDeferSplits * attn_decode_keys_per_split(head_dim, kv_half);
}

Sequence::~Sequence() {
  // The context (and its stream) must still be open: free drivers first.
  if (s) hipStreamSynchronize(s);
  for (int i = 0; i < 2; i++) {
    if (step_graph[i]) hipGraphExecDestroy(step_graph[i]);
    if (gen_graph[i]) hipGraphExecDestroy(gen_graph[i]);
    if (sample_graph[i]) hipGraphExecDestroy(sample_graph[i]);
  }
  if (ev0) hipEventDestroy(ev0);
  if (ev1) hipEventDestroy(ev1);
  for (auto &e : stream_ev)
    if (e) hipEventDestroy(e);
  if (stream_host) hipHostFree(stream_host);
  for (void *p : allocations) hipFree(p);
}

int Sequence::alloc(uint64_t bytes, void **out) {
  void *p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 256) != hipSuccess)
    return fail(BCH_ERR_ALLOCATION, "cannot allocate %llu bytes", (unsigned long long)bytes);
  if (hipMemset(p, 0, bytes ? bytes : 256) != hipSuccess) return fail(BCH_ERR_ALLOCATION, "cannot clear memory");
  allocations.push_back(p);
  *out = p;
  return BCH_OK;
}

int Sequence::upload(Uploader &up) {
  void *w;
  BCH_TRY(alloc(up.total, &w));
  weights = static_cast<uint8_t *>(w);
  for (size_t i = 0; i < up.items.size(); i++)
    if (hipMemcpy(weights + up.offsets[i], up.items[i].first, up.items[i].second, hipMemcpyHostToDevice) != hipSuccess)
      return fail(BCH_ERR_ALLOCATION, "cannot copy the weights to the device");
  for (auto &f : up.fixups) *f.first = weights + up.offsets[f.second];
  // A copy from pageable host memory may return before its DMA has landed,
  // and the model's stream (non-blocking) does not wait for the null
  // stream: the first kernels to read the weights (the expansions, right
  // after this) must not start before the copies are done.
  return check_hip(hipDeviceSynchronize(), "weight upload");
}

static bool env_on(const char *name) {
  const char *e = getenv(name);
  return e && *e && *e != '0';
}

// The library path is on (BCH_NO_BLAS unset), the batch can exceed
// kBlasPairMinTokens, and the matrix (or pair) of `weights` weights in
// `format` is large enough or BCH_BLAS_PAIR=1 takes every size.
bool Sequence::blas_wanted(uint32_t format, uint64_t weights, uint64_t min_weights) const {
  return !env_on("BCH_NO_BLAS") && batch > kBlasPairMinTokens && expand_f16_supported(format, n_embd) &&
         (weights >= min_weights || env_on("BCH_BLAS_PAIR"));
}

int Sequence::expand_pair(const DevMatrix &gate, const DevMatrix &up, uint32_t n_ff, _Float16 **out) {
  *out = nullptr;
  // Smaller pairs run as fast on the Q4_K tile (Qwen3.5-0.8B, LFM2-350M at
  // 512 tokens).
  if (n_ff % 4 || gate.format != up.format || !blas_wanted(gate.format, 2ull * n_ff * n_embd, kBlasPairMinWeights))
    return BCH_OK;
  const uint64_t half = (uint64_t)n_ff * n_embd;
  BCH_TRY(alloc_t(2 * half, out));
  run_expand_f16(s, gate.format, gate.data, n_ff, n_embd, *out);
  run_expand_f16(s, up.format, up.data, n_ff, n_embd, *out + half);
  any_pair = true;
  return BCH_OK;
}

int Sequence::finish_pairs(uint32_t n_ff) {
  if (!any_pair) return BCH_OK;
  BCH_TRY(alloc_t((uint64_t)batch * 2 * n_ff, &pair_out));
  BCH_TRY(alloc_t((uint64_t)batch, &pair_us));
  BCH_TRY(blas_prepare());
  return check_hip(hipStreamSynchronize(s), "weight expansion");
}

int Sequence::alloc_common() {
  BCH_TRY(alloc_t(n_vocab, &logits));
  BCH_TRY(alloc_t((uint64_t)n_ctx + 2, &tokens));
  BCH_TRY(alloc_t(4, &dpos));
  BCH_TRY(alloc_t(4, &greedy));
  BCH_TRY(alloc_t(kArgmaxPartials, &argmax_partials));
  BCH_TRY(alloc_t(1, &rng));
  BCH_TRY(check_hip(hipEventCreate(&ev0), "create event"));
  return check_hip(hipEventCreate(&ev1), "create event");
}

int Sequence::busy_check() const {
  if (ctx->recording || ctx->committed > ctx->waited)
    return fail(BCH_ERR_BUSY, "the backend has recorded work in flight");
  return BCH_OK;
}

int Sequence::set_dpos(uint32_t value) {
  dpos_host = value;
  return check_hip(hipMemcpyAsync(dpos, &dpos_host, 4, hipMemcpyHostToDevice, s), "write position");
}

int Sequence::finish() {
  hipEventRecord(ev1, s);
  BCH_TRY(check_hip(hipEventSynchronize(ev1), "the GPU failed to run the work"));
  float ms = 0.f;
  hipEventElapsedTime(&ms, ev0, ev1);
  last_gpu_seconds = ms * 1e-3;
  return check_hip(hipGetLastError(), "launch");
}

// Grow the trace buffer to hold `rows` tokens per activation
// (Lfm2Metal::ensure_trace_rows, lfm2_metal.rs:764-779).
int Sequence::ensure_trace_rows(uint32_t rows) {
  if (rows <= trace_rows) return BCH_OK;
  if (trace) {
    hipStreamSynchronize(s);
    hipFree(trace);
    for (auto &p : allocations)
      if (p == trace) p = nullptr;
    trace = nullptr;
  }
  BCH_TRY(alloc_t((uint64_t)(n_layers + 2) * rows * n_embd, &trace));
  trace_rows = rows;
  return BCH_OK;
}

// Capture one decode step (preceded by the sampler when given) as a graph.
int Sequence::capture(bool greedy_input, const SampleArgs *sampler, bool short_ctx, hipGraphExec_t *out) {
  BCH_TRY(check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture"));
  if (sampler) run_sample(s, *sampler);
  record_step(s, greedy_input, false, short_ctx);
  hipGraph_t g;
  BCH_TRY(check_hip(hipStreamEndCapture(s, &g), "end capture"));
  hipError_t e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  return check_hip(e, "instantiate graph");
}

// One greedy decode step (the argmax of the previous step's logits as its
// token) at position pos, as a graph replay unless graphs are off.
int Sequence::launch_gen_step(uint32_t pos) {
  const bool sh = short_at(pos);
  if (!use_graphs()) {
    record_step(s, true, false, sh);
    return BCH_OK;
  }
  if (!gen_graph[sh]) BCH_TRY(capture(true, nullptr, sh, &gen_graph[sh]));
  return check_hip(hipGraphLaunch(gen_graph[sh], s), "launch decode graph");
}

int Sequence::reset() {
  BCH_TRY(busy_check());
  // A new sequence starts from zero recurrent state; the caches need no
  // clearing (lfm2_metal.rs:237-247).
  for (auto &r : state_regions())
    if (r.second) BCH_TRY(check_hip(hipMemsetAsync(r.first, 0, r.second, s), "clear state"));
  BCH_TRY(check_hip(hipStreamSynchronize(s), "reset"));
  n_past = 0;
  resets++;
  have_logits = false;
  return BCH_OK;
}

int Sequence::step(uint32_t token, float *out_logits, float *trace_embedding, float *trace_layers,
                   float *trace_final) {
  BCH_TRY(busy_check());
  if (n_past >= n_ctx) return fail(BCH_ERR_CONTEXT_FULL, "the context is full");
  if (token >= n_vocab) return fail(BCH_ERR_TOKEN, "token %u is outside the vocabulary of %u", token, n_vocab);
  const bool traced = trace_embedding || trace_layers || trace_final;
  if (traced) BCH_TRY(ensure_trace_rows(1));
  token_host = token;
  BCH_TRY(check_hip(hipMemcpyAsync(tokens + n_past, &token_host, 4, hipMemcpyHostToDevice, s), "write token"));
  BCH_TRY(set_dpos(n_past));
  hipEventRecord(ev0, s);
  const bool sh = short_at(n_past);
  if (traced) {
    record_step(s, false, true, sh);
  } else if (use_graphs()) {
    if (!step_graph[sh]) BCH_TRY(capture(false, nullptr, sh, &step_graph[sh]));
    BCH_TRY(check_hip(hipGraphLaunch(step_graph[sh], s), "launch step graph"));
  } else {
    record_step(s, false, false, sh);
  }
  BCH_TRY(finish());
  const uint32_t n = n_embd;
  const uint64_t tstride = (uint64_t)trace_rows * n;
  if (out_logits)
    BCH_TRY(check_hip(hipMemcpy(out_logits, logits, (uint64_t)n_vocab * 4, hipMemcpyDeviceToHost), "read logits"));
  if (trace_embedding)
    BCH_TRY(check_hip(hipMemcpy(trace_embedding, trace, (uint64_t)n * 4, hipMemcpyDeviceToHost), "read trace"));
  if (trace_layers)
    for (uint32_t il = 0; il < n_layers; il++)
      BCH_TRY(check_hip(hipMemcpy(trace_layers + (uint64_t)il * n, trace + (1 + il) * tstride, (uint64_t)n * 4,
                                  hipMemcpyDeviceToHost),
                        "read trace"));
  if (trace_final)
    BCH_TRY(check_hip(hipMemcpy(trace_final, trace + (1 + n_layers) * tstride, (uint64_t)n * 4, hipMemcpyDeviceToHost),
                      "read trace"));
  n_past++;
  have_logits = true;
  return BCH_OK;
}

int Sequence::prefill(const uint32_t *toks, uint32_t n_tokens, float *out_logits, float *trace_embedding,
                      float *trace_layers, float *trace_final) {
  BCH_TRY(busy_check());
  if (n_tokens == 0) return fail(BCH_ERR_ARGUMENT, "the prompt must hold a token");
  if (n_tokens > n_ctx - n_past)
    return fail(BCH_ERR_CONTEXT_FULL, "the prompt of %u tokens exceeds the %u free positions", n_tokens,
                n_ctx - n_past);
  for (uint32_t i = 0; i < n_tokens; i++)
    if (toks[i] >= n_vocab) return fail(BCH_ERR_TOKEN, "token %u is outside the vocabulary of %u", toks[i], n_vocab);
  BCH_TRY(check_hip(hipMemcpyAsync(tokens + n_past, toks, (uint64_t)n_tokens * 4, hipMemcpyHostToDevice, s),
                    "write tokens"));
  const bool traced = trace_embedding || trace_layers || trace_final;
  if (traced) BCH_TRY(ensure_trace_rows(batch));
  const uint32_t n = n_embd;
  const uint64_t tstride = (uint64_t)trace_rows * n;
  double gpu = 0.0;
  for (uint32_t done = 0; done < n_tokens; done += batch) {
    const uint32_t count = std::min(batch, n_tokens - done);
    const bool last = done + count == n_tokens;
    hipEventRecord(ev0, s);
    record_batch(s, n_past + done, count, last, traced);
    // A traced batch finishes before the next overwrites the trace rows, as
    // in the reference (lfm2_metal.rs:727-746); others run back to back.
    if (traced || last) {
      BCH_TRY(finish());
      gpu += last_gpu_seconds;
    }
    if (traced) {
      const uint64_t rows = (uint64_t)count * n * 4;
      if (trace_embedding)
        BCH_TRY(check_hip(hipMemcpy(trace_embedding + (uint64_t)done * n, trace, rows, hipMemcpyDeviceToHost),
                          "read trace"));
      if (trace_final)
        BCH_TRY(check_hip(hipMemcpy(trace_final + (uint64_t)done * n, trace + (1 + n_layers) * tstride, rows,
                                    hipMemcpyDeviceToHost),
                          "read trace"));
      if (trace_layers)
        for (uint32_t il = 0; il < n_layers; il++)
          BCH_TRY(check_hip(hipMemcpy(trace_layers + ((uint64_t)il * n_tokens + done) * n, trace + (1 + il) * tstride,
                                      rows, hipMemcpyDeviceToHost),
                            "read trace"));
    }
  }
  last_gpu_seconds = gpu;
  if (out_logits)
    BCH_TRY(check_hip(hipMemcpy(out_logits, logits, (uint64_t)n_vocab * 4, hipMemcpyDeviceToHost), "read logits"));
  n_past += n_tokens;
  have_logits = true;
  return BCH_OK;
}

int Sequence::greedy_token(uint32_t *token) {
  BCH_TRY(busy_check());
  if (n_past == 0 || !have_logits) return fail(BCH_ERR_ARGUMENT, "generation needs a prompt first");
  hipEventRecord(ev0, s);
  run_argmax(s, logits, greedy, n_vocab, nullptr, false);
  BCH_TRY(finish());
  return check_hip(hipMemcpy(token, greedy, 4, hipMemcpyDeviceToHost), "read token");
}

int Sequence::generate(uint32_t *out, uint32_t n) {
  BCH_TRY(busy_check());
  if (n_past == 0 || !have_logits) return fail(BCH_ERR_ARGUMENT, "generation needs a prompt first");
  if (n > n_ctx - n_past) return fail(BCH_ERR_CONTEXT_FULL, "%u tokens exceed the %u free positions", n, n_ctx - n_past);
  if (n == 0) return BCH_OK;
  // Each replay writes argmax(logits) into tokens[dpos + 1], advances dpos
  // and runs the step there; dpos starts at the last consumed position.  The
  // current logits (from a prefill, a step or a restore) are reduced to
  // argmax partials once; every step then leaves its own.
  BCH_TRY(set_dpos(n_past - 1));
  hipEventRecord(ev0, s);
  run_argmax_partials(s, logits, n_vocab, argmax_partials, kArgmaxPartials);
  // Replay i runs the step at position n_past + i.
  for (uint32_t i = 0; i < n; i++) BCH_TRY(launch_gen_step(n_past + i));
  BCH_TRY(finish());
  BCH_TRY(check_hip(hipMemcpy(out, tokens + n_past, (uint64_t)n * 4, hipMemcpyDeviceToHost), "read tokens"));
  n_past += n;
  return BCH_OK;
}

// Lfm2Metal::generate_next (lfm2_metal.rs:413-420): consume the current
// greedy selection and n - 1 more, returning the selection after each of the
// n steps; the last stays unconsumed (it is the next greedy_token).
int Sequence::generate_next(uint32_t *out, uint32_t n) {
  BCH_TRY(busy_check());
  if (n_past == 0 || !have_logits) return fail(BCH_ERR_ARGUMENT, "generation needs a prompt first");
  if (n > n_ctx - n_past) return fail(BCH_ERR_CONTEXT_FULL, "%u tokens exceed the %u free positions", n, n_ctx - n_past);
  if (n == 0) return BCH_OK;
  BCH_TRY(set_dpos(n_past - 1));
  hipEventRecord(ev0, s);
  run_argmax_partials(s, logits, n_vocab, argmax_partials, kArgmaxPartials);
  // Replay i runs the step at position n_past + i.
  for (uint32_t i = 0; i < n; i++) BCH_TRY(launch_gen_step(n_past + i));
  // The selection after the last step goes one past the consumed tokens
  // (the ring holds n_ctx + 2 entries).
  run_argmax_pick(s, argmax_partials, kArgmaxPartials, tokens + n_past + n);
  BCH_TRY(finish());
  BCH_TRY(check_hip(hipMemcpy(out, tokens + n_past + 1, (uint64_t)n * 4, hipMemcpyDeviceToHost), "read tokens"));
  n_past += n;
  return BCH_OK;
}

int Sequence::generate_sampled(uint32_t *out, uint32_t n, const bch_sampling *settings, uint64_t seed) {
  BCH_TRY(busy_check());
  if (!settings) return fail(BCH_ERR_ARGUMENT, "no sampling settings");
  if (n_past == 0 || !have_logits) return fail(BCH_ERR_ARGUMENT, "generation needs a prompt first");
  if (n > n_ctx - n_past) return fail(BCH_ERR_CONTEXT_FULL, "%u tokens exceed the %u free positions", n, n_ctx - n_past);
  if (n == 0) return BCH_OK;
  // Each replay samples the current logits into tokens[dpos + 1], advances
  // dpos and runs the step there; the settings are captured into the graph.
  BCH_TRY(set_dpos(n_past - 1));
  rng_host = seed;
  BCH_TRY(check_hip(hipMemcpyAsync(rng, &rng_host, 8, hipMemcpyHostToDevice, s), "seed the sampler"));
  SampleArgs sa{};
  sa.logits = logits;
  sa.n = n_vocab;
  sa.recent = tokens;
  sa.dpos = dpos;
  sa.out = tokens;
  sa.rng = rng;
  sa.temperature = settings->temperature;
  sa.top_p = settings->top_p;
  sa.min_p = settings->min_p;
  sa.penalty = settings->repeat_penalty;
  sa.top_k = settings->top_k;
  hipEventRecord(ev0, s);
  if (use_graphs()) {
    // Replay i runs the step at position n_past + i.
    for (uint32_t i = 0; i < n; i++) {
      const bool sh = short_at(n_past + i);
      if (sample_graph[sh] && memcmp(&sample_settings[sh], settings, sizeof(bch_sampling)) != 0) {
        hipGraphExecDestroy(sample_graph[sh]);
        sample_graph[sh] = nullptr;
      }
      if (!sample_graph[sh]) {
        BCH_TRY(capture(false, &sa, sh, &sample_graph[sh]));
        sample_settings[sh] = *settings;
      }
      BCH_TRY(check_hip(hipGraphLaunch(sample_graph[sh], s), "launch sampling graph"));
    }
  } else {
    for (uint32_t i = 0; i < n; i++) {
      run_sample(s, sa);
      record_step(s, false, false, short_at(n_past + i));
    }
  }
  BCH_TRY(finish());
  BCH_TRY(check_hip(hipMemcpy(out, tokens + n_past, (uint64_t)n * 4, hipMemcpyDeviceToHost), "read tokens"));
  n_past += n;
  return BCH_OK;
}

// Lfm2Metal::generate_stream (lfm2_metal.rs:425-560).  The first token is
// the argmax of the current logits and needs no step; each step then runs
// the token at the next position (the decode graph reduces the previous
// logits' argmax keys into it) and a small kernel picks the token it
// selects into a slot that is copied to pinned host memory.  Up to
// kStreamInFlight steps are queued ahead of the host, so the GPU does not
// wait for `emit`; once emit returns 0 no further step is queued, but the
// queued ones still run.  `gained` (room for max_tokens) receives the tokens
// the sequence consumed, n_gained of them: every emitted token but the last,
// possibly followed by tokens selected after the last emitted one.
int Sequence::generate_stream(uint32_t max_tokens, bch_emit_fn emit, void *user, uint32_t *gained,
                              uint32_t *n_gained) {
  BCH_TRY(busy_check());
  if (!emit || !n_gained) return fail(BCH_ERR_ARGUMENT, "generate_stream needs an emit callback and n_gained");
  *n_gained = 0;
  if (max_tokens == 0) return BCH_OK;
  if (!gained) return fail(BCH_ERR_ARGUMENT, "generate_stream needs room for the gained tokens");
  uint32_t first;
  BCH_TRY(greedy_token(&first));
  if (!emit(first, user)) return BCH_OK;
  const uint32_t steps = std::min(max_tokens - 1, n_ctx - n_past);
  if (steps == 0) return BCH_OK;
  if (!stream_dev) {
    BCH_TRY(alloc_t(kStreamInFlight, &stream_dev));
    BCH_TRY(check_hip(hipHostMalloc(reinterpret_cast<void **>(&stream_host), kStreamInFlight * 4, hipHostMallocDefault),
                      "allocate pinned slots"));
    for (auto &e : stream_ev) BCH_TRY(check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "create event"));
  }
  const uint32_t start = n_past;
  BCH_TRY(set_dpos(n_past - 1));
  hipEventRecord(ev0, s);
  run_argmax_partials(s, logits, n_vocab, argmax_partials, kArgmaxPartials);
  bool pending[kStreamInFlight] = {};
  bool emitting = true;
  uint32_t committed = 0;
  int rc = BCH_OK;
  auto drain = [&](int slot) -> int {
    pending[slot] = false;
    BCH_TRY(check_hip(hipEventSynchronize(stream_ev[slot]), "the GPU failed to run a decode step"));
    if (emitting) emitting = emit(stream_host[slot], user) != 0;
    return BCH_OK;
  };
  for (uint32_t step = 0; step < steps; step++) {
    const int slot = (int)(step % kStreamInFlight);
    if (pending[slot] && (rc = drain(slot)) != BCH_OK) break;
    if (!emitting) break;
    if ((rc = launch_gen_step(start + step)) != BCH_OK) break;
    run_argmax_pick(s, argmax_partials, kArgmaxPartials, stream_dev + slot);
    if ((rc = check_hip(hipMemcpyAsync(stream_host + slot, stream_dev + slot, 4, hipMemcpyDeviceToHost, s),
                        "read a selected token")) != BCH_OK)
      break;
    hipEventRecord(stream_ev[slot], s);
    pending[slot] = true;
    committed++;
  }
  // The steps still in flight finish in submission order, their tokens' order.
  for (int k = 0; k < kStreamInFlight; k++) {
    const int slot = (int)((committed + k) % kStreamInFlight);
    if (pending[slot]) {
      const int r = drain(slot);
      if (rc == BCH_OK) rc = r;
    }
  }
  hipEventRecord(ev1, s);
  hipEventSynchronize(ev1);
  float ms = 0.f;
  hipEventElapsedTime(&ms, ev0, ev1);
  last_gpu_seconds = ms * 1e-3;
  n_past += committed;
  BCH_TRY(rc);
  BCH_TRY(check_hip(hipGetLastError(), "launch"));
  BCH_TRY(check_hip(hipMemcpy(gained, tokens + start, (uint64_t)committed * 4, hipMemcpyDeviceToHost), "read tokens"));
  *n_gained = committed;
  return BCH_OK;
}

// Checkpoint blob: resets (u64), n_past (u32), have_logits (u32), the state
// regions in order, the logits (lfm2_metal.rs:86-97 keeps resets and n_past).
uint64_t Sequence::checkpoint_bytes() const {
  uint64_t b = 16 + (uint64_t)n_vocab * 4;
  for (auto &r : state_regions()) b += r.second;
  return b;
}

int Sequence::checkpoint(void *blob, uint64_t bytes) {
  BCH_TRY(busy_check());
  if (bytes != checkpoint_bytes()) return fail(BCH_ERR_ARGUMENT, "checkpoint buffer of the wrong size");
  char *p = static_cast<char *>(blob);
  memcpy(p, &resets, 8);
  memcpy(p + 8, &n_past, 4);
  const uint32_t have = have_logits;
  memcpy(p + 12, &have, 4);
  p += 16;
  for (auto &r : state_regions()) {
    BCH_TRY(check_hip(hipMemcpy(p, r.first, r.second, hipMemcpyDeviceToHost), "read state"));
    p += r.second;
  }
  return check_hip(hipMemcpy(p, logits, (uint64_t)n_vocab * 4, hipMemcpyDeviceToHost), "read logits");
}

int Sequence::restore(const void *blob, uint64_t bytes) {
  BCH_TRY(busy_check());
  if (bytes != checkpoint_bytes()) return fail(BCH_ERR_ARGUMENT, "the checkpoint comes from a different model or context");
  const char *p = static_cast<const char *>(blob);
  uint64_t saved_resets;
  uint32_t saved_past, have;
  memcpy(&saved_resets, p, 8);
  memcpy(&saved_past, p + 8, 4);
  memcpy(&have, p + 12, 4);
  if (saved_resets != resets) return fail(BCH_ERR_ARGUMENT, "the checkpoint predates a reset");
  if (saved_past > n_ctx) return fail(BCH_ERR_ARGUMENT, "the checkpoint comes from a different model or context");
  p += 16;
  for (auto &r : state_regions()) {
    BCH_TRY(check_hip(hipMemcpy(r.first, p, r.second, hipMemcpyHostToDevice), "write state"));
    p += r.second;
  }
  BCH_TRY(check_hip(hipMemcpy(logits, p, (uint64_t)n_vocab * 4, hipMemcpyHostToDevice), "write logits"));
  n_past = saved_past;
  have_logits = have != 0;
  return BCH_OK;
}

}  // namespace bch
