"""GPU parity of the LFM2 driver (bch_lfm2_*) against the oracle's forward pass.

Mirrors crates/bobcat/tests/lfm2_reference.rs with the oracle standing in for
the transformers dumps (the oracle itself is pinned to transformers in
tests/test_oracle_lfm2.py):
  * every layer's output, the final norm and the logits of each step within
    1e-4 with an f32 KV cache and 5e-3 with an f16 cache (:17-25);
  * greedy decoding reproduces the oracle's tokens (allowing a flip only where
    the oracle's top-2 logits differ by less than 1e-3, the north-star rule);
  * prefill == steps (:117-151), reset == fresh (:155-185), checkpoint and
    restore (:190-238), generate == repeated greedy steps (:243-350);
  * the error paths of Lfm2Metal (context full, token outside the vocabulary,
    generation without a prompt).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd import BobcatError
from bobcat_amd.lfm2 import (LFM2_TINY, LFM2_TINY_F16, LFM2_TINY_MIXED, LFM2_TINY_MOE, LFM2_TINY_WIDE, Lfm2Hip,
                              Lfm2Weights)

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-4
HALF_TOLERANCE = 5e-3


def set_grouped(monkeypatch, grouped):
    """Decode attention with every query head of a KV group in one workgroup
    (the long-context layout) from the first split on, instead of only when
    the one-head grid would exceed a round of workgroups."""
    if grouped:
        monkeypatch.setenv("BCH_ATTN_GROUPED_ABOVE", "0")


def rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    d = np.abs(got - want)
    if np.isnan(d).any():
        return float("inf")
    return float(d.max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module", params=[LFM2_TINY, LFM2_TINY_F16, LFM2_TINY_MOE, LFM2_TINY_MIXED], ids=lambda c: c.name)
def weights(request):
    return Lfm2Weights(request.param, seed=7)


def prompt(cfg, n, seed=1):
    return np.random.default_rng(seed).integers(0, cfg.n_vocab, n).tolist()


@pytest.mark.parametrize("grouped", [False, True], ids=["head_per_wg", "grouped"])
@pytest.mark.parametrize("kv_half", [False, True])
def test_steps_match_oracle_layer_by_layer(hip, weights, kv_half, grouped, monkeypatch):
    set_grouped(monkeypatch, grouped)
    cfg = weights.cfg
    tol = HALF_TOLERANCE if kv_half else TOLERANCE
    gpu = Lfm2Hip(hip, weights, n_ctx=48, kv_half=kv_half)
    cpu = oracle.Lfm2State(weights, n_ctx=48)
    worst = np.zeros(cfg.n_layers + 3)
    for tok in prompt(cfg, 20):
        lg, (emb, layers, final) = gpu.step(tok, trace=True)
        wl, (wemb, wlayers, wfinal) = cpu.step(tok, trace=True)
        errs = [rel(emb, wemb)]
        errs += [rel(layers[i * cfg.n_embd:(i + 1) * cfg.n_embd], wlayers[i * cfg.n_embd:(i + 1) * cfg.n_embd])
                 for i in range(cfg.n_layers)]
        errs += [rel(final, wfinal), rel(lg, wl)]
        worst = np.maximum(worst, errs)
    assert worst.max() < tol, worst
    gpu.close()


@pytest.mark.parametrize("kv_half", [False, True])
def test_prefill_trace_matches_oracle(hip, weights, kv_half):
    """The batched pass traced for every token (lfm2_reference.rs:581-640 with
    batched = true): the prefill GEMM's half-precision weights and inputs
    bound it by 5e-3."""
    cfg = weights.cfg
    toks = prompt(cfg, 20, seed=11)
    gpu = Lfm2Hip(hip, weights, n_ctx=48, kv_half=kv_half)
    lg, (emb, layers, final) = gpu.prefill(toks, trace=True)
    cpu = oracle.Lfm2State(weights, n_ctx=48)
    worst = np.zeros(cfg.n_layers + 3)
    for t, tok in enumerate(toks):
        wl, (wemb, wlayers, wfinal) = cpu.step(tok, trace=True)
        errs = [rel(emb[t], wemb)]
        errs += [rel(layers[i, t], wlayers[i * cfg.n_embd:(i + 1) * cfg.n_embd]) for i in range(cfg.n_layers)]
        errs += [rel(final[t], wfinal), rel(lg, wl) if t + 1 == len(toks) else 0.0]
        worst = np.maximum(worst, errs)
    print(cfg.name, kv_half, "worst per layer", np.array2string(worst, formatter={'float_kind': lambda v: f'{v:.1e}'}))
    # The prefill GEMM equals the product of half-rounded weights and
    # half-rounded inputs to 1e-5 (test_gpu_ops.py::test_matmul_other_formats).
    # The mixed-format model's random Q8_0/Q6_K layers amplify that rounding
    # (its layer outputs drift by up to ~3e-2 while its logits stay within
    # 1e-3), so its bound is 5e-2; the other models stay within the 5e-3 of
    # lfm2_reference.rs:21-25.
    bound = 5e-2 if cfg.tensor_formats else HALF_TOLERANCE
    assert worst[-1] < HALF_TOLERANCE, worst
    assert worst.max() < bound, worst
    gpu.close()


def test_prefill_library_pair_matches_oracle(hip, monkeypatch):
    """A prefill batch of more than 128 tokens with the SwiGLU pair on the
    library GEMM over the expanded fp16 weights (forced for this small
    model with BCH_BLAS_PAIR=1; by default only pairs of 2^24 weights or
    more take it), its SwiGLU writing the down projection's fp16 inputs:
    every layer of every token against the oracle within the prefill bound,
    and against the same prompt on the fused Q4_K tile (BCH_NO_BLAS=1),
    which sums the same fp16 products in another order."""
    w = Lfm2Weights(LFM2_TINY, seed=21)
    cfg = w.cfg
    toks = prompt(cfg, 160, seed=22)
    monkeypatch.setenv("BCH_BLAS_PAIR", "1")
    gpu = Lfm2Hip(hip, w, n_ctx=192, kv_half=False)
    lg, (emb, layers, final) = gpu.prefill(toks, trace=True)
    nxt = gpu.step(7)
    gpu.close()
    monkeypatch.setenv("BCH_NO_BLAS", "1")
    tile = Lfm2Hip(hip, w, n_ctx=192, kv_half=False)
    lg_tile = tile.prefill(toks)
    nxt_tile = tile.step(7)
    tile.close()
    assert rel(lg, lg_tile) < 1e-4 and rel(nxt, nxt_tile) < 1e-4, (rel(lg, lg_tile), rel(nxt, nxt_tile))
    cpu = oracle.Lfm2State(w, n_ctx=192)
    worst = 0.0
    for t, tok in enumerate(toks):
        wl, (wemb, wlayers, wfinal) = cpu.step(tok, trace=True)
        for i in range(cfg.n_layers):
            worst = max(worst, rel(layers[i, t], wlayers[i * cfg.n_embd:(i + 1) * cfg.n_embd]))
    assert worst < HALF_TOLERANCE, worst
    assert rel(lg, wl) < HALF_TOLERANCE
    assert rel(nxt, cpu.step(7)) < HALF_TOLERANCE


def greedy_oracle(weights, tokens, n_gen, n_ctx):
    """Oracle greedy continuation and, per step, the gap between its top-2 logits."""
    cpu = oracle.Lfm2State(weights, n_ctx=n_ctx)
    for t in tokens:
        lg = cpu.step(t)
    out, gaps = [], []
    for _ in range(n_gen):
        top = np.argsort(lg)[-2:]
        gaps.append(float(lg[top[1]] - lg[top[0]]))
        nxt = int(np.argmax(lg))
        out.append(nxt)
        lg = cpu.step(nxt)
    return out, gaps


def assert_greedy_matches(got, want, gaps):
    for i, (g, w) in enumerate(zip(got, want)):
        if g != w:
            assert gaps[i] < 1e-3, f"token {i}: {g} vs oracle {w} (top-2 gap {gaps[i]:.3g})"
            return  # the sequences legitimately diverge after a near-tie


def test_greedy_generation_matches_oracle(hip, weights):
    cfg = weights.cfg
    toks = prompt(cfg, 16, seed=2)
    want, gaps = greedy_oracle(weights, toks, 24, n_ctx=64)
    gpu = Lfm2Hip(hip, weights, n_ctx=64, kv_half=False)
    gpu.prefill(toks)
    got = gpu.generate(24)
    assert_greedy_matches(got.tolist(), want, gaps)
    assert gpu.n_past == 16 + 24
    gpu.close()


def test_prefill_matches_steps(hip, weights):
    """lfm2_reference.rs:117-151: one prefill of the prompt equals one step per token."""
    cfg = weights.cfg
    toks = prompt(cfg, 70, seed=3)  # spans two attention query batches
    a = Lfm2Hip(hip, weights, n_ctx=96)
    b = Lfm2Hip(hip, weights, n_ctx=96)
    la = a.prefill(toks)
    for t in toks:
        lb = b.step(t)
    assert rel(la, lb) < HALF_TOLERANCE
    # Continuations agree too.
    assert rel(a.step(5), b.step(5)) < HALF_TOLERANCE
    a.close()
    b.close()


def test_prefill_in_batches_matches_one_batch(hip):
    """A prompt longer than the 512-token prefill batch runs in two batches."""
    w = Lfm2Weights(LFM2_TINY, seed=9)
    toks = prompt(LFM2_TINY, 600, seed=4)
    a = Lfm2Hip(hip, w, n_ctx=700)
    la = a.prefill(toks)
    b = Lfm2Hip(hip, w, n_ctx=700)
    b.prefill(toks[:300])
    lb = b.prefill(toks[300:])
    assert rel(la, lb) < HALF_TOLERANCE
    a.close()
    b.close()


@pytest.mark.parametrize("grouped", [False, True], ids=["head_per_wg", "grouped"])
@pytest.mark.parametrize("kv_half", [False, True])
def test_decode_across_attention_splits(hip, kv_half, grouped, monkeypatch):
    """Decode steps at positions 1020-1027 cross the split boundary at 1024
    (a split holds 128 f32 or 256 f16 positions of a 64-wide head), so the
    number of splits, and with it the cross-workgroup combine, changes
    between steps (8 to 9 f32 splits, 4 to 5 f16)."""
    set_grouped(monkeypatch, grouped)
    w = Lfm2Weights(LFM2_TINY, seed=11)
    toks = prompt(LFM2_TINY, 1028, seed=6)
    gpu = Lfm2Hip(hip, w, n_ctx=1100, kv_half=kv_half)
    cpu = oracle.Lfm2State(w, n_ctx=1100)
    gpu.prefill(toks[:1020], logits=False)
    for t in toks[:1020]:
        cpu.step(t)
    tol = HALF_TOLERANCE if kv_half else TOLERANCE
    for t in toks[1020:]:
        got, want = gpu.step(t), cpu.step(t)
        assert rel(got, want) < tol, (t, rel(got, want))
    gpu.close()


@pytest.mark.parametrize("kv_half", [False, True])
def test_decode_across_deferred_combine(hip, kv_half):
    """A 1,024-wide attention output: decode steps with at most four
    attention splits (f16: positions below 1,024) leave the splits' combine
    to the out projection's input staging, later ones combine in the
    attention launch.  Steps at 1018-1029 cross from one form to the other
    (f32 splits hold 128 positions, so the f32 cache crosses at 512 and stays
    past it), each against the oracle; then generate() across the boundary
    (one replay per position, the graph chosen per position) against the
    oracle's greedy continuation."""
    w = Lfm2Weights(LFM2_TINY_WIDE, seed=13)
    toks = prompt(LFM2_TINY_WIDE, 1030, seed=10)
    gpu = Lfm2Hip(hip, w, n_ctx=1100, kv_half=kv_half)
    cpu = oracle.Lfm2State(w, n_ctx=1100)
    gpu.prefill(toks[:1018], logits=False)
    for t in toks[:1018]:
        cpu.step(t)
    tol = HALF_TOLERANCE if kv_half else TOLERANCE
    for t in toks[1018:]:
        got, want = gpu.step(t), cpu.step(t)
        assert rel(got, want) < tol, (t, rel(got, want))
    gpu.close()
    start = toks[:1016]
    want, gaps = greedy_oracle(w, start, 16, n_ctx=1100)
    gpu = Lfm2Hip(hip, w, n_ctx=1100, kv_half=kv_half)
    gpu.prefill(start)
    assert_greedy_matches(gpu.generate(16).tolist(), want, gaps)
    gpu.close()


@pytest.mark.parametrize("grouped", [False, True], ids=["head_per_wg", "grouped"])
@pytest.mark.parametrize("kv_half", [False, True])
def test_long_context_decode(hip, kv_half, grouped, monkeypatch):
    """A driver sized for a long context (n_ctx 8192: 64 splits of 128 f32 or
    32 of 256 f16 positions, four query heads per KV head) launches a grid of
    that many splits; steps at positions
    1020-1027 run with 4 to 9 live splits and the parallel split combine,
    against the oracle, and against a driver sized for 1100."""
    set_grouped(monkeypatch, grouped)
    w = Lfm2Weights(LFM2_TINY_F16, seed=12)
    toks = prompt(LFM2_TINY_F16, 1028, seed=9)
    big = Lfm2Hip(hip, w, n_ctx=8192, kv_half=kv_half)
    small = Lfm2Hip(hip, w, n_ctx=1100, kv_half=kv_half)
    cpu = oracle.Lfm2State(w, n_ctx=1100)
    big.prefill(toks[:1020], logits=False)
    small.prefill(toks[:1020], logits=False)
    for t in toks[:1020]:
        cpu.step(t, logits=False)
    tol = HALF_TOLERANCE if kv_half else TOLERANCE
    for t in toks[1020:]:
        got, per_head, want = big.step(t), small.step(t), cpu.step(t)
        assert rel(got, want) < tol, (t, rel(got, want))
        assert rel(got, per_head) < 1e-5, (t, rel(got, per_head))
    big.close()
    small.close()


def test_long_context_prefill_key_splits(hip):
    """A 40-token prefill after 2,900 cached positions (f16 cache, n_ctx 8192)
    splits the keys of the MFMA prefill attention over several workgroups,
    each split's partials combined afterwards; its logits and the next steps
    against the oracle."""
    w = Lfm2Weights(LFM2_TINY_F16, seed=14)
    toks = prompt(LFM2_TINY_F16, 2944, seed=15)
    gpu = Lfm2Hip(hip, w, n_ctx=8192, kv_half=True)
    cpu = oracle.Lfm2State(w, n_ctx=3000)
    gpu.prefill(toks[:2900], logits=False)
    for t in toks[:2939]:
        cpu.step(t, logits=False)
    got, want = gpu.prefill(toks[2900:2940]), cpu.step(toks[2939])
    assert rel(got, want) < HALF_TOLERANCE, rel(got, want)
    for t in toks[2940:]:
        got, want = gpu.step(t), cpu.step(t)
        assert rel(got, want) < HALF_TOLERANCE, (t, rel(got, want))
    gpu.close()


def test_reset_matches_fresh_state(hip, weights):
    cfg = weights.cfg
    toks = prompt(cfg, 10, seed=5)
    a = Lfm2Hip(hip, weights, n_ctx=32)
    a.prefill(prompt(cfg, 7, seed=6))
    a.generate(3)
    a.reset()
    assert a.n_past == 0
    la = a.prefill(toks)
    b = Lfm2Hip(hip, weights, n_ctx=32)
    lb = b.prefill(toks)
    assert rel(la, lb) < TOLERANCE
    a.close()
    b.close()


def test_checkpoint_restore_continues(hip, weights):
    cfg = weights.cfg
    a = Lfm2Hip(hip, weights, n_ctx=64)
    a.prefill(prompt(cfg, 12, seed=7))
    ck = a.checkpoint()
    first = a.generate(8)
    a.restore(ck)
    assert a.n_past == 12
    again = a.generate(8)
    assert np.array_equal(first, again)
    a.reset()
    with pytest.raises(BobcatError):
        a.restore(ck)  # predates the reset
    a.close()


def test_generate_matches_greedy_steps(hip, weights):
    """generate() on the GPU graph equals greedy_token() + step() on the host."""
    cfg = weights.cfg
    toks = prompt(cfg, 9, seed=8)
    a = Lfm2Hip(hip, weights, n_ctx=64)
    b = Lfm2Hip(hip, weights, n_ctx=64)
    a.prefill(toks)
    b.prefill(toks)
    got = a.generate(12).tolist()
    want = []
    for _ in range(12):
        t = b.greedy_token()
        assert b.greedy_token() == t  # selection leaves the state unchanged
        want.append(t)
        b.step(t)
    assert got == want
    a.close()
    b.close()


def test_error_paths(hip):
    w = Lfm2Weights(LFM2_TINY, seed=1)
    m = Lfm2Hip(hip, w, n_ctx=4)
    with pytest.raises(BobcatError) as e:
        m.generate(1)
    assert "prompt" in str(e.value)
    with pytest.raises(BobcatError) as e:
        m.step(LFM2_TINY.n_vocab)
    assert e.value.status == 16  # Token
    m.prefill([1, 2, 3])
    with pytest.raises(BobcatError) as e:
        m.prefill([1, 2])
    assert e.value.status == 15  # ContextFull
    m.step(4)
    with pytest.raises(BobcatError) as e:
        m.step(5)
    assert e.value.status == 15
    m.close()


def test_restore_continues_against_oracle(hip, weights):
    """lfm2_reference.rs:190-238: a restored state continues as the checkpointed
    one did, straight into generation and through more prompt after later
    tokens changed the histories, logits and cache positions; the continuation
    is checked against the oracle stepping prefix + suffix."""
    cfg = weights.cfg
    prefix, suffix = prompt(cfg, 12, seed=21), prompt(cfg, 5, seed=22)
    gpu = Lfm2Hip(hip, weights, n_ctx=64, kv_half=False)
    gpu.prefill(prefix, logits=False)
    ck = gpu.checkpoint()
    first = gpu.generate(8)
    gpu.prefill(prompt(cfg, 3, seed=23), logits=False)
    gpu.restore(ck)
    assert gpu.n_past == len(prefix)
    assert np.array_equal(gpu.generate(8), first), "generation after a restore"
    gpu.restore(ck)
    got = gpu.prefill(suffix)
    cpu = oracle.Lfm2State(weights, n_ctx=64)
    for t in prefix + suffix:
        want = cpu.step(t)
    # The suffix runs as a prefill batch, whose GEMM rounds weights to f16.
    assert rel(got, want) < HALF_TOLERANCE, rel(got, want)
    # ...and the next steps after the restored prompt.
    for t in prompt(cfg, 4, seed=24):
        assert rel(gpu.step(t), cpu.step(t)) < HALF_TOLERANCE
    gpu.reset()
    with pytest.raises(BobcatError):
        gpu.restore(ck)
    gpu.close()


def test_streaming_matches_generate(hip, weights):
    """lfm2_reference.rs:240-292: the stream emits what generate picks, stops
    where the caller stops it, and reports every token its steps ran,
    including those past the stop and at the end of the context."""
    cfg = weights.cfg
    toks = prompt(cfg, 4, seed=25)
    gpu = Lfm2Hip(hip, weights, n_ctx=20)
    gpu.prefill(toks, logits=False)
    ck = gpu.checkpoint()
    expected = gpu.generate(16).tolist()
    after = gpu.greedy_token()

    gpu.restore(ck)
    emitted = []
    gained = gpu.generate_stream(17, lambda t: emitted.append(t) or True)
    assert emitted[:16] == expected, "streamed tokens"
    assert emitted[16] == after, "the selection after the last position"
    assert gained == expected, "tokens a full stream ran"
    assert gpu.n_past == 20

    gpu.restore(ck)
    emitted = []
    gained = gpu.generate_stream(17, lambda t: emitted.append(t) or len(emitted) < 5)
    assert emitted == expected[:5], "tokens up to the stop"
    assert len(gained) >= 4, "a stopped stream ran the tokens before its last"
    assert gained == expected[:len(gained)], "tokens a stopped stream ran"
    assert gpu.n_past == 4 + len(gained)
    # The sequence goes on from where the stream left it.
    nxt = gpu.generate(20 - gpu.n_past).tolist()
    assert gained + nxt == expected

    gpu.restore(ck)
    assert gpu.generate_stream(0, lambda t: True) == []
    emitted = []
    assert gpu.generate_stream(1, lambda t: emitted.append(t) or True) == []
    assert emitted == expected[:1] and gpu.n_past == 4
    assert gpu.generate_stream(5, lambda t: False) == []
    assert gpu.n_past == 4
    gpu.close()


def test_greedy_selection_preserves_sequence_state(hip, weights):
    """lfm2_reference.rs:296-350: greedy_token consumes nothing, and
    generate_next continues from it in chunks as generate would."""
    cfg = weights.cfg
    toks = prompt(cfg, 4, seed=26)
    for kv_half in (True, False):
        gpu = Lfm2Hip(hip, weights, n_ctx=20, kv_half=kv_half)
        with pytest.raises(BobcatError):
            gpu.greedy_token()
        gpu.prefill(toks, logits=False)
        ck = gpu.checkpoint()
        expected = gpu.generate(16).tolist()
        nxt = gpu.greedy_token()
        with pytest.raises(BobcatError):
            gpu.generate(1)  # full context
        assert gpu.greedy_token() == nxt
        for chunk in (1, 3, 8):
            gpu.restore(ck)
            streamed = [gpu.greedy_token()]
            assert gpu.greedy_token() == streamed[0], "repeated selection"
            assert gpu.generate_next(0).size == 0
            assert gpu.greedy_token() == streamed[0], "empty continuation"
            while len(streamed) < 16:
                streamed += gpu.generate_next(min(chunk, 16 - len(streamed))).tolist()
            assert streamed == expected, "early selection changes generation"
            assert gpu.generate(1).tolist() == [expected[15]]
            assert gpu.greedy_token() == nxt, "selection advances the sequence"
        gpu.reset()
        with pytest.raises(BobcatError):
            gpu.greedy_token()
        gpu.close()


def test_gguf_model_matches_direct_upload(hip, weights, tmp_path):
    """The model written as an LFM2 GGUF file (tensor names and metadata of
    real files) and loaded through bch_gguf_open + bch_lfm2_model_from_gguf
    decodes bit-identically to the same weights uploaded directly."""
    from bobcat_amd.gguf import GgufWeights, lfm2_to_gguf

    cfg = weights.cfg
    path = tmp_path / "m.gguf"
    lfm2_to_gguf(weights, path)
    gw = GgufWeights(path, cfg)
    toks = prompt(cfg, 9, seed=41)
    a = Lfm2Hip(hip, weights, n_ctx=32)
    b = Lfm2Hip(hip, gw, n_ctx=32)
    assert np.array_equal(a.prefill(toks), b.prefill(toks))
    assert np.array_equal(a.generate(6), b.generate(6))
    a.close()
    b.close()
