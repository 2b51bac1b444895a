"""GPU parity of BASELINE configs[3] part 2 at its real size: the LFM2 2.6B
model (8 KV heads of 64, f16 KV cache) over a 32,768-token prompt, and a
second request that reuses the first 30,000 tokens' state.

The oracle cannot run 32K positions of a 2.6B model within a test, so the
long run is pinned by the invariants the reference's own model tests use
(crates/bobcat/tests/lfm2_reference.rs:117-238; engine.rs:561-584):

* prefill == steps: the last-token logits of a 32,768-token prefill equal a
  prefill of the first 32,760 tokens followed by 8 decode steps (the decode
  attention over ~32K keys, its key splits and the MFMA prefill attention
  with key splits meet at the same numbers) within the 5e-3 half-precision
  bound;
* shared prefix == fresh: restoring the checkpoint taken after the 30,000
  shared tokens and prefilling only the 2,768-token tail gives the logits of
  the whole prompt prefilled from scratch, and the same 128 greedy tokens
  (a flip allowed only where the fresh run's top-2 logits differ by < 1e-3).

And against the oracle itself at the long-context attention shape: a
4,096-token prompt and 32 greedy tokens of the same model
(tests/golden/greedy_lfm2-2.6b-ctx4k.npz, written by
tests/golden/make_greedy.py), with the f32 cache and with the f16 cache,
under the same near-tie rule.
"""
from __future__ import annotations

import numpy as np
import pytest

from bobcat_amd.lfm2 import LFM2_2_6B, Lfm2Hip, Lfm2Weights
from golden.make_greedy import LONG, WEIGHT_SEED, digest, fixture_path

pytestmark = pytest.mark.gpu

HALF_TOLERANCE = 5e-3
TIE = 1e-3
LONG_PROMPT, SHARED, GEN, TAIL_STEPS = 32768, 30000, 128, 8


def rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def top2_gap(lg):
    top = np.sort(np.asarray(lg, np.float64))[-2:]
    return float(top[1] - top[0])


def first_divergence(got, want, gaps):
    """Index where got leaves want, or None; raises if that is not a near-tie."""
    for i, (g, w) in enumerate(zip(got, want)):
        if g != w:
            assert gaps[i] < TIE, f"token {i}: {g} vs {w} (top-2 gap {gaps[i]:.3g})"
            return i
    return None


@pytest.fixture(scope="module")
def weights():
    w = Lfm2Weights(LFM2_2_6B, seed=WEIGHT_SEED)
    yield w
    del w


def prompts(seed=7):
    rng = np.random.default_rng(seed)
    p1 = rng.integers(0, LFM2_2_6B.n_vocab, LONG_PROMPT).astype(np.uint32)
    p2 = p1.copy()
    p2[SHARED:] = rng.integers(0, LFM2_2_6B.n_vocab, LONG_PROMPT - SHARED)
    return p1, p2


@pytest.mark.timeout(600)
def test_prefill_equals_steps_at_32k(hip, weights):
    p1, _ = prompts()
    m = Lfm2Hip(hip, weights, n_ctx=LONG_PROMPT + GEN, kv_half=True)
    full = m.prefill(p1)
    m.reset()
    m.prefill(p1[:-TAIL_STEPS], logits=False)
    for t in p1[-TAIL_STEPS:]:
        stepped = m.step(int(t))
    assert m.n_past == LONG_PROMPT
    m.close()
    r = rel(stepped, full)
    print(f"32K prefill vs prefill + {TAIL_STEPS} steps: max relative difference {r:.3g}")
    assert r < HALF_TOLERANCE, r
    if int(np.argmax(stepped)) != int(np.argmax(full)):
        assert top2_gap(full) < TIE


@pytest.mark.timeout(900)
def test_shared_prefix_reuse_equals_fresh(hip, weights):
    p1, p2 = prompts()
    m = Lfm2Hip(hip, weights, n_ctx=LONG_PROMPT + GEN, kv_half=True)
    # Request 1: the shared prefix, a checkpoint there, then its own tail.
    m.prefill(p1[:SHARED], logits=False)
    ck = m.checkpoint()
    m.prefill(p1[SHARED:], logits=False)
    m.generate(8)
    # Request 2 from the checkpoint: only its 2,768-token tail is prefilled.
    m.restore(ck)
    assert m.n_past == SHARED
    lg_reused = m.prefill(p2[SHARED:])
    reused = m.generate(GEN).tolist()  # starts with the selection after the prefill
    # Request 2 from scratch, step by step so every step's top-2 gap is known.
    m.reset()
    lg_fresh = m.prefill(p2)
    fresh, gaps, lg = [], [], lg_fresh
    for _ in range(GEN):
        tok = int(np.argmax(lg))
        fresh.append(tok)
        gaps.append(top2_gap(lg))
        lg = m.step(tok)
    m.close()
    r = rel(lg_reused, lg_fresh)
    at = first_divergence(reused, fresh, gaps)
    print(f"reuse vs fresh: logits {r:.3g}, 128 tokens {'identical' if at is None else f'near-tie flip at {at}'}")
    assert r < HALF_TOLERANCE, r


@pytest.mark.timeout(900)
def test_4k_prompt_matches_oracle(hip, weights):
    name = "lfm2-2.6b-ctx4k"
    path = fixture_path(name)
    if not path.exists():
        pytest.skip(f"{path.name} not generated (tests/golden/make_greedy.py {name})")
    fix = np.load(path)
    assert str(fix["digest"]) == digest(weights), "the seeded weight generator changed; regenerate the fixture"
    _, n_prompt, n_gen = LONG[name]
    prompt = fix["prompt"].tolist()
    assert len(prompt) == n_prompt
    want = fix["tokens"].tolist()
    for kv_half in (False, True):
        m = Lfm2Hip(hip, weights, n_ctx=n_prompt + n_gen + 8, kv_half=kv_half)
        lg = m.prefill(prompt)
        r = rel(lg, fix["logits0"])
        got = m.generate(n_gen).tolist()
        m.close()
        at = first_divergence(got, want, fix["gaps"])
        print(f"4K prompt, {'f16' if kv_half else 'f32'} cache: logits {r:.3g}, {n_gen} tokens "
              f"{'identical' if at is None else f'near-tie flip at {at}'}")
        assert r < HALF_TOLERANCE, r
