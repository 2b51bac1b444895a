"""GPU parity of the Qwen3.5 driver (bch_qwen35_*) and the DeltaNet kernels
against the oracle.

The driver follows tests/test_gpu_lfm2.py, with the oracle's Qwen3.5 forward
pass (pinned to transformers in tests/test_oracle_qwen35.py) as the
reference: every layer's output and the logits of each step within 1e-4 with
an f32 KV cache (5e-3 with f16), prefill traces, greedy ids (a flip allowed
only where the oracle's top-2 logits differ by less than 1e-3), prefill ==
steps, generate == greedy steps, checkpoint/restore and reset.

The kernels are checked on their own against float64 restatements of the
formulas of qwen35.rs:448-511 (the convolution, the gates, the gated delta
rule with L2-normalised queries and keys, the gated output norm) and of
attention_gate (gdn.metal:300-322), within 1e-5 relative — the tolerance of
the reference's metal_gdn.rs.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd._lib import DeltaShape
from bobcat_amd.qwen35 import (QWEN35_TINY, QWEN35_TINY_64, QWEN35_TINY_V192, QWEN35_TINY_V256, QWEN35_TINY_V1024,
                               Qwen35Config, Qwen35Hip, Qwen35Weights)

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-4
PREFILL_TOLERANCE = 1e-3
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


@pytest.fixture(scope="module", params=[QWEN35_TINY, QWEN35_TINY_64, QWEN35_TINY_V256, QWEN35_TINY_V192,
                                        QWEN35_TINY_V1024],
                ids=lambda c: c.name)
def weights(request):
    return Qwen35Weights(request.param, seed=7)


def prompt(cfg, n, seed=1):
    return np.random.default_rng(seed).integers(0, cfg.n_vocab, n).tolist()


@pytest.mark.parametrize("grouped", [False, True], ids=["head_per_wg", "grouped"])
@pytest.mark.parametrize("kv_half", [False, True])
def test_steps_match_oracle_layer_by_layer(hip, weights, kv_half, grouped, monkeypatch):
    set_grouped(monkeypatch, grouped)
    cfg = weights.cfg
    tol = HALF_TOLERANCE if kv_half else TOLERANCE
    gpu = Qwen35Hip(hip, weights, n_ctx=40, kv_half=kv_half)
    cpu = oracle.Qwen35State(weights, n_ctx=40)
    for t, tok in enumerate(prompt(cfg, 20)):
        lg, (emb, layers, final) = gpu.step(tok, trace=True)
        wlg, (wemb, wlayers, wfinal) = cpu.step(tok, trace=True)
        assert rel(emb, wemb) < 1e-6
        for il in range(cfg.n_layers):
            sl = slice(il * cfg.n_embd, (il + 1) * cfg.n_embd)
            assert rel(layers[sl], wlayers[sl]) < tol, (t, il, rel(layers[sl], wlayers[sl]))
        assert rel(final, wfinal) < tol
        assert rel(lg, wlg) < tol, t
    gpu.close()


@pytest.mark.parametrize("kv_half", [False, True])
def test_prefill_trace_matches_oracle(hip, weights, kv_half):
    """The batched pass against the oracle's token-by-token steps.  The
    prefill GEMM rounds weights and inputs to half precision (the weights
    as the reference's expanded half tiles), so with an f32 KV cache the
    layers match within 1e-3 relative rather than the decode path's 1e-4."""
    cfg = weights.cfg
    tol = HALF_TOLERANCE if kv_half else PREFILL_TOLERANCE
    toks = prompt(cfg, 30, seed=2)
    gpu = Qwen35Hip(hip, weights, n_ctx=40, kv_half=kv_half)
    lg, (emb, layers, final) = gpu.prefill(toks, trace=True)
    cpu = oracle.Qwen35State(weights, n_ctx=40)
    for t, tok in enumerate(toks):
        wlg, (wemb, wlayers, wfinal) = cpu.step(tok, trace=True)
        for il in range(cfg.n_layers):
            w = wlayers[il * cfg.n_embd:(il + 1) * cfg.n_embd]
            assert rel(layers[il, t], w) < tol, (t, il, rel(layers[il, t], w))
    assert rel(lg, wlg) < tol
    gpu.close()


@pytest.mark.parametrize("kv_half", [False, True])
def test_hidden_matches_oracle_final_norm(hip, weights, kv_half):
    """Gpu::hidden (crates/bobcat-cli/src/backend.rs:150-160) through
    bch_qwen35_hidden: a new sequence, each token's final-norm row, against
    the oracle's final norm after each step (qwen35.rs, the input of the
    output projection), within the prefill bound; it also starts over (the
    rows do not depend on what ran before) and leaves the sequence at the
    prompt's length."""
    cfg = weights.cfg
    tol = HALF_TOLERANCE if kv_half else PREFILL_TOLERANCE
    toks = prompt(cfg, 25, seed=8)
    gpu = Qwen35Hip(hip, weights, n_ctx=40, kv_half=kv_half)
    gpu.prefill(prompt(cfg, 7, seed=9))  # something to start over from
    got = gpu.hidden(toks)
    assert gpu.n_past == len(toks)
    again = gpu.hidden(toks)
    gpu.close()
    assert np.array_equal(got, again)
    cpu = oracle.Qwen35State(weights, n_ctx=40)
    for t, tok in enumerate(toks):
        _, (_, _, wfinal) = cpu.step(tok, trace=True)
        assert rel(got[t], wfinal) < tol, (t, rel(got[t], wfinal))


def test_greedy_generation_matches_oracle(hip, weights):
    cfg = weights.cfg
    toks = prompt(cfg, 9, seed=3)
    cpu = oracle.Qwen35State(weights, n_ctx=64)
    for t in toks:
        lg = cpu.step(t)
    want, gaps = [], []
    for _ in range(20):
        top2 = np.sort(lg)[-2:]
        gaps.append(float(top2[1] - top2[0]))
        nxt = int(np.argmax(lg))
        want.append(nxt)
        lg = cpu.step(nxt)
    gpu = Qwen35Hip(hip, weights, n_ctx=64, kv_half=False)
    gpu.prefill(toks)
    got = [gpu.greedy_token()] + gpu.generate(19).tolist()
    gpu.close()
    for i, (g, w) in enumerate(zip(got, want)):
        if g != w:
            assert gaps[i] < 1e-3, (i, got, want)
            break


def test_prefill_matches_steps_and_generate(hip, weights):
    cfg = weights.cfg
    toks = prompt(cfg, 70, seed=5)  # two attention query batches
    a = Qwen35Hip(hip, weights, n_ctx=100)
    b = Qwen35Hip(hip, weights, n_ctx=100)
    la = a.prefill(toks)
    for t in toks:
        lb = b.step(t)
    assert rel(la, lb) < HALF_TOLERANCE
    ga = a.generate(6).tolist()
    gb = []
    t = int(np.argmax(lb))
    for _ in range(6):
        gb.append(t)
        t = int(np.argmax(b.step(t)))
    assert ga == gb
    a.close()
    b.close()


def test_checkpoint_restore_and_reset(hip, weights):
    cfg = weights.cfg
    toks = prompt(cfg, 12, seed=6)
    m = Qwen35Hip(hip, weights, n_ctx=64, kv_half=False)
    m.prefill(toks[:8])
    blob = m.checkpoint()
    first = m.step(toks[8])
    m.step(toks[9])
    m.restore(blob)
    again = m.step(toks[8])
    assert rel(again, first) < 1e-6
    m.reset()
    fresh = Qwen35Hip(hip, weights, n_ctx=64, kv_half=False)
    assert rel(m.prefill(toks), fresh.prefill(toks)) < 1e-6
    m.close()
    fresh.close()


def test_restore_continues_against_oracle(hip, weights):
    """A restored DeltaNet/conv state continues through more prompt as the
    oracle stepping prefix + suffix does (lfm2_reference.rs:190-238's check on
    the Qwen3.5 driver)."""
    cfg = weights.cfg
    prefix, suffix = prompt(cfg, 10, seed=31), prompt(cfg, 6, seed=32)
    m = Qwen35Hip(hip, weights, n_ctx=64, kv_half=False)
    m.prefill(prefix, logits=False)
    ck = m.checkpoint()
    first = m.generate(6)
    m.prefill(prompt(cfg, 3, seed=33), logits=False)
    m.restore(ck)
    assert np.array_equal(m.generate(6), first)
    m.restore(ck)
    got = m.prefill(suffix)
    cpu = oracle.Qwen35State(weights, n_ctx=64)
    for t in prefix + suffix:
        want = cpu.step(t)
    # The suffix runs as a prefill batch, whose GEMM rounds weights to f16.
    assert rel(got, want) < HALF_TOLERANCE, rel(got, want)
    for t in prompt(cfg, 3, seed=34):
        assert rel(m.step(t), cpu.step(t)) < HALF_TOLERANCE
    m.close()


def test_streaming_matches_generate(hip, weights):
    cfg = weights.cfg
    m = Qwen35Hip(hip, weights, n_ctx=24)
    m.prefill(prompt(cfg, 6, seed=35), logits=False)
    ck = m.checkpoint()
    expected = m.generate(18).tolist()
    after = m.greedy_token()
    m.restore(ck)
    emitted = []
    assert m.generate_stream(40, lambda t: emitted.append(t) or True) == expected
    assert emitted == expected + [after]
    m.restore(ck)
    emitted = []
    gained = m.generate_stream(40, lambda t: emitted.append(t) or len(emitted) < 7)
    assert emitted == expected[:7] and gained == expected[:len(gained)] and len(gained) >= 6
    m.restore(ck)
    streamed = [m.greedy_token()]
    while len(streamed) < 18:
        streamed += m.generate_next(min(4, 18 - len(streamed))).tolist()
    assert streamed == expected
    m.close()


# ---------------------------------------------------------------- kernels

def run(hip, fn):
    hip.begin()
    fn()
    hip.end()


def silu(x):
    return x / (1 + np.exp(-x))


@pytest.mark.parametrize("n_k,n_v,dk,dv,n_tokens", [(2, 2, 128, 128, 1), (2, 4, 64, 64, 7), (16, 16, 128, 128, 33)])
def test_gdn_ops_match_float64(hip, n_k, n_v, dk, dv, n_tokens):
    rng = np.random.default_rng(n_v * 100 + n_tokens)
    key_dim, value_dim = n_k * dk, n_v * dv
    conv_dim, K = 2 * key_dim + value_dim, 4
    x = rng.standard_normal((n_tokens, conv_dim)).astype(np.float32)
    taps = rng.uniform(-0.5, 0.5, (conv_dim, K)).astype(np.float32)
    hist = rng.standard_normal((conv_dim, K - 1)).astype(np.float32)
    beta = rng.standard_normal((n_tokens, n_v)).astype(np.float32)
    alpha = rng.standard_normal((n_tokens, n_v)).astype(np.float32)
    a = (-np.exp(rng.uniform(-2, 1, n_v))).astype(np.float32)
    dt = rng.uniform(-1, 1, n_v).astype(np.float32)
    state = (rng.standard_normal((n_v, dk, dv)) * 0.1).astype(np.float32)
    nw = (1 + 0.1 * rng.uniform(-1, 1, dv)).astype(np.float32)
    z = rng.standard_normal((n_tokens, value_dim)).astype(np.float32)

    xb, tb, hb = hip.buffer_from(x), hip.buffer_from(taps), hip.buffer_from(hist)
    yb = hip.new_buffer(x.nbytes)
    bb, ab, a_b, db = hip.buffer_from(beta), hip.buffer_from(alpha), hip.buffer_from(a), hip.buffer_from(dt)
    sb, ob = hip.buffer_from(state), hip.new_buffer(n_tokens * value_dim * 4)
    wb, zb = hip.buffer_from(nw), hip.buffer_from(z)
    shape = DeltaShape(n_k, n_v, dk, dv)
    from bobcat_amd._lib import lib
    import ctypes as C
    from bobcat_amd.backend import _view

    def call(fn, *args):
        assert fn(hip.handle, *args) == 0, lib().bch_last_error()

    q_scale = 1 / np.sqrt(dk)
    run(hip, lambda: (call(lib().bch_gdn_conv, _view(xb.at(0)), _view(tb.at(0)), _view(hb.at(0)), _view(yb.at(0)),
                           conv_dim, K, n_tokens),
                      call(lib().bch_gdn_gates, _view(bb.at(0)), _view(ab.at(0)), _view(a_b.at(0)), _view(db.at(0)),
                           n_v, n_tokens * n_v),
                      call(lib().bch_gdn_recurrence, _view(yb.at(0)), _view(bb.at(0)), _view(ab.at(0)),
                           _view(sb.at(0)), _view(ob.at(0)), C.byref(shape), n_tokens, C.c_float(q_scale)),
                      call(lib().bch_gdn_gated_norm, _view(ob.at(0)), _view(wb.at(0)), _view(zb.at(0)), dv,
                           n_tokens * n_v, C.c_float(1e-6))))
    y = hip.read(yb.at(0), np.empty_like(x))
    got_hist = hip.read(hb.at(0), np.empty_like(hist))
    got_state = hip.read(sb.at(0), np.empty_like(state))
    got = hip.read(ob.at(0), np.empty((n_tokens, value_dim), np.float32))

    # float64 restatement (qwen35.rs:448-511).
    h = hist.astype(np.float64).copy()
    conv = np.empty((n_tokens, conv_dim))
    for t in range(n_tokens):
        s = taps[:, K - 1] * x[t] + (taps[:, :K - 1] * h).sum(1)
        conv[t] = silu(s)
        h = np.concatenate([h[:, 1:], x[t][:, None].astype(np.float64)], 1)
    assert rel(y, conv) < 1e-5
    assert rel(got_hist, h) < 1e-6
    S = state.astype(np.float64).copy()
    want = np.empty((n_tokens, value_dim))
    for t in range(n_tokens):
        q = conv[t, :key_dim].reshape(n_k, dk)
        k = conv[t, key_dim:2 * key_dim].reshape(n_k, dk)
        v = conv[t, 2 * key_dim:].reshape(n_v, dv)
        q = q / np.sqrt((q * q).sum(1, keepdims=True) + 1e-6) * q_scale
        k = k / np.sqrt((k * k).sum(1, keepdims=True) + 1e-6)
        for hh in range(n_v):
            kh = hh % n_k
            b = 1 / (1 + np.exp(-float(beta[t, hh])))
            sp = float(alpha[t, hh] + dt[hh])
            decay = np.exp(float(a[hh]) * (sp if sp > 20 else np.log1p(np.exp(sp))))
            S[hh] *= decay
            rem = k[kh] @ S[hh]
            delta = (v[hh] - rem) * b
            S[hh] += np.outer(k[kh], delta)
            o = q[kh] @ S[hh]
            o = o / np.sqrt((o * o).mean() + 1e-6) * nw
            want[t, hh * dv:(hh + 1) * dv] = o * silu(z[t, hh * dv:(hh + 1) * dv].astype(np.float64))
    assert rel(got_state, S) < 1e-5
    assert rel(got, want) < 1e-5


def test_attention_gate_matches_float64(hip):
    rng = np.random.default_rng(3)
    n_tokens, heads, hd = 5, 8, 256
    q_dim = heads * hd
    attn = rng.standard_normal((n_tokens, q_dim)).astype(np.float32)
    qg = rng.standard_normal((n_tokens, 2 * q_dim)).astype(np.float32)
    ab, gb = hip.buffer_from(attn), hip.buffer_from(qg)
    from bobcat_amd._lib import lib
    from bobcat_amd.backend import _view
    hip.begin()
    assert lib().bch_attention_gate(hip.handle, _view(ab.at(0)), _view(gb.at(0)), hd, q_dim, n_tokens) == 0
    hip.end()
    got = hip.read(ab.at(0), np.empty_like(attn))
    gate = qg.reshape(n_tokens, heads, 2, hd)[:, :, 1, :].reshape(n_tokens, q_dim).astype(np.float64)
    assert rel(got, attn * (1 / (1 + np.exp(-gate)))) < 1e-6


@pytest.mark.parametrize("head_dim", [64, 256])
@pytest.mark.parametrize("grouped", [False, True], ids=["head_per_wg", "grouped"])
@pytest.mark.parametrize("kv_half", [False, True])
def test_long_context_gated_decode(hip, kv_half, grouped, head_dim, monkeypatch):
    """Four query heads per KV head in a driver sized for 8192 positions: the
    gated decode kernel over a grid of many splits; steps at positions
    1020-1027 (4 to 33 live splits, combined in parallel) against the
    oracle."""
    set_grouped(monkeypatch, grouped)
    cfg = Qwen35Config("qwen3.5-group4", n_embd=256, n_ff=512, n_vocab=500, n_layers=4, n_heads=4,
                       n_kv_heads=1, head_dim=head_dim, n_rot=32, n_k_heads=2, n_v_heads=4, k_head_dim=64,
                       v_head_dim=64)
    w = Qwen35Weights(cfg, seed=13)
    toks = prompt(cfg, 1028, seed=10)
    gpu = Qwen35Hip(hip, w, n_ctx=8192, kv_half=kv_half)
    cpu = oracle.Qwen35State(w, n_ctx=1100)
    gpu.prefill(toks[:1020], logits=False)
    for t in toks[:1020]:
        cpu.step(t, logits=False)
    tol = HALF_TOLERANCE if kv_half else TOLERANCE
    for t in toks[1020:]:
        got, want = gpu.step(t), cpu.step(t)
        assert rel(got, want) < tol, (t, rel(got, want))
    gpu.close()


def delta_rule_f64(y, beta, decay, state, n_k, n_v, dk, dv, q_scale):
    """The gated delta rule of qwen35.rs:475-511 in float64, token by token,
    all heads at once: S *= decay; delta = beta (v - S^T k); S += k delta^T;
    o = S^T q, with q and k L2-normalised (eps 1e-6) and q times q_scale."""
    key_dim = n_k * dk
    S = state.astype(np.float64).copy()
    out = np.empty((y.shape[0], n_v * dv))
    heads = np.arange(n_v) % n_k
    for t in range(y.shape[0]):
        yt = y[t].astype(np.float64)
        q = yt[:key_dim].reshape(n_k, dk)
        k = yt[key_dim:2 * key_dim].reshape(n_k, dk)
        v = yt[2 * key_dim:].reshape(n_v, dv)
        q = q / np.sqrt((q * q).sum(1, keepdims=True) + 1e-6) * q_scale
        k = k / np.sqrt((k * k).sum(1, keepdims=True) + 1e-6)
        q, k = q[heads], k[heads]
        S *= decay[t].astype(np.float64)[:, None, None]
        rem = np.einsum("hr,hrc->hc", k, S)
        delta = (v - rem) * beta[t].astype(np.float64)[:, None]
        S += k[:, :, None] * delta[:, None, :]
        out[t] = np.einsum("hr,hrc->hc", q, S).reshape(-1)
    return out, S


@pytest.mark.parametrize("n_k,n_v,dk,dv,n_tokens", [(16, 16, 128, 128, 1), (16, 16, 128, 128, 63),
                                                    (16, 16, 128, 128, 64), (16, 16, 128, 128, 65),
                                                    (16, 16, 128, 128, 512), (2, 4, 64, 64, 130),
                                                    (1, 2, 128, 256, 100)])
def test_gdn_chunked_matches_float64(hip, n_k, n_v, dk, dv, n_tokens):
    """The chunked (WY) prefill form against the sequential recurrence in
    float64 (qwen35.rs:475-511) at chunk boundaries 1/63/64/65/512 of the
    Qwen3.5-0.8B head shape (16 heads of 128 x 128 states), within 1e-5 of
    the largest output and state entry; and against the GPU's own sequential
    kernel (bch_gdn_recurrence) on the same inputs."""
    from bobcat_amd._lib import lib
    import ctypes as C
    from bobcat_amd.backend import _view

    rng = np.random.default_rng(1000 + n_tokens + dv)
    key_dim, value_dim = n_k * dk, n_v * dv
    conv_dim = 2 * key_dim + value_dim
    y = rng.standard_normal((n_tokens, conv_dim)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (n_tokens, n_v)).astype(np.float32)
    decay = np.exp(-rng.uniform(0.0, 2.5, (n_tokens, n_v))).astype(np.float32)
    state = (rng.standard_normal((n_v, dk, dv)) * 0.1).astype(np.float32)
    q_scale = 1 / np.sqrt(dk)
    shape = DeltaShape(n_k, n_v, dk, dv)
    scratch = lib().bch_gdn_chunk_scratch_floats(C.byref(shape), n_tokens)
    assert scratch == n_v * -(-n_tokens // 64) * (64 * (3 * dk + dv) + 64 * 64 + 64)
    yb, bb, db = hip.buffer_from(y), hip.buffer_from(beta), hip.buffer_from(decay)
    sb, s2 = hip.buffer_from(state), hip.buffer_from(state)
    ob, o2 = hip.new_buffer(n_tokens * value_dim * 4), hip.new_buffer(n_tokens * value_dim * 4)
    wb = hip.new_buffer(scratch * 4)

    def call(fn, *args):
        assert fn(hip.handle, *args) == 0, lib().bch_last_error()

    run(hip, lambda: (call(lib().bch_gdn_recurrence_chunked, _view(yb.at(0)), _view(bb.at(0)), _view(db.at(0)),
                           _view(sb.at(0)), _view(ob.at(0)), C.byref(shape), n_tokens, C.c_float(q_scale),
                           _view(wb.at(0))),
                      call(lib().bch_gdn_recurrence, _view(yb.at(0)), _view(bb.at(0)), _view(db.at(0)),
                           _view(s2.at(0)), _view(o2.at(0)), C.byref(shape), n_tokens, C.c_float(q_scale))))
    got = hip.read(ob.at(0), np.empty((n_tokens, value_dim), np.float32))
    got_state = hip.read(sb.at(0), np.empty_like(state))
    seq = hip.read(o2.at(0), np.empty((n_tokens, value_dim), np.float32))
    want, want_state = delta_rule_f64(y, beta, decay, state, n_k, n_v, dk, dv, q_scale)
    print(f"chunked vs f64: out {rel(got, want):.2e} state {rel(got_state, want_state):.2e}; "
          f"sequential kernel vs f64: {rel(seq, want):.2e}")
    assert rel(got, want) < 1e-5
    assert rel(got_state, want_state) < 1e-5
    assert rel(got, seq) < 1e-5


def test_gguf_model_matches_direct_upload(hip, weights, tmp_path):
    """The model written as a qwen35 GGUF file and loaded through
    bch_qwen35_model_from_gguf decodes bit-identically to the direct upload."""
    from bobcat_amd.gguf import GgufWeights, qwen35_to_gguf

    cfg = weights.cfg
    path = tmp_path / "q.gguf"
    qwen35_to_gguf(weights, path)
    gw = GgufWeights(path, cfg)
    toks = prompt(cfg, 9, seed=41)
    a = Qwen35Hip(hip, weights, n_ctx=32)
    b = Qwen35Hip(hip, gw, n_ctx=32)
    assert np.array_equal(a.prefill(toks), b.prefill(toks))
    assert np.array_equal(a.generate(6), b.generate(6))
    a.close()
    b.close()
