"""GPU parity of bch_attention_decode, the decode attention step the model
drivers run per attention layer: q/k RMS norm, NeoX RoPE, the cache store of
the new key and value, and causal GQA attention over positions 0..pos
(lfm2.rs:515-555).

The expected values are the oracle's restatement of that block: its
rms_norm and rope_neox per head, the cache rows as the kernel must leave
them (the new key and value, rounded to f16 for an f16 cache), and its
attention over the cache.  Two consecutive positions per case, so the
second call also checks that the scratch (position word, split counters,
partials) carries nothing from the first.  Shapes: the LFM2-2.6B/8B heads
(32 x 8 of 64) at short and long contexts, including 32,770 positions (129
splits, the grouped layout), an f32 cache, LFM2-350M's groups of two, and
Qwen3.5's heads of 256 with a 64-element rotary part; each with the default
layout choice and with the grouped layout forced.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd.backend import attention_decode_scratch_floats

pytestmark = pytest.mark.gpu

EPS = 1e-5
THETA = 1_000_000.0
CASES = [
    # heads, kv heads, head dim, rotary elements, f16 cache, position
    (32, 8, 64, 64, True, 100),
    (32, 8, 64, 64, True, 5000),
    (32, 8, 64, 64, True, 32770),
    (32, 8, 64, 64, False, 2000),
    (16, 8, 64, 64, True, 1500),
    (8, 2, 256, 64, True, 3000),
    (8, 2, 256, 64, False, 700),
]


def expected(q, k, v, qn, kn, kc, vc, heads, kv, hd, n_rot, half, pos):
    """The oracle's attention block for position pos; kc/vc [n][kv*hd] f32
    hold positions < pos and receive row pos."""
    def norm_rope(x, w):
        out = oracle.rms_norm(x, w, EPS)
        out[:n_rot] = oracle.rope_neox(out[:n_rot], pos, THETA)
        return out

    qr = np.concatenate([norm_rope(q[h * hd:(h + 1) * hd], qn) for h in range(heads)])
    kr = np.concatenate([norm_rope(k[h * hd:(h + 1) * hd], kn) for h in range(kv)])
    kc[pos] = kr.astype(np.float16).astype(np.float32) if half else kr
    vc[pos] = v.astype(np.float16).astype(np.float32) if half else v
    out = oracle.attention(qr, kc[:pos + 1].reshape(-1), vc[:pos + 1].reshape(-1), heads, kv, hd, pos, 1)
    return out, kr


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("heads,kv,hd,n_rot,half,pos", CASES)
def test_attention_decode_matches_oracle(hip, monkeypatch, grouped, heads, kv, hd, n_rot, half, pos):
    if grouped:
        monkeypatch.setenv("BCH_ATTN_GROUPED_ABOVE", "0")
    else:
        monkeypatch.delenv("BCH_ATTN_GROUPED_ABOVE", raising=False)
    print(f"attention_decode {heads}x{kv}x{hd} rot {n_rot} half {half} pos {pos} grouped {grouped}", flush=True)
    rng = np.random.default_rng(pos * 7 + heads)
    n_ctx = pos + 8
    kvd = kv * hd
    kc = np.zeros((n_ctx, kvd), np.float32)
    vc = np.zeros((n_ctx, kvd), np.float32)
    kc[:pos] = rng.standard_normal((pos, kvd), np.float32)
    vc[:pos] = rng.standard_normal((pos, kvd), np.float32)
    if half:
        kc, vc = kc.astype(np.float16).astype(np.float32), vc.astype(np.float16).astype(np.float32)
    ctype = np.float16 if half else np.float32
    kb, vb = hip.buffer_from(kc.astype(ctype)), hip.buffer_from(vc.astype(ctype))
    qn = (1.0 + 0.3 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.3 * rng.standard_normal(hd)).astype(np.float32)
    qnb, knb = hip.buffer_from(qn), hip.buffer_from(kn)
    sb = hip.new_buffer(attention_decode_scratch_floats(heads, hd, n_ctx, half) * 4)
    ob = hip.new_buffer(heads * hd * 4)
    try:
        for p in (pos, pos + 1):
            q = rng.standard_normal(heads * hd).astype(np.float32) * 2
            k = rng.standard_normal(kvd).astype(np.float32) * 2
            v = rng.standard_normal(kvd).astype(np.float32)
            qb, kb1, vb1 = hip.buffer_from(q), hip.buffer_from(k), hip.buffer_from(v)
            hip.begin()
            hip.attention_decode(qb.at(0), kb1.at(0), vb1.at(0), qnb.at(0), knb.at(0), EPS, THETA, n_rot,
                                 kb.at(0), vb.at(0), half, sb.at(0), ob.at(0), heads, kv, hd, p, n_ctx)
            hip.end()
            got = hip.read(ob.at(0), np.empty(heads * hd, np.float32))
            want, kr = expected(q, k, v, qn, kn, kc, vc, heads, kv, hd, n_rot, half, p)
            err = float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())
            assert err < 2e-5, (p, err)
            # The stored rows: the value exactly, the normalised and rotated
            # key within its own rounding (one f16 ulp, or 1e-5 in f32).
            row = hip.read(kb.at(p * kvd * (2 if half else 4)), np.empty(kvd, ctype)).astype(np.float32)
            vrow = hip.read(vb.at(p * kvd * (2 if half else 4)), np.empty(kvd, ctype)).astype(np.float32)
            assert np.array_equal(vrow, vc[p])
            tol = np.abs(kr) * (2.0 ** -10 if half else 1e-5) + 1e-6
            assert (np.abs(row - kr) <= tol).all()
            kc[p] = row  # later positions attend to what the kernel stored
            for b in (qb, kb1, vb1):
                b.free()
    finally:
        for b in (kb, vb, qnb, knb, sb, ob):
            b.free()
