"""Pins the CPU oracle (oracle/bobcat_oracle.c) before anything is checked against it.

Each oracle function is checked against something other than its own formula:
the reference's known-answer blocks (metal_matmul.rs:29-58), IEEE conversion
as numpy implements it, an independent vectorised numpy decoder of each
block layout, closed forms, invariants and brute force.  A plausible slip
(dropped term, swapped nibble, wrong scale byte, wrong sign) fails one of
them.

Pinning status per oracle function:
  orc_f16_to_f32 / orc_f32_to_f16 / orc_bf16_to_f32  exhaustive / random vs numpy IEEE
  orc_q4k_scale_min       all 2^24 byte triples per block pattern class, known answers
  orc_dequantize Q4_K     known answers + independent numpy decoder, bit-exact
  orc_dequantize Q5_K/Q6_K/Q8_0/Q4_0/F16/BF16  independent numpy decoders, bit-exact
  orc_matvec / orc_dot    float64 brute force
  orc_rms_norm            closed form on constant vectors + float64 brute force
  orc_rope_neox           identity at pos 0, norm preservation, relative-position invariance
  orc_softmax / orc_silu  closed forms and invariants
  orc_lfm2_route          brute-force top-k
  orc_lfm2_step           transformers' Lfm2ForCausalLM (tests/test_oracle_lfm2.py)
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd.synth import pack_q4k_scales, q4k_blocks
from tests._gen import Random, matmul_q4k_weights

F32, F16, Q4_0, Q8_0, Q4K, Q5K, Q6K, BF16 = 0, 1, 2, 8, 12, 13, 14, 30


# --------------------------------------------------------------------- #
# Independent numpy decoders, written from the block layouts.
# --------------------------------------------------------------------- #
def np_scale_min(s: np.ndarray):
    """[n, 12] scale bytes -> ([n, 8] scales, [n, 8] mins) from the bit layout."""
    s = s.astype(np.uint32)
    sc = np.empty(s.shape[:-1] + (8,), np.uint32)
    mn = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 0x3F
    mn[..., :4] = s[..., 4:8] & 0x3F
    sc[..., 4:] = (s[..., 8:12] & 0x0F) + 16 * (s[..., 0:4] >> 6)
    mn[..., 4:] = (s[..., 8:12] >> 4) + 16 * (s[..., 4:8] >> 6)
    return sc, mn


def np_q4k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = np_scale_min(b[:, 4:16])
    q = b[:, 16:].reshape(-1, 4, 32)
    nib = np.empty((b.shape[0], 8, 32), np.float32)
    nib[:, 0::2] = q & 0xF
    nib[:, 1::2] = q >> 4
    scale = d[:, None] * sc.astype(np.float32)          # f32 product, rounded
    minimum = dmin[:, None] * mn.astype(np.float32)
    out = scale[:, :, None] * nib - minimum[:, :, None]   # two separate roundings
    return out.reshape(-1).astype(np.float32)


def np_q5k(blocks):
    b = blocks.reshape(-1, 176)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    sc, mn = np_scale_min(b[:, 4:16])
    high = b[:, 16:48]
    q = b[:, 48:].reshape(-1, 4, 32)
    v = np.empty((b.shape[0], 8, 32), np.float32)
    for j in range(8):
        base = (q[:, j // 2] >> (4 * (j % 2))) & 0xF
        v[:, j] = base | (((high >> j) & 1) << 4)
    scale = d[:, None] * sc.astype(np.float32)
    minimum = dmin[:, None] * mn.astype(np.float32)
    return (scale[:, :, None] * v - minimum[:, :, None]).reshape(-1).astype(np.float32)


def np_q6k(blocks):
    b = blocks.reshape(-1, 210)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    out = np.empty((b.shape[0], 256), np.float32)
    for i in range(256):
        half, r = divmod(i, 128)
        quarter, l = divmod(r, 32)
        low_byte = b[:, half * 64 + l + (32 if quarter in (1, 3) else 0)]
        low = (low_byte & 0xF) if quarter < 2 else (low_byte >> 4)
        hi = (b[:, 128 + half * 32 + l] >> (2 * quarter)) & 3
        q = (low.astype(np.int32) | (hi.astype(np.int32) << 4)) - 32
        sc = b[:, 192 + half * 8 + l // 16 + 2 * quarter].view(np.int8).astype(np.float32)
        out[:, i] = (d * sc) * q.astype(np.float32)
    return out.reshape(-1)


def np_q8_0(blocks):
    b = blocks.reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    return (b[:, 2:].view(np.int8).astype(np.float32) * d).reshape(-1)


def np_q4_0(blocks):
    b = blocks.reshape(-1, 18)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:]
    v = np.concatenate([(q & 0xF).astype(np.int32) - 8, (q >> 4).astype(np.int32) - 8], axis=1)
    return (v.astype(np.float32) * d).reshape(-1)


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


# --------------------------------------------------------------------- #
# Conversions
# --------------------------------------------------------------------- #
def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert bits_equal(got[~nan], want[~nan])


def test_f32_to_f16_rounds_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 2.99e-8,
                  np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_bf16_and_f16_dequantize_match_numpy():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 65536, 4096, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7F80) != 0x7F80]  # finite bf16
    got = oracle.dequantize(BF16, bits.view(np.uint8), bits.size)
    assert bits_equal(got, (bits.astype(np.uint32) << 16).view(np.float32))
    h = rng.standard_normal(4096).astype(np.float16)
    assert bits_equal(oracle.dequantize(F16, h.view(np.uint8), h.size), h.astype(np.float32))


# --------------------------------------------------------------------- #
# Q4_K
# --------------------------------------------------------------------- #
def test_q4k_scale_min_known_answers():
    # Scale bytes 0x11 give (17, 17) for blocks 0-3 and (1, 1) for blocks 4-7
    # (the deterministic blocks of metal_matmul.rs:46-51).
    s = bytes([0x11] * 12)
    for j in range(8):
        assert oracle.q4k_scale_min(j, s) == ((17, 17) if j < 4 else (1, 1))
    # Every (scale, min) pair survives the pack -> unpack round trip.
    for v in range(64):
        sc = np.arange(8, dtype=np.uint8) * 0 + v
        mn = (63 - sc).astype(np.uint8)
        packed = pack_q4k_scales(sc[None], mn[None])[0].tobytes()
        for j in range(8):
            assert oracle.q4k_scale_min(j, packed) == (v, 63 - v)


def test_q4k_scale_min_exhaustive_bytes():
    """Each scale/min of block j depends on at most 3 bytes; enumerate all
    256 values of every byte that feeds it against the numpy bit decoder."""
    rng = np.random.default_rng(3)
    base = rng.integers(0, 256, 12, dtype=np.uint8)
    for pos in range(12):
        trial = np.repeat(base[None], 256, axis=0)
        trial[:, pos] = np.arange(256, dtype=np.uint8)
        sc, mn = np_scale_min(trial)
        for row in range(0, 256, 1):
            s = trial[row].tobytes()
            for j in range(8):
                assert oracle.q4k_scale_min(j, s) == (sc[row, j], mn[row, j])


def test_q4k_known_answer_blocks():
    # d = 1.0, dmin = 0, scales 1, mins 0: values are the nibbles themselves.
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[4:16] = pack_q4k_scales(np.ones((1, 8), np.uint8), np.zeros((1, 8), np.uint8))[0]
    q = np.arange(128, dtype=np.uint8)
    blk[16:] = q
    got = oracle.dequantize(Q4K, blk, 256)
    want = np.concatenate([np.concatenate([q[32 * p:32 * p + 32] & 0xF, q[32 * p:32 * p + 32] >> 4])
                           for p in range(4)]).astype(np.float32)
    assert bits_equal(got, want)
    # The reference's deterministic matmul blocks: d = dmin = 0.125, scales 0x11.
    w = matmul_q4k_weights(1, 256)
    got = oracle.dequantize(Q4K, w, 256)
    qb = w[16:144]
    for j in range(8):
        sc = 17 if j < 4 else 1
        nib = (qb[32 * (j // 2):32 * (j // 2) + 32] >> (4 * (j % 2))) & 0xF
        want = np.float32(0.125 * sc) * nib.astype(np.float32) - np.float32(0.125 * sc)
        assert bits_equal(got[32 * j:32 * j + 32], want.astype(np.float32))


def test_q4k_matches_independent_decoder():
    rng = np.random.default_rng(4)
    blocks = rng.integers(0, 256, (512, 144), dtype=np.uint8)
    blocks[:, 0:4] = rng.uniform(-0.02, 0.02, (512, 2)).astype(np.float16).view(np.uint8)
    assert bits_equal(oracle.dequantize(Q4K, blocks, 512 * 256), np_q4k(blocks))
    cfg = q4k_blocks(rng, 256)
    assert bits_equal(oracle.dequantize(Q4K, cfg, 256 * 256), np_q4k(cfg))


def test_q4k_reference_generator_blocks():
    """Blocks from the xorshift generator of metal_matvec.rs (seed :284)."""
    r = Random(0x9E3779B97F4A7C15)
    w = r.blocks(144 * 64, 144, [0, 2])
    assert bits_equal(oracle.dequantize(Q4K, w, 64 * 256), np_q4k(w))


@pytest.mark.parametrize("fmt,nbytes,ne,dec,scales", [
    (Q5K, 176, 256, np_q5k, [0, 2]),
    (Q6K, 210, 256, np_q6k, [208]),
    (Q8_0, 34, 32, np_q8_0, [0]),
    (Q4_0, 18, 32, np_q4_0, [0]),
])
def test_other_formats_match_independent_decoders(fmt, nbytes, ne, dec, scales):
    r = Random(0x60E7927B081DA5EF)
    w = r.blocks(nbytes * 40, nbytes, scales)
    assert bits_equal(oracle.dequantize(fmt, w, 40 * ne), dec(w))


# --------------------------------------------------------------------- #
# Vector ops
# --------------------------------------------------------------------- #
def test_matvec_matches_float64_brute_force():
    rng = np.random.default_rng(5)
    rows, cols = 37, 512
    w = rng.integers(0, 256, rows * cols // 256 * 144, dtype=np.uint8).reshape(-1, 144)
    w[:, 0:4] = rng.uniform(1e-3, 1e-2, (w.shape[0], 2)).astype(np.float16).view(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    dense = np_q4k(w).reshape(rows, cols).astype(np.float64)
    want = (dense @ x.astype(np.float64)).astype(np.float32)
    for threads in (1, 3):
        oracle.set_threads(threads)
        got = oracle.matvec(Q4K, w, rows, cols, x)
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    oracle.set_threads(1)
    f = rng.standard_normal((rows, cols)).astype(np.float32)
    got = oracle.matvec(F32, f, rows, cols, x)
    np.testing.assert_allclose(got, (f.astype(np.float64) @ x).astype(np.float32), rtol=1e-6)


def test_rms_norm_closed_form():
    x = np.full(64, 3.0, np.float32)
    w = np.full(64, 2.0, np.float32)
    # mean(x²) = 9 -> scale = 1/sqrt(9 + eps) ~ 1/3
    np.testing.assert_allclose(oracle.rms_norm(x, w, 0.0), np.full(64, 2.0), rtol=1e-7)
    rng = np.random.default_rng(6)
    x = rng.standard_normal(300).astype(np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    s = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-5), w * (x * np.float32(s)), rtol=1e-6)


def test_rope_properties():
    rng = np.random.default_rng(7)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    assert np.array_equal(oracle.rope_neox(q, 0, 1e6), q)
    r = oracle.rope_neox(q, 123, 1e6)
    pair = lambda v: np.hypot(v[:32], v[32:])
    np.testing.assert_allclose(pair(r), pair(q), rtol=1e-5)
    # Scores depend only on the relative position.
    a = oracle.dot(oracle.rope_neox(q, 10, 1e4), oracle.rope_neox(k, 7, 1e4))
    b = oracle.dot(oracle.rope_neox(q, 503, 1e4), oracle.rope_neox(k, 500, 1e4))
    assert abs(a - b) < 1e-3 * (np.abs(q).sum() + 1)
    # Element 0 pairs with element 32 and turns by exactly pos radians.
    e = np.zeros(64, np.float32)
    e[0] = 1.0
    r = oracle.rope_neox(e, 2, 1e6)
    np.testing.assert_allclose([r[0], r[32]], [np.cos(2.0), np.sin(2.0)], rtol=1e-6)


def test_softmax_and_silu_closed_forms():
    np.testing.assert_allclose(oracle.softmax(np.array([0.0, np.log(2.0)], np.float32)),
                               [1 / 3, 2 / 3], rtol=1e-6)
    rng = np.random.default_rng(8)
    x = rng.standard_normal(100).astype(np.float32) * 10
    p = oracle.softmax(x)
    assert abs(p.astype(np.float64).sum() - 1) < 1e-6
    np.testing.assert_allclose(oracle.softmax(x + 5.0), p, rtol=1e-5)
    assert oracle.silu(0.0) == 0.0
    for v in (-3.0, -0.5, 0.7, 4.0):
        assert abs((oracle.silu(v) - oracle.silu(-v)) - v) < 1e-6
    assert abs(oracle.silu(50.0) - 50.0) < 1e-6


def test_route_brute_force():
    rng = np.random.default_rng(9)
    for _ in range(50):
        logits = rng.standard_normal(32).astype(np.float32)
        bias = (rng.standard_normal(32) * 0.1).astype(np.float32)
        # A few exact ties exercise the lower-index rule.
        logits[5] = logits[9]
        bias[5] = bias[9]
        w, experts = oracle.route(logits, bias, 4)
        sig = 1 / (1 + np.exp(-logits.astype(np.float32)))
        key = sig + bias
        order = sorted(range(32), key=lambda e: (-key[e], e))
        assert experts[:4] == order[:4]
        norm = sig[order[:4]].sum() + 1e-6
        np.testing.assert_allclose(w[order[:4]], sig[order[:4]] / norm, rtol=1e-5)


# --- Sampler::sample (crates/bobcat-cli/src/sampler.rs:75-111) with the draw given ---
#
# Cases whose answers the mathematics fixes, each chosen so that a plausible
# slip fails: the top-p cut (`position(cumulative >= top_p) + 1`), the min-p
# floor relative to the first candidate, the temperature applied to the log
# probabilities, and the draw walking the kept candidates.

SAMPLE_P = np.log(np.array([0.5, 0.3, 0.2], np.float32))


def st(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, penalty=1.0):
    return oracle.Sampling(temperature, top_k, top_p, min_p, penalty)


def test_sample_top_p_keeps_the_prefix_and_renormalises():
    # p = [0.5, 0.3, 0.2]; top_p 0.75 keeps two, renormalised to [0.625, 0.375].
    s = st(top_p=0.75)
    assert [oracle.sample_u(SAMPLE_P, [], s, u) for u in (0.0, 0.62, 0.63, 0.999)] == [0, 0, 1, 1]


def test_sample_temperature_squares_at_one_half():
    # T = 0.5 on log-probabilities: q ∝ p² = [0.25, 0.09, 0.04] / 0.38.
    s = st(temperature=0.5)
    q0, q01 = 0.25 / 0.38, 0.34 / 0.38  # 0.65789..., 0.89473...
    cases = [(q0 - 1e-3, 0), (q0 + 1e-3, 1), (q01 - 1e-3, 1), (q01 + 1e-3, 2)]
    assert [oracle.sample_u(SAMPLE_P, [], s, u) for u, _ in cases] == [t for _, t in cases]


def test_sample_min_p_drops_below_the_floor():
    # min_p 0.5: floor 0.25 drops p = 0.2 and keeps 0.3; kept mass renormalised to [0.625, 0.375].
    s = st(min_p=0.5)
    assert [oracle.sample_u(SAMPLE_P, [], s, u) for u in (0.62, 0.63, 0.999)] == [0, 1, 1]


def test_sample_top_p_equal_to_a_cumulative_sum():
    # Four equal logits: p = 0.25 each, exact in float32, cumulative 0.5 after two.
    # `>=` with `+ 1` keeps two ([0.5, 0.5]); `>` would keep three and `+ 0` one.
    # (Equal logits keep the lowest ids first here; sort_unstable in the
    # reference leaves their order open, but not how many are kept.)
    lg = np.zeros(4, np.float32)
    s = st(top_p=0.5)
    assert oracle.sample_u(lg, [], s, 0.45) == 0
    assert oracle.sample_u(lg, [], s, 0.70) == 1  # three kept would give id 2, one kept id 0
    assert oracle.sample_u(lg, [], s, 0.999) == 1


def test_sample_top_k_then_penalty_order():
    # Penalty first (3.0 -> 1.5 for a positive logit), then top-k 1 keeps the new largest.
    lg = np.array([0.1, 3.0, 2.0], np.float32)
    assert oracle.sample_u(lg, [1], st(top_k=1, penalty=2.0), 0.9) == 2
    # A negative logit is multiplied: -1 -> -2 falls below -1.5.
    lg = np.array([-1.5, -1.0], np.float32)
    assert oracle.sample_u(lg, [1, 1, 1], st(top_k=1, penalty=2.0), 0.5) == 0


def test_generator_invariants():
    # The state advances by the wyrand increment on every draw (mod 2^64);
    # temperature 0 draws nothing.
    c0 = 0x2D358DCCAA6C78A5
    seed = 12345
    state = seed
    lg = np.array([1.0, 0.5, 0.2], np.float32)
    for n in range(1, 6):
        _, state = oracle.sample(lg, [], st(), state)
        assert state == (seed + n * c0) % (1 << 64)
    _, after = oracle.sample(lg, [], st(temperature=0.0), state)
    assert after == state
    # Rng::f32 maps a 32-bit draw's 23 high bits into [0, 1).
    assert oracle.u32_to_f32(0) == 0.0
    assert oracle.u32_to_f32(0x80000000) == 0.5
    assert oracle.u32_to_f32(0xFFFFFFFF) == 1.0 - 2.0 ** -23
    assert oracle.u32_to_f32(0x1FF) == 0.0  # the low 9 bits do not reach the mantissa
