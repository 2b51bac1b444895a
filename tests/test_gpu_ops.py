"""GPU parity of the element-wise, normalisation, attention, convolution and
prefill-GEMM kernels against the oracle.

Follows crates/bobcat/tests/metal_attention.rs (7 shape cases, f16 and f32
caches, batched == single-query within 1e-6, double-precision reference
within 1e-6 absolute), metal_matmul.rs (deterministic blocks, 1e-4 relative
to the largest output, every store mode) and the conv/norm checks of
metal_gdn.rs's tolerance style (1e-5 relative).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd.backend import Format, Store, attention_scratch_floats
from bobcat_amd.synth import q4k_matrix
from tests._gen import Random, matmul_inputs, matmul_q4k_weights

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    d = np.abs(got - want)
    if np.isnan(d).any():
        return float("inf")
    m = np.abs(want).max()
    return float(d.max() / m) if m > 0 else float(d.max())


def run(hip, fn):
    hip.begin()
    fn()
    hip.end()


def test_rms_norm(hip):
    rnd = Random(7)
    n, rows = 2048, 5
    x = rnd.units(n * rows) * 3
    w = 1 + 0.5 * rnd.units(n)
    xb, wb, ob = hip.buffer_from(x), hip.buffer_from(w), hip.new_buffer(n * rows * 4)
    run(hip, lambda: hip.rms_norm(xb.at(0), wb.at(0), ob.at(0), n, rows, 1e-5))
    got = hip.read(ob.at(0), np.empty(n * rows, np.float32))
    want = np.concatenate([oracle.rms_norm(x[r * n:(r + 1) * n], w, 1e-5) for r in range(rows)])
    assert rel_err(got, want) < 1e-6


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("head_dim,n_rot,src_head_stride", [(64, 64, 64), (256, 64, 512), (128, 128, 128)])
def test_norm_rope(hip, half, head_dim, n_rot, src_head_stride):
    rnd = Random(11)
    n_heads, n_tokens, pos = 4, 3, 1000
    src_stride = n_heads * src_head_stride
    src = rnd.units(n_tokens * src_stride) * 2
    w = 1 + 0.5 * rnd.units(head_dim)
    dst_stride = n_heads * head_dim
    sb, wb = hip.buffer_from(src), hip.buffer_from(w)
    db = hip.new_buffer(n_tokens * dst_stride * (2 if half else 4))
    run(hip, lambda: hip.norm_rope(sb.at(0), db.at(0), half, wb.at(0), n_heads, head_dim, n_rot,
                                   src_head_stride, pos, n_tokens, src_stride, dst_stride, 1e6, 1e-5))
    got = hip.read(db.at(0), np.empty(n_tokens * dst_stride, np.float16 if half else np.float32))
    want = np.empty(n_tokens * dst_stride, np.float32)
    for t in range(n_tokens):
        for h in range(n_heads):
            s = src[t * src_stride + h * src_head_stride:][:head_dim]
            v = oracle.rms_norm(s, w, 1e-5)
            v[:n_rot] = oracle.rope_neox(v[:n_rot], pos + t, 1e6)
            want[t * dst_stride + h * head_dim:][:head_dim] = v
    if half:
        # Each element rounds to half once; compare in half precision.
        assert np.abs(got.astype(np.float32) - want).max() <= 2 ** -10 * np.abs(want).max()
    else:
        assert rel_err(got, want) < 1e-5


def test_convert_half_is_bit_exact(hip):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(10000) * 10.0 ** rng.integers(-6, 4, 10000)).astype(np.float32)
    xb, ob = hip.buffer_from(x), hip.new_buffer(x.size * 2)
    run(hip, lambda: hip.convert_half(xb.at(0), ob.at(0), x.size))
    got = hip.read(ob.at(0), np.empty(x.size, np.uint16))
    want = np.array([oracle.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt", [Format.Q4K, Format.F16, Format.F32])
def test_embed_is_bit_exact(hip, fmt):
    rng = np.random.default_rng(4)
    n_vocab, n_embd = 300, 1024
    if fmt == Format.Q4K:
        w = q4k_matrix(rng, n_vocab, n_embd)
    else:
        w = rng.standard_normal(n_vocab * n_embd).astype(np.float16 if fmt == Format.F16 else np.float32).view(np.uint8)
    tokens = np.array([5, 299, 0, 17, 5], np.uint32)
    wb, tb, ob = hip.buffer_from(w), hip.buffer_from(tokens), hip.new_buffer(tokens.size * n_embd * 4)
    run(hip, lambda: hip.embed(fmt, wb.at(0), n_vocab, tb.at(0), ob.at(0), n_embd, tokens.size))
    got = hip.read(ob.at(0), np.empty(tokens.size * n_embd, np.float32))
    rb = w.size // n_vocab
    want = np.concatenate([oracle.dequantize(int(fmt), w[t * rb:(t + 1) * rb], n_embd) for t in tokens])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_argmax_ties_go_to_lowest_index(hip):
    rng = np.random.default_rng(5)
    for n in (1, 7, 1024, 65536, 151936):
        x = rng.standard_normal(n).astype(np.float32)
        if n > 10:
            x[n // 3] = x[n // 2] = x[-1] = x.max() + 1  # three-way tie
        xb, ob = hip.buffer_from(x), hip.new_buffer(4)
        run(hip, lambda: hip.argmax(xb.at(0), ob.at(0), n))
        got = int(hip.read(ob.at(0), np.empty(1, np.uint32))[0])
        assert got == int(np.argmax(x)), (n, got)


@pytest.mark.parametrize("batch", [False, True])
def test_short_conv(hip, batch):
    """Carried history across calls of 1, 2, 7, 1, 64 and 3 tokens."""
    rnd = Random(13)
    n_embd, k = 1024, 3
    taps = rnd.units(n_embd * k)
    hist = np.zeros((k - 1) * n_embd, np.float32)
    tb, hb = hip.buffer_from(taps), hip.buffer_from(hist)
    for n_tok in (1, 2, 7, 1, 64, 3):
        bcx = rnd.units(n_tok * 3 * n_embd) if n_tok < 8 else \
            np.random.default_rng(n_tok).uniform(-1, 1, n_tok * 3 * n_embd).astype(np.float32)
        bb, ob = hip.buffer_from(bcx), hip.new_buffer(n_tok * n_embd * 4)
        if batch:
            run(hip, lambda: hip.short_conv_batch(bb.at(0), tb.at(0), hb.at(0), ob.at(0), n_embd, k, n_tok))
        else:
            run(hip, lambda: hip.short_conv(bb.at(0), tb.at(0), hb.at(0), ob.at(0), n_embd, k, n_tok))
        got = hip.read(ob.at(0), np.empty(n_tok * n_embd, np.float32))
        want, hist = oracle.short_conv(bcx, taps, hist, n_embd, k, n_tok)
        assert rel_err(got, want) < 1e-5
        got_hist = hip.read(hb.at(0), np.empty(hist.size, np.float32))
        assert np.array_equal(got_hist, hist)


ATTENTION_CASES = [(0, 7, 4, 1, 32), (63, 7, 4, 2, 64), (64, 73, 4, 1, 128), (63, 70, 4, 2, 64),
                   (129, 5, 2, 2, 32), (63, 9, 8, 2, 256), (65, 70, 8, 2, 256)]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("first,queries,heads,kv_heads,dim", ATTENTION_CASES)
def test_attention(hip, half, first, queries, heads, kv_heads, dim):
    """metal_attention.rs:11-160 restated."""
    keys = first + queries
    context = keys + 67
    q_dim, kv_dim = heads * dim, kv_heads * dim
    i = np.arange(queries * q_dim)
    q = (((i * 19) % 97 - 48) / 67.0).astype(np.float32)
    j = np.arange(keys * kv_dim)
    k = (((j * 29) % 83 - 41) / 53.0).astype(np.float32)
    v = (((j * 31) % 83 - 41) / 53.0).astype(np.float32)
    if half:
        k, v = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
        kb, vb = hip.buffer_from(k.astype(np.float16)), hip.buffer_from(v.astype(np.float16))
    else:
        kb, vb = hip.buffer_from(k), hip.buffer_from(v)
    qb = hip.buffer_from(q)
    sb = hip.new_buffer(attention_scratch_floats(heads, dim, context, queries) * 4)
    tiled, separate = hip.new_buffer(q.nbytes), hip.new_buffer(q.nbytes)
    run(hip, lambda: hip.attention(qb.at(0), kb.at(0), vb.at(0), half, sb.at(0), tiled.at(0), heads,
                                   kv_heads, dim, first, queries, context))
    for qi in range(queries):
        run(hip, lambda: hip.attention(qb.floats(qi * q_dim), kb.at(0), vb.at(0), half, sb.at(0),
                                       separate.floats(qi * q_dim), heads, kv_heads, dim, first + qi, 1,
                                       context))
    got = hip.read(tiled.at(0), np.empty(q.size, np.float32))
    single = hip.read(separate.at(0), np.empty(q.size, np.float32))
    assert np.abs(got - single).max() < 1e-6
    # Double-precision reference (metal_attention.rs:116-156), 1e-6 absolute.
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(dim)))
    group = heads // kv_heads
    K = k.reshape(keys, kv_heads, dim).astype(np.float64)
    V = v.reshape(keys, kv_heads, dim).astype(np.float64)
    Q = q.reshape(queries, heads, dim).astype(np.float64)
    want = np.empty((queries, heads, dim))
    for qi in range(queries):
        n = first + qi + 1
        for h in range(heads):
            s = K[:n, h // group] @ Q[qi, h] * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            want[qi, h] = p @ V[:n, h // group]
    assert np.abs(got - want.reshape(-1)).max() < 1e-6
    # And the oracle's own restatement of lfm2.rs:520-556.
    orc = oracle.attention(q, k, v, heads, kv_heads, dim, first, queries)
    assert np.abs(got - orc).max() < 1e-6


def matmul_check(hip, fmt, weights, n_rows, n_cols, n_tokens, store, tol, inputs=None):
    x = matmul_inputs(n_tokens, n_cols) if inputs is None else inputs
    prior = ((np.arange(n_tokens * n_rows) * 11 % 53 - 26) / 32.0).astype(np.float32)
    oracle.set_threads(8)
    want = prior.copy().reshape(n_tokens, n_rows)
    for t in range(n_tokens):
        prod = oracle.matvec(int(fmt), weights, n_rows, n_cols, x[t * n_cols:(t + 1) * n_cols])
        if store == Store.OVERWRITE:
            want[t] = prod
        elif store == Store.ACCUMULATE:
            want[t] += prod
        else:
            want[t] = np.array([oracle.silu(float(g)) for g in want[t]], np.float32) * prod
    wb, xb, yb = hip.buffer_from(weights), hip.buffer_from(x), hip.buffer_from(prior)
    run(hip, lambda: hip.matmul(fmt, wb.at(0), n_rows, n_cols, xb.at(0), yb.at(0), n_tokens, store))
    got = hip.read(yb.at(0), np.empty(n_tokens * n_rows, np.float32))
    err = rel_err(got, want.reshape(-1))
    assert err < tol, (fmt, store, n_rows, n_cols, n_tokens, err)


@pytest.mark.parametrize("store", [Store.OVERWRITE, Store.ACCUMULATE, Store.SWIGLU])
@pytest.mark.parametrize("n_rows,n_cols,n_tokens", [(64, 256, 32), (70, 256, 33), (128, 512, 64),
                                                    (1024, 1024, 1), (192, 1024, 100)])
def test_matmul_deterministic_blocks(hip, store, n_rows, n_cols, n_tokens):
    """metal_matmul.rs:17-108: d = dmin = 0.125 and scale bytes 0x11 make every
    weight exact in half precision, so the 1e-4 bound holds as in the reference."""
    w = matmul_q4k_weights(n_rows, n_cols)
    matmul_check(hip, Format.Q4K, w, n_rows, n_cols, n_tokens, store, 1e-4)


def test_matmul_random_q4k(hip):
    """Random config-1 blocks: weights round to half in the tile (as the
    reference's expanded half tiles do), bounded by the 5e-3 half tolerance
    of lfm2_reference.rs:21-25 relative to the largest output."""
    rng = np.random.default_rng(9)
    n_rows, n_cols, n_tokens = 512, 2048, 77
    w = q4k_matrix(rng, n_rows, n_cols)
    x = rng.standard_normal(n_tokens * n_cols).astype(np.float32)
    matmul_check(hip, Format.Q4K, w, n_rows, n_cols, n_tokens, Store.OVERWRITE, 5e-3, inputs=x)


def half_inputs(x):
    """The prefill GEMM's inputs: each token scaled by the power of two that
    puts its largest magnitude in [2^13, 2^14), rounded to fp16, unscaled."""
    x = np.asarray(x, np.float32)
    mx = np.abs(x).max(axis=1, keepdims=True)
    _, ex = np.frexp(mx)
    scale = np.ldexp(1.0, np.clip(14 - ex, -100, 100)).astype(np.float32)
    scale[mx == 0] = 1.0
    return (x * scale).astype(np.float16).astype(np.float64) / scale


@pytest.mark.parametrize("fmt", [Format.Q4K, Format.Q6K, Format.Q8_0, Format.Q4_0, Format.Q5K])
def test_matmul_other_formats(hip, fmt):
    """The prefill GEMM on every block format of real files: each weight is
    the scalar path's dequantised value rounded to half (as the reference's
    expanded half tiles, lfm2_metal.rs:936-985) and each token's inputs are
    rounded to half after a power-of-two scaling, so the result equals the
    product of those two roundings within 1e-5 (fp32 accumulation), and the
    exact product within 5e-3."""
    from bobcat_amd.synth import block_matrix

    rng = np.random.default_rng(int(fmt))
    n_rows, n_cols, n_tokens = 200, 512, 45
    w = block_matrix(rng, int(fmt), n_rows, n_cols)
    x = rng.standard_normal((n_tokens, n_cols)).astype(np.float32)
    dense = oracle.dequantize(int(fmt), w, n_rows * n_cols).reshape(n_rows, n_cols)
    exact = x.astype(np.float64) @ dense.astype(np.float64).T
    halves = half_inputs(x) @ dense.astype(np.float16).astype(np.float64).T
    wb, xb, yb = hip.buffer_from(w), hip.buffer_from(x), hip.new_buffer(n_tokens * n_rows * 4)
    run(hip, lambda: hip.matmul(fmt, wb.at(0), n_rows, n_cols, xb.at(0), yb.at(0), n_tokens, Store.OVERWRITE))
    got = hip.read(yb.at(0), np.empty((n_tokens, n_rows), np.float32))
    scale = np.abs(exact).max()
    assert np.abs(got - halves).max() / scale < 1e-5
    assert np.abs(got - exact).max() / scale < 5e-3


@pytest.mark.parametrize("n_rows,n_cols,n_tokens", [(2048, 10752, 300), (10752, 2048, 512), (512, 2048, 512),
                                                    (6144, 2048, 200), (6144, 2048, 512), (64, 512, 129)])
@pytest.mark.parametrize("store", [Store.OVERWRITE, Store.ACCUMULATE, Store.SWIGLU])
def test_matmul_tiles_and_splits(hip, n_rows, n_cols, n_tokens, store):
    """Config-scale shapes through every tile choice (256- and 128-token
    tiles, 128-, 96- and 64-row tiles) and column split (up to 8 splits,
    added by the reduction), against the product of the half-rounded
    operands."""
    rng = np.random.default_rng(n_rows + n_tokens)
    w = q4k_matrix(rng, n_rows, n_cols)
    x = rng.standard_normal((n_tokens, n_cols)).astype(np.float32)
    dense = oracle.dequantize(int(Format.Q4K), w, n_rows * n_cols).reshape(n_rows, n_cols)
    prod = half_inputs(x) @ dense.astype(np.float16).astype(np.float64).T
    prior = rng.standard_normal((n_tokens, n_rows)).astype(np.float32)
    if store == Store.OVERWRITE:
        want = prod
    elif store == Store.ACCUMULATE:
        want = prior + prod
    else:
        want = prior / (1.0 + np.exp(-prior.astype(np.float64))) * prod
    wb, xb, yb = hip.buffer_from(w), hip.buffer_from(x), hip.buffer_from(prior)
    run(hip, lambda: hip.matmul(Format.Q4K, wb.at(0), n_rows, n_cols, xb.at(0), yb.at(0), n_tokens, store))
    got = hip.read(yb.at(0), np.empty((n_tokens, n_rows), np.float32))
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


def test_matmul_f16(hip):
    rng = np.random.default_rng(10)
    n_rows, n_cols, n_tokens = 96, 512, 40
    w = (rng.standard_normal(n_rows * n_cols) * 0.1).astype(np.float16).view(np.uint8)
    matmul_check(hip, Format.F16, w, n_rows, n_cols, n_tokens, Store.ACCUMULATE, 1e-4)


def test_matmul_inputs_beyond_half_range(hip):
    """Activations far outside fp16 range (a random-init model's residual
    stream reaches 1e8) must not overflow the half-precision input split."""
    rng = np.random.default_rng(12)
    n_rows, n_cols, n_tokens = 128, 512, 17
    w = q4k_matrix(rng, n_rows, n_cols)
    x = (rng.standard_normal(n_tokens * n_cols) * 10.0 ** rng.integers(-3, 9, n_tokens * n_cols)).astype(np.float32)
    matmul_check(hip, Format.Q4K, w, n_rows, n_cols, n_tokens, Store.OVERWRITE, 5e-3, inputs=x)
