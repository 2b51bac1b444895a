"""GPU parity of the MFMA prefill attention (bch_attention_prefill) against a
float64 restatement of causal GQA softmax attention and against the
reference-shaped bch_attention path.

Inputs follow crates/bobcat/tests/metal_attention.rs:19-48 (the q/k/v
formulas (i·19%97−48)/67, (i·29%83−41)/53, (i·31%83−41)/53 over an f16
cache) on the reference's shapes that this kernel takes (f16 cache, heads of
64, 128 or 256, ≤ 4 query heads per KV head) plus prefill-sized batches.  The
queries and probabilities enter the MFMA products as f16 high + low parts
(~22 bits), so the bound is 1e-5 absolute (outputs are below 1 in
magnitude) instead of the op-level kernel's 1e-6.
"""
from __future__ import annotations

import numpy as np
import pytest

from bobcat_amd import BobcatError
from bobcat_amd.backend import attention_scratch_floats

pytestmark = pytest.mark.gpu

ATTENTION_LIMITS = 9
CASES = [(63, 7, 4, 2, 64), (64, 73, 4, 1, 128), (63, 70, 4, 2, 64), (0, 512, 32, 8, 64), (100, 200, 16, 4, 128),
         (37, 1, 4, 1, 64), (0, 33, 8, 8, 64), (5, 70, 8, 2, 256), (0, 130, 8, 2, 256)]


def run(hip, fn):
    hip.begin()
    fn()
    hip.end()


def inputs(first, queries, heads, kv_heads, dim):
    keys = first + queries
    q_dim, kv_dim = heads * dim, kv_heads * dim
    i = np.arange(queries * q_dim)
    q = (((i * 19) % 97 - 48) / 67.0).astype(np.float32)
    j = np.arange(keys * kv_dim)
    k = (((j * 29) % 83 - 41) / 53.0).astype(np.float16)
    v = (((j * 31) % 83 - 41) / 53.0).astype(np.float16)
    return q, k, v


def reference(q, k, v, first, queries, heads, kv_heads, dim):
    keys = first + queries
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(dim)))
    group = heads // kv_heads
    K = k.astype(np.float64).reshape(keys, kv_heads, dim)
    V = v.astype(np.float64).reshape(keys, kv_heads, dim)
    Q = q.astype(np.float64).reshape(queries, heads, dim)
    want = np.empty((queries, heads, dim))
    for h in range(heads):
        Kh, Vh = K[:, h // group], V[:, h // group]
        S = Q[:, h] @ Kh.T * scale                                 # [queries, keys]
        mask = np.arange(keys)[None, :] > (first + np.arange(queries))[:, None]
        S[mask] = -np.inf
        P = np.exp(S - S.max(axis=1, keepdims=True))
        want[:, h] = (P / P.sum(axis=1, keepdims=True)) @ Vh
    return want.reshape(-1)


@pytest.mark.parametrize("first,queries,heads,kv_heads,dim", CASES)
def test_attention_prefill_matches_float64(hip, first, queries, heads, kv_heads, dim):
    q, k, v = inputs(first, queries, heads, kv_heads, dim)
    context = first + queries + 5
    qb, kb, vb = hip.buffer_from(q), hip.buffer_from(k), hip.buffer_from(v)
    out = hip.new_buffer(q.nbytes)
    print(f"attention_prefill first={first} queries={queries} heads={heads}/{kv_heads} dim={dim}", flush=True)
    run(hip, lambda: hip.attention_prefill(qb.at(0), kb.at(0), vb.at(0), out.at(0), heads, kv_heads, dim, first,
                                           queries, context))
    got = hip.read(out.at(0), np.empty(q.size, np.float32))
    want = reference(q, k, v, first, queries, heads, kv_heads, dim)
    assert np.abs(got - want).max() < 1e-5

    # The op-level kernel on the same inputs (metal_attention.rs's 1e-6 path).
    sb = hip.new_buffer(attention_scratch_floats(heads, dim, context, queries) * 4)
    tiled = hip.new_buffer(q.nbytes)
    run(hip, lambda: hip.attention(qb.at(0), kb.at(0), vb.at(0), True, sb.at(0), tiled.at(0), heads, kv_heads, dim,
                                   first, queries, context))
    other = hip.read(tiled.at(0), np.empty(q.size, np.float32))
    assert np.abs(got - other).max() < 1e-5


def test_attention_prefill_limits(hip):
    b = hip.new_buffer(1 << 20)
    for heads, kv_heads, dim in [(4, 1, 512), (10, 2, 64), (8, 1, 64), (4, 1, 32)]:
        hip.begin()
        with pytest.raises(BobcatError) as e:
            hip.attention_prefill(b.at(0), b.at(0), b.at(0), b.at(0), heads, kv_heads, dim, 0, 1, 16)
        hip.discard()
        assert e.value.status == ATTENTION_LIMITS
