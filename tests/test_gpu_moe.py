"""GPU parity of the mixture-of-experts kernels (moe_route, matvec_experts_swiglu,
matvec_experts_down) against the oracle.

The reference's own MoE checks compare the routed block with the CPU
`Model::moe_block` (crates/bobcat/src/lfm2.rs:413-440) through the model
tests; here each op is checked on its own:
  * the route: the oracle's `route` (lfm2.rs:691-709, pinned by brute force
    and by transformers' Lfm2MoeForCausalLM) applied to float64 router
    logits — the picked experts must be identical unless two biased scores
    are within 1e-5 of each other, and the weights within 1e-5;
  * the fused RMS norm of the route launch against `orc_rms_norm` (1e-6);
  * the expert SwiGLU rows and the weighted expert down-sum against the
    oracle's dequantised matrices in float64, within 1e-5 of the row
    term-scale (the GEMV contract of metal_matvec.rs:16-19);
  * the reference's limits (n_experts <= 128, 1 <= n_used <= 8,
    backend.rs:2728-2734) as ExpertLimits errors.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd import BobcatError
from bobcat_amd.backend import Format, NormSpec
from bobcat_amd.synth import q4k_matrix
from tests.test_gpu_ops import half_inputs

pytestmark = pytest.mark.gpu

EXPERT_LIMITS = 12


def run(hip, fn):
    hip.begin()
    fn()
    hip.end()


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


@pytest.mark.parametrize("n_experts,n_used,n_cols,n_tokens,fused", [
    (32, 4, 2048, 1, True), (32, 4, 2048, 7, False), (8, 2, 256, 3, True), (128, 8, 1024, 2, True),
    (5, 5, 512, 1, False)])
def test_moe_route_matches_oracle(hip, n_experts, n_used, n_cols, n_tokens, fused):
    rng = np.random.default_rng(n_experts * 131 + n_used)
    x = (rng.standard_normal(n_tokens * n_cols) * 2).astype(np.float32)
    router = (rng.standard_normal(n_experts * n_cols) / np.sqrt(n_cols)).astype(np.float32)
    bias = rng.uniform(-0.05, 0.05, n_experts).astype(np.float32)
    nw = (1 + 0.2 * rng.uniform(-1, 1, n_cols)).astype(np.float32)
    xb, rb, bb, wb = hip.buffer_from(x), hip.buffer_from(router), hip.buffer_from(bias), hip.buffer_from(nw)
    nb = hip.new_buffer(n_tokens * n_cols * 4)
    route = hip.new_buffer(2 * n_used * n_tokens * 4)
    norm = NormSpec(wb.at(0), 1e-5) if fused else None
    run(hip, lambda: hip.moe_route(xb.at(0), norm, nb.at(0), rb.at(0), bb.at(0), route.at(0), n_cols, n_experts,
                                   n_used, n_tokens))
    got = hip.read(route.at(0), np.empty(2 * n_used * n_tokens, np.uint32)).reshape(n_tokens, 2 * n_used)
    normed = hip.read(nb.at(0), np.empty(n_tokens * n_cols, np.float32)) if fused else None
    R = router.reshape(n_experts, n_cols).astype(np.float64)
    for t in range(n_tokens):
        xt = x[t * n_cols:(t + 1) * n_cols]
        if fused:
            xt = oracle.rms_norm(xt, nw, 1e-5)
            m = np.abs(xt).max()
            assert np.abs(normed[t * n_cols:(t + 1) * n_cols] - xt).max() <= 1e-6 * m
        logits = (R @ xt.astype(np.float64)).astype(np.float32)
        weights, order = oracle.route(logits, bias, n_used)
        ids = got[t, :n_used].tolist()
        w = got[t, n_used:].view(np.float32)
        biased = sigmoid(logits.astype(np.float64)) + bias
        gaps = np.diff(np.sort(biased)[::-1])
        if ids != order[:n_used]:
            # Only a near-tie at the boundary may pick differently.
            assert np.abs(gaps).min() < 1e-5, (t, ids, order[:n_used])
            continue
        assert np.abs(w - np.array([weights[e] for e in ids])).max() < 1e-5, t


def expert_case(rng, n_experts, rows, cols):
    return q4k_matrix(rng, n_experts * rows, cols)


def dense(w, rows, cols):
    return oracle.dequantize(int(Format.Q4K), w, rows * cols).reshape(rows, cols).astype(np.float64)


@pytest.mark.parametrize("n_experts,n_used,n_ff,n_embd", [(8, 2, 256, 256), (32, 4, 1792, 2048), (4, 4, 512, 1024)])
def test_experts_swiglu_and_down_match_oracle(hip, n_experts, n_used, n_ff, n_embd):
    rng = np.random.default_rng(n_ff + n_embd)
    gate = expert_case(rng, n_experts, n_ff, n_embd)
    up = expert_case(rng, n_experts, n_ff, n_embd)
    down = expert_case(rng, n_experts, n_embd, n_ff)
    x = rng.standard_normal(n_embd).astype(np.float32)
    ids = rng.choice(n_experts, n_used, replace=False).astype(np.uint32)
    wts = rng.uniform(0.05, 0.5, n_used).astype(np.float32)
    route_np = np.concatenate([ids, wts.view(np.uint32)])
    gb, ub, db = hip.buffer_from(gate), hip.buffer_from(up), hip.buffer_from(down)
    xb, rtb = hip.buffer_from(x), hip.buffer_from(route_np)
    yb = hip.new_buffer(n_used * n_ff * 4)
    run(hip, lambda: hip.matvec_experts_swiglu(Format.Q4K, gb.at(0), ub.at(0), n_ff, n_embd, n_experts, xb.at(0),
                                               rtb.at(0), n_used, yb.at(0), 1))
    got = hip.read(yb.at(0), np.empty(n_used * n_ff, np.float32)).reshape(n_used, n_ff)
    rb = n_embd // 256 * 144
    ffn = np.empty((n_used, n_ff), np.float32)
    for k, e in enumerate(ids):
        G = dense(gate[e * n_ff * rb:(e + 1) * n_ff * rb], n_ff, n_embd)
        U = dense(up[e * n_ff * rb:(e + 1) * n_ff * rb], n_ff, n_embd)
        g, u = G @ x, U @ x
        silu = g / (1 + np.exp(-g))
        want = silu * u
        # Propagate the GEMV bound (1e-5 of each row's term-scale) through
        # silu(g)·u: |silu'| <= 1.1.
        sg, su = np.abs(G) @ np.abs(x), np.abs(U) @ np.abs(x)
        bound = 1e-5 * (1.1 * sg * np.abs(u) + np.abs(silu) * su) + 1e-30
        assert (np.abs(got[k] - want) <= bound).all(), (k, (np.abs(got[k] - want) / bound).max())
        ffn[k] = want.astype(np.float32)

    # The down projections of those rows, weighted and added to a residual.
    resid = rng.standard_normal(n_embd).astype(np.float32)
    fb, hb = hip.buffer_from(ffn), hip.buffer_from(resid)
    run(hip, lambda: hip.matvec_experts_down(Format.Q4K, db.at(0), n_embd, n_ff, n_experts, fb.at(0), rtb.at(0),
                                             n_used, hb.at(0), 1))
    got = hip.read(hb.at(0), np.empty(n_embd, np.float32))
    rbd = n_ff // 256 * 144
    want = resid.astype(np.float64).copy()
    scale = np.zeros(n_embd)
    for k, e in enumerate(ids):
        D = dense(down[e * n_embd * rbd:(e + 1) * n_embd * rbd], n_embd, n_ff)
        want += float(wts[k]) * (D @ ffn[k].astype(np.float64))
        scale += float(wts[k]) * (np.abs(D) @ np.abs(ffn[k].astype(np.float64)))
    assert np.abs(got - want).max() / max(scale.max(), np.abs(resid).max()) < 1e-5


def test_expert_limits(hip):
    x = hip.new_buffer(256 * 4)
    route = hip.new_buffer(64 * 4)
    router = hip.new_buffer(200 * 256 * 4)
    for n_experts, n_used in [(129, 4), (32, 9), (32, 0), (4, 5)]:
        hip.begin()
        with pytest.raises(BobcatError) as e:
            hip.moe_route(x.at(0), None, None, router.at(0), x.at(0), route.at(0), 256, n_experts, n_used, 1)
        hip.discard()
        assert e.value.status == EXPERT_LIMITS


@pytest.mark.parametrize("n_experts,n_used,n_ff,n_embd,n_tokens", [
    (32, 4, 1792, 2048, 300), (8, 2, 256, 512, 65), (4, 4, 512, 256, 1), (128, 8, 256, 256, 40)])
def test_grouped_experts_match_oracle(hip, n_experts, n_used, n_ff, n_embd, n_tokens):
    """The batched (prefill) path of lfm2_metal.rs:1317-1380: moe_group's
    grouping (expert by expert, token order within), matmul_experts (SwiGLU
    with shared token inputs, then down on the entries' rows) and moe_combine
    (slots summed in route order, then added).  Weights round to half in the
    MFMA tiles as the reference's expanded half tiles do, and each input row
    rounds to half after a power-of-two scaling (the reference's expert tiles
    take half inputs, matmul.metal:509-518), so the products are compared
    with half-rounded weights and inputs in float64, within 1e-5 of each
    row's term-scale."""
    rng = np.random.default_rng(n_experts * 7 + n_tokens)
    gate = expert_case(rng, n_experts, n_ff, n_embd)
    up = expert_case(rng, n_experts, n_ff, n_embd)
    down = expert_case(rng, n_experts, n_embd, n_ff)
    x = rng.standard_normal((n_tokens, n_embd)).astype(np.float32)
    ids = np.stack([rng.choice(n_experts, n_used, replace=False) for _ in range(n_tokens)]).astype(np.uint32)
    wts = rng.uniform(0.05, 0.5, (n_tokens, n_used)).astype(np.float32)
    route_np = np.concatenate([ids, wts.view(np.uint32)], axis=1).reshape(-1)
    n_entries = n_tokens * n_used

    rtb = hip.buffer_from(route_np)
    offb, entb = hip.new_buffer((n_experts + 1) * 4), hip.new_buffer(n_entries * 4)
    run(hip, lambda: hip.moe_group(rtb.at(0), offb.at(0), entb.at(0), n_experts, n_used, n_tokens))
    offsets = hip.read(offb.at(0), np.empty(n_experts + 1, np.uint32))
    entries = hip.read(entb.at(0), np.empty(n_entries, np.uint32))
    flat = ids.reshape(-1)
    want_entries = np.concatenate([np.nonzero(flat == e)[0] for e in range(n_experts)]).astype(np.uint32)
    want_offsets = np.concatenate([[0], np.cumsum([(flat == e).sum() for e in range(n_experts)])]).astype(np.uint32)
    assert (offsets == want_offsets).all() and (entries == want_entries).all()

    gb, ub, db, xb = hip.buffer_from(gate), hip.buffer_from(up), hip.buffer_from(down), hip.buffer_from(x)
    ffb, outb = hip.new_buffer(n_entries * n_ff * 4), hip.new_buffer(n_entries * n_embd * 4)
    run(hip, lambda: hip.matmul_experts(Format.Q4K, gb.at(0), ub.at(0), n_ff, n_embd, n_experts, xb.at(0), True,
                                        offb.at(0), entb.at(0), n_used, ffb.at(0), n_tokens))
    ffn = hip.read(ffb.at(0), np.empty(n_entries * n_ff, np.float32)).reshape(n_entries, n_ff)
    rb, rbd = n_embd // 256 * 144, n_ff // 256 * 144

    def half_dense(w, e, rows, cols, row_bytes):
        return dense(w[e * rows * row_bytes:(e + 1) * rows * row_bytes], rows, cols).astype(np.float16) \
            .astype(np.float64)

    used = sorted(set(flat.tolist()))
    xh = half_inputs(x)
    for e in used:
        G, U = half_dense(gate, e, n_ff, n_embd, rb), half_dense(up, e, n_ff, n_embd, rb)
        for v in np.nonzero(flat == e)[0]:
            xv = xh[v // n_used]
            g, u = G @ xv, U @ xv
            silu = g / (1 + np.exp(-g))
            sg, su = np.abs(G) @ np.abs(xv), np.abs(U) @ np.abs(xv)
            bound = 1e-5 * (1.1 * sg * np.abs(u) + np.abs(silu) * su) + 1e-30
            assert (np.abs(ffn[v] - silu * u) <= bound).all(), (e, v, (np.abs(ffn[v] - silu * u) / bound).max())

    run(hip, lambda: hip.matmul_experts(Format.Q4K, db.at(0), None, n_embd, n_ff, n_experts, ffb.at(0), False,
                                        offb.at(0), entb.at(0), n_used, outb.at(0), n_tokens))
    out = hip.read(outb.at(0), np.empty(n_entries * n_embd, np.float32)).reshape(n_entries, n_embd)
    fh = half_inputs(ffn)
    for e in used:
        D = half_dense(down, e, n_embd, n_ff, rbd)
        for v in np.nonzero(flat == e)[0]:
            fv = fh[v]
            want, scale = D @ fv, np.abs(D) @ np.abs(fv)
            assert np.abs(out[v] - want).max() <= 1e-5 * scale.max() + 1e-30, (e, v)

    resid = rng.standard_normal((n_tokens, n_embd)).astype(np.float32)
    hb = hip.buffer_from(resid)
    run(hip, lambda: hip.moe_combine(outb.at(0), rtb.at(0), hb.at(0), n_embd, n_used, n_tokens))
    got = hip.read(hb.at(0), np.empty(n_tokens * n_embd, np.float32)).reshape(n_tokens, n_embd)
    want = resid.copy()
    for t in range(n_tokens):
        acc = np.zeros(n_embd, np.float32)
        for s in range(n_used):
            acc = acc + wts[t, s] * out[t * n_used + s]
        want[t] = resid[t] + acc
    assert np.abs(got - want).max() <= 1e-6 * max(1.0, float(np.abs(want).max()))
