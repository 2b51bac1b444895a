"""Benchmark: bobcat's per-token LM loop on one MI355X.

Prints ONE JSON line (the driver's contract).  Legs:
  * model — pp512/tg128 on a random-init LFM2-style model (default: the
            2.6B config of BASELINE.json configs[3], the north-star target).
            Protocol of bobcat-bench (docs/performance/eval.md:7-13,
            bobcat_bench.rs:91-173): 512 random prompt ids, then greedy
            tokens; prefill rate = 512 / TTFT (TTFT includes the first output
            token), decode rate = 127 / (t_last - t_first).  One "step" is one
            such round.  `value` is the decode rate over the timed rounds.
  * gemv  — BASELINE config 1: Q4_K dequant-GEMV, W [8192 x 2048], timed
            over 64 rotating copies of W (604 MB > the 256 MB MALL) with HIP
            events on the backend's own stream: the `roofline` object.
  * long  — BASELINE configs[3] part 2 (2.6B only): 128 greedy steps after a
            32,768-token prompt, and a second request that reuses the KV
            cache of a shared 30,000-token prefix: the `long_context` object.
  * models — the other BASELINE model configs (Qwen3.5-0.8B with a 16K-token
            prefill, LFM2-8B-A1B, LFM2-350M): pp512/tg128 each, in `models`.
  * cpu   — the oracle (a C restatement of the reference's scalar Rust path)
            decoding the same model on the host, on a bounded sample: one
            core (the reference's scalar path is single-threaded; `value`)
            and the host share of 16 threads, plus the config-1 GEMV.
Every model's greedy tokens are compared with the oracle's run of the same
seeded model and prompt (tests/golden/greedy_<model>.npz):
`greedy_matches_oracle`.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--model lfm2-2.6b]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
GEMV_ROWS, GEMV_COLS = 8192, 2048
GEMV_BYTES = GEMV_ROWS * GEMV_COLS // 256 * 144 + GEMV_COLS * 4 + GEMV_ROWS * 4  # 9,478,144
PROMPT, GEN = 512, 128
LONG_PROMPT, LONG_SHARED = 32768, 30000
READ_THREADS = 256 * 1024
COPY_BYTES = 64 << 20
ROOT = os.path.dirname(os.path.abspath(__file__))
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "matvec_q4k_config1_traffic.txt")


def measured_traffic():
    """HBM bytes per config-1 GEMV launch from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE scaled by the calibration launches), or
    None when there is none."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def host_threads() -> int:
    """Threads of the host share this process may use: OMP_NUM_THREADS when
    the environment sets the share (the GPU box does), else the CPUs this
    process may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return max(1, os.cpu_count() or 1)


def gemv_leg(hip, reps: int, copies: int = 64):
    from bobcat_amd.backend import Format
    from bobcat_amd.synth import gemv_case

    w, x = gemv_case()
    wbytes = w.nbytes
    big_bytes = wbytes * copies
    big = hip.new_buffer(big_bytes)
    for c in range(copies):
        hip.write(big.at(c * wbytes), w)
    xb = hip.buffer_from(x)
    yb = hip.new_buffer(GEMV_ROWS * 4)

    def run(n: int, rotate: bool = True) -> float:
        hip.begin()
        for i in range(n):
            off = (i % copies) * wbytes if rotate else 0
            hip.matvec(Format.Q4K, big.at(off), GEMV_ROWS, GEMV_COLS, xb.at(0), yb.at(0))
        return hip.end()

    run(copies)
    launches = reps * copies
    per_launch = run(launches) / launches
    hot = run(copies, rotate=False) / copies

    # Calibration launches of known traffic, for scaling the FETCH_SIZE and
    # WRITE_SIZE counters of a profiled run: read_sum reads all of `big`, copy
    # moves COPY_BYTES.
    sums = hip.new_buffer(READ_THREADS * 4)
    hip.begin()
    hip.read_sum(big.at(0), big_bytes // 16, sums.at(0), READ_THREADS)
    hip.end()
    dst = hip.new_buffer(COPY_BYTES)
    hip.begin()
    hip.copy(big.at(0), dst.at(0), COPY_BYTES // 4)
    hip.end()
    sums.free()
    dst.free()
    big.free()
    return dict(us=per_launch * 1e6, gbs=GEMV_BYTES / per_launch / 1e9, launches=launches,
                hot_us=hot * 1e6, hot_gbs=GEMV_BYTES / hot / 1e9)


def decode_gemv_leg(hip, reps: int = 8, budget: int = 640 << 20):
    """The slab GEMVs of one LFM2-2.6B decode token, each at its model shape,
    for per-kernel counters: the SwiGLU pair (10752 x 2048, RMS-normalised
    input), the down projection (2048 x 10752, accumulating), the conv layer's
    in_proj with its gated short convolution (6144 x 2048) and out_proj/wo
    (2048 x 2048, accumulating).  Each shape rotates over enough copies of
    its weights (together ~640 MB, beyond the 256 MB MALL) that every launch
    reads from HBM, as in the model.  Returns microseconds per launch."""
    from bobcat_amd.backend import Format, NormSpec
    from bobcat_amd.synth import q4k_matrix

    rng = np.random.default_rng(11)
    n = 2048
    x = hip.buffer_from(rng.standard_normal(10752).astype(np.float32))
    nw = hip.buffer_from((1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    y = hip.new_buffer(10752 * 4)
    taps = hip.buffer_from((0.1 * rng.standard_normal(3 * n)).astype(np.float32))
    hist = hip.new_buffer(2 * n * 4)
    conv_out = hip.new_buffer(n * 4)
    norm = NormSpec(nw.at(0), 1e-5)
    out = {}
    shapes = [("swiglu_10752x2048", 10752, 2048, 2), ("down_2048x10752", 2048, 10752, 1),
              ("conv_in_6144x2048", 6144, 2048, 1), ("out_proj_2048x2048", 2048, 2048, 1)]
    for name, rows, cols, mats in shapes:
        w = q4k_matrix(rng, rows, cols)
        copies = max(2, min(64, budget // (mats * w.nbytes)))
        big = hip.new_buffer(copies * mats * w.nbytes)
        for c in range(copies * mats):
            hip.write(big.at(c * w.nbytes), w)

        def launch(i):
            at = (i % copies) * mats * w.nbytes
            if name.startswith("swiglu"):
                hip.matvec_swiglu(Format.Q4K, big.at(at), big.at(at + w.nbytes), rows, cols, x.at(0), norm, y.at(0))
            elif name.startswith("conv"):
                hip.matvec_conv(Format.Q4K, big.at(at), cols, x.at(0), norm, taps.at(0), hist.at(0), conv_out.at(0),
                                n, 3)
            else:
                hip.matvec(Format.Q4K, big.at(at), rows, cols, x.at(0), y.at(0), accumulate=True)

        def run(k):
            hip.begin()
            for i in range(k):
                launch(i)
            return hip.end()

        run(copies)
        out[name] = round(run(reps * copies) / (reps * copies) * 1e6, 3)
        big.free()
    for b in (x, nw, y, taps, hist, conv_out):
        b.free()
    return out


def attn_decode_leg(hip, pos: int = LONG_PROMPT + 2, layers: int = 8, reps: int = 8):
    """The decode attention of one LFM2-2.6B attention layer at a 32K context
    (32 query heads over 8 KV heads of 64, f16 cache), through
    bch_attention_decode, for per-kernel counters: the q/k norm, RoPE and
    cache store of the new position, then attention over pos + 1 keys.
    `layers` distinct caches (67 MB each, together beyond the 256 MB MALL)
    are used in turn, as the model's layers are.  Returns microseconds per
    launch and the algorithmic rate (the K and V rows read once)."""
    from bobcat_amd.backend import attention_decode_scratch_floats

    heads, kv, hd, n_ctx = 32, 8, 64, LONG_PROMPT + GEN
    rng = np.random.default_rng(13)
    layer = n_ctx * kv * hd * 2
    cache = rng.standard_normal(n_ctx * kv * hd).astype(np.float16)
    kc = hip.new_buffer(layers * layer)
    vc = hip.new_buffer(layers * layer)
    for i in range(layers):
        hip.write(kc.at(i * layer), cache)
        hip.write(vc.at(i * layer), cache)
    q = hip.buffer_from(rng.standard_normal(heads * hd).astype(np.float32))
    k = hip.buffer_from(rng.standard_normal(kv * hd).astype(np.float32))
    v = hip.buffer_from(rng.standard_normal(kv * hd).astype(np.float32))
    qn = hip.buffer_from((1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    kn = hip.buffer_from((1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    sc = hip.new_buffer(attention_decode_scratch_floats(heads, hd, n_ctx, True) * 4)
    out = hip.new_buffer(heads * hd * 4)

    def run(n):
        hip.begin()
        for i in range(n):
            at = (i % layers) * layer
            hip.attention_decode(q.at(0), k.at(0), v.at(0), qn.at(0), kn.at(0), 1e-5, 1e6, hd, kc.at(at), vc.at(at),
                                 True, sc.at(0), out.at(0), heads, kv, hd, pos, n_ctx)
        return hip.end()

    run(layers)
    per = run(reps * layers) / (reps * layers)
    for b in (kc, vc, q, k, v, qn, kn, sc, out):
        b.free()
    kv_bytes = 2 * (pos + 1) * kv * hd * 2
    return dict(keys=pos + 1, us=round(per * 1e6, 3), kv_mb=round(kv_bytes / 1e6, 2),
                gbs=round(kv_bytes / per / 1e9, 1))


def oracle_tokens(name: str):
    """The oracle's 128 greedy tokens (and top-2 gaps) for the same seeded model
    and prompt, from the committed fixture tests/golden/greedy_<name>.npz
    (written on the CPU by tests/golden/make_greedy.py), or None."""
    path = os.path.join(ROOT, "tests", "golden", f"greedy_{name}.npz")
    if not os.path.exists(path):
        return None
    f = np.load(path)
    return f["tokens"].tolist(), f["gaps"].tolist()


def greedy_match(got, name: str):
    """(matches, identical_prefix): matches when the GPU's greedy tokens equal
    the oracle's, or first differ where the oracle's top-2 logits are within
    1e-3 (the north-star rule)."""
    ref = oracle_tokens(name)
    if ref is None:
        return None, None
    want, gaps = ref
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            return gaps[i] < 1e-3, i
    return True, min(len(got), len(want))


def model_leg(hip, weights, steps: int, warmup: int, seed: int = 42):
    from bobcat_amd.lfm2 import Lfm2Hip
    from bobcat_amd.qwen35 import Qwen35Hip, Qwen35Weights

    cfg = weights.cfg
    Lfm2Hip = Qwen35Hip if isinstance(weights, Qwen35Weights) else Lfm2Hip
    rng = np.random.default_rng(seed)  # the prompt of tests/golden/make_greedy.py
    prompt = rng.integers(0, cfg.n_vocab, PROMPT).astype(np.uint32)
    m = Lfm2Hip(hip, weights, n_ctx=PROMPT + GEN, kv_half=True)
    rounds = []
    first_tokens = None
    for r in range(warmup + steps):
        m.reset()
        t0 = time.perf_counter()
        m.prefill(prompt, logits=False)
        first = m.greedy_token()
        t1 = time.perf_counter()
        toks = m.generate(GEN - 1)
        t2 = time.perf_counter()
        gpu_decode = m.last_gpu_seconds
        if r >= warmup:
            rounds.append(dict(ttft=t1 - t0, decode=t2 - t1, gpu_decode=gpu_decode))
        # generate() starts from the selection greedy_token() made; the 128th
        # token is the selection after the last step.
        assert toks[0] == first
        first_tokens = toks.tolist() + [m.greedy_token()]
    m.close()
    ttft = sum(x["ttft"] for x in rounds)
    dec = sum(x["decode"] for x in rounds)
    gdec = sum(x["gpu_decode"] for x in rounds)
    n = len(rounds)
    return dict(prefill_tok_s=PROMPT * n / ttft, decode_tok_s=(GEN - 1) * n / dec,
                decode_tok_s_device=(GEN - 1) * n / gdec, ms_per_step=(ttft + dec) / n * 1e3,
                ttft_ms=ttft / n * 1e3, tpot_ms=dec / n / (GEN - 1) * 1e3, tokens=first_tokens)


def long_leg(hip, weights, seed: int = 7):
    """BASELINE configs[3] part 2: 128 greedy steps after a 32,768-token random
    prompt, then a second request sharing the first 30,000 prompt tokens.

    Request 1 prefills the shared prefix, takes a checkpoint there (as the
    reference's engine does at a prompt's turn boundary, engine.rs:561-584),
    prefills the rest and decodes.  Request 2 restores the checkpoint (the KV
    cache of the prefix stays in HBM, lfm2_metal.rs:86-97), prefills only its
    own 2,768-token tail and decodes; its tokens are checked against the same
    request run from scratch."""
    from bobcat_amd.lfm2 import Lfm2Hip

    cfg = weights.cfg
    rng = np.random.default_rng(seed)
    prompt1 = rng.integers(0, cfg.n_vocab, LONG_PROMPT).astype(np.uint32)
    prompt2 = prompt1.copy()
    prompt2[LONG_SHARED:] = rng.integers(0, cfg.n_vocab, LONG_PROMPT - LONG_SHARED)
    m = Lfm2Hip(hip, weights, n_ctx=LONG_PROMPT + GEN, kv_half=True)
    m.reset()
    t0 = time.perf_counter()
    m.prefill(prompt1[:LONG_SHARED], logits=False)
    ck = m.checkpoint()
    m.prefill(prompt1[LONG_SHARED:], logits=False)
    m.greedy_token()
    t1 = time.perf_counter()
    m.generate(GEN - 1)
    t2 = time.perf_counter()
    gpu_decode = m.last_gpu_seconds
    # Request 2 with the shared prefix reused.
    m.restore(ck)
    t3 = time.perf_counter()
    m.prefill(prompt2[LONG_SHARED:], logits=False)
    first = m.greedy_token()
    t4 = time.perf_counter()
    reused = [first] + m.generate(GEN - 1).tolist()
    # Request 2 from scratch, for the reuse check and the TTFT it saves.
    m.reset()
    t5 = time.perf_counter()
    m.prefill(prompt2, logits=False)
    first = m.greedy_token()
    t6 = time.perf_counter()
    fresh = [first] + m.generate(GEN - 1).tolist()
    m.close()
    return dict(prompt=LONG_PROMPT, shared_prefix=LONG_SHARED,
                prefill_tok_s=round(LONG_PROMPT / (t1 - t0), 1),
                decode_tok_s=round((GEN - 1) / (t2 - t1), 1),
                decode_tok_s_device=round((GEN - 1) / gpu_decode, 1),
                reuse_ttft_ms=round((t4 - t3) * 1e3, 2), fresh_ttft_ms=round((t6 - t5) * 1e3, 2),
                reuse_matches_fresh=reused == fresh,
                reuse_matching_prefix=next((i for i, (a, b) in enumerate(zip(reused, fresh)) if a != b), GEN))


def long_prefill(hip, weights, n: int, seed: int = 9) -> float:
    """Prefill rate of an n-token random prompt (f16 KV cache), after a warm-up."""
    from bobcat_amd.qwen35 import Qwen35Hip

    prompt = np.random.default_rng(seed).integers(0, weights.cfg.n_vocab, n).astype(np.uint32)
    m = Qwen35Hip(hip, weights, n_ctx=n + 8, kv_half=True)
    m.prefill(prompt[:1024], logits=False)
    m.reset()
    t0 = time.perf_counter()
    m.prefill(prompt, logits=False)
    m.greedy_token()
    dt = time.perf_counter() - t0
    m.close()
    return n / dt


def cpu_model_rate(weights, budget_s: float, threads: int):
    """Decode steps of the oracle on the host: the reference's scalar path
    (f64-accumulating matvec, lfm2.rs:308-394 / qwen35.rs:280-516) restated in
    C, rows split over `threads` threads.  Bounded: a short prompt, then steps
    until the budget (at least one)."""
    import oracle

    oracle.set_threads(threads)
    st = (oracle.Qwen35State if hasattr(weights.cfg, "n_k_heads") else oracle.Lfm2State)(weights, n_ctx=64)
    rng = np.random.default_rng(42)
    for t in rng.integers(0, weights.cfg.n_vocab, 2):
        st.step(int(t), logits=False)
    n, t0 = 0, time.perf_counter()
    tok = 1
    while True:
        lg = st.step(tok)
        tok = int(np.argmax(lg))
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= 32:
            break
    dt = time.perf_counter() - t0
    return dict(tok_s=n / dt, steps=n, seconds=dt)


def cpu_gdn_layer_us(weights, threads: int, budget_s: float = 2.0):
    """One Gated DeltaNet layer step of Qwen3.5-0.8B by the oracle
    (qwen35.rs:430-516: the input projections, convolution, recurrence over
    16 heads' 128 x 128 states, gated norm and output projection)."""
    import oracle

    oracle.set_threads(threads)
    st = oracle.Qwen35State(weights, n_ctx=8)
    st.step(1, logits=False)
    layer = next(i for i in range(weights.cfg.n_layers) if not weights.cfg.is_attention(i))
    n, t0 = 0, time.perf_counter()
    while True:
        st.delta_step(layer)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    return (time.perf_counter() - t0) / n * 1e6


def cpu_gemv_us(w, x, threads: int, budget_s: float = 2.0):
    """The oracle's config-1 Q4_K matvec (scalar.rs:213-220) on `threads` threads."""
    import oracle

    oracle.set_threads(threads)
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.matvec(12, w, GEMV_ROWS, GEMV_COLS, x)
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    return (time.perf_counter() - t0) / n * 1e6


def host_cpu():
    """(online cores, model name) of the host."""
    cores = os.sysconf("SC_NPROCESSORS_ONLN") if hasattr(os, "sysconf") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return int(cores), model


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def gemm_leg(hip, reps: int = 20):
    """The prefill GEMM at LFM2-2.6B's shapes for a 512-token batch: the FFN
    gate projection (10752 x 2048) and down projection (2048 x 10752) on
    Q4_K weights, each launch timed over `reps` repetitions with HIP events
    (each includes the input conversion to fp16).  TFLOP/s counts the
    2·rows·cols·tokens of the product; the fraction is of MI355X's dense
    fp16 MFMA peak."""
    from bobcat_amd.backend import Format, Store
    from bobcat_amd.synth import q4k_matrix

    rng = np.random.default_rng(5)
    out = {}
    for name, rows, cols, store in (("ffn_gate_10752x2048", 10752, 2048, Store.OVERWRITE),
                                    ("ffn_down_2048x10752", 2048, 10752, Store.ACCUMULATE)):
        w = hip.buffer_from(q4k_matrix(rng, rows, cols))
        x = hip.buffer_from(rng.standard_normal(PROMPT * cols).astype(np.float32))
        y = hip.new_buffer(PROMPT * rows * 4)

        def run(n):
            hip.begin()
            for _ in range(n):
                hip.matmul(Format.Q4K, w.at(0), rows, cols, x.at(0), y.at(0), PROMPT, store)
            return hip.end()

        run(3)
        sec = run(reps) / reps
        tflops = 2.0 * rows * cols * PROMPT / sec / 1e12
        out[name] = {"us": round(sec * 1e6, 2), "tflops": round(tflops, 1),
                     "mfma_frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
        for b in (w, x, y):
            b.free()
    out["peak_tflops"] = MFMA_F16_PEAK_TFLOPS
    return out


def cpu_baseline(weights, gemv_case, budget_s: float):
    """The reference's CPU path (the oracle) on the host, in the same run: the
    model's decode rate single-threaded (the reference's scalar path runs on
    one core) and over the GPU's host share; one decode token of LFM2-350M
    and one Gated DeltaNet layer step of Qwen3.5-0.8B
    on both; and the config-1 GEMV time."""
    from bobcat_amd.lfm2 import LFM2_350M, Lfm2Weights
    from bobcat_amd.qwen35 import QWEN35_0_8B, Qwen35Weights

    online, model = host_cpu()
    threads = host_threads()
    one = cpu_model_rate(weights, budget_s / 2, 1)
    many = cpu_model_rate(weights, budget_s / 2, threads)
    small = Lfm2Weights(LFM2_350M, seed=WEIGHT_SEED)
    small_one = cpu_model_rate(small, 2.0, 1)
    small_many = cpu_model_rate(small, 2.0, threads)
    del small
    qwen = Qwen35Weights(QWEN35_0_8B, seed=WEIGHT_SEED)
    gdn_one, gdn_many = cpu_gdn_layer_us(qwen, 1), cpu_gdn_layer_us(qwen, threads)
    del qwen
    w, x = gemv_case
    return dict(one_core=one, all_cores=many, threads=threads, online_cores=online, cpu_model=model,
                gemv_us_1=cpu_gemv_us(w, x, 1), gemv_us_all=cpu_gemv_us(w, x, threads),
                lfm2_350m=dict(one_core=small_one, all_cores=small_many),
                gdn_layer_us=dict(one_core=gdn_one, all_cores=gdn_many))


def model_summary(cfg, mres, name: str):
    wb = cfg.weight_bytes()
    mean_ctx = PROMPT + GEN / 2
    n_attn = (len(cfg.attention_layers) if hasattr(cfg, "attention_layers")
              else sum(cfg.is_attention(i) for i in range(cfg.n_layers)))
    kv_bytes = n_attn * mean_ctx * 2 * cfg.n_kv_heads * cfg.head_dim * 2
    token_bytes = wb["total"] + kv_bytes
    decode_gbs = mres["decode_tok_s_device"] * token_bytes / 1e9
    match, prefix = greedy_match(mres["tokens"], name)
    return token_bytes, decode_gbs, dict(
        prefill_tok_s=round(mres["prefill_tok_s"], 1), decode_tok_s=round(mres["decode_tok_s"], 1),
        decode_tok_s_device=round(mres["decode_tok_s_device"], 1), ttft_ms=round(mres["ttft_ms"], 3),
        tpot_ms=round(mres["tpot_ms"], 4), decode_bytes_per_token=int(token_bytes),
        decode_hbm_gbs=round(decode_gbs, 1), decode_roofline_frac=round(decode_gbs / HBM_PEAK_GBS, 4),
        greedy_matches_oracle=match, greedy_identical_prefix=prefix)


# The seeded random-init weights of tests/golden/make_greedy.py, so the
# generated tokens can be checked against the oracle's fixtures.
WEIGHT_SEED = 3
SIDE_MODELS = ("qwen3.5-0.8b", "lfm2-8b-a1b", "lfm2-350m")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed pp512/tg128 rounds")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--model", default="lfm2-2.6b")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-long", action="store_true", help="skip the 32K-context leg")
    ap.add_argument("--skip-side", action="store_true", help="skip the other model configs")
    ap.add_argument("--long-only", action="store_true", help="only the 32K-context leg (for profiling)")
    ap.add_argument("--gemv-only", action="store_true", help="only the config-1 GEMV leg (for profiling)")
    ap.add_argument("--gemm-only", action="store_true", help="only the prefill GEMM leg (for profiling)")
    ap.add_argument("--decode-gemv-only", action="store_true",
                    help="only the 2.6B decode GEMV shapes (for profiling)")
    ap.add_argument("--attn-decode-only", action="store_true",
                    help="only the 2.6B decode attention at a 32K context (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the decode loop is single-device (as in the reference) "
              "and this build has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2

    from bobcat_amd.backend import Hip
    from bobcat_amd.lfm2 import CONFIGS, Lfm2Weights
    from bobcat_amd.qwen35 import CONFIGS as QWEN_CONFIGS, Qwen35Weights
    from bobcat_amd.synth import gemv_case

    def weights_of(name):
        if name in QWEN_CONFIGS:
            return Qwen35Weights(QWEN_CONFIGS[name], seed=WEIGHT_SEED)
        return Lfm2Weights(CONFIGS[name], seed=WEIGHT_SEED)

    side = {}
    with Hip() as hip:
        name, cus = hip.device_info()
        log(f"device: {name}, {cus} CUs")
        if args.long_only:
            lres = long_leg(hip, weights_of(args.model))
            log(f"long context: {lres}")
            return 0
        if args.gemm_only:
            log(f"prefill gemm: {gemm_leg(hip)}")
            return 0
        if args.decode_gemv_only:
            log(f"decode gemv: {decode_gemv_leg(hip)}")
            return 0
        if args.attn_decode_only:
            log(f"decode attention: {attn_decode_leg(hip)}")
            return 0
        g = gemv_leg(hip, reps=10)
        log(f"gemv: {g}")
        if args.gemv_only:
            return 0
        gm = gemm_leg(hip)
        log(f"prefill gemm: {gm}")
        t = time.perf_counter()
        weights = weights_of(args.model)
        cfg = weights.cfg
        log(f"generated {cfg.name} weights in {time.perf_counter() - t:.1f}s")
        mres = model_leg(hip, weights, args.steps, args.warmup)
        log(f"model: { {k: v for k, v in mres.items() if k != 'tokens'} }")
        lres = None
        if not args.skip_long and cfg.name == "lfm2-2.6b":
            lres = long_leg(hip, weights)
            log(f"long context: {lres}")
        if not args.skip_side:
            for sname in SIDE_MODELS:
                if sname == cfg.name:
                    continue
                sw = weights_of(sname)
                sres = model_leg(hip, sw, steps=2, warmup=1)
                side[sname] = model_summary(sw.cfg, sres, sname)[2]
                if sname.startswith("qwen"):
                    side[sname]["prefill_16k_tok_s"] = round(long_prefill(hip, sw, 16384), 1)
                log(f"{sname}: {side[sname]}")
                del sw
    cpu = None if args.skip_cpu else cpu_baseline(weights, gemv_case(), args.cpu_seconds)
    if cpu:
        log(f"cpu: {cpu}")

    token_bytes, decode_gbs, summary = model_summary(cfg, mres, cfg.name)
    line = {
        "metric": "decode tok/s (pp512/tg128, 1 GPU)",
        "value": round(mres["decode_tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mres["ms_per_step"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4k-f32",
        "data": "synthetic (random-init weights of the config's shapes, seed 3; 512 random prompt ids, seed 42)",
        "config": {"workload": f"{cfg.name} pp512/tg128 (BASELINE configs[3])" if cfg.name == "lfm2-2.6b"
                   else f"{cfg.name} pp512/tg128", "prompt": PROMPT, "generated": GEN, "kv_cache": "f16",
                   "parallelism": "none"},
        **{k: v for k, v in summary.items() if k != "decode_tok_s"},
        "long_context": lres,
        "models": side or None,
        "prefill_gemm": gm,
        "roofline": {"kernel": "matvec_q4k (config 1, 8192x2048)", "bound": "hbm",
                     "achieved": round(g["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "us_per_launch": round(g["us"], 3)},
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["one_core"]["tok_s"], 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{cpu['one_core']['steps']} decode steps of {cfg.name} by the oracle (C restatement of "
                      f"the reference's scalar path, f64 accumulate) on one core",
            "all_cores": {"value": round(cpu["all_cores"]["tok_s"], 4), "cores": cpu["threads"],
                          "sample": f"{cpu['all_cores']['steps']} decode steps, rows over {cpu['threads']} threads"},
            "host": {"online_cores": cpu["online_cores"], "cpu_model": cpu["cpu_model"]},
            "gemv_config1_us": {"1_core": round(cpu["gemv_us_1"], 1),
                                f"{cpu['threads']}_cores": round(cpu["gemv_us_all"], 1)},
            "lfm2_350m_decode_tok_s": {"1_core": round(cpu["lfm2_350m"]["one_core"]["tok_s"], 3),
                                       f"{cpu['threads']}_cores": round(cpu["lfm2_350m"]["all_cores"]["tok_s"], 3)},
            "qwen35_gdn_layer_step_us": {"1_core": round(cpu["gdn_layer_us"]["one_core"], 1),
                                         f"{cpu['threads']}_cores": round(cpu["gdn_layer_us"]["all_cores"], 1)}},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
