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
  * cpu   — the oracle (a C restatement of the reference's scalar Rust path)
            decoding the same model on the host cores, on a bounded sample.

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
    # The GPU box gives one GPU a 16-core share, whatever os.cpu_count() says.
    return max(1, min(16, os.cpu_count() or 1))


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


def model_leg(hip, weights, steps: int, warmup: int, seed: int = 42):
    from bobcat_amd.lfm2 import Lfm2Hip
    from bobcat_amd.qwen35 import Qwen35Hip, Qwen35Weights

    cfg = weights.cfg
    Lfm2Hip = Qwen35Hip if isinstance(weights, Qwen35Weights) else Lfm2Hip
    rng = np.random.default_rng(seed)
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
        first_tokens = [first] + toks.tolist()
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


def cpu_leg(weights, budget_s: float, threads: int):
    """Decode steps of the oracle on the host: the reference's scalar path
    (f64-accumulating matvec, lfm2.rs:308-394) restated in C, rows split over
    `threads` threads.  Bounded: a short prompt, then steps until the budget."""
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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed pp512/tg128 rounds")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--model", default="lfm2-2.6b")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-long", action="store_true", help="skip the 32K-context leg")
    ap.add_argument("--long-only", action="store_true", help="only the 32K-context leg (for profiling)")
    ap.add_argument("--gemv-only", action="store_true", help="only the config-1 GEMV leg (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the decode loop is single-device (as in the reference) "
              "and this build has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2

    from bobcat_amd.backend import Hip
    from bobcat_amd.lfm2 import CONFIGS, Lfm2Weights
    from bobcat_amd.qwen35 import CONFIGS as QWEN_CONFIGS, Qwen35Weights

    if args.model in QWEN_CONFIGS:
        cfg, Lfm2Weights = QWEN_CONFIGS[args.model], Qwen35Weights
    else:
        cfg = CONFIGS[args.model]
    with Hip() as hip:
        name, cus = hip.device_info()
        log(f"device: {name}, {cus} CUs")
        if args.long_only:
            lres = long_leg(hip, Lfm2Weights(cfg, seed=0))
            log(f"long context: {lres}")
            return 0
        g = gemv_leg(hip, reps=10)
        log(f"gemv: {g}")
        if args.gemv_only:
            return 0
        t = time.perf_counter()
        weights = Lfm2Weights(cfg, seed=0)
        log(f"generated {cfg.name} weights in {time.perf_counter() - t:.1f}s")
        mres = model_leg(hip, weights, args.steps, args.warmup)
        log(f"model: { {k: v for k, v in mres.items() if k != 'tokens'} }")
        lres = None
        if not args.skip_long and cfg.name == "lfm2-2.6b":
            lres = long_leg(hip, weights)
            log(f"long context: {lres}")
    threads = host_threads()
    cpu = None if args.skip_cpu else cpu_leg(weights, args.cpu_seconds, threads)
    if cpu:
        log(f"cpu: {cpu} ({threads} threads)")

    wb = cfg.weight_bytes()
    # Bytes a decode token streams: all layer matrices + the output matrix
    # + the KV cache read at the mean context of tg128 after pp512.
    mean_ctx = PROMPT + GEN / 2
    n_attn = (len(cfg.attention_layers) if hasattr(cfg, "attention_layers")
              else sum(cfg.is_attention(i) for i in range(cfg.n_layers)))
    kv_bytes = n_attn * mean_ctx * 2 * cfg.n_kv_heads * cfg.head_dim * 2
    token_bytes = wb["total"] + kv_bytes
    decode_gbs = mres["decode_tok_s_device"] * token_bytes / 1e9
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
        "data": "synthetic (random-init weights of the config's shapes, 512 random prompt ids)",
        "config": {"workload": f"{cfg.name} pp512/tg128 (BASELINE configs[3])" if cfg.name == "lfm2-2.6b"
                   else f"{cfg.name} pp512/tg128", "prompt": PROMPT, "generated": GEN, "kv_cache": "f16",
                   "parallelism": "none"},
        "prefill_tok_s": round(mres["prefill_tok_s"], 1),
        "decode_tok_s_device": round(mres["decode_tok_s_device"], 1),
        "ttft_ms": round(mres["ttft_ms"], 3),
        "tpot_ms": round(mres["tpot_ms"], 4),
        "decode_bytes_per_token": int(token_bytes),
        "decode_hbm_gbs": round(decode_gbs, 1),
        "decode_roofline_frac": round(decode_gbs / HBM_PEAK_GBS, 4),
        "long_context": lres,
        "roofline": {"kernel": "matvec_q4k (config 1, 8192x2048)", "bound": "hbm",
                     "achieved": round(g["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "us_per_launch": round(g["us"], 3)},
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["tok_s"], 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{cpu['steps']} decode steps of {cfg.name} by the oracle (C restatement of the "
                      f"reference's scalar path, f64 accumulate, rows over {threads} threads)"},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
