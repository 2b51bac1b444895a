"""Benchmark: bobcat's per-token LM loop on one MI355X.

Prints ONE JSON line (the driver's contract).  Legs:
  * gemv  — BASELINE config 1: Q4_K dequant-GEMV, W [8192 x 2048], x ~ N(0,1),
            timed over 64 rotating copies of W (604 MB > the 256 MB MALL) with
            HIP events on the backend's own stream; gives the roofline object.
  * cpu   — the oracle's scalar GEMV (1 thread, f64 accumulate, the
            reference's scalar path restated) on a bounded sample.
  * model — LFM2 decode/prefill (pp512/tg128), once the driver is built.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
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


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_leg(hip, steps: int, warmup: int, copies: int = 64):
    from bobcat_amd.backend import Format
    from bobcat_amd.synth import gemv_case

    w, x = gemv_case()
    wbytes = w.nbytes
    big = hip.new_buffer(wbytes * copies)
    for c in range(copies):
        hip.write(big.at(c * wbytes), w)
    xb = hip.buffer_from(x)
    yb = hip.new_buffer(GEMV_ROWS * 4)

    def run(n: int) -> float:
        hip.begin()
        for i in range(n):
            hip.matvec(Format.Q4K, big.at((i % copies) * wbytes), GEMV_ROWS, GEMV_COLS, xb.at(0), yb.at(0))
        return hip.end()

    run(max(warmup, 1) * copies)
    launches = steps * copies
    seconds = run(launches)
    per_launch = seconds / launches
    achieved = GEMV_BYTES / per_launch / 1e9
    # Cache-resident rate on one copy (for the record; not the roofline figure).
    hip.begin()
    for _ in range(copies):
        hip.matvec(Format.Q4K, big.at(0), GEMV_ROWS, GEMV_COLS, xb.at(0), yb.at(0))
    hot = hip.end() / copies
    big.free()
    return dict(us_per_launch=per_launch * 1e6, gbs=achieved, launches=launches,
                hot_us=hot * 1e6, hot_gbs=GEMV_BYTES / hot / 1e9)


def cpu_leg(budget_s: float = 10.0):
    import oracle
    from bobcat_amd.synth import gemv_case

    w, x = gemv_case()
    oracle.set_threads(1)
    oracle.matvec(12, w, GEMV_ROWS, GEMV_COLS, x)  # warm
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        oracle.matvec(12, w, GEMV_ROWS, GEMV_COLS, x)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return dict(us=dt * 1e6, gbs=GEMV_BYTES / dt / 1e9, reps=n)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the decode loop is single-device, as in the reference).", file=sys.stderr)
        return 2

    from bobcat_amd.backend import Hip

    with Hip() as hip:
        name, cus = hip.device_info()
        log(f"device: {name}, {cus} CUs")
        g = gemv_leg(hip, args.steps, args.warmup)
        log(f"gemv: {g}")
    cpu = None if args.skip_cpu else cpu_leg(args.cpu_seconds)
    if cpu:
        log(f"cpu: {cpu}")

    line = {
        "metric": "Q4_K GEMV GB/s vs HBM peak (config 1, 8192x2048)",
        "value": round(g["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["us_per_launch"] * 64 / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4k-f32",
        "data": "synthetic (seeded Q4_K blocks, x ~ N(0,1))",
        "config": {"workload": "config1_q4k_gemv_8192x2048", "rotating_copies": 64,
                   "parallelism": "none"},
        "roofline": {"bound": "hbm", "achieved": round(g["gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": None if cpu is None else {
            "value": round(cpu["gbs"], 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{cpu['reps']} scalar GEMVs of config 1 (oracle, f64 accumulate)"},
        "gemv_us": round(g["us_per_launch"], 3),
        "gemv_hot_gbs": round(g["hot_gbs"], 1),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
