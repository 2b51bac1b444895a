"""Writes the full-size greedy fixtures (tests/golden/greedy_<model>.npz).

For each BASELINE model config (LFM2 350M, Qwen3.5 0.8B, LFM2 2.6B, LFM2
8B-A1B) with its seeded random-init weights, the CPU oracle (oracle/, the
restatement of lfm2.rs / qwen35.rs Model::step) runs a 512-token seeded prompt
and then 128 greedy steps, as the reference's model tests do on real files
(crates/bobcat/tests/lfm2_reference.rs:117-350).  Stored per model:

  prompt      the prompt ids
  tokens      the 128 greedy ids
  gaps        per step, the oracle's top-1 minus top-2 logit
  logits0     the logits after the prompt (the first greedy step's input)
  digest      sha256 over a few weight tensors, so a test notices when the
              seeded weight generator no longer makes the same model

Run once on the CPU: ``python tests/golden/make_greedy.py [model ...]`` (about
15 minutes on 8 threads for all four).  The GPU tests regenerate the weights
from the same seeds and compare against these files.
"""
from __future__ import annotations

import hashlib
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from bobcat_amd.lfm2 import LFM2_2_6B, LFM2_8B_A1B, LFM2_350M, Lfm2Weights  # noqa: E402
from bobcat_amd.qwen35 import QWEN35_0_8B, Qwen35Weights  # noqa: E402

HERE = Path(__file__).resolve().parent
WEIGHT_SEED = 3
PROMPT_SEED = 42
N_PROMPT = 512
N_GEN = 128

MODELS = {
    "lfm2-350m": (LFM2_350M, Lfm2Weights, oracle.Lfm2State),
    "qwen3.5-0.8b": (QWEN35_0_8B, Qwen35Weights, oracle.Qwen35State),
    "lfm2-2.6b": (LFM2_2_6B, Lfm2Weights, oracle.Lfm2State),
    "lfm2-8b-a1b": (LFM2_8B_A1B, Lfm2Weights, oracle.Lfm2State),
}
# Long-context fixtures: (model, prompt length, greedy steps).  The 2.6B at a
# 4,096-token prompt reaches the long-context attention shape (8 KV heads of
# 64 over thousands of keys, several key splits in prefill and decode).
LONG = {
    "lfm2-2.6b-ctx4k": ("lfm2-2.6b", 4096, 32),
}


def digest(weights) -> str:
    """sha256 over the first and last tensors the generator makes."""
    keys = list(weights.arrays)
    h = hashlib.sha256()
    for k in keys[:3] + keys[-3:]:
        h.update(k.encode())
        h.update(np.ascontiguousarray(weights.arrays[k]).view(np.uint8).tobytes())
    return h.hexdigest()


def prompt_ids(n_vocab: int, n: int = N_PROMPT) -> np.ndarray:
    return np.random.default_rng(PROMPT_SEED).integers(0, n_vocab, n).astype(np.uint32)


def fixture_path(name: str) -> Path:
    return HERE / f"greedy_{name}.npz"


def make(name: str) -> None:
    base, n_prompt, n_gen = LONG.get(name, (name, N_PROMPT, N_GEN))
    cfg, wcls, scls = MODELS[base]
    t0 = time.time()
    weights = wcls(cfg, seed=WEIGHT_SEED)
    prompt = prompt_ids(cfg.n_vocab, n_prompt)
    cpu = scls(weights, n_ctx=n_prompt + n_gen + 8)
    for t in prompt:
        lg = cpu.step(int(t))
    logits0 = lg.copy()
    toks, gaps = [], []
    for _ in range(n_gen):
        top = np.argsort(lg, kind="stable")[-2:]
        gaps.append(float(lg[top[1]] - lg[top[0]]))
        nxt = int(np.argmax(lg))
        toks.append(nxt)
        lg = cpu.step(nxt)
    np.savez_compressed(fixture_path(name), prompt=prompt, tokens=np.array(toks, np.uint32),
                        gaps=np.array(gaps, np.float32), logits0=logits0, digest=np.array(digest(weights)))
    print(f"{name}: {time.time() - t0:.0f} s, min gap {min(gaps):.3g}", flush=True)


if __name__ == "__main__":
    oracle.set_threads(int(os.environ.get("ORC_THREADS", os.cpu_count() or 8)))
    for n in sys.argv[1:] or list(MODELS):
        make(n)
