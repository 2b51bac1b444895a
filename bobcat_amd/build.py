"""Build libbobcat_hip.so for gfx950 in-tree.

Every ``csrc/*.hip`` file compiles with hipcc to an object under
``bobcat_amd/_build/`` (in parallel), and the objects link into
``bobcat_amd/libbobcat_hip.so``.  Run ``python -m bobcat_amd.build``.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libbobcat_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# gfx950 only.  Packed-FP32 instructions stay off: the compiler must not
# form v_pk_{add,mul,fma}_f32 from scalar or float2 code.
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-value",
    "-Wno-unused-result",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    if os.environ.get("BCH_INCREMENTAL") == "1" and obj.exists():
        # Development shortcut: keep an object newer than its source and every header.
        newest = max(p.stat().st_mtime for p in [src, *CSRC.glob("*.h"), PKG.parent / "include" / "bobcat_hip.h"])
        if obj.stat().st_mtime > newest:
            return obj
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns about the packed-fp32 feature; anything else
    # is worth showing.
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(LIB), *map(str, objs),
           "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
