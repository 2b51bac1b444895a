"""CPU checks of the C-ABI boundary (no GPU needed).

* libbobcat_hip.so loads and exports every entry point include/bobcat_hip.h
  declares, and the ctypes binding declares exactly those;
* the pure functions answer without a device (row sizes, attention scratch
  size of backend.rs:2739-2748);
* without a GPU, opening the backend fails with the NoDevice status rather
  than falling back to anything;
* the product package never imports the oracle.
"""
from __future__ import annotations

import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "bobcat_hip.h"


def declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(bch_\w+)\s*\(", text))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("bch_open", "bch_matvec", "bch_matvec_swiglu", "bch_matvec_conv", "bch_matmul", "bch_attention",
                 "bch_norm_rope", "bch_embed", "bch_argmax", "bch_lfm2_new", "bch_lfm2_generate"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from bobcat_amd import _lib

    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_matches_header():
    from bobcat_amd import _lib

    assert set(_lib.PROTOTYPES) == declared()
    _lib.lib()
    assert not _lib.MISSING


def test_row_bytes_and_scratch_sizes():
    from bobcat_amd import _lib

    lib = _lib.lib()
    assert lib.bch_row_bytes(12, 2048) == 8 * 144
    assert lib.bch_row_bytes(14, 256) == 210
    assert lib.bch_row_bytes(1, 1024) == 2048
    assert lib.bch_row_bytes(8, 64) == 68
    assert lib.bch_row_bytes(12, 100) == 0  # not a whole super-block
    assert lib.bch_row_bytes(99, 256) == 0  # unknown format
    # min(nq, 64) * heads * ceil(n_ctx / 64) * (head_dim + 2)
    assert lib.bch_attention_scratch_floats(32, 64, 640, 1) == 1 * 32 * 10 * 66
    assert lib.bch_attention_scratch_floats(16, 64, 100, 500) == 64 * 16 * 2 * 66


def test_no_device_is_an_error_not_a_fallback():
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    from bobcat_amd import BobcatError
    from bobcat_amd.backend import Hip

    with pytest.raises(BobcatError) as e:
        Hip()
    assert e.value.status == 1  # NoDevice


def test_product_never_imports_the_oracle():
    for path in (ROOT / "bobcat_amd").rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(import oracle|from oracle)", text, re.M), path


def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
