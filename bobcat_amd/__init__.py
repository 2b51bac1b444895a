"""bobcat_amd: an MI355X (gfx950) backend for bobcat's per-token LM loop.

The compute path is libbobcat_hip.so (hand-written HIP kernels and a C++
driver behind the C ABI of include/bobcat_hip.h).  This package holds the
Python mirror of that ABI (`backend.Hip`, `lfm2.Lfm2Hip`) used by the tests
and the benchmark.
"""
from ._lib import BobcatError, lib  # noqa: F401

__all__ = ["BobcatError", "lib"]
