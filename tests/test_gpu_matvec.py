"""GPU parity of the dequantisation and matrix-vector kernels against the oracle.

Mirrors crates/bobcat/tests/metal_matvec.rs: every mode (plain, fused norm,
accumulate, SwiGLU) on the reference's shapes (:26-36), weights from its
xorshift generator (:57-92), and its tolerance, 1e-5 relative to the largest
row sum of |w·x| (:16-19, :115-129, :236-244).  Dequantisation is bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from bobcat_amd.backend import Format, NormSpec
from bobcat_amd.synth import q4k_matrix
from tests._gen import Random

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5
NORM_EPS = 1e-5
SHAPES = [(1, 32), (7, 64), (7, 256), (1000, 1024), (1024, 1024), (3072, 1024), (4608, 1024),
          (1024, 4608), (65536, 1024)]
BLOCK = {Format.Q4K: (256, 144, [0, 2]), Format.F16: (1, 2, []), Format.F32: (1, 4, []),
         Format.Q8_0: (32, 34, [0]), Format.Q4_0: (32, 18, [0]), Format.Q5K: (256, 176, [0, 2]),
         Format.Q6K: (256, 210, [208])}
# Columns a row must be a multiple of on the GPU (Q8_0/Q4_0 units are two blocks).
COLS = {Format.Q4K: 256, Format.Q5K: 256, Format.Q6K: 256, Format.Q8_0: 64, Format.Q4_0: 64}


def make_weights(rnd: Random, fmt: Format, rows: int, cols: int, big_rng) -> np.ndarray:
    n_el, n_b, scales = BLOCK[fmt]
    nbytes = rows * cols // n_el * n_b
    if fmt in COLS:
        if nbytes <= 1 << 20:
            return rnd.blocks(nbytes, n_b, scales)
        # Large shapes: the same distribution from numpy (the xorshift in
        # Python would take minutes).
        w = big_rng.integers(0, 256, nbytes, dtype=np.uint8).reshape(-1, n_b)
        for at in scales:
            exp = big_rng.integers(5, 9, w.shape[0]).astype(np.uint16)
            man = big_rng.integers(0, 1024, w.shape[0]).astype(np.uint16)
            w[:, at:at + 2] = ((exp << 10) | man).view(np.uint8).reshape(-1, 2)
        return w.reshape(-1)
    vals = rnd.units(rows * cols) if rows * cols <= 1 << 18 else \
        big_rng.uniform(-1, 1, rows * cols).astype(np.float32)
    return (vals.astype(np.float16) if fmt == Format.F16 else vals).view(np.uint8)


def dense(fmt, w, rows, cols):
    return oracle.dequantize(int(fmt), w, rows * cols).reshape(rows, cols)


def term_scale(fmt, w, rows, cols, x):
    """Largest row sum of |w·x| (metal_matvec.rs:115-129), in row chunks."""
    row_bytes = w.size // rows
    ax = np.abs(x.astype(np.float64))
    best = 0.0
    for r0 in range(0, rows, 4096):
        r1 = min(rows, r0 + 4096)
        d = dense(fmt, w[r0 * row_bytes:r1 * row_bytes], r1 - r0, cols)
        best = max(best, float((np.abs(d.astype(np.float64)) @ ax).max()))
    return best


def launch_error(hip, rnd, fmt, mode, rows, cols, big_rng):
    gate_w = make_weights(rnd, fmt, rows, cols, big_rng)
    up_w = make_weights(rnd, fmt, rows, cols, big_rng)
    x = rnd.units(cols) if cols <= 4608 else big_rng.uniform(-1, 1, cols).astype(np.float32)
    norm_w = (1.0 + 0.5 * rnd.units(cols)).astype(np.float32)
    prior = rnd.units(rows) if rows <= 4608 else big_rng.uniform(-1, 1, rows).astype(np.float32)

    inp = oracle.rms_norm(x, norm_w, NORM_EPS) if mode in ("norm", "swiglu") else x
    oracle.set_threads(8)
    want = oracle.matvec(int(fmt), gate_w, rows, cols, inp)
    if mode == "accumulate":
        want = want + prior
    elif mode == "swiglu":
        up = oracle.matvec(int(fmt), up_w, rows, cols, inp)
        want = np.array([oracle.silu(float(g)) for g in want], np.float32) * up

    gate = hip.buffer_from(gate_w)
    upb = hip.buffer_from(up_w)
    xb = hip.buffer_from(x)
    nb = hip.buffer_from(norm_w)
    y = hip.buffer_from(prior)
    norm = NormSpec(nb.at(0), NORM_EPS)
    hip.begin()
    if mode == "swiglu":
        hip.matvec_swiglu(fmt, gate.at(0), upb.at(0), rows, cols, xb.at(0), norm, y.at(0))
    else:
        hip.matvec(fmt, gate.at(0), rows, cols, xb.at(0), y.at(0),
                   norm if mode == "norm" else None, mode == "accumulate")
    hip.end()
    got = hip.read(y.at(0), np.empty(rows, np.float32))
    for b in (gate, upb, xb, nb, y):
        b.free()
    if mode == "swiglu":
        scale = float(np.abs(want).max())
    else:
        scale = max(term_scale(fmt, gate_w, rows, cols, inp), float(np.abs(want).max()))
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    if np.isnan(diff).any():
        return float("inf")
    return float(diff.max() / scale)


@pytest.mark.parametrize("fmt", [Format.Q4K, Format.Q8_0, Format.Q4_0, Format.Q5K, Format.Q6K])
def test_matvec_kernels_match_scalar(hip, fmt):
    """metal_matvec.rs:39-45's five block formats over its shapes and modes."""
    rnd = Random(0x9E3779B97F4A7C15)
    big = np.random.default_rng(11)
    failures = []
    for mode in ("plain", "norm", "accumulate", "swiglu"):
        for rows, cols in SHAPES:
            if cols % COLS[fmt]:
                continue
            print(f"matvec {fmt.name} {mode} {rows}x{cols}", flush=True)
            err = launch_error(hip, rnd, fmt, mode, rows, cols, big)
            if not err < TOLERANCE:
                failures.append(f"{fmt.name} {mode} {rows}x{cols}: {err:.3e}")
    assert not failures, failures


def test_float_matvec_matches_scalar(hip):
    """metal_matvec.rs:249-274: F16 and F32 on (7, 256) and (1000, 1024)."""
    rnd = Random(0x60E7927B081DA5EF)
    big = np.random.default_rng(12)
    for fmt in (Format.F16, Format.F32):
        for mode in ("plain", "norm", "accumulate", "swiglu"):
            for rows, cols in [(7, 256), (1000, 1024), (65536, 1024)]:
                err = launch_error(hip, rnd, fmt, mode, rows, cols, big)
                assert err < TOLERANCE, (fmt.name, mode, rows, cols, err)


def test_q4k_gemv_config1_tolerance(hip):
    """BASELINE config 1 at full size (8192 x 2048) within the 1e-3 relative bound."""
    rng = np.random.default_rng(0x9E3779B97F4A7C15)
    w = q4k_matrix(rng, 8192, 2048)
    x = rng.standard_normal(2048).astype(np.float32)
    oracle.set_threads(8)
    want = oracle.matvec(12, w, 8192, 2048, x)
    wb, xb, yb = hip.buffer_from(w), hip.buffer_from(x), hip.new_buffer(8192 * 4)
    hip.begin()
    hip.matvec(Format.Q4K, wb.at(0), 8192, 2048, xb.at(0), yb.at(0))
    hip.end()
    got = hip.read(yb.at(0), np.empty(8192, np.float32))
    scale = term_scale(Format.Q4K, w, 8192, 2048, x)
    assert np.abs(got - want).max() / scale < TOLERANCE
    rel = np.abs(got - want) / np.maximum(np.abs(want), 1e-30)
    # Per-element relative error away from cancellation.
    big = np.abs(want) > 1e-2 * np.abs(want).max()
    assert rel[big].max() < 1e-3


@pytest.mark.parametrize("cols", [2048, 4096])
def test_q4k_gemv_block_dynamic_range(hip, cols):
    """Inputs whose 32-element blocks mix magnitudes 1e6 apart (one value of
    ~1e3 among values of ~1e-3).  The Q4_K decode GEMV quantises each block's
    inputs to 22-bit fixed point relative to the block's largest |x| < 2^E,
    an absolute error of at most 2^(E-22) per input.  Checked against the
    oracle at the reference's term-scale bound (metal_matvec.rs:16-19), and
    every row against that quantisation bound itself: |err_r| <=
    sum over blocks b of sum_l |w_rl| * 2^(E_b - 22), plus the reference's
    1e-5 of the row's own term scale for the f32 arithmetic."""
    rows = 2048
    rng = np.random.default_rng(31)
    w = q4k_matrix(rng, rows, cols)
    x = (rng.standard_normal(cols) * 1e-3).astype(np.float32)
    blocks = x.reshape(-1, 32)
    big_at = rng.integers(0, 32, blocks.shape[0])
    blocks[np.arange(blocks.shape[0]), big_at] = (rng.choice([-1.0, 1.0], blocks.shape[0]) *
                                                  rng.uniform(500, 1500, blocks.shape[0])).astype(np.float32)
    x = blocks.reshape(-1)
    oracle.set_threads(8)
    want = oracle.matvec(12, w, rows, cols, x).astype(np.float64)
    wb, xb, yb = hip.buffer_from(w), hip.buffer_from(x), hip.new_buffer(rows * 4)
    hip.begin()
    hip.matvec(Format.Q4K, wb.at(0), rows, cols, xb.at(0), yb.at(0))
    hip.end()
    got = hip.read(yb.at(0), np.empty(rows, np.float32)).astype(np.float64)
    err = np.abs(got - want)
    assert err.max() / term_scale(Format.Q4K, w, rows, cols, x) < TOLERANCE
    wd = np.abs(dense(Format.Q4K, w, rows, cols).astype(np.float64))
    exp = np.frexp(np.abs(blocks.astype(np.float64)).max(axis=1))[1]  # max|x| < 2^E
    quant = wd.reshape(rows, -1, 32).sum(axis=2) @ np.ldexp(1.0, exp - 22)
    accum = TOLERANCE * (wd @ np.abs(x.astype(np.float64)))  # f32 arithmetic, per row
    assert (err <= quant + accum).all(), float((err / (quant + accum)).max())
    print(f"dynamic range {cols} cols: worst error {float((err / (quant + accum)).max()):.3g} of the bound")


@pytest.mark.parametrize("fmt,nbytes,ne,scales", [
    (Format.Q4K, 144, 256, [0, 2]), (Format.Q5K, 176, 256, [0, 2]), (Format.Q6K, 210, 256, [208]),
    (Format.Q8_0, 34, 32, [0]), (Format.Q4_0, 18, 32, [0]), (Format.F16, 2, 1, []),
    (Format.BF16, 2, 1, []), (Format.F32, 4, 1, []),
])
def test_dequantize_bit_exact(hip, fmt, nbytes, ne, scales):
    rnd = Random(0x9E3779B97F4A7C15 ^ int(fmt))
    rows, cols = 9, 512
    if ne > 1:
        w = rnd.blocks(rows * cols // ne * nbytes, nbytes, scales)
    else:
        w = np.random.default_rng(int(fmt)).standard_normal(rows * cols).astype(
            np.float32 if fmt == Format.F32 else np.float16)
        if fmt == Format.BF16:
            w = (np.random.default_rng(3).standard_normal(rows * cols).astype(np.float32)
                 .view(np.uint32) >> 16).astype(np.uint16)
        w = w.view(np.uint8)
    want = oracle.dequantize(int(fmt), w, rows * cols)
    wb, ob = hip.buffer_from(w), hip.new_buffer(rows * cols * 4)
    hip.begin()
    hip.dequantize(fmt, wb.at(0), rows, cols, ob.at(0))
    hip.end()
    got = hip.read(ob.at(0), np.empty(rows * cols, np.float32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_q4k_config1_bit_exact(hip):
    rng = np.random.default_rng(5)
    w = q4k_matrix(rng, 512, 2048)
    want = oracle.dequantize(12, w, 512 * 2048)
    wb, ob = hip.buffer_from(w), hip.new_buffer(512 * 2048 * 4)
    hip.begin()
    hip.dequantize(Format.Q4K, wb.at(0), 512, 2048, ob.at(0))
    hip.end()
    got = hip.read(ob.at(0), np.empty(512 * 2048, np.float32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
