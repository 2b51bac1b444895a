"""Seeded synthetic weights in GGUF block layouts.

There is no network and no checkpoint, so benchmarks and tests run on
random-init weights of the reference architectures.  Q4_K super-blocks
follow the layout of crates/bobcat/src/scalar.rs:127-152: fp16 d and dmin,
12 bytes packing eight 6-bit (scale, min) pairs, then 128 bytes of nibbles.
"""
from __future__ import annotations

import numpy as np

Q4K_BYTES = 144
Q4K_WEIGHTS = 256


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack 6-bit scales and minimums [..., 8] into the 12 scale bytes [..., 12].

    The inverse of q4k_scale_min (scalar.rs:116-125): blocks 0-3 keep their
    low six bits in bytes j and j+4, blocks 4-7 keep their low nibbles in
    byte j+4 and their top two bits in the top bits of bytes j-4 and j.
    """
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0xF) | ((mn[..., 4:8] & 0xF) << 4)
    return out


def q4k_blocks(rng: np.random.Generator, n_blocks: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """n_blocks random Q4_K super-blocks as uint8 [n_blocks, 144].

    d and dmin ~ U(d_range) rounded to fp16, 6-bit scales and minimums
    ~ U{0..63}, nibbles ~ U{0..15}.
    """
    out = np.empty((n_blocks, Q4K_BYTES), np.uint8)
    d = rng.uniform(*d_range, size=(n_blocks, 2)).astype(np.float16)
    out[:, 0:4] = d.view(np.uint8).reshape(n_blocks, 4)
    sc = rng.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    out[:, 4:16] = pack_q4k_scales(sc, mn)
    out[:, 16:] = rng.integers(0, 256, size=(n_blocks, 128), dtype=np.uint8)
    return out


def q4k_matrix(rng: np.random.Generator, n_rows: int, n_cols: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """A random Q4_K matrix as flat uint8 bytes (row-major rows of super-blocks)."""
    assert n_cols % Q4K_WEIGHTS == 0
    n_blocks = n_rows * (n_cols // Q4K_WEIGHTS)
    # Generate in slabs so multi-GB matrices stay within memory.
    out = np.empty(n_blocks * Q4K_BYTES, np.uint8)
    slab = 1 << 20
    for start in range(0, n_blocks, slab):
        n = min(slab, n_blocks - start)
        out[start * Q4K_BYTES:(start + n) * Q4K_BYTES] = q4k_blocks(rng, n, d_range).reshape(-1)
    return out


def gemv_case(seed: int = 0x9E3779B97F4A7C15, n_rows: int = 8192, n_cols: int = 2048):
    """W [n_rows x n_cols] Q4_K and x ~ N(0,1) f32 [n_cols]."""
    rng = np.random.default_rng(seed)
    w = q4k_matrix(rng, n_rows, n_cols)
    x = rng.standard_normal(n_cols).astype(np.float32)
    return w, x


# Block layouts of the other GGUF formats: (weights per block, bytes per
# block, byte offsets of the fp16 scales, their range).
BLOCK_FORMATS = {
    2: (32, 18, [0], (2e-3, 2e-2)),            # Q4_0: d, 16 bytes of nibbles
    8: (32, 34, [0], (1e-3, 1e-2)),            # Q8_0: d, 32 int8
    13: (256, 176, [0, 2], (1e-3, 1e-2)),      # Q5_K: d, dmin, 12 scale bytes, qh[32], qs[128]
    14: (256, 210, [208], (1e-3, 1e-2)),       # Q6_K: ql[128], qh[64], 16 int8 scales, d
}


def block_matrix(rng: np.random.Generator, fmt: int, n_rows: int, n_cols: int) -> np.ndarray:
    """A random matrix of a GGUF block format as flat bytes: every byte
    uniform, then each fp16 scale field set to U(range) (for Q6_K the int8
    sub-block scales stay uniform bytes)."""
    if fmt == 12:
        return q4k_matrix(rng, n_rows, n_cols)
    ne, nb, scales, (lo, hi) = BLOCK_FORMATS[fmt]
    assert n_cols % ne == 0
    n_blocks = n_rows * n_cols // ne
    w = rng.integers(0, 256, n_blocks * nb, dtype=np.uint8).reshape(n_blocks, nb)
    for at in scales:
        w[:, at:at + 2] = rng.uniform(lo, hi, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)
