"""Input generators restated from the reference's kernel tests.

`Random` is the xorshift64 of crates/bobcat/tests/metal_matvec.rs:57-92
(seeds at :256 and :284); the deterministic patterns are those of
crates/bobcat/tests/metal_matmul.rs:29-64 and metal_attention.rs:19-48.
"""
from __future__ import annotations

import numpy as np

MASK = (1 << 64) - 1


class Random:
    def __init__(self, seed: int):
        self.s = seed & MASK

    def next(self) -> int:
        s = self.s
        s ^= (s << 13) & MASK
        s ^= s >> 7
        s ^= (s << 17) & MASK
        self.s = s
        return s

    def unit(self) -> float:
        """A float in [-1, 1): 24 random bits, exact in f32 (metal_matvec.rs:68-71)."""
        return np.float32((self.next() >> 40) / (1 << 23) - 1.0)

    def units(self, n: int) -> np.ndarray:
        return np.array([self.unit() for _ in range(n)], np.float32)

    def scale_bits(self) -> int:
        """fp16 bits of a scale in [2^-10, 2^-6) (metal_matvec.rs:75-79)."""
        exponent = 5 + self.next() % 4
        mantissa = self.next() & 0x3FF
        return (exponent << 10) | mantissa

    def blocks(self, n_bytes: int, block_bytes: int, scales) -> np.ndarray:
        """Random blocks with an fp16 scale at each offset in `scales` (:83-91)."""
        out = np.array([self.next() & 0xFF for _ in range(n_bytes)], np.uint8)
        blocks = out.reshape(-1, block_bytes)
        for b in blocks:
            for at in scales:
                v = self.scale_bits()
                b[at] = v & 0xFF
                b[at + 1] = v >> 8
        return out


def matmul_q4k_weights(n_rows: int, n_cols: int) -> np.ndarray:
    """Deterministic Q4_K blocks of metal_matmul.rs:29-58: d = dmin = fp16
    0x3000 (0.125), scale bytes 0x11, quants (block*17 + i*13) % 251."""
    n_blocks = n_rows * n_cols // 256
    out = np.zeros((n_blocks, 144), np.uint8)
    out[:, 0:2] = [0x00, 0x30]
    out[:, 2:4] = [0x00, 0x30]
    out[:, 4:16] = 0x11
    b = np.arange(n_blocks)[:, None]
    i = np.arange(128)[None, :]
    out[:, 16:] = ((b * 17 + i * 13) % 251).astype(np.uint8)
    return out.reshape(-1)


def matmul_inputs(n_tokens: int, n_cols: int, divisor: float = 64.0) -> np.ndarray:
    i = np.arange(n_tokens * n_cols)
    return (((i * 19) % 97 - 48) / divisor).astype(np.float32)
