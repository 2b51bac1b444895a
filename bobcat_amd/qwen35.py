"""Qwen3.5 on the MI355X backend: configs, random-init weights, and `Qwen35Hip`,
the Python mirror of the C driver (bch_qwen35_*), itself the counterpart of
`Qwen35Metal` (crates/bobcat/src/qwen35_metal.rs).

Models are random-init with the reference architecture's shapes
(qwen35.rs:31-145): three Gated DeltaNet layers to one gated-attention layer,
Q4_K matrices, F32 norms (stored as the GGUF does, the +1 of the zero-centred
norms baked in), F32 convolution taps, and a tied output matrix.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._lib import Matrix, Qwen35Layer, Qwen35Model, check, lib
from .backend import Format, Hip
from .lfm2 import SequenceHip, _matrix


@dataclass
class Qwen35Config:
    """qwen35::Hyperparameters plus the layer pattern."""
    name: str
    n_embd: int
    n_ff: int
    n_vocab: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    n_rot: int
    n_k_heads: int
    n_v_heads: int
    k_head_dim: int
    v_head_dim: int
    conv_kernel: int = 4
    rope_theta: float = 1e7
    norm_eps: float = 1e-6
    attention_every: int = 4  # layer il is attention when (il + 1) % attention_every == 0
    embd_format: int = Format.Q4K
    layer_format: int = Format.Q4K

    def is_attention(self, il: int) -> bool:
        return (il + 1) % self.attention_every == 0

    @property
    def key_dim(self) -> int:
        return self.n_k_heads * self.k_head_dim

    @property
    def value_dim(self) -> int:
        return self.n_v_heads * self.v_head_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    @property
    def hp(self) -> dict:
        return dict(n_layers=self.n_layers, n_embd=self.n_embd, n_vocab=self.n_vocab)

    def weight_bytes(self) -> dict:
        """Bytes a decode step streams: matrices, output, and the DeltaNet states read and written."""
        rb = lambda fmt, cols: cols // 256 * 144 if fmt == Format.Q4K else cols * (2 if fmt == Format.F16 else 4)
        n, lf = self.n_embd, self.layer_format
        q, kv = self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim
        layers = state = 0
        for il in range(self.n_layers):
            if self.is_attention(il):
                layers += (2 * q + 2 * kv) * rb(lf, n) + n * rb(lf, q)
            else:
                layers += (self.conv_dim + self.value_dim + 2 * self.n_v_heads) * rb(lf, n) + n * rb(lf, self.value_dim)
                state += 2 * self.n_v_heads * self.k_head_dim * self.v_head_dim * 4
            layers += 2 * self.n_ff * rb(lf, n) + n * rb(lf, self.n_ff)
        output = self.n_vocab * rb(self.embd_format, n)
        return dict(layers=layers, output=output, state=state, total=layers + output + state)


# Qwen3.5-style 0.8B (18 DeltaNet + 6 gated attention).
QWEN35_0_8B = Qwen35Config("qwen3.5-0.8b", n_embd=1024, n_ff=3584, n_vocab=151936, n_layers=24, n_heads=8,
                           n_kv_heads=2, head_dim=256, n_rot=64, n_k_heads=16, n_v_heads=16, k_head_dim=128,
                           v_head_dim=128)
# Small shapes for parity tests against the CPU oracle.
QWEN35_TINY = Qwen35Config("qwen3.5-tiny", n_embd=256, n_ff=512, n_vocab=1000, n_layers=4, n_heads=2,
                           n_kv_heads=1, head_dim=256, n_rot=64, n_k_heads=2, n_v_heads=2, k_head_dim=128,
                           v_head_dim=128)
QWEN35_TINY_64 = Qwen35Config("qwen3.5-tiny-64", n_embd=256, n_ff=768, n_vocab=777, n_layers=4, n_heads=4,
                              n_kv_heads=2, head_dim=64, n_rot=32, n_k_heads=2, n_v_heads=4, k_head_dim=64,
                              v_head_dim=64)
# Value heads of 256 with key heads of 64, and of 192 with 128: the decode
# step's 1024- and 768-lane workgroups with the fused gated norm.
QWEN35_TINY_V256 = Qwen35Config("qwen3.5-tiny-v256", n_embd=256, n_ff=512, n_vocab=500, n_layers=4, n_heads=2,
                                n_kv_heads=1, head_dim=128, n_rot=64, n_k_heads=1, n_v_heads=2, k_head_dim=64,
                                v_head_dim=256)
QWEN35_TINY_V192 = Qwen35Config("qwen3.5-tiny-v192", n_embd=256, n_ff=512, n_vocab=500, n_layers=4, n_heads=2,
                                n_kv_heads=1, head_dim=128, n_rot=32, n_k_heads=2, n_v_heads=4, k_head_dim=128,
                                v_head_dim=192)
# Eight value heads of 128 (1,024 values, as the 0.8B's 2,048): the decode
# step's gated norm staged by the out projection's slab launch.
QWEN35_TINY_V1024 = Qwen35Config("qwen3.5-tiny-v1024", n_embd=256, n_ff=512, n_vocab=500, n_layers=4, n_heads=2,
                                 n_kv_heads=1, head_dim=128, n_rot=64, n_k_heads=4, n_v_heads=8, k_head_dim=128,
                                 v_head_dim=128)
CONFIGS = {c.name: c for c in (QWEN35_0_8B, QWEN35_TINY, QWEN35_TINY_64, QWEN35_TINY_V256, QWEN35_TINY_V192,
                               QWEN35_TINY_V1024)}


@dataclass
class Qwen35Weights:
    """Host tensors of a random-init model and the bch_qwen35_model struct over them."""
    cfg: Qwen35Config
    seed: int = 0
    arrays: dict = field(default_factory=dict)

    def __post_init__(self):
        cfg, rng = self.cfg, np.random.default_rng(self.seed)
        n, q, kv = cfg.n_embd, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        a = self.arrays
        vec = lambda size, spread: (1.0 + spread * rng.uniform(-1, 1, size)).astype(np.float32)
        self._layers = (Qwen35Layer * cfg.n_layers)()
        fp = lambda arr: arr.ctypes.data_as(C.POINTER(C.c_float))

        def mat(key, fmt, rows, cols):
            a[key] = _matrix(fmt, rows, cols, rng)
            return Matrix(int(fmt), rows, cols, a[key].ctypes.data)

        def keep(key, arr):
            a[key] = np.ascontiguousarray(arr, np.float32)
            return fp(a[key])

        lf = cfg.layer_format
        for il in range(cfg.n_layers):
            L = self._layers[il]
            L.attn_norm = keep(f"{il}.attn_norm", vec(n, 0.1))
            L.ffn_norm = keep(f"{il}.ffn_norm", vec(n, 0.1))
            if cfg.is_attention(il):
                L.is_attention = 1
                L.wq = mat(f"{il}.wq", lf, 2 * q, n)
                L.wk = mat(f"{il}.wk", lf, kv, n)
                L.wv = mat(f"{il}.wv", lf, kv, n)
                L.wo = mat(f"{il}.wo", lf, n, q)
                L.q_norm = keep(f"{il}.q_norm", vec(cfg.head_dim, 0.1))
                L.k_norm = keep(f"{il}.k_norm", vec(cfg.head_dim, 0.1))
            else:
                L.qkv = mat(f"{il}.qkv", lf, cfg.conv_dim, n)
                L.z = mat(f"{il}.z", lf, cfg.value_dim, n)
                L.beta = mat(f"{il}.beta", lf, cfg.n_v_heads, n)
                L.alpha = mat(f"{il}.alpha", lf, cfg.n_v_heads, n)
                L.conv_taps = keep(f"{il}.conv", rng.uniform(-0.5, 0.5, cfg.conv_dim * cfg.conv_kernel))
                L.dt_bias = keep(f"{il}.dt_bias", rng.uniform(-1, 1, cfg.n_v_heads))
                # -exp(A_log) with A_log ~ U(-2, 1), decays between ~0.1 and ~1.
                L.a = keep(f"{il}.a", -np.exp(rng.uniform(-2, 1, cfg.n_v_heads)))
                L.ssm_norm = keep(f"{il}.ssm_norm", vec(cfg.v_head_dim, 0.1))
                L.out = mat(f"{il}.out", lf, n, cfg.value_dim)
            L.gate = mat(f"{il}.gate", lf, cfg.n_ff, n)
            L.up = mat(f"{il}.up", lf, cfg.n_ff, n)
            L.down = mat(f"{il}.down", lf, n, cfg.n_ff)
        embd = mat("token_embd", cfg.embd_format, cfg.n_vocab, n)
        self.c_model = Qwen35Model(
            n_layers=cfg.n_layers, n_embd=n, n_ff=cfg.n_ff, n_vocab=cfg.n_vocab, n_heads=cfg.n_heads,
            n_kv_heads=cfg.n_kv_heads, head_dim=cfg.head_dim, n_rot=cfg.n_rot, rope_theta=cfg.rope_theta,
            norm_eps=cfg.norm_eps, conv_kernel=cfg.conv_kernel, n_k_heads=cfg.n_k_heads, n_v_heads=cfg.n_v_heads,
            k_head_dim=cfg.k_head_dim, v_head_dim=cfg.v_head_dim, layers=self._layers, token_embd=embd,
            output=embd, output_norm=keep("output_norm", vec(n, 0.1)))

    @property
    def hp(self) -> dict:
        return self.cfg.hp


class Qwen35Hip(SequenceHip):
    """bch_qwen35: one Qwen3.5 sequence on the GPU (Qwen35Metal's API)."""
    _prefix = "bch_qwen35_"

    def hidden(self, tokens) -> np.ndarray:
        """Gpu::hidden: a new sequence of `tokens`; each token's final-norm row [n_tokens, n_embd]."""
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty((t.size, self.cfg.n_embd), np.float32)
        check(self._fn("hidden")(self.handle, t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size,
                                    out.ctypes.data_as(C.POINTER(C.c_float))))
        return out
