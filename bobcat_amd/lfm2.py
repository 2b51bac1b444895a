"""LFM2 on the MI355X backend: configs, random-init weights, and `Lfm2Hip`,
the Python mirror of the C driver (bch_lfm2_*), itself the counterpart of
`Lfm2Metal` (crates/bobcat/src/lfm2_metal.rs:125-779).

There are no checkpoints offline, so models are random-init with the
reference architecture's shapes (lfm2.rs:17-49, 150-170, 868-1004): Q4_K
matrices from the BASELINE config-1 block distribution, F32 norms and
convolution taps, and a tied output matrix.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from ._lib import EMIT_FN, Lfm2Layer, Lfm2Model, Matrix, check, lib
from .backend import Format, Hip
from .synth import block_matrix, q4k_matrix


@dataclass
class Lfm2Config:
    """lfm2::Hyperparameters plus the layer pattern."""
    name: str
    n_embd: int
    n_ff: int
    n_heads: int
    n_kv_heads: int
    n_vocab: int
    attention_layers: list
    n_layers: int
    head_dim: int = 64
    conv_kernel: int = 3
    rope_theta: float = 1e6
    norm_eps: float = 1e-5
    embd_format: int = Format.Q4K
    layer_format: int = Format.Q4K
    # Mixture of experts (lfm2.rs:17-49): layers from n_dense_layers on use
    # n_experts experts of width n_ff_expert, n_experts_used per token.
    n_experts: int = 0
    n_experts_used: int = 0
    n_ff_expert: int = 0
    n_dense_layers: int = 0
    # Per-tensor formats overriding layer_format/embd_format, keyed by tensor
    # name ("wv") or layer and name ("3.down"), as real Q4_K_M files mix
    # formats (lfm2_reference.rs:45-49).
    tensor_formats: dict = field(default_factory=dict)

    def format_of(self, key: str, default: int) -> int:
        return self.tensor_formats.get(key, self.tensor_formats.get(key.split(".", 1)[-1], default))

    def is_moe(self, il: int) -> bool:
        return self.n_experts > 0 and il >= self.n_dense_layers

    @property
    def hp(self) -> dict:
        return dict(n_layers=self.n_layers, n_embd=self.n_embd, n_ff=self.n_ff, n_heads=self.n_heads,
                    n_kv_heads=self.n_kv_heads, head_dim=self.head_dim, n_vocab=self.n_vocab,
                    conv_kernel=self.conv_kernel)

    def weight_bytes(self) -> dict:
        """Bytes of the matrices a decode step streams (for roofline accounting)."""
        rb = lambda fmt, cols: cols // 256 * 144 if fmt == Format.Q4K else cols * (2 if fmt == Format.F16 else 4)
        n, q, kv = self.n_embd, self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim
        layers = 0
        for il in range(self.n_layers):
            if il in self.attention_layers:
                layers += (q + 2 * kv) * rb(self.layer_format, n) + n * rb(self.layer_format, q)
            else:
                layers += 3 * n * rb(self.layer_format, n) + n * rb(self.layer_format, n)
            if self.is_moe(il):  # the router (F32) and the picked experts
                layers += self.n_experts * n * 4 + self.n_experts_used * (
                    2 * self.n_ff_expert * rb(self.layer_format, n) + n * rb(self.layer_format, self.n_ff_expert))
            else:
                layers += 2 * self.n_ff * rb(self.layer_format, n) + n * rb(self.layer_format, self.n_ff)
        output = self.n_vocab * rb(self.embd_format, n)
        return dict(layers=layers, output=output, total=layers + output)


# LFM2-style 350M (10 conv + 6 GQA layers, fp16 tied
# embedding).  The attention layers sit where LFM2-350M keeps them.
LFM2_350M = Lfm2Config("lfm2-350m", n_embd=1024, n_ff=4608, n_heads=16, n_kv_heads=8, n_vocab=65536,
                       attention_layers=[2, 5, 8, 10, 12, 14], n_layers=16, embd_format=Format.F16)
# LFM2-style 2.6B (22 conv + 8 GQA layers, Q4_K tied
# embedding); the 8 attention layers are spread over the stack.
LFM2_2_6B = Lfm2Config("lfm2-2.6b", n_embd=2048, n_ff=10752, n_heads=32, n_kv_heads=8, n_vocab=65536,
                       attention_layers=[2, 5, 8, 12, 16, 20, 24, 27], n_layers=30)
# Small shapes for parity tests against the CPU oracle.
LFM2_TINY = Lfm2Config("lfm2-tiny", n_embd=256, n_ff=512, n_heads=4, n_kv_heads=2, n_vocab=1000,
                       attention_layers=[1, 3], n_layers=4)
LFM2_TINY_F16 = Lfm2Config("lfm2-tiny-f16", n_embd=256, n_ff=768, n_heads=4, n_kv_heads=1, n_vocab=777,
                           attention_layers=[0, 2], n_layers=3, embd_format=Format.F16)
# LFM2-style 8B-A1B (18 conv + 6 GQA layers; the
# first 2 layers dense, the rest 32 experts, top 4, expert width 1792).
LFM2_8B_A1B = Lfm2Config("lfm2-8b-a1b", n_embd=2048, n_ff=7168, n_heads=32, n_kv_heads=8, n_vocab=65536,
                         attention_layers=[2, 6, 10, 14, 18, 21], n_layers=24, n_experts=32, n_experts_used=4,
                         n_ff_expert=1792, n_dense_layers=2)
LFM2_TINY_MOE = Lfm2Config("lfm2-tiny-moe", n_embd=256, n_ff=512, n_heads=4, n_kv_heads=2, n_vocab=1000,
                           attention_layers=[1, 3], n_layers=4, n_experts=8, n_experts_used=2, n_ff_expert=256,
                           n_dense_layers=1)
# A tiny model whose tensors mix the formats of real files: attn_v and the
# tied embedding in Q6_K (as Q4_K_M files keep them), Q8_0, Q4_0 and Q5_K
# matrices elsewhere.
LFM2_TINY_MIXED = Lfm2Config("lfm2-tiny-mixed", n_embd=256, n_ff=512, n_heads=4, n_kv_heads=2, n_vocab=1000,
                             attention_layers=[1, 3], n_layers=4,
                             tensor_formats={"wv": Format.Q6K, "token_embd": Format.Q6K, "0.out_proj": Format.Q8_0,
                                             "1.wo": Format.Q4_0, "2.down": Format.Q6K, "3.up": Format.Q5K,
                                             "3.gate": Format.Q5K, "0.in_proj": Format.Q8_0})
# A tiny model with 16 query heads of 64 (a 1,024-wide attention output, as
# LFM2-350M's), so its decode takes the short-context form whose out
# projection combines the attention splits (positions below 1,024 with an
# f16 cache).
LFM2_TINY_WIDE = Lfm2Config("lfm2-tiny-wide", n_embd=256, n_ff=512, n_heads=16, n_kv_heads=4, n_vocab=1000,
                            attention_layers=[0, 2], n_layers=3)
CONFIGS = {c.name: c for c in (LFM2_350M, LFM2_2_6B, LFM2_TINY, LFM2_TINY_F16, LFM2_8B_A1B, LFM2_TINY_MOE,
                               LFM2_TINY_MIXED, LFM2_TINY_WIDE)}


def _matrix(fmt: int, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    if fmt == Format.Q4K:
        return q4k_matrix(rng, rows, cols)
    if fmt in (Format.Q4_0, Format.Q8_0, Format.Q5K, Format.Q6K):
        return block_matrix(rng, int(fmt), rows, cols)
    if fmt == Format.F16:
        return rng.standard_normal(rows * cols, dtype=np.float32).astype(np.float16).view(np.uint8)
    return rng.standard_normal(rows * cols, dtype=np.float32).view(np.uint8)


@dataclass
class Lfm2Weights:
    """Host tensors of a random-init model and the bch_lfm2_model struct over them."""
    cfg: Lfm2Config
    seed: int = 0
    arrays: dict = field(default_factory=dict)

    def __post_init__(self):
        cfg, rng = self.cfg, np.random.default_rng(self.seed)
        n, q, kv = cfg.n_embd, cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        a = self.arrays
        vec = lambda size, spread: (1.0 + spread * rng.uniform(-1, 1, size)).astype(np.float32)
        self._layers = (Lfm2Layer * cfg.n_layers)()
        fp = lambda arr: arr.ctypes.data_as(C.POINTER(C.c_float))

        def mat(key, fmt, rows, cols):
            fmt = cfg.format_of(key, fmt)
            a[key] = _matrix(fmt, rows, cols, rng)
            return Matrix(int(fmt), rows, cols, a[key].ctypes.data)

        lf = cfg.layer_format
        for il in range(cfg.n_layers):
            L = self._layers[il]
            a[f"{il}.attn_norm"] = vec(n, 0.1)
            a[f"{il}.ffn_norm"] = vec(n, 0.1)
            L.attn_norm, L.ffn_norm = fp(a[f"{il}.attn_norm"]), fp(a[f"{il}.ffn_norm"])
            if il in cfg.attention_layers:
                L.is_attention = 1
                L.wq = mat(f"{il}.wq", lf, q, n)
                L.wk = mat(f"{il}.wk", lf, kv, n)
                L.wv = mat(f"{il}.wv", lf, kv, n)
                L.wo = mat(f"{il}.wo", lf, n, q)
                a[f"{il}.q_norm"] = vec(cfg.head_dim, 0.1)
                a[f"{il}.k_norm"] = vec(cfg.head_dim, 0.1)
                L.q_norm, L.k_norm = fp(a[f"{il}.q_norm"]), fp(a[f"{il}.k_norm"])
            else:
                L.in_proj = mat(f"{il}.in_proj", lf, 3 * n, n)
                L.out_proj = mat(f"{il}.out_proj", lf, n, n)
                a[f"{il}.taps"] = rng.uniform(-0.5, 0.5, n * cfg.conv_kernel).astype(np.float32)
                L.conv_taps = fp(a[f"{il}.taps"])
            if cfg.is_moe(il):
                L.is_moe = 1
                ne, nff = cfg.n_experts, cfg.n_ff_expert
                # Router logits ~N(0, 1) on a normalised token.
                a[f"{il}.router"] = (rng.standard_normal(ne * n) / np.sqrt(n)).astype(np.float32)
                L.router = Matrix(int(Format.F32), ne, n, a[f"{il}.router"].ctypes.data)
                a[f"{il}.expert_bias"] = rng.uniform(-0.05, 0.05, ne).astype(np.float32)
                L.expert_bias = fp(a[f"{il}.expert_bias"])
                L.gate_exps = mat(f"{il}.gate_exps", lf, ne * nff, n)
                L.up_exps = mat(f"{il}.up_exps", lf, ne * nff, n)
                L.down_exps = mat(f"{il}.down_exps", lf, ne * n, nff)
            else:
                L.gate = mat(f"{il}.gate", lf, cfg.n_ff, n)
                L.up = mat(f"{il}.up", lf, cfg.n_ff, n)
                L.down = mat(f"{il}.down", lf, n, cfg.n_ff)
        embd = mat("token_embd", cfg.embd_format, cfg.n_vocab, n)
        a["output_norm"] = vec(n, 0.1)
        self.c_model = Lfm2Model(
            n_layers=cfg.n_layers, n_embd=n, n_ff=cfg.n_ff, n_experts=cfg.n_experts,
            n_experts_used=cfg.n_experts_used, n_ff_expert=cfg.n_ff_expert,
            n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads, head_dim=cfg.head_dim, n_vocab=cfg.n_vocab,
            conv_kernel=cfg.conv_kernel, rope_theta=cfg.rope_theta, norm_eps=cfg.norm_eps,
            layers=self._layers, token_embd=embd, output=embd, output_norm=fp(a["output_norm"]))

    @property
    def hp(self) -> dict:
        return self.cfg.hp


class SequenceHip:
    """One sequence of a model driver on the GPU (the API of Lfm2Metal and
    Qwen35Metal); subclasses name the C functions' prefix."""
    _prefix = ""

    def _fn(self, name: str):
        return getattr(lib(), self._prefix + name)

    def __init__(self, hip: Hip, weights: Lfm2Weights, n_ctx: int, kv_half: bool = True):
        self.hip, self.weights, self.cfg = hip, weights, weights.cfg
        h = C.c_void_p()
        check(self._fn("new")(hip.handle, C.byref(weights.c_model), n_ctx, int(kv_half), C.byref(h)))
        self.handle = h.value
        self.n_ctx = n_ctx
        hip._dependents.add(self)

    def close(self):
        if self.handle:
            self._fn("free")(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def n_past(self) -> int:
        return self._fn("n_past")(self.handle)

    @property
    def last_gpu_seconds(self) -> float:
        return self._fn("last_gpu_seconds")(self.handle)

    def reset(self) -> None:
        check(self._fn("reset")(self.handle))

    def step(self, token: int, logits: bool = True, trace: bool = False):
        cfg = self.cfg
        lg = np.empty(cfg.n_vocab, np.float32) if logits else None
        te = np.empty(cfg.n_embd, np.float32) if trace else None
        tl = np.empty(cfg.n_layers * cfg.n_embd, np.float32) if trace else None
        tf = np.empty(cfg.n_embd, np.float32) if trace else None
        ptr = lambda a: None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))
        check(self._fn("step")(self.handle, token, ptr(lg), ptr(te), ptr(tl), ptr(tf)))
        return (lg, (te, tl, tf)) if trace else lg

    def prefill(self, tokens, logits: bool = True, trace: bool = False):
        """Returns the last token's logits, or (logits, (embedding, layers, final)) with
        `trace`: embedding and final [n_tokens, n_embd], layers [n_layers, n_tokens, n_embd]."""
        cfg = self.cfg
        t = np.ascontiguousarray(tokens, np.uint32)
        lg = np.empty(cfg.n_vocab, np.float32) if logits else None
        te = np.empty((t.size, cfg.n_embd), np.float32) if trace else None
        tl = np.empty((cfg.n_layers, t.size, cfg.n_embd), np.float32) if trace else None
        tf = np.empty((t.size, cfg.n_embd), np.float32) if trace else None
        ptr = lambda a: None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))
        check(self._fn("prefill")(self.handle, t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size,
                                     ptr(lg), ptr(te), ptr(tl), ptr(tf)))
        return (lg, (te, tl, tf)) if trace else lg

    def greedy_token(self) -> int:
        t = C.c_uint32()
        check(self._fn("greedy_token")(self.handle, C.byref(t)))
        return t.value

    def generate(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        check(self._fn("generate")(self.handle, out.ctypes.data_as(C.POINTER(C.c_uint32)), n))
        return out

    def generate_next(self, n: int) -> np.ndarray:
        """Lfm2Metal::generate_next: consume the current selection and n - 1 more; the
        selection after each of the n steps."""
        out = np.empty(max(n, 1), np.uint32)
        check(self._fn("generate_next")(self.handle, out.ctypes.data_as(C.POINTER(C.c_uint32)), n))
        return out[:n]

    def generate_stream(self, max_tokens: int, emit) -> list:
        """Lfm2Metal::generate_stream: emit(token) -> bool per selected token; returns the
        tokens the sequence gained (every emitted token but the last, and possibly tokens
        selected after it)."""
        errors = []

        def cb(token, _user):
            try:
                return 1 if emit(int(token)) else 0
            except Exception as e:  # an exception in emit stops the stream and is re-raised
                errors.append(e)
                return 0

        fn = EMIT_FN(cb)
        gained = np.empty(max(max_tokens, 1), np.uint32)
        n = C.c_uint32()
        check(self._fn("generate_stream")(self.handle, max_tokens, fn, None,
                                          gained.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(n)))
        if errors:
            raise errors[0]
        return gained[:n.value].tolist()

    def generate_sampled(self, n: int, settings, seed: int) -> np.ndarray:
        """n tokens drawn by the GPU sampler (settings: a bch_sampling)."""
        out = np.empty(n, np.uint32)
        check(self._fn("generate_sampled")(self.handle, out.ctypes.data_as(C.POINTER(C.c_uint32)), n,
                                              C.byref(settings), seed))
        return out

    def checkpoint(self) -> bytes:
        nb = self._fn("checkpoint_bytes")(self.handle)
        buf = (C.c_uint8 * nb)()
        check(self._fn("checkpoint")(self.handle, buf, nb))
        return bytes(buf)

    def restore(self, blob: bytes) -> None:
        buf = (C.c_uint8 * len(blob)).from_buffer_copy(blob)
        check(self._fn("restore")(self.handle, buf, len(blob)))


class Lfm2Hip(SequenceHip):
    """bch_lfm2: one LFM2 sequence on the GPU (Lfm2Metal's API)."""
    _prefix = "bch_lfm2_"
