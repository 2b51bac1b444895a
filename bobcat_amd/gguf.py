"""GGUF files: the reader over the library's parser (bch_gguf_*, the
counterpart of crates/bobcat-gguf), a writer of the same format, and the
export of a random-init model in the tensor naming of real LFM2 / Qwen3.5
files (lfm2.rs:737-1004, qwen35.rs:630-745), so that a file takes the same
path into the drivers as a downloaded one (bch_*_model_from_gguf).

Format (GGUF v3, little-endian): magic "GGUF", version, tensor count,
metadata count; metadata entries (key string, type, value); tensor infos
(name, n_dims, ne[n_dims] innermost first, ggml type, offset); padding to
general.alignment (32); tensor data, each tensor at an aligned offset.
"""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np

from ._lib import GgufTensor, Lfm2Layer, Lfm2Model, Qwen35Layer, Qwen35Model, check, lib

MAGIC = 0x46554747
ALIGNMENT = 32
# Metadata value types.
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FIXED = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
          U64: "<Q", I64: "<q", F64: "<d"}
# ggml type id -> (elements per block, bytes per block)
BLOCKS = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
          14: (256, 210)}


def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


class GgufWriter:
    """Collects metadata and tensors, then writes one GGUF v3 file."""

    def __init__(self):
        self.meta: list[tuple[str, int, object]] = []
        self.tensors: list[tuple[str, tuple, int, bytes]] = []

    def add(self, key: str, vtype: int, value) -> None:
        self.meta.append((key, vtype, value))

    def add_u32(self, key, v):
        self.add(key, U32, int(v))

    def add_f32(self, key, v):
        self.add(key, F32, float(v))

    def add_string(self, key, v):
        self.add(key, STRING, v)

    def add_array(self, key, element: int, values) -> None:
        self.add(key, ARRAY, (element, list(values)))

    def add_tensor(self, name: str, shape: tuple, ggml_type: int, data) -> None:
        """shape innermost first (ne0 = row length)."""
        raw = np.ascontiguousarray(data).view(np.uint8).tobytes()
        block, nbytes = BLOCKS[ggml_type]
        n = int(np.prod(shape))
        assert shape[0] % block == 0 and n // block * nbytes == len(raw), (name, shape, ggml_type, len(raw))
        self.tensors.append((name, tuple(int(d) for d in shape), ggml_type, raw))

    @staticmethod
    def _value(vtype: int, value) -> bytes:
        if vtype == STRING:
            return _string(value)
        if vtype == ARRAY:
            element, values = value
            out = struct.pack("<IQ", element, len(values))
            for v in values:
                out += _string(v) if element == STRING else struct.pack(_FIXED[element], v)
            return out
        return struct.pack(_FIXED[vtype], value)

    def to_bytes(self) -> bytes:
        out = bytearray(struct.pack("<IIQQ", MAGIC, 3, len(self.tensors), len(self.meta)))
        for key, vtype, value in self.meta:
            out += _string(key) + struct.pack("<I", vtype) + self._value(vtype, value)
        offset = 0
        offsets = []
        for name, shape, t, raw in self.tensors:
            offsets.append(offset)
            out += _string(name) + struct.pack("<I", len(shape))
            out += b"".join(struct.pack("<Q", d) for d in shape)
            out += struct.pack("<IQ", t, offset)
            offset = (offset + len(raw) + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
        out += b"\0" * (-len(out) % ALIGNMENT)
        for (name, shape, t, raw), off in zip(self.tensors, offsets):
            out += raw
            out += b"\0" * (-len(out) % ALIGNMENT)
        return bytes(out)

    def write(self, path) -> None:
        Path(path).write_bytes(self.to_bytes())


class Gguf:
    """A parsed GGUF file (bch_gguf_open / bch_gguf_parse)."""

    def __init__(self, path=None, data: bytes | None = None):
        h = C.c_void_p()
        if path is not None:
            check(lib().bch_gguf_open(str(path).encode(), C.byref(h)))
            self._keep = None
        else:
            self._keep = C.create_string_buffer(bytes(data), len(data)) if data else None
            check(lib().bch_gguf_parse(self._keep, len(data), C.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().bch_gguf_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def u32(self, key: str) -> int:
        v = C.c_uint32()
        check(lib().bch_gguf_u32(self.handle, key.encode(), C.byref(v)))
        return v.value

    def f32(self, key: str) -> float:
        v = C.c_float()
        check(lib().bch_gguf_f32(self.handle, key.encode(), C.byref(v)))
        return v.value

    def string(self, key: str) -> bytes:
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().bch_gguf_string(self.handle, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value) if n.value else b""

    def array_u32(self, key: str) -> list:
        n = C.c_uint64()
        check(lib().bch_gguf_array_len(self.handle, key.encode(), C.byref(n)))
        out = []
        for i in range(n.value):
            v = C.c_uint32()
            check(lib().bch_gguf_array_u32(self.handle, key.encode(), i, C.byref(v)))
            out.append(v.value)
        return out

    def array_strings(self, key: str) -> list:
        n = C.c_uint64()
        check(lib().bch_gguf_array_len(self.handle, key.encode(), C.byref(n)))
        out = []
        for i in range(n.value):
            p, ln = C.c_void_p(), C.c_uint64()
            check(lib().bch_gguf_array_string(self.handle, key.encode(), i, C.byref(p), C.byref(ln)))
            out.append(C.string_at(p.value, ln.value) if ln.value else b"")
        return out

    def tensor(self, name: str) -> GgufTensor:
        t = GgufTensor()
        check(lib().bch_gguf_tensor(self.handle, name.encode(), C.byref(t)))
        return t

    def tensors(self) -> list:
        out = []
        for i in range(lib().bch_gguf_n_tensors(self.handle)):
            t = GgufTensor()
            check(lib().bch_gguf_tensor_at(self.handle, i, C.byref(t)))
            out.append(t)
        return out

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = self.tensor(name)
        return np.frombuffer(C.string_at(t.data, t.bytes), np.uint8)

    def lfm2_model(self):
        """(bch_lfm2_model, layers) filled from the file (bch_lfm2_model_from_gguf)."""
        layers = (Lfm2Layer * 512)()
        m = Lfm2Model()
        check(lib().bch_lfm2_model_from_gguf(self.handle, C.byref(m), layers, 512))
        return m, layers

    def qwen35_model(self):
        layers = (Qwen35Layer * 512)()
        m = Qwen35Model()
        check(lib().bch_qwen35_model_from_gguf(self.handle, C.byref(m), layers, 512))
        return m, layers


class GgufWeights:
    """A model loaded from a GGUF file, usable wherever Lfm2Weights /
    Qwen35Weights are (it keeps the file mapped while the struct is used)."""

    def __init__(self, path, cfg):
        self.gguf = Gguf(path)
        self.cfg = cfg
        if hasattr(cfg, "n_k_heads"):
            self.c_model, self._layers = self.gguf.qwen35_model()
        else:
            self.c_model, self._layers = self.gguf.lfm2_model()

    @property
    def hp(self) -> dict:
        return self.cfg.hp


def _vector(w: GgufWriter, name: str, arr: np.ndarray, shape=None) -> None:
    a = np.ascontiguousarray(arr, np.float32)
    w.add_tensor(name, shape or (a.size,), 0, a)


def lfm2_to_gguf(weights, path) -> None:
    """Write a random-init LFM2 model (bobcat_amd.lfm2.Lfm2Weights) as an
    "lfm2" / "lfm2moe" GGUF file with the tensor names of real files."""
    cfg, a = weights.cfg, weights.arrays
    moe = cfg.n_experts > 0
    arch = "lfm2moe" if moe else "lfm2"
    w = GgufWriter()
    w.add_string("general.architecture", arch)
    w.add_u32("general.alignment", ALIGNMENT)
    w.add_u32(f"{arch}.block_count", cfg.n_layers)
    w.add_u32(f"{arch}.embedding_length", cfg.n_embd)
    w.add_u32(f"{arch}.feed_forward_length", cfg.n_ff)
    w.add_u32(f"{arch}.attention.head_count", cfg.n_heads)
    w.add_array(f"{arch}.attention.head_count_kv", U32,
                [cfg.n_kv_heads if il in cfg.attention_layers else 0 for il in range(cfg.n_layers)])
    w.add_u32(f"{arch}.shortconv.l_cache", cfg.conv_kernel)
    w.add_f32(f"{arch}.rope.freq_base", cfg.rope_theta)
    w.add_f32(f"{arch}.attention.layer_norm_rms_epsilon", cfg.norm_eps)
    if moe:
        w.add_u32(f"{arch}.expert_gating_func", 2)
        w.add_u32(f"{arch}.expert_count", cfg.n_experts)
        w.add_u32(f"{arch}.expert_used_count", cfg.n_experts_used)
        w.add_u32(f"{arch}.expert_feed_forward_length", cfg.n_ff_expert)
        w.add_u32(f"{arch}.leading_dense_block_count", cfg.n_dense_layers)
    n, hd = cfg.n_embd, cfg.head_dim

    def mat(name, key, rows, cols, experts=None):
        fmt = cfg.format_of(key, cfg.layer_format if key != "token_embd" else cfg.embd_format)
        shape = (cols, rows) if experts is None else (cols, rows // experts, experts)
        w.add_tensor(name, shape, int(fmt), a[key])

    for il in range(cfg.n_layers):
        b = f"blk.{il}."
        _vector(w, b + "attn_norm.weight", a[f"{il}.attn_norm"])
        _vector(w, b + "ffn_norm.weight", a[f"{il}.ffn_norm"])
        if il in cfg.attention_layers:
            q, kv = cfg.n_heads * hd, cfg.n_kv_heads * hd
            mat(b + "attn_q.weight", f"{il}.wq", q, n)
            mat(b + "attn_k.weight", f"{il}.wk", kv, n)
            mat(b + "attn_v.weight", f"{il}.wv", kv, n)
            mat(b + "attn_output.weight", f"{il}.wo", n, q)
            _vector(w, b + "attn_q_norm.weight", a[f"{il}.q_norm"])
            _vector(w, b + "attn_k_norm.weight", a[f"{il}.k_norm"])
        else:
            mat(b + "shortconv.in_proj.weight", f"{il}.in_proj", 3 * n, n)
            mat(b + "shortconv.out_proj.weight", f"{il}.out_proj", n, n)
            _vector(w, b + "shortconv.conv.weight", a[f"{il}.taps"], (cfg.conv_kernel, n))
        if cfg.is_moe(il):
            ne, nff = cfg.n_experts, cfg.n_ff_expert
            w.add_tensor(b + "ffn_gate_inp.weight", (n, ne), 0, a[f"{il}.router"])
            w.add_tensor(b + "exp_probs_b.bias", (ne,), 0, a[f"{il}.expert_bias"])
            mat(b + "ffn_gate_exps.weight", f"{il}.gate_exps", ne * nff, n, ne)
            mat(b + "ffn_up_exps.weight", f"{il}.up_exps", ne * nff, n, ne)
            mat(b + "ffn_down_exps.weight", f"{il}.down_exps", ne * n, nff, ne)
        else:
            mat(b + "ffn_gate.weight", f"{il}.gate", cfg.n_ff, n)
            mat(b + "ffn_up.weight", f"{il}.up", cfg.n_ff, n)
            mat(b + "ffn_down.weight", f"{il}.down", n, cfg.n_ff)
    mat("token_embd.weight", "token_embd", cfg.n_vocab, n)
    _vector(w, "token_embd_norm.weight", a["output_norm"])
    w.write(path)


def qwen35_to_gguf(weights, path) -> None:
    """Write a random-init Qwen3.5 model (Qwen35Weights) as a "qwen35" GGUF file."""
    cfg, a = weights.cfg, weights.arrays
    w = GgufWriter()
    w.add_string("general.architecture", "qwen35")
    w.add_u32("general.alignment", ALIGNMENT)
    w.add_u32("qwen35.block_count", cfg.n_layers)
    w.add_u32("qwen35.embedding_length", cfg.n_embd)
    w.add_u32("qwen35.feed_forward_length", cfg.n_ff)
    w.add_u32("qwen35.attention.head_count", cfg.n_heads)
    w.add_u32("qwen35.attention.head_count_kv", cfg.n_kv_heads)
    w.add_u32("qwen35.attention.key_length", cfg.head_dim)
    w.add_u32("qwen35.attention.value_length", cfg.head_dim)
    w.add_u32("qwen35.rope.dimension_count", cfg.n_rot)
    w.add_f32("qwen35.rope.freq_base", cfg.rope_theta)
    w.add_f32("qwen35.attention.layer_norm_rms_epsilon", cfg.norm_eps)
    w.add_u32("qwen35.ssm.conv_kernel", cfg.conv_kernel)
    w.add_u32("qwen35.ssm.group_count", cfg.n_k_heads)
    w.add_u32("qwen35.ssm.time_step_rank", cfg.n_v_heads)
    w.add_u32("qwen35.ssm.state_size", cfg.k_head_dim)
    w.add_u32("qwen35.ssm.inner_size", cfg.value_dim)
    n = cfg.n_embd
    lf = int(cfg.layer_format)

    def mat(name, key, rows, cols, fmt=lf):
        w.add_tensor(name, (cols, rows), fmt, a[key])

    for il in range(cfg.n_layers):
        b = f"blk.{il}."
        if cfg.is_attention(il):
            q, kv = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
            mat(b + "attn_q.weight", f"{il}.wq", 2 * q, n)
            mat(b + "attn_k.weight", f"{il}.wk", kv, n)
            mat(b + "attn_v.weight", f"{il}.wv", kv, n)
            mat(b + "attn_output.weight", f"{il}.wo", n, q)
            _vector(w, b + "attn_q_norm.weight", a[f"{il}.q_norm"])
            _vector(w, b + "attn_k_norm.weight", a[f"{il}.k_norm"])
        else:
            mat(b + "attn_qkv.weight", f"{il}.qkv", cfg.conv_dim, n)
            mat(b + "attn_gate.weight", f"{il}.z", cfg.value_dim, n)
            mat(b + "ssm_beta.weight", f"{il}.beta", cfg.n_v_heads, n)
            mat(b + "ssm_alpha.weight", f"{il}.alpha", cfg.n_v_heads, n)
            _vector(w, b + "ssm_conv1d.weight", a[f"{il}.conv"], (cfg.conv_kernel, cfg.conv_dim))
            _vector(w, b + "ssm_dt.bias", a[f"{il}.dt_bias"])
            _vector(w, b + "ssm_a", a[f"{il}.a"])
            _vector(w, b + "ssm_norm.weight", a[f"{il}.ssm_norm"])
            mat(b + "ssm_out.weight", f"{il}.out", n, cfg.value_dim)
        _vector(w, b + "attn_norm.weight", a[f"{il}.attn_norm"])
        _vector(w, b + "post_attention_norm.weight", a[f"{il}.ffn_norm"])
        mat(b + "ffn_gate.weight", f"{il}.gate", cfg.n_ff, n)
        mat(b + "ffn_up.weight", f"{il}.up", cfg.n_ff, n)
        mat(b + "ffn_down.weight", f"{il}.down", n, cfg.n_ff)
    mat("token_embd.weight", "token_embd", cfg.n_vocab, n, int(cfg.embd_format))
    _vector(w, "output_norm.weight", a["output_norm"])
    w.write(path)
