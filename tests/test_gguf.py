"""GGUF files on the CPU (no GPU needed): the library's parser
(bch_gguf_*) against the reference's malformed-file tests
(crates/bobcat-gguf/tests/malformed.rs:105-153) — a small valid file parses,
every truncation of it fails, and twelve corrupted headers fail — plus a
writer round trip over every metadata and tensor type, and the model loaders
(bch_lfm2_model_from_gguf / bch_qwen35_model_from_gguf, lfm2.rs:186-232,
737-1004, qwen35.rs:630-745) filling the same model a direct upload gets."""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

from bobcat_amd import BobcatError
from bobcat_amd.gguf import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, Gguf, GgufWeights,
                             GgufWriter, lfm2_to_gguf, qwen35_to_gguf)

Q8_0 = (32, 34)
ROWS = 2


class Builder:
    """malformed.rs:19-84: two metadata entries and one Q8_0 tensor of two rows."""

    def __init__(self):
        b = bytearray()
        put32 = lambda v: b.extend(struct.pack("<I", v))
        put64 = lambda v: b.extend(struct.pack("<Q", v))
        puts = lambda s: (put64(len(s)), b.extend(s.encode()))
        put32(0x46554747)
        put32(3)
        put64(1)
        self.n_kv_at = len(b)
        put64(2)
        puts("general.architecture")
        put32(8)
        puts("test")
        puts("general.alignment")
        put32(4)
        self.alignment_at = len(b)
        put32(32)
        puts("weight")
        self.n_dims_at = len(b)
        put32(2)
        self.ne0_at = len(b)
        put64(Q8_0[0])
        self.ne1_at = len(b)
        put64(ROWS)
        self.type_at = len(b)
        put32(8)
        self.offset_at = len(b)
        put64(0)
        b.extend(b"\0" * (-len(b) % 32))
        b.extend(b"\1" * (ROWS * Q8_0[1]))
        self.bytes = bytes(b)

    def with_u32(self, at, v):
        b = bytearray(self.bytes)
        b[at:at + 4] = struct.pack("<I", v)
        return bytes(b)

    def with_u64(self, at, v):
        b = bytearray(self.bytes)
        b[at:at + 8] = struct.pack("<Q", v)
        return bytes(b)


def test_valid_file_parses():
    b = Builder()
    g = Gguf(data=b.bytes)
    t = g.tensor("weight")
    assert t.offset == len(b.bytes) - ROWS * Q8_0[1] and t.bytes == ROWS * Q8_0[1]
    assert t.n_dims == 2 and list(t.ne) == [32, 2, 1, 1] and t.type == 8
    assert g.string("general.architecture") == b"test"
    assert g.u32("general.alignment") == 32


def test_every_truncation_fails():
    b = Builder()
    for size in range(len(b.bytes)):
        with pytest.raises(BobcatError) as e:
            Gguf(data=b.bytes[:size])
        assert e.value.status == 18, size


@pytest.mark.parametrize("case", [
    "huge metadata count", "alignment of 3", "alignment of 0", "zero dimensions", "five dimensions",
    "row of 31 Q8_0 elements", "zero-sized dimension", "overflowing shape", "unknown tensor type",
    "misaligned offset", "offset past the end", "offset wrapping around"])
def test_corrupted_headers_fail(case):
    b = Builder()
    bytes_ = {
        "huge metadata count": lambda: b.with_u64(b.n_kv_at, 1 << 62),
        "alignment of 3": lambda: b.with_u32(b.alignment_at, 3),
        "alignment of 0": lambda: b.with_u32(b.alignment_at, 0),
        "zero dimensions": lambda: b.with_u32(b.n_dims_at, 0),
        "five dimensions": lambda: b.with_u32(b.n_dims_at, 5),
        "row of 31 Q8_0 elements": lambda: b.with_u64(b.ne0_at, 31),
        "zero-sized dimension": lambda: b.with_u64(b.ne1_at, 0),
        "overflowing shape": lambda: b.with_u64(b.ne1_at, 1 << 62),
        "unknown tensor type": lambda: b.with_u32(b.type_at, 99),
        "misaligned offset": lambda: b.with_u64(b.offset_at, 1),
        "offset past the end": lambda: b.with_u64(b.offset_at, 32),
        "offset wrapping around": lambda: b.with_u64(b.offset_at, (1 << 64) - 32),
    }[case]()
    with pytest.raises(BobcatError) as e:
        Gguf(data=bytes_)
    assert e.value.status == 18


def test_not_gguf_and_versions():
    b = Builder()
    with pytest.raises(BobcatError, match="not a GGUF file"):
        Gguf(data=b"GGUX" + b.bytes[4:])
    with pytest.raises(BobcatError, match="unsupported GGUF version 4"):
        Gguf(data=b.with_u32(4, 4))
    Gguf(data=b.with_u32(4, 2))  # version 2 reads the same


def test_duplicates_fail():
    w = GgufWriter()
    w.add_u32("a", 1)
    w.add_u32("a", 2)
    with pytest.raises(BobcatError, match="appears twice"):
        Gguf(data=w.to_bytes())
    w = GgufWriter()
    w.add_tensor("t", (4,), 0, np.zeros(4, np.float32))
    w.add_tensor("t", (4,), 0, np.zeros(4, np.float32))
    with pytest.raises(BobcatError, match="appears twice"):
        Gguf(data=w.to_bytes())


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(3)
    w = GgufWriter()
    for key, t, v in [("u8", U8, 200), ("i8", I8, -5), ("u16", U16, 60000), ("i16", I16, 7), ("u32", U32, 4000000000),
                      ("i32", I32, 12), ("u64", U64, 9), ("i64", I64, 3), ("f32", F32, 1.5), ("f64", F64, 0.25),
                      ("b", BOOL, True), ("s", STRING, "héllo")]:
        w.add(key, t, v)
    w.add_array("arr", U32, [0, 8, 0, 8])
    w.add_array("strs", STRING, ["a", "", "xyz"])
    tensors = {}
    for name, t, shape in [("f32", 0, (64, 3)), ("f16", 1, (64, 2)), ("q4_0", 2, (64, 2)), ("q8_0", 8, (32, 3)),
                           ("q4k", 12, (256, 2)), ("q5k", 13, (256, 1)), ("q6k", 14, (512, 1)), ("bf16", 30, (8,))]:
        from bobcat_amd.gguf import BLOCKS
        ne, nb = BLOCKS[t]
        data = rng.integers(0, 256, int(np.prod(shape)) // ne * nb, dtype=np.uint8)
        w.add_tensor(name, shape, t, data)
        tensors[name] = (t, shape, data)
    path = tmp_path / "x.gguf"
    w.write(path)
    g = Gguf(path)
    assert g.u32("u8") == 200 and g.u32("u16") == 60000 and g.u32("u32") == 4000000000 and g.u32("i32") == 12
    with pytest.raises(BobcatError):
        g.u32("i8")  # negative: no u32
    assert g.f32("f32") == 1.5 and g.f32("f64") == 0.25
    assert g.string("s") == "héllo".encode()
    assert g.array_u32("arr") == [0, 8, 0, 8]
    assert g.array_strings("strs") == [b"a", b"", b"xyz"]
    assert [t.name.decode() for t in g.tensors()] == list(tensors)
    for name, (t, shape, data) in tensors.items():
        info = g.tensor(name)
        assert info.type == t and list(info.ne)[:len(shape)] == list(shape) and info.offset % 32 == 0
        assert np.array_equal(g.tensor_bytes(name), data)


def _matrices_equal(a, b):
    if (a.format, a.n_rows, a.n_cols) != (b.format, b.n_rows, b.n_cols):
        return False
    if not a.data:
        return not b.data
    from bobcat_amd._lib import lib
    rb = lib().bch_row_bytes(a.format, a.n_cols) * a.n_rows
    return C.string_at(a.data, rb) == C.string_at(b.data, rb)


def _vec_equal(pa, pb, n):
    if not pa:
        return not pb
    return C.string_at(C.cast(pa, C.c_void_p).value, 4 * n) == C.string_at(C.cast(pb, C.c_void_p).value, 4 * n)


@pytest.mark.parametrize("name", ["lfm2-tiny", "lfm2-tiny-moe", "lfm2-tiny-mixed"])
def test_lfm2_model_from_gguf(tmp_path, name):
    from bobcat_amd.lfm2 import CONFIGS, Lfm2Weights

    cfg = CONFIGS[name]
    w = Lfm2Weights(cfg, seed=5)
    path = tmp_path / f"{name}.gguf"
    lfm2_to_gguf(w, path)
    g = GgufWeights(path, cfg)
    a, b = w.c_model, g.c_model
    for f in ("n_layers", "n_embd", "n_ff", "n_experts", "n_experts_used", "n_ff_expert", "n_heads", "n_kv_heads",
              "head_dim", "n_vocab", "conv_kernel"):
        assert getattr(a, f) == getattr(b, f), f
    assert np.float32(a.rope_theta) == np.float32(b.rope_theta) and np.float32(a.norm_eps) == np.float32(b.norm_eps)
    assert _matrices_equal(a.token_embd, b.token_embd) and _matrices_equal(a.output, b.output)
    assert _vec_equal(a.output_norm, b.output_norm, cfg.n_embd)
    n, hd = cfg.n_embd, cfg.head_dim
    for il in range(cfg.n_layers):
        la, lb = a.layers[il], b.layers[il]
        assert (la.is_attention, la.is_moe) == (lb.is_attention, lb.is_moe)
        assert _vec_equal(la.attn_norm, lb.attn_norm, n) and _vec_equal(la.ffn_norm, lb.ffn_norm, n)
        for m in ("in_proj", "out_proj", "wq", "wk", "wv", "wo", "gate", "up", "down", "router", "gate_exps",
                  "up_exps", "down_exps"):
            assert _matrices_equal(getattr(la, m), getattr(lb, m)), (il, m)
        if la.is_attention:
            assert _vec_equal(la.q_norm, lb.q_norm, hd) and _vec_equal(la.k_norm, lb.k_norm, hd)
        else:
            assert _vec_equal(la.conv_taps, lb.conv_taps, n * cfg.conv_kernel)
        if la.is_moe:
            assert _vec_equal(la.expert_bias, lb.expert_bias, cfg.n_experts)


@pytest.mark.parametrize("name", ["qwen3.5-tiny", "qwen3.5-tiny-64"])
def test_qwen35_model_from_gguf(tmp_path, name):
    from bobcat_amd.qwen35 import CONFIGS, Qwen35Weights

    cfg = CONFIGS[name]
    w = Qwen35Weights(cfg, seed=5)
    path = tmp_path / f"{name}.gguf"
    qwen35_to_gguf(w, path)
    g = GgufWeights(path, cfg)
    a, b = w.c_model, g.c_model
    for f in ("n_layers", "n_embd", "n_ff", "n_vocab", "n_heads", "n_kv_heads", "head_dim", "n_rot", "conv_kernel",
              "n_k_heads", "n_v_heads", "k_head_dim", "v_head_dim"):
        assert getattr(a, f) == getattr(b, f), f
    assert _matrices_equal(a.token_embd, b.token_embd)
    for il in range(cfg.n_layers):
        la, lb = a.layers[il], b.layers[il]
        assert la.is_attention == lb.is_attention
        for m in ("wq", "wk", "wv", "wo", "qkv", "z", "beta", "alpha", "out", "gate", "up", "down"):
            assert _matrices_equal(getattr(la, m), getattr(lb, m)), (il, m)
        if not la.is_attention:
            assert _vec_equal(la.a, lb.a, cfg.n_v_heads) and _vec_equal(la.dt_bias, lb.dt_bias, cfg.n_v_heads)
            assert _vec_equal(la.conv_taps, lb.conv_taps, cfg.conv_dim * cfg.conv_kernel)
            assert _vec_equal(la.ssm_norm, lb.ssm_norm, cfg.v_head_dim)


def test_model_load_errors(tmp_path):
    from bobcat_amd.lfm2 import LFM2_TINY, Lfm2Weights

    w = GgufWriter()
    w.add_string("general.architecture", "llama")
    with pytest.raises(BobcatError, match="architecture") as e:
        Gguf(data=w.to_bytes()).lfm2_model()
    assert e.value.status == 19
    # A file without one layer's out_proj.
    lw = Lfm2Weights(LFM2_TINY, seed=1)
    path = tmp_path / "t.gguf"
    lfm2_to_gguf(lw, path)
    raw = path.read_bytes()
    bad = raw.replace(b"blk.0.shortconv.out_proj.weight", b"blk.0.shortconv.out_prox.weight")
    with pytest.raises(BobcatError, match="missing tensor blk.0.shortconv.out_proj.weight"):
        Gguf(data=bad).lfm2_model()
