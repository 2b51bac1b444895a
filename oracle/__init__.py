"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (bobcat_oracle.c).

The oracle restates bobcat's scalar reference path (crates/bobcat/src/scalar.rs,
crates/bobcat/src/lfm2.rs) in C.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may load it, as the checker or as the timed CPU
baseline; nothing in bobcat_amd/ imports it.

Parity status of each oracle function (how it is pinned) is listed in
tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libbobcat_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = C.CDLL(str(LIB_PATH))
        fp, vp, u32, u64 = C.POINTER(C.c_float), C.c_void_p, C.c_uint32, C.c_uint64
        sig = {
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_row_bytes": (u64, [u32, u32]),
            "orc_q4k_scale_min": (None, [C.c_int, vp, vp, vp]),
            "orc_dequantize": (C.c_int, [u32, vp, u64, fp]),
            "orc_dot": (C.c_float, [fp, fp, u64]),
            "orc_set_threads": (None, [C.c_int]),
            "orc_get_threads": (C.c_int, []),
            "orc_matvec": (C.c_int, [u32, vp, u32, u32, fp, fp]),
            "orc_rms_norm": (None, [fp, fp, u64, C.c_float, fp]),
            "orc_rope_neox": (None, [fp, u32, u32, C.c_float]),
            "orc_silu": (C.c_float, [C.c_float]),
            "orc_softmax": (None, [fp, u64]),
            "orc_lfm2_route": (None, [fp, fp, u32, u32, C.POINTER(u32)]),
            "orc_short_conv": (None, [fp, fp, fp, fp, u32, u32, u32]),
            "orc_attention": (None, [fp, fp, fp, fp, u32, u32, u32, u32, u32]),
            "orc_lfm2_state_new": (vp, [vp, u32]),
            "orc_lfm2_state_free": (None, [vp]),
            "orc_lfm2_n_past": (u32, [vp]),
            "orc_lfm2_step": (C.c_int, [vp, vp, u32, fp, fp, fp, fp]),
            "orc_qwen35_state_new": (vp, [vp, u32]),
            "orc_qwen35_state_free": (None, [vp]),
            "orc_qwen35_n_past": (u32, [vp]),
            "orc_qwen35_step": (C.c_int, [vp, vp, u32, fp, fp, fp, fp]),
            "orc_qwen35_delta_step": (C.c_int, [vp, vp, u32]),
            "orc_sample": (u32, [fp, u32, C.POINTER(u32), u32, vp, C.POINTER(C.c_uint64)]),
            "orc_wyrand": (C.c_uint64, [C.POINTER(C.c_uint64)]),
            "orc_sample_u": (u32, [fp, u32, C.POINTER(u32), u32, vp, C.c_float]),
            "orc_u32_to_f32": (C.c_float, [u32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def dequantize(fmt: int, data: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    data = np.ascontiguousarray(data)
    assert lib().orc_dequantize(int(fmt), data.ctypes.data, n, _fp(out)) == 0
    return out


def matvec(fmt: int, weights: np.ndarray, n_rows: int, n_cols: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(n_rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    weights = np.ascontiguousarray(weights)
    assert lib().orc_matvec(int(fmt), weights.ctypes.data, n_rows, n_cols, _fp(x), _fp(y)) == 0
    return y


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm(_fp(x), _fp(w), x.size, eps, _fp(out))
    return out


def rope_neox(v: np.ndarray, pos: int, theta: float) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().orc_rope_neox(_fp(v), v.size, pos, theta)
    return v


def silu(x: float) -> float:
    return lib().orc_silu(x)


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, np.float32)
    lib().orc_softmax(_fp(x), x.size)
    return x


def dot(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().orc_dot(_fp(a), _fp(b), a.size)


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def q4k_scale_min(j: int, scales: bytes) -> tuple[int, int]:
    s = (C.c_uint8 * 12).from_buffer_copy(bytes(scales))
    a, b = C.c_uint8(), C.c_uint8()
    lib().orc_q4k_scale_min(j, s, C.byref(a), C.byref(b))
    return a.value, b.value


def route(scores: np.ndarray, bias: np.ndarray, n_used: int):
    s = np.array(scores, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    experts = (C.c_uint32 * s.size)()
    lib().orc_lfm2_route(_fp(s), _fp(b), s.size, n_used, experts)
    return s, list(experts)


class Sampling(C.Structure):
    """bch_sampling / bobcat::Sampling."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float)]


def sample(logits, recent, settings: Sampling, state: int):
    """Sampler::sample; returns (token, the generator state after the draw)."""
    lg = np.array(logits, np.float32)
    rc = np.ascontiguousarray(recent, np.uint32)
    st = C.c_uint64(state)
    tok = lib().orc_sample(_fp(lg), lg.size, rc.ctypes.data_as(C.POINTER(C.c_uint32)), rc.size,
                           C.cast(C.byref(settings), C.c_void_p), C.byref(st))
    return int(tok), int(st.value)


def sample_u(logits, recent, settings: Sampling, u: float) -> int:
    """Sampler::sample with the draw `u` (0 <= u < 1) given instead of generated."""
    lg = np.array(logits, np.float32)
    rc = np.ascontiguousarray(recent, np.uint32)
    return int(lib().orc_sample_u(_fp(lg), lg.size, rc.ctypes.data_as(C.POINTER(C.c_uint32)), rc.size,
                                  C.cast(C.byref(settings), C.c_void_p), u))


def u32_to_f32(x: int) -> float:
    """fastrand's Rng::f32 of a 32-bit draw."""
    return float(lib().orc_u32_to_f32(x))


def short_conv(bcx: np.ndarray, taps: np.ndarray, hist: np.ndarray, n_embd: int, k: int, n_tokens: int):
    """Returns (out, new_history); `hist` is not modified."""
    bcx = np.ascontiguousarray(bcx, np.float32)
    taps = np.ascontiguousarray(taps, np.float32)
    h = np.array(hist, np.float32)
    out = np.empty(n_tokens * n_embd, np.float32)
    lib().orc_short_conv(_fp(bcx), _fp(taps), _fp(h), _fp(out), n_embd, k, n_tokens)
    return out, h


def attention(q, kc, vc, n_heads, n_kv, hd, first_pos, n_queries):
    q = np.ascontiguousarray(q, np.float32)
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    out = np.empty(n_queries * n_heads * hd, np.float32)
    lib().orc_attention(_fp(q), _fp(kc), _fp(vc), _fp(out), n_heads, n_kv, hd, first_pos, n_queries)
    return out


class Lfm2State:
    """lfm2::State and Model::step on the CPU (lfm2.rs:308-394, 565-629)."""

    def __init__(self, model, n_ctx: int):
        """`model` is a bobcat_amd.lfm2.Lfm2Weights (keeps the ctypes struct alive)."""
        self.model = model
        self.n_vocab = model.hp["n_vocab"]
        self.n_embd = model.hp["n_embd"]
        self.n_layers = model.hp["n_layers"]
        self.handle = lib().orc_lfm2_state_new(C.addressof(model.c_model), n_ctx)
        assert self.handle

    def step(self, token: int, logits: bool = True, trace: bool = False):
        lg = np.empty(self.n_vocab, np.float32) if logits else None
        te = np.empty(self.n_embd, np.float32) if trace else None
        tl = np.empty(self.n_layers * self.n_embd, np.float32) if trace else None
        tf = np.empty(self.n_embd, np.float32) if trace else None
        rc = lib().orc_lfm2_step(C.addressof(self.model.c_model), self.handle, token,
                                 *(None if a is None else _fp(a) for a in (lg, te, tl, tf)))
        if rc != 0:
            raise ValueError({-1: "context full", -2: "token outside the vocabulary"}[rc])
        return (lg, (te, tl, tf)) if trace else lg

    @property
    def n_past(self) -> int:
        return lib().orc_lfm2_n_past(self.handle)

    def __del__(self):
        try:
            lib().orc_lfm2_state_free(self.handle)
        except Exception:
            pass


class Qwen35State:
    """qwen35::State and Model::step on the CPU (qwen35.rs:280-516, 533-640)."""

    def __init__(self, model, n_ctx: int):
        """`model` is a bobcat_amd.qwen35.Qwen35Weights."""
        self.model = model
        cfg = model.cfg
        self.n_vocab, self.n_embd, self.n_layers = cfg.n_vocab, cfg.n_embd, cfg.n_layers
        self.handle = lib().orc_qwen35_state_new(C.addressof(model.c_model), n_ctx)
        assert self.handle

    def step(self, token: int, logits: bool = True, trace: bool = False):
        lg = np.empty(self.n_vocab, np.float32) if logits else None
        te = np.empty(self.n_embd, np.float32) if trace else None
        tl = np.empty(self.n_layers * self.n_embd, np.float32) if trace else None
        tf = np.empty(self.n_embd, np.float32) if trace else None
        rc = lib().orc_qwen35_step(C.addressof(self.model.c_model), self.handle, token,
                                   *(None if a is None else _fp(a) for a in (lg, te, tl, tf)))
        if rc != 0:
            raise ValueError({-1: "context full", -2: "token outside the vocabulary"}[rc])
        return (lg, (te, tl, tf)) if trace else lg

    def delta_step(self, layer: int) -> None:
        """One Gated DeltaNet layer (Model::delta_net) on the current input; timing only."""
        if lib().orc_qwen35_delta_step(C.addressof(self.model.c_model), self.handle, layer) != 0:
            raise ValueError(f"layer {layer} is not a DeltaNet layer")

    def __del__(self):
        try:
            lib().orc_qwen35_state_free(self.handle)
        except Exception:
            pass
