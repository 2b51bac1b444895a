"""`Hip`: the op-level backend, a Python mirror of `bobcat_metal::Metal`.

Method names, argument order and meaning follow the Metal backend
(crates/bobcat-metal/src/backend.rs:1027-2699), so the kernel tests read like
the reference's own tests (crates/bobcat/tests/metal_*.rs).  Every call goes
through the C ABI of libbobcat_hip.so; errors raise `BobcatError` carrying
the bch_status code of the matching `bobcat_metal::Error` variant.
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from ._lib import BobcatError, Norm as _Norm, ProfileEntry, View as _View, check, lib


class Format(IntEnum):
    """Weight formats; values are ggml type ids (bobcat-gguf/src/lib.rs:137-148)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4K = 12
    Q5K = 13
    Q6K = 14
    BF16 = 30


class Store(IntEnum):
    """bobcat_metal::Store (backend.rs:360-370)."""
    OVERWRITE = 0
    ACCUMULATE = 1
    SWIGLU = 2


class Buffer:
    """A device buffer (bobcat_metal::Buffer, backend.rs:302-325)."""

    def __init__(self, hip: "Hip", handle: int, length: int):
        self.hip = hip
        self.handle = handle
        self.len = length

    def at(self, offset: int) -> "ViewRef":
        return ViewRef(self, offset)

    def floats(self, index: int) -> "ViewRef":
        return ViewRef(self, 4 * index)

    @property
    def device_ptr(self) -> int:
        return lib().bch_buffer_device_ptr(self.handle)

    def free(self) -> None:
        if self.handle:
            lib().bch_buffer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass(frozen=True)
class ViewRef:
    """A position inside a buffer (bobcat_metal::View, backend.rs:337-341)."""
    buffer: Buffer
    offset: int

    def c(self) -> _View:
        return _View(self.buffer.handle, self.offset)


@dataclass(frozen=True)
class NormSpec:
    """bobcat_metal::Norm (backend.rs:344-350)."""
    weight: ViewRef
    eps: float

    def c(self) -> _Norm:
        return _Norm(self.weight.c(), self.eps)


def _view(v: ViewRef) -> _View:
    return v.c()


class Hip:
    """One device context with one stream (Metal::open, backend.rs:1083)."""

    def __init__(self):
        handle = C.c_void_p()
        check(lib().bch_open(C.byref(handle)))
        self.handle = handle.value
        self._buffers: list[Buffer] = []
        # Objects that hold device state of this context (model drivers);
        # they close before the context does.
        self._dependents = weakref.WeakSet()

    def close(self) -> None:
        if self.handle:
            for d in list(self._dependents):
                d.close()
            for b in self._buffers:
                b.free()
            lib().bch_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def device_info(self) -> tuple[str, int]:
        name = C.create_string_buffer(256)
        cus = C.c_uint32()
        check(lib().bch_device_info(self.handle, name, 256, C.byref(cus)))
        return name.value.decode(), cus.value

    # -- buffers ---------------------------------------------------------
    def new_buffer(self, length: int) -> Buffer:
        h = C.c_void_p()
        check(lib().bch_buffer_new(self.handle, length, C.byref(h)))
        b = Buffer(self, h.value, length)
        self._buffers.append(b)
        return b

    def buffer_from(self, array: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(array)
        h = C.c_void_p()
        check(lib().bch_buffer_from_host(self.handle, a.ctypes.data, a.nbytes, C.byref(h)))
        b = Buffer(self, h.value, a.nbytes)
        self._buffers.append(b)
        return b

    def write(self, view: ViewRef, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data)
        check(lib().bch_write(self.handle, _view(view), a.ctypes.data, a.nbytes))

    def read(self, view: ViewRef, out: np.ndarray) -> np.ndarray:
        assert out.flags.c_contiguous
        check(lib().bch_read(self.handle, _view(view), out.ctypes.data, out.nbytes))
        return out

    # -- recording -------------------------------------------------------
    def begin(self) -> None:
        check(lib().bch_begin(self.handle))

    def discard(self) -> None:
        lib().bch_discard(self.handle)

    def barrier(self) -> None:
        lib().bch_barrier(self.handle)

    def commit(self) -> int:
        t = C.c_uint64()
        check(lib().bch_commit(self.handle, C.byref(t)))
        return t.value

    def wait(self, ticket: int) -> float:
        s = C.c_double()
        check(lib().bch_wait(self.handle, ticket, C.byref(s)))
        return s.value

    def end(self) -> float:
        s = C.c_double()
        check(lib().bch_end(self.handle, C.byref(s)))
        return s.value

    def set_profiling(self, enabled: bool) -> None:
        lib().bch_set_profiling(self.handle, int(enabled))

    def profile(self) -> list[dict]:
        out = []
        for i in range(lib().bch_profile_count(self.handle)):
            e = ProfileEntry()
            check(lib().bch_profile_get(self.handle, i, C.byref(e)))
            out.append(dict(name=e.name.decode(), n_rows=e.n_rows, n_cols=e.n_cols, calls=e.calls,
                            seconds=e.seconds, bytes=e.bytes))
        return out

    # -- ops ---------------------------------------------------------------
    def dequantize(self, fmt, weights, n_rows, n_cols, out):
        check(lib().bch_dequantize(self.handle, int(fmt), _view(weights), n_rows, n_cols, _view(out)))

    def matvec(self, fmt, weights, n_rows, n_cols, x, y, norm: NormSpec | None = None,
               accumulate: bool = False):
        n = C.byref(norm.c()) if norm is not None else None
        check(lib().bch_matvec(self.handle, int(fmt), _view(weights), n_rows, n_cols, _view(x),
                               _view(y), n, int(accumulate)))

    def matvec_swiglu(self, fmt, gate, up, n_rows, n_cols, x, norm: NormSpec, y):
        check(lib().bch_matvec_swiglu(self.handle, int(fmt), _view(gate), _view(up), n_rows, n_cols,
                                      _view(x), norm.c(), _view(y)))

    def matvec_conv(self, fmt, weights, n_cols, x, norm: NormSpec | None, taps, history, out,
                    n_embd, kernel_size):
        n = C.byref(norm.c()) if norm is not None else None
        check(lib().bch_matvec_conv(self.handle, int(fmt), _view(weights), n_cols, _view(x), n,
                                    _view(taps), _view(history), _view(out), n_embd, kernel_size))

    def short_conv(self, bcx, taps, history, out, n_embd, kernel_size, n_tokens):
        check(lib().bch_short_conv(self.handle, _view(bcx), _view(taps), _view(history), _view(out),
                                   n_embd, kernel_size, n_tokens))

    def short_conv_batch(self, bcx, taps, history, out, n_embd, kernel_size, n_tokens):
        check(lib().bch_short_conv_batch(self.handle, _view(bcx), _view(taps), _view(history),
                                         _view(out), n_embd, kernel_size, n_tokens))

    def rms_norm(self, x, weight, out, n, n_rows, eps):
        check(lib().bch_rms_norm(self.handle, _view(x), _view(weight), _view(out), n, n_rows, eps))

    def norm_rope(self, src, dst, dst_half, weight, n_heads, head_dim, n_rot, src_head_stride, pos,
                  n_tokens, src_stride, dst_stride, theta, eps):
        check(lib().bch_norm_rope(self.handle, _view(src), _view(dst), int(dst_half), _view(weight),
                                  n_heads, head_dim, n_rot, src_head_stride, pos, n_tokens,
                                  src_stride, dst_stride, theta, eps))

    def convert_half(self, src, dst, n):
        check(lib().bch_convert_half(self.handle, _view(src), _view(dst), n))

    def copy(self, src, dst, n):
        check(lib().bch_copy(self.handle, _view(src), _view(dst), n))

    def embed(self, fmt, weights, n_vocab, tokens, out, n_embd, n_tokens):
        check(lib().bch_embed(self.handle, int(fmt), _view(weights), n_vocab, _view(tokens),
                              _view(out), n_embd, n_tokens))

    def attention(self, q, k_cache, v_cache, kv_half, scratch, out, n_heads, n_kv_heads, head_dim,
                  first_pos, n_queries, n_ctx):
        check(lib().bch_attention(self.handle, _view(q), _view(k_cache), _view(v_cache), int(kv_half),
                                  _view(scratch), _view(out), n_heads, n_kv_heads, head_dim,
                                  first_pos, n_queries, n_ctx))

    def attention_prefill(self, q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, first_pos, n_queries,
                          n_ctx):
        check(lib().bch_attention_prefill(self.handle, _view(q), _view(k_cache), _view(v_cache), _view(out),
                                          n_heads, n_kv_heads, head_dim, first_pos, n_queries, n_ctx))

    def attention_decode(self, q, k, v, q_norm, k_norm, eps, rope_theta, n_rot, k_cache, v_cache, kv_half, scratch,
                         out, n_heads, n_kv_heads, head_dim, pos, n_ctx):
        check(lib().bch_attention_decode(self.handle, _view(q), _view(k), _view(v), _view(q_norm), _view(k_norm),
                                         eps, rope_theta, n_rot, _view(k_cache), _view(v_cache), int(kv_half),
                                         _view(scratch), _view(out), n_heads, n_kv_heads, head_dim, pos, n_ctx))

    def matmul(self, fmt, weights, n_rows, n_cols, x, y, n_tokens, store: Store):
        check(lib().bch_matmul(self.handle, int(fmt), _view(weights), n_rows, n_cols, _view(x),
                               _view(y), n_tokens, int(store)))

    def read_sum(self, src, n_vectors, out, n_threads):
        check(lib().bch_read_sum(self.handle, _view(src), n_vectors, _view(out), n_threads))

    def moe_route(self, x, norm: NormSpec | None, normed, router, bias, route, n_cols, n_experts, n_used,
                  n_tokens):
        n = C.byref(norm.c()) if norm is not None else None
        check(lib().bch_moe_route(self.handle, _view(x), n, _view(normed if normed is not None else x),
                                  _view(router), _view(bias), _view(route), n_cols, n_experts, n_used, n_tokens))

    def matvec_experts_swiglu(self, fmt, gate, up, n_rows, n_cols, n_experts, x, route, n_used, y, n_tokens):
        check(lib().bch_matvec_experts_swiglu(self.handle, int(fmt), _view(gate), _view(up), n_rows, n_cols,
                                              n_experts, _view(x), _view(route), n_used, _view(y), n_tokens))

    def matvec_experts_down(self, fmt, weights, n_rows, n_cols, n_experts, x, route, n_used, y, n_tokens):
        check(lib().bch_matvec_experts_down(self.handle, int(fmt), _view(weights), n_rows, n_cols, n_experts,
                                            _view(x), _view(route), n_used, _view(y), n_tokens))

    def moe_group(self, route, offsets, entries, n_experts, n_used, n_tokens):
        check(lib().bch_moe_group(self.handle, _view(route), _view(offsets), _view(entries), n_experts, n_used,
                                  n_tokens))

    def matmul_experts(self, fmt, weights, up, n_rows, n_cols, n_experts, x, shared_input, offsets, entries,
                       n_used, y, n_tokens):
        upv = C.byref(_view(up)) if up is not None else None
        check(lib().bch_matmul_experts(self.handle, int(fmt), _view(weights), upv, n_rows, n_cols, n_experts,
                                       _view(x), int(bool(shared_input)), _view(offsets), _view(entries), n_used,
                                       _view(y), n_tokens))

    def moe_combine(self, x, route, y, n_embd, n_used, n_tokens):
        check(lib().bch_moe_combine(self.handle, _view(x), _view(route), _view(y), n_embd, n_used, n_tokens))

    def sample(self, logits, n_vocab, recent, n_recent, settings, rng_state, out):
        check(lib().bch_sample(self.handle, _view(logits), n_vocab, _view(recent), n_recent, C.byref(settings),
                               _view(rng_state), _view(out)))

    def sample_draw(self, logits, n_vocab, recent, n_recent, settings, u, out):
        check(lib().bch_sample_draw(self.handle, _view(logits), n_vocab, _view(recent), n_recent, C.byref(settings),
                                    u, _view(out)))

    def argmax(self, x, out, n):
        check(lib().bch_argmax(self.handle, _view(x), _view(out), n))


def attention_scratch_floats(n_heads: int, head_dim: int, n_ctx: int, n_queries: int) -> int:
    return lib().bch_attention_scratch_floats(n_heads, head_dim, n_ctx, n_queries)


def attention_decode_scratch_floats(n_heads: int, head_dim: int, n_ctx: int, kv_half: bool) -> int:
    return lib().bch_attention_decode_scratch_floats(n_heads, head_dim, n_ctx, int(kv_half))


def row_bytes(fmt: int, n_cols: int) -> int:
    return lib().bch_row_bytes(int(fmt), n_cols)


__all__ = ["Hip", "Buffer", "ViewRef", "NormSpec", "Format", "Store", "BobcatError",
           "attention_scratch_floats", "attention_decode_scratch_floats", "row_bytes"]
