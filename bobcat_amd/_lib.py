"""ctypes binding of libbobcat_hip.so (the C ABI declared in include/bobcat_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libbobcat_hip.so"


class BobcatError(RuntimeError):
    """A failed backend call: `status` is a bch_status code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{STATUS_NAMES.get(status, status)}] {message}")
        self.status = status


STATUS_NAMES = {
    0: "OK", 1: "NoDevice", 2: "Allocation", 3: "NotRecording", 4: "AlreadyRecording",
    5: "OutOfBounds", 6: "ForeignBuffer", 7: "Busy", 8: "Access", 9: "AttentionLimits",
    10: "UnsupportedFormat", 11: "DeltaNetLimits", 12: "ExpertLimits", 13: "Execution",
    14: "Argument", 15: "ContextFull", 16: "Token", 17: "GateShape", 18: "Gguf", 19: "Model",
}
STATUS = {v: k for k, v in STATUS_NAMES.items()}


class View(C.Structure):
    _fields_ = [("buffer", C.c_void_p), ("offset", C.c_uint64)]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float)]


class DeltaShape(C.Structure):
    _fields_ = [("n_k_heads", C.c_uint32), ("n_v_heads", C.c_uint32), ("k_dim", C.c_uint32), ("v_dim", C.c_uint32)]


class Norm(C.Structure):
    _fields_ = [("weight", View), ("eps", C.c_float)]


class ProfileEntry(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("n_rows", C.c_uint32), ("n_cols", C.c_uint32),
                ("calls", C.c_uint64), ("seconds", C.c_double), ("bytes", C.c_uint64)]


class Matrix(C.Structure):
    _fields_ = [("format", C.c_uint32), ("n_rows", C.c_uint32), ("n_cols", C.c_uint32),
                ("data", C.c_void_p)]


class GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4), ("type", C.c_uint32),
                ("data", C.c_void_p), ("offset", C.c_uint64), ("bytes", C.c_uint64)]


_FP = C.POINTER(C.c_float)
# bch_emit_fn: int (*)(uint32_t token, void *user)
EMIT_FN = C.CFUNCTYPE(C.c_int, C.c_uint32, C.c_void_p)


class Lfm2Layer(C.Structure):
    _fields_ = [
        ("is_attention", C.c_uint32), ("is_moe", C.c_uint32),
        ("attn_norm", _FP), ("ffn_norm", _FP),
        ("conv_taps", _FP), ("in_proj", Matrix), ("out_proj", Matrix),
        ("wq", Matrix), ("wk", Matrix), ("wv", Matrix), ("wo", Matrix),
        ("q_norm", _FP), ("k_norm", _FP),
        ("gate", Matrix), ("up", Matrix), ("down", Matrix),
        ("router", Matrix), ("expert_bias", _FP),
        ("gate_exps", Matrix), ("up_exps", Matrix), ("down_exps", Matrix),
    ]


class Qwen35Layer(C.Structure):
    _fields_ = [
        ("is_attention", C.c_uint32), ("attn_norm", _FP), ("ffn_norm", _FP),
        ("wq", Matrix), ("wk", Matrix), ("wv", Matrix), ("wo", Matrix), ("q_norm", _FP), ("k_norm", _FP),
        ("qkv", Matrix), ("z", Matrix), ("beta", Matrix), ("alpha", Matrix),
        ("conv_taps", _FP), ("dt_bias", _FP), ("a", _FP), ("ssm_norm", _FP), ("out", Matrix),
        ("gate", Matrix), ("up", Matrix), ("down", Matrix),
    ]


class Qwen35Model(C.Structure):
    _fields_ = [
        ("n_layers", C.c_uint32), ("n_embd", C.c_uint32), ("n_ff", C.c_uint32), ("n_vocab", C.c_uint32),
        ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("n_rot", C.c_uint32),
        ("rope_theta", C.c_float), ("norm_eps", C.c_float), ("conv_kernel", C.c_uint32),
        ("n_k_heads", C.c_uint32), ("n_v_heads", C.c_uint32), ("k_head_dim", C.c_uint32),
        ("v_head_dim", C.c_uint32), ("layers", C.POINTER(Qwen35Layer)),
        ("token_embd", Matrix), ("output", Matrix), ("output_norm", _FP),
    ]


class Lfm2Model(C.Structure):
    _fields_ = [
        ("n_layers", C.c_uint32), ("n_embd", C.c_uint32), ("n_ff", C.c_uint32),
        ("n_experts", C.c_uint32), ("n_experts_used", C.c_uint32), ("n_ff_expert", C.c_uint32),
        ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("n_vocab", C.c_uint32), ("conv_kernel", C.c_uint32),
        ("rope_theta", C.c_float), ("norm_eps", C.c_float),
        ("layers", C.POINTER(Lfm2Layer)), ("token_embd", Matrix), ("output", Matrix),
        ("output_norm", _FP),
    ]


_u32, _u64, _int, _vp, _f32, _dbl = C.c_uint32, C.c_uint64, C.c_int, C.c_void_p, C.c_float, C.c_double

# name -> (restype, argtypes).  Every declaration of include/bobcat_hip.h.
PROTOTYPES = {
    "bch_last_error": (C.c_char_p, []),
    "bch_row_bytes": (_u64, [_u32, _u32]),
    "bch_open": (_int, [C.POINTER(_vp)]),
    "bch_close": (None, [_vp]),
    "bch_device_info": (_int, [_vp, C.c_char_p, C.c_size_t, C.POINTER(_u32)]),
    "bch_buffer_new": (_int, [_vp, _u64, C.POINTER(_vp)]),
    "bch_buffer_from_host": (_int, [_vp, _vp, _u64, C.POINTER(_vp)]),
    "bch_buffer_free": (None, [_vp]),
    "bch_buffer_len": (_u64, [_vp]),
    "bch_buffer_device_ptr": (_vp, [_vp]),
    "bch_write": (_int, [_vp, View, _vp, _u64]),
    "bch_read": (_int, [_vp, View, _vp, _u64]),
    "bch_begin": (_int, [_vp]),
    "bch_discard": (None, [_vp]),
    "bch_barrier": (None, [_vp]),
    "bch_commit": (_int, [_vp, C.POINTER(_u64)]),
    "bch_wait": (_int, [_vp, _u64, C.POINTER(_dbl)]),
    "bch_end": (_int, [_vp, C.POINTER(_dbl)]),
    "bch_set_profiling": (None, [_vp, _int]),
    "bch_profile_count": (_u32, [_vp]),
    "bch_profile_get": (_int, [_vp, _u32, C.POINTER(ProfileEntry)]),
    "bch_dequantize": (_int, [_vp, _u32, View, _u32, _u32, View]),
    "bch_matvec": (_int, [_vp, _u32, View, _u32, _u32, View, View, C.POINTER(Norm), _int]),
    "bch_matvec_swiglu": (_int, [_vp, _u32, View, View, _u32, _u32, View, Norm, View]),
    "bch_matvec_conv": (_int, [_vp, _u32, View, _u32, View, C.POINTER(Norm), View, View, View, _u32, _u32]),
    "bch_short_conv": (_int, [_vp, View, View, View, View, _u32, _u32, _u32]),
    "bch_short_conv_batch": (_int, [_vp, View, View, View, View, _u32, _u32, _u32]),
    "bch_rms_norm": (_int, [_vp, View, View, View, _u32, _u32, _f32]),
    "bch_norm_rope": (_int, [_vp, View, View, _int, View, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                             _u32, _f32, _f32]),
    "bch_convert_half": (_int, [_vp, View, View, _u32]),
    "bch_copy": (_int, [_vp, View, View, _u32]),
    "bch_embed": (_int, [_vp, _u32, View, _u32, View, View, _u32, _u32]),
    "bch_attention": (_int, [_vp, View, View, View, _int, View, View, _u32, _u32, _u32, _u32, _u32, _u32]),
    "bch_attention_prefill": (_int, [_vp, View, View, View, View, _u32, _u32, _u32, _u32, _u32, _u32]),
    "bch_attention_scratch_floats": (_u64, [_u32, _u32, _u32, _u32]),
    "bch_attention_decode": (_int, [_vp, View, View, View, View, View, C.c_float, C.c_float, _u32, View, View, _int,
                                    View, View, _u32, _u32, _u32, _u32, _u32]),
    "bch_attention_decode_scratch_floats": (_u64, [_u32, _u32, _u32, _int]),
    "bch_matmul": (_int, [_vp, _u32, View, _u32, _u32, View, View, _u32, _u32]),
    "bch_matmul_noalloc": (_int, [_vp, _u32, View, _u32, _u32, View, View, _u32, _u32]),
    "bch_matmul_noalloc_max_bytes": (_u64, []),
    "bch_argmax": (_int, [_vp, View, View, _u32]),
    "bch_read_sum": (_int, [_vp, View, _u64, View, _u32]),
    "bch_route_bytes": (_u64, [_u32, _u32]),
    "bch_gdn_conv": (_int, [_vp, View, View, View, View, _u32, _u32, _u32]),
    "bch_gdn_gates": (_int, [_vp, View, View, View, View, _u32, _u32]),
    "bch_gdn_recurrence": (_int, [_vp, View, View, View, View, View, C.POINTER(DeltaShape), _u32, C.c_float]),
    "bch_gdn_chunk_scratch_floats": (_u64, [C.POINTER(DeltaShape), _u32]),
    "bch_gdn_recurrence_chunked": (_int, [_vp, View, View, View, View, View, C.POINTER(DeltaShape), _u32, C.c_float,
                                          View]),
    "bch_gdn_gated_norm": (_int, [_vp, View, View, View, _u32, _u32, C.c_float]),
    "bch_attention_gate": (_int, [_vp, View, View, _u32, _u32, _u32]),
    "bch_qwen35_new": (_int, [_vp, C.POINTER(Qwen35Model), _u32, _int, C.POINTER(_vp)]),
    "bch_qwen35_free": (None, [_vp]),
    "bch_qwen35_n_past": (_u32, [_vp]),
    "bch_qwen35_reset": (_int, [_vp]),
    "bch_qwen35_step": (_int, [_vp, _u32, _FP, _FP, _FP, _FP]),
    "bch_qwen35_prefill": (_int, [_vp, C.POINTER(C.c_uint32), _u32, _FP, _FP, _FP, _FP]),
    "bch_qwen35_hidden": (_int, [_vp, C.POINTER(C.c_uint32), _u32, _FP]),
    "bch_qwen35_greedy_token": (_int, [_vp, C.POINTER(C.c_uint32)]),
    "bch_qwen35_generate": (_int, [_vp, C.POINTER(C.c_uint32), _u32]),
    "bch_qwen35_generate_next": (_int, [_vp, C.POINTER(C.c_uint32), _u32]),
    "bch_qwen35_generate_stream": (_int, [_vp, _u32, EMIT_FN, _vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    "bch_qwen35_generate_sampled": (_int, [_vp, C.POINTER(C.c_uint32), _u32, C.POINTER(Sampling), _u64]),
    "bch_qwen35_checkpoint_bytes": (_u64, [_vp]),
    "bch_qwen35_checkpoint": (_int, [_vp, _vp, _u64]),
    "bch_qwen35_restore": (_int, [_vp, _vp, _u64]),
    "bch_qwen35_last_gpu_seconds": (C.c_double, [_vp]),
    "bch_sample": (_int, [_vp, View, _u32, View, _u32, C.POINTER(Sampling), View, View]),
    "bch_sample_draw": (_int, [_vp, View, _u32, View, _u32, C.POINTER(Sampling), C.c_float, View]),
    "bch_lfm2_generate_sampled": (_int, [_vp, C.POINTER(C.c_uint32), _u32, C.POINTER(Sampling), _u64]),
    "bch_moe_route": (_int, [_vp, View, C.POINTER(Norm), View, View, View, View, _u32, _u32, _u32, _u32]),
    "bch_matvec_experts_swiglu": (_int, [_vp, _u32, View, View, _u32, _u32, _u32, View, View, _u32, View, _u32]),
    "bch_matvec_experts_down": (_int, [_vp, _u32, View, _u32, _u32, _u32, View, View, _u32, View, _u32]),
    "bch_moe_group": (_int, [_vp, View, View, View, _u32, _u32, _u32]),
    "bch_matmul_experts": (_int, [_vp, _u32, View, C.POINTER(View), _u32, _u32, _u32, View, C.c_int, View, View,
                                  _u32, View, _u32]),
    "bch_moe_combine": (_int, [_vp, View, View, View, _u32, _u32, _u32]),
    "bch_lfm2_new": (_int, [_vp, C.POINTER(Lfm2Model), _u32, _int, C.POINTER(_vp)]),
    "bch_lfm2_free": (None, [_vp]),
    "bch_lfm2_n_past": (_u32, [_vp]),
    "bch_lfm2_reset": (_int, [_vp]),
    "bch_lfm2_step": (_int, [_vp, _u32, _FP, _FP, _FP, _FP]),
    "bch_lfm2_prefill": (_int, [_vp, C.POINTER(_u32), _u32, _FP, _FP, _FP, _FP]),
    "bch_lfm2_greedy_token": (_int, [_vp, C.POINTER(_u32)]),
    "bch_lfm2_generate": (_int, [_vp, C.POINTER(_u32), _u32]),
    "bch_lfm2_generate_next": (_int, [_vp, C.POINTER(_u32), _u32]),
    "bch_lfm2_generate_stream": (_int, [_vp, _u32, EMIT_FN, _vp, C.POINTER(_u32), C.POINTER(_u32)]),
    "bch_gguf_parse": (_int, [_vp, _u64, C.POINTER(_vp)]),
    "bch_gguf_open": (_int, [C.c_char_p, C.POINTER(_vp)]),
    "bch_gguf_free": (None, [_vp]),
    "bch_gguf_bytes": (_vp, [_vp, C.POINTER(_u64)]),
    "bch_gguf_u32": (_int, [_vp, C.c_char_p, C.POINTER(_u32)]),
    "bch_gguf_f32": (_int, [_vp, C.c_char_p, C.POINTER(C.c_float)]),
    "bch_gguf_bool": (_int, [_vp, C.c_char_p, C.POINTER(_int)]),
    "bch_gguf_string": (_int, [_vp, C.c_char_p, C.POINTER(_vp), C.POINTER(_u64)]),
    "bch_gguf_array_len": (_int, [_vp, C.c_char_p, C.POINTER(_u64)]),
    "bch_gguf_array_u32": (_int, [_vp, C.c_char_p, _u64, C.POINTER(_u32)]),
    "bch_gguf_array_string": (_int, [_vp, C.c_char_p, _u64, C.POINTER(_vp), C.POINTER(_u64)]),
    "bch_gguf_tensor": (_int, [_vp, C.c_char_p, C.POINTER(GgufTensor)]),
    "bch_gguf_n_tensors": (_u64, [_vp]),
    "bch_gguf_tensor_at": (_int, [_vp, _u64, C.POINTER(GgufTensor)]),
    "bch_lfm2_model_from_gguf": (_int, [_vp, C.POINTER(Lfm2Model), C.POINTER(Lfm2Layer), _u32]),
    "bch_qwen35_model_from_gguf": (_int, [_vp, C.POINTER(Qwen35Model), C.POINTER(Qwen35Layer), _u32]),
    "bch_lfm2_checkpoint_bytes": (_u64, [_vp]),
    "bch_lfm2_checkpoint": (_int, [_vp, _vp, _u64]),
    "bch_lfm2_restore": (_int, [_vp, _vp, _u64]),
    "bch_lfm2_last_gpu_seconds": (_dbl, [_vp]),
}

_lib = None
# Declared entry points the loaded library does not export.
MISSING: list[str] = []


def lib() -> C.CDLL:
    """Load libbobcat_hip.so once; raise if it is missing or lacks a symbol."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m bobcat_amd.build` "
                "(the HIP backend has no fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(handle, name, None)
            if fn is None:
                MISSING.append(name)
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise BobcatError(status, lib().bch_last_error().decode())
