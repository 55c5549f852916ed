"""ctypes declarations for liboxbitnet.so (include/oxbitnet.h, include/oxbitnet_ops.h).

The library is the only compute path: importing the package never falls back
to anything else, and every call that fails raises NativeError with the
library's message.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboxbitnet.so")


class NativeError(RuntimeError):
    pass


_lib = None

vp = C.c_void_p
i32 = C.c_int32
f32 = C.c_float
sz = C.c_size_t


class ModelInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layers", "hidden", "ffn", "heads", "kv_heads",
                                        "head_dim", "vocab", "max_seq")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("relu2", C.c_int),
        ("weight_bytes", C.c_size_t), ("kv_f32", C.c_int)]


class GenerateOptions(C.Structure):  # include/oxbitnet.h OxBitNetGenerateOptions
    _fields_ = [("max_tokens", C.c_size_t), ("temperature", C.c_float), ("top_k", C.c_size_t),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_size_t)]


class LoadProgress(C.Structure):
    _fields_ = [("phase", C.c_int), ("loaded", C.c_uint64), ("total", C.c_uint64),
                ("fraction", C.c_double)]


ProgressFn = C.CFUNCTYPE(None, C.POINTER(LoadProgress), C.c_void_p)
TokenFn = C.CFUNCTYPE(C.c_int32, C.c_char_p, C.c_size_t, C.c_void_p)
LogFn = C.CFUNCTYPE(None, C.c_int, C.c_char_p, C.c_size_t, C.c_void_p)


class LoadOptions(C.Structure):
    _fields_ = [("on_progress", ProgressFn), ("progress_userdata", C.c_void_p),
                ("cache_dir", C.c_char_p)]


class ChatMessage(C.Structure):
    _fields_ = [("role", C.c_char_p), ("content", C.c_char_p)]


# name -> (restype, argtypes)
SIGNATURES = {
    # plumbing
    "oxb_last_error": (C.c_char_p, []),
    "oxb_device_malloc": (vp, [sz]),
    "oxb_device_free": (C.c_int, [vp]),
    "oxb_memcpy_h2d": (C.c_int, [vp, vp, sz, vp]),
    "oxb_memcpy_d2h": (C.c_int, [vp, vp, sz, vp]),
    "oxb_memcpy_d2d": (C.c_int, [vp, vp, sz, vp]),
    "oxb_memset_d": (C.c_int, [vp, C.c_int, sz, vp]),
    "oxb_stream_create": (vp, []),
    "oxb_stream_destroy": (C.c_int, [vp]),
    "oxb_stream_sync": (C.c_int, [vp]),
    "oxb_device_sync": (C.c_int, []),
    "oxb_event_create": (vp, []),
    "oxb_event_destroy": (C.c_int, [vp]),
    "oxb_event_record": (C.c_int, [vp, vp]),
    "oxb_event_sync": (C.c_int, [vp]),
    "oxb_event_elapsed_ms": (C.c_float, [vp, vp]),
    "oxb_stream_begin_capture": (C.c_int, [vp]),
    "oxb_stream_end_capture": (vp, [vp]),
    "oxb_graph_launch": (C.c_int, [vp, vp]),
    "oxb_graph_destroy": (C.c_int, [vp]),
    "oxb_device_info": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                  C.POINTER(C.c_size_t)]),
    # kernels
    "oxb_repack_i2s_tiled": (C.c_int, [vp, vp, i32, i32, vp]),
    "oxb_gemv_i8": (C.c_int, [vp, vp, vp, vp, vp, i32, i32, vp, vp, vp]),
    "oxb_bitlinear_gemv": (C.c_int, [vp, vp, vp, f32, vp, i32, i32, vp, i32, vp, vp, vp, vp]),
    "oxb_bitlinear_gateup": (C.c_int, [vp, vp, vp, f32, vp, i32, i32, vp, vp]),
    "oxb_bitlinear_qkv": (C.c_int, [vp, vp, vp, f32, vp, i32, i32, i32, i32, vp, vp, vp, i32, vp,
                                    vp, vp]),
    "oxb_rope_table": (C.c_int, [vp, i32, i32, f32]),
    "oxb_norm_quant_rows": (C.c_int, [vp, vp, f32, i32, i32, vp, vp, vp, vp]),
    "oxb_quantize_rows_tiled": (C.c_int, [vp, vp, f32, i32, i32, vp, vp, vp, vp]),
    "oxb_gemm_i8": (C.c_int, [vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, i32, vp]),
    "oxb_gemm_ws_bytes": (C.c_size_t, [i32, i32, i32]),
    "oxb_gemm_i8_ws": (C.c_int, [vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, i32, vp, C.c_size_t,
                                 vp]),
    "oxb_gemm_qkv": (C.c_int, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, i32,
                               vp, vp]),
    "oxb_attn_decode": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp]),
    "oxb_attn_decode_fused_supported": (C.c_int, [i32, i32, i32, i32]),
    "oxb_attn_decode_fused": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "oxb_sample_logits": (C.c_int32, [vp, C.c_size_t, C.c_float, C.c_size_t, C.c_float, vp,
                                      C.c_size_t, C.c_float]),
    "oxb_sample_ws_bytes": (C.c_size_t, [i32]),
    "oxb_sample_device": (C.c_int, [vp, i32, C.c_float, C.c_size_t, C.c_float, vp, i32, vp, vp,
                                    vp, C.c_size_t, vp]),
    "oxb_attn_decode_noalloc": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "oxb_attn_decode_head_v8": (C.c_int, [vp, vp, vp, vp, vp, i32, C.c_size_t, C.c_size_t, i32,
                                          i32, i32, i32, i32, i32, vp, vp]),
    "oxb_qkv_attn_decode": (C.c_int, [vp, vp, vp, vp, f32, vp, vp, vp, vp, vp, vp, vp, i32, i32,
                                      i32, i32, i32, vp, vp]),
    "oxb_attn_decode_head": (C.c_int, [vp, vp, vp, vp, i32, C.c_size_t, i32, i32, i32, i32, i32,
                                       i32, vp, vp]),
    "oxb_attn_prefill": (C.c_int, [vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, vp]),
    "oxb_embedding": (C.c_int, [vp, i32, i32, vp, i32, vp, vp, vp]),
    "oxb_lm_head_argmax": (C.c_int, [vp, vp, f32, vp, i32, i32, vp, vp, vp, i32, vp]),
    "oxb_repack_lm": (C.c_int, [vp, vp, i32, i32, vp]),
    "oxb_lm_bytes": (C.c_size_t, [i32, i32]),
    # model
    "oxb_model_load": (vp, [C.c_char_p, C.c_int]),
    "oxb_model_load_kv": (vp, [C.c_char_p, C.c_int, C.c_int]),
    "oxb_tokenizer_load": (vp, [C.c_char_p]),
    "oxb_tokenizer_free": (None, [vp]),
    "oxb_tokenizer_encode": (C.c_int, [vp, C.c_char_p, C.c_int, vp, C.c_int]),
    "oxb_tokenizer_decode_one": (C.c_int, [vp, C.c_int32, vp, C.c_int]),
    "oxb_tokenizer_chat": (C.c_int, [vp, vp, vp, C.c_int, vp, C.c_int]),
    "oxb_tokenizer_info": (C.c_int, [vp, vp]),
    "oxb_model_free": (None, [vp]),
    "oxb_model_get_info": (C.c_int, [vp, C.POINTER(ModelInfo)]),
    "oxb_model_reset": (C.c_int, [vp]),
    "oxb_model_forward": (C.c_int, [vp, vp, C.c_int, vp]),
    "oxb_model_decode_greedy": (C.c_int, [vp, C.c_int, vp]),
    "oxb_model_position": (C.c_int, [vp]),
    "oxb_model_set_token": (C.c_int, [vp, i32]),
    "oxb_model_step": (C.c_int, [vp, vp]),
    "oxb_model_set_sampling": (C.c_int, [vp, C.c_float, C.c_size_t, C.c_float, C.c_size_t, vp,
                                         C.c_int]),
    "oxb_attn_decode_batch": (C.c_int, [vp, vp, vp, vp, i32, C.c_size_t, i32, i32, i32, i32, i32,
                                        vp, vp, vp]),
    "oxb_attn_decode_batch_v8": (C.c_int, [vp, vp, vp, vp, vp, i32, C.c_size_t, C.c_size_t, i32,
                                           i32, i32, i32, i32, vp, vp, vp]),
    "oxb_lm_head_argmax_batch": (C.c_int, [vp, C.c_size_t, vp, f32, vp, i32, i32, vp, vp, i32,
                                           vp, i32, i32, i32, vp]),
    "oxb_batch_create": (vp, [vp, i32, i32]),
    "oxb_batch_free": (None, [vp]),
    "oxb_batch_prefill": (C.c_int, [vp, i32, vp, i32]),
    "oxb_batch_decode_greedy": (C.c_int, [vp, i32, vp]),
    "oxb_batch_position": (C.c_int, [vp, i32]),
    "oxb_batch_logits": (C.c_int, [vp, vp]),
    # reference C ABI
    "oxbitnet_set_logger": (None, [LogFn, vp, C.c_uint8]),
    "oxbitnet_default_generate_options": (GenerateOptions, []),
    "oxbitnet_default_load_options": (LoadOptions, []),
    "oxbitnet_load": (vp, [C.c_char_p, C.POINTER(LoadOptions)]),
    "oxbitnet_free": (None, [vp]),
    "oxbitnet_generate": (C.c_int32, [vp, C.c_char_p, C.POINTER(GenerateOptions), TokenFn, vp]),
    "oxbitnet_chat": (C.c_int32, [vp, C.POINTER(ChatMessage), C.c_size_t,
                                  C.POINTER(GenerateOptions), TokenFn, vp]),
    "oxbitnet_error_message": (C.c_char_p, []),
}


def lib():
    """Load liboxbitnet.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeError(f"{LIB_PATH} is missing: build it with `python 0xbitnet_amd/build.py`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().oxb_last_error()
    return msg.decode() if msg else "unknown error"


def check(rc: int, what: str = "") -> int:
    if rc != 0:
        raise NativeError(f"{what}: {last_error()}" if what else last_error())
    return rc
