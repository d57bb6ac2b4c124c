"""ctypes bindings of libllambda_hip.so -- the foreign-function layer.

This is the Python counterpart of the reference's CFFI declarations for its
native bridge (llambda.lisp:82-127): one binding per exported function of
include/llambda_hip.h.  Loading fails loudly when the library is missing;
there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("LLAMBDA_HIP_LIBRARY", os.path.join(HERE, "libllambda_hip.so"))

_lock = threading.Lock()
_lib = None

# LLAMBDA_HIP_INPUT_ERROR: a MoE run met the reference's own error for its
# input; the session stays usable
INPUT_ERROR = -2
# LLAMBDA_HIP_STREAM_READ_WORDS: words of llambda_hip_stream_read's output
STREAM_READ_WORDS = 4096

c_int = ctypes.c_int
c_size = ctypes.c_size_t
c_i64 = ctypes.c_int64
c_void_p = ctypes.c_void_p
c_char_p = ctypes.c_char_p
c_float_p = ctypes.POINTER(ctypes.c_float)


class MoeDesc(ctypes.Structure):
    """llambda_hip_moe_desc."""
    _fields_ = [
        ("variant", c_int),
        ("hidden", c_i64),
        ("expert_count", c_i64),
        ("top_k", c_i64),
        ("expert_ffn", c_i64),
        ("shared_ffn", c_i64),
        ("router", c_void_p),
        ("shared_gate_inp", c_void_p),
        ("router_bias", c_void_p),
        ("expert_weights_scale", ctypes.c_float),
        ("expert_weights_norm", c_int),
        ("gate_type", c_int), ("gate_exps", c_void_p),
        ("up_type", c_int), ("up_exps", c_void_p),
        ("down_type", c_int), ("down_exps", c_void_p),
        ("shared_gate_type", c_int), ("shared_gate", c_void_p),
        ("shared_up_type", c_int), ("shared_up", c_void_p),
        ("shared_down_type", c_int), ("shared_down", c_void_p),
        ("latent_down_type", c_int), ("latent_down", c_void_p),
        ("latent_up_type", c_int), ("latent_up", c_void_p),
        ("latent_in", c_i64),
        ("latent_out", c_i64),
    ]


class TensorRef(ctypes.Structure):
    """llambda_hip_tensor_ref."""
    _fields_ = [("type", c_int), ("data", c_void_p), ("bytes", c_size)]


class LlamaLayer(ctypes.Structure):
    """llambda_hip_llama_layer."""
    _fields_ = [
        ("attn_norm", c_void_p),
        ("attn_q", TensorRef), ("attn_k", TensorRef), ("attn_v", TensorRef),
        ("attn_output", TensorRef),
        ("ffn_norm", c_void_p),
        ("ffn_gate", TensorRef), ("ffn_up", TensorRef), ("ffn_down", TensorRef),
    ]


class LlamaDesc(ctypes.Structure):
    """llambda_hip_llama_desc."""
    _fields_ = [
        ("hidden", c_i64), ("layer_count", c_i64), ("head_count", c_i64),
        ("kv_head_count", c_i64), ("ffn", c_i64), ("vocab", c_i64), ("rope_dimension", c_i64),
        ("norm_epsilon", ctypes.c_float), ("rope_base", ctypes.c_float),
        ("rope_factors", c_void_p), ("rope_factor_count", c_i64),
        ("context", c_i64),
        ("weights_on_device", c_int),
        ("token_embd", TensorRef), ("output", TensorRef),
        ("output_norm", c_void_p),
        ("layers", ctypes.POINTER(LlamaLayer)),
    ]


class Sampling(ctypes.Structure):
    """llambda_hip_sampling."""
    _fields_ = [("history", c_void_p), ("history_count", c_size),
                ("repetition_penalty", ctypes.c_float), ("top_k", c_i64),
                ("top_p", ctypes.c_float), ("temperature", ctypes.c_float),
                ("random_value", ctypes.c_float)]


class GgufTensor(ctypes.Structure):
    """llambda_hip_gguf_tensor."""
    _fields_ = [("name", c_void_p), ("name_length", c_size), ("dimension_count", ctypes.c_uint32),
                ("dimensions", ctypes.c_uint64 * 4), ("type", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("element_count", ctypes.c_uint64),
                ("supported", c_int), ("byte_size", ctypes.c_uint64),
                ("data_offset", ctypes.c_uint64), ("data", c_void_p)]


class GgufValue(ctypes.Structure):
    """llambda_hip_gguf_value."""
    _fields_ = [("key", c_void_p), ("key_length", c_size), ("type", ctypes.c_uint32),
                ("element_type", ctypes.c_uint32), ("count", ctypes.c_uint64),
                ("u", ctypes.c_uint64), ("i", ctypes.c_int64), ("f", ctypes.c_double),
                ("string", c_void_p), ("string_length", c_size)]


# name -> (restype, argtypes); the complete export list of include/llambda_hip.h
SIGNATURES = {
    "llambda_hip_probe": (c_int, []),
    "llambda_hip_bridge_version": (c_char_p, []),
    "llambda_hip_runtime_version": (c_char_p, []),
    "llambda_hip_last_error": (c_char_p, []),
    "llambda_hip_sha256": (c_int, [c_void_p, c_size, c_char_p, c_size]),
    "llambda_hip_session_create": (c_int, [c_char_p, c_char_p, c_char_p, ctypes.POINTER(c_void_p)]),
    "llambda_hip_session_create_packed": (c_int, [c_void_p, c_size, c_int, c_i64, c_i64,
                                                  ctypes.POINTER(c_void_p)]),
    "llambda_hip_session_destroy": (None, [c_void_p]),
    "llambda_hip_session_input_element_count": (c_size, [c_void_p]),
    "llambda_hip_session_output_element_count": (c_size, [c_void_p]),
    "llambda_hip_session_run": (c_int, [c_void_p, c_void_p, c_size, c_void_p, c_size]),
    "llambda_hip_session_run_batch": (c_int, [c_void_p, c_void_p, c_size, c_void_p, c_size, c_size]),
    "llambda_hip_session_run_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_void_p]),
    "llambda_hip_session_dequantize": (c_int, [c_void_p, c_void_p, c_size]),
    "llambda_hip_moe_session_create": (c_int, [ctypes.POINTER(MoeDesc), ctypes.POINTER(c_void_p)]),
    "llambda_hip_moe_session_destroy": (None, [c_void_p]),
    "llambda_hip_moe_session_hidden_size": (c_size, [c_void_p]),
    "llambda_hip_moe_session_expert_count": (c_size, [c_void_p]),
    "llambda_hip_moe_session_run": (c_int, [c_void_p, c_void_p, c_size, c_void_p, c_size, c_size,
                                            c_void_p, c_void_p, c_void_p]),
    "llambda_hip_moe_session_run_device": (c_int, [c_void_p, c_void_p, c_void_p, c_size, c_void_p]),
    "llambda_hip_moe_session_sync": (c_int, [c_void_p, c_void_p]),
    "llambda_hip_moe_session_run_device_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_size,
                                                           c_void_p]),
    "llambda_hip_select_top_k": (c_int, [c_void_p, c_size, c_size, c_size, c_void_p, c_void_p]),
    "llambda_hip_stream_read": (c_int, [c_void_p, c_size, c_void_p, c_void_p]),
    "llambda_hip_llama_session_create": (c_int, [ctypes.POINTER(LlamaDesc),
                                                 ctypes.POINTER(c_void_p)]),
    "llambda_hip_llama_session_destroy": (None, [c_void_p]),
    "llambda_hip_llama_session_vocab": (c_size, [c_void_p]),
    "llambda_hip_llama_session_step": (c_int, [c_void_p, c_i64, c_i64, c_void_p, c_size]),
    "llambda_hip_llama_session_step_device": (c_int, [c_void_p, c_i64, c_i64, c_void_p, c_void_p,
                                                      c_int]),
    "llambda_hip_llama_session_logits": (c_int, [c_void_p, c_void_p, c_size]),
    "llambda_hip_llama_session_write_kv": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p,
                                                   c_void_p, c_int]),
    "llambda_hip_llama_session_read_kv": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p,
                                                  c_void_p]),
    "llambda_hip_llama_session_sync": (c_int, [c_void_p, c_void_p]),
    "llambda_hip_sampler_create": (c_int, [c_size, ctypes.POINTER(c_void_p)]),
    "llambda_hip_sampler_destroy": (None, [c_void_p]),
    "llambda_hip_sampler_sample": (c_int, [c_void_p, c_void_p, c_size, c_int,
                                           ctypes.POINTER(Sampling), ctypes.POINTER(c_i64)]),
    "llambda_hip_llama_session_sample": (c_int, [c_void_p, c_void_p, ctypes.POINTER(Sampling),
                                                 ctypes.POINTER(c_i64)]),
    "llambda_hip_gguf_open": (c_int, [c_char_p, ctypes.POINTER(c_void_p)]),
    "llambda_hip_gguf_close": (None, [c_void_p]),
    "llambda_hip_gguf_header": (c_int, [c_void_p, ctypes.POINTER(ctypes.c_uint32),
                                        ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(ctypes.c_uint64)]),
    "llambda_hip_gguf_mapping": (c_void_p, [c_void_p, ctypes.POINTER(c_size)]),
    "llambda_hip_gguf_tensor_info": (c_int, [c_void_p, ctypes.c_uint64,
                                             ctypes.POINTER(GgufTensor)]),
    "llambda_hip_gguf_find_tensor": (c_i64, [c_void_p, c_char_p]),
    "llambda_hip_gguf_kv": (c_int, [c_void_p, ctypes.c_uint64, ctypes.POINTER(GgufValue)]),
    "llambda_hip_gguf_kv_element": (c_int, [c_void_p, ctypes.c_uint64, ctypes.c_uint64,
                                            ctypes.POINTER(GgufValue)]),
}


class NativeLibraryMissing(RuntimeError):
    pass


def library_path() -> str:
    return LIB_PATH


def lib():
    """The loaded library (loaded once).  Raises NativeLibraryMissing when the
    shared object has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} is missing; build it with `python -m llambda_amd.build`")
            L = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = L
    return _lib


def last_error() -> str:
    msg = lib().llambda_hip_last_error()
    return msg.decode(errors="replace") if msg else ""
