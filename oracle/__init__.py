"""ctypes front end of the CPU oracle (oracle/llambda_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this module, and only as the
parity checker or the reported CPU baseline.  The product path
(``llambda_amd``) never imports it.

The C restatement follows the reference's CPU kernels (llambda.lisp); see the
header of ``llambda_oracle.h`` for which check pins each function.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

TYPE_F32 = 0
TYPE_Q5_0 = 6
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile; returns the library path."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class OracleError(RuntimeError):
    pass


class MoeDesc(ctypes.Structure):
    _fields_ = [
        ("variant", ctypes.c_int),
        ("hidden", ctypes.c_int64),
        ("expert_count", ctypes.c_int64),
        ("top_k", ctypes.c_int64),
        ("expert_ffn", ctypes.c_int64),
        ("shared_ffn", ctypes.c_int64),
        ("router", ctypes.c_void_p),
        ("shared_gate_inp", ctypes.c_void_p),
        ("router_bias", ctypes.c_void_p),
        ("expert_weights_scale", ctypes.c_float),
        ("expert_weights_norm", ctypes.c_int),
        ("gate_type", ctypes.c_int), ("gate_exps", ctypes.c_void_p),
        ("up_type", ctypes.c_int), ("up_exps", ctypes.c_void_p),
        ("down_type", ctypes.c_int), ("down_exps", ctypes.c_void_p),
        ("shared_gate_type", ctypes.c_int), ("shared_gate", ctypes.c_void_p),
        ("shared_up_type", ctypes.c_int), ("shared_up", ctypes.c_void_p),
        ("shared_down_type", ctypes.c_int), ("shared_down", ctypes.c_void_p),
        ("latent_in", ctypes.c_int64),
        ("latent_down_type", ctypes.c_int), ("latent_down", ctypes.c_void_p),
        ("latent_up_type", ctypes.c_int), ("latent_up", ctypes.c_void_p),
        ("latent_out", ctypes.c_int64),
    ]


class OTensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("data", ctypes.c_void_p)]


class LlamaLayerDesc(ctypes.Structure):
    _fields_ = [("attn_norm", ctypes.c_void_p), ("attn_q", OTensor), ("attn_k", OTensor),
                ("attn_v", OTensor), ("attn_output", OTensor), ("ffn_norm", ctypes.c_void_p),
                ("ffn_gate", OTensor), ("ffn_up", OTensor), ("ffn_down", OTensor)]


class LlamaDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int64), ("layer_count", ctypes.c_int64),
                ("heads", ctypes.c_int64), ("kv_heads", ctypes.c_int64), ("ffn", ctypes.c_int64),
                ("vocab", ctypes.c_int64), ("rope_dim", ctypes.c_int64),
                ("norm_eps", ctypes.c_float), ("rope_base", ctypes.c_float),
                ("rope_factors", ctypes.c_void_p), ("rope_factor_count", ctypes.c_int64),
                ("token_embd", OTensor), ("output", OTensor), ("output_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(LlamaLayerDesc))]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_last_error.restype = ctypes.c_char_p
        L.oracle_row_bytes.restype = ctypes.c_int64
        L.oracle_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
        L.oracle_fp16_to_f32.argtypes = [ctypes.c_uint16, ctypes.POINTER(ctypes.c_float)]
        L.oracle_get_scale_min_k4.argtypes = [ctypes.c_void_p, ctypes.c_int,
                                              ctypes.POINTER(ctypes.c_int),
                                              ctypes.POINTER(ctypes.c_int)]
        L.oracle_dequantize.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_void_p]
        L.oracle_dot_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.POINTER(ctypes.c_float)]
        L.oracle_dot_product.restype = ctypes.c_float
        L.oracle_dot_product.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.oracle_gemv.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.oracle_select_top_k.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_void_p, ctypes.c_void_p]
        for name in ("oracle_sigmoid", "oracle_silu", "oracle_relu_squared"):
            f = getattr(L, name)
            f.restype = ctypes.c_float
            f.argtypes = [ctypes.c_float]
        L.oracle_moe_forward.argtypes = [ctypes.POINTER(MoeDesc), ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.oracle_rms_norm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_float, ctypes.c_void_p]
        L.oracle_rope_head.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_float, ctypes.c_void_p,
                                       ctypes.c_int64]
        L.oracle_softmax.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        L.oracle_attention.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        L.oracle_llama_step.argtypes = [ctypes.POINTER(LlamaDesc), ctypes.c_void_p,
                                        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_void_p, ctypes.c_int]
        L.oracle_llama_step_hidden.argtypes = [ctypes.POINTER(LlamaDesc), ctypes.c_void_p,
                                               ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        i64p = ctypes.c_void_p
        L.oracle_repetition_penalty.argtypes = [ctypes.c_void_p, ctypes.c_int64, i64p,
                                                ctypes.c_int64, ctypes.c_float]
        L.oracle_top_k.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
        L.oracle_top_p.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                   ctypes.c_float]
        L.oracle_sample_from_probabilities.restype = ctypes.c_int64
        L.oracle_sample_from_probabilities.argtypes = [ctypes.c_void_p, ctypes.c_int64,
                                                       ctypes.c_float]
        L.oracle_sample_token.argtypes = [ctypes.c_void_p, ctypes.c_int64, i64p, ctypes.c_int64,
                                          ctypes.c_float, ctypes.c_int64, ctypes.c_float,
                                          ctypes.c_float, ctypes.c_float, ctypes.c_void_p]
        _lib = L
    return _lib


def _check(status: int) -> None:
    if status != 0:
        raise OracleError(lib().oracle_last_error().decode())


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def row_bytes(type_tag: int, columns: int) -> int:
    n = lib().oracle_row_bytes(type_tag, columns)
    if n < 0:
        raise OracleError(lib().oracle_last_error().decode())
    return n


def columns_of(type_tag: int, row_byte_count: int) -> int:
    """Columns of one packed row of row_byte_count bytes (its smallest block
    of 1, 32 or 256 weights, whichever the type takes)."""
    for block in (1, 32, 256):
        if lib().oracle_row_bytes(type_tag, block) > 0:
            return row_byte_count // row_bytes(type_tag, block) * block
    raise OracleError(f"unknown GGML type tag {type_tag}")


def fp16_to_f32(bits: int) -> float:
    out = ctypes.c_float()
    _check(lib().oracle_fp16_to_f32(bits, ctypes.byref(out)))
    return out.value


def get_scale_min_k4(scales: bytes, index: int):
    buf = np.frombuffer(bytes(scales), dtype=np.uint8).copy()
    sc, m = ctypes.c_int(), ctypes.c_int()
    lib().oracle_get_scale_min_k4(buf.ctypes.data, index, ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequantize(type_tag: int, data: np.ndarray, elements: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(elements, dtype=np.float32)
    _check(lib().oracle_dequantize(type_tag, data.ctypes.data, elements, out.ctypes.data))
    return out


def dot_row(type_tag: int, row: np.ndarray, x: np.ndarray) -> float:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = ctypes.c_float()
    _check(lib().oracle_dot_row(type_tag, row.ctypes.data, x.ctypes.data, x.size,
                                ctypes.byref(out)))
    return out.value


def dot_product(left: np.ndarray, right: np.ndarray) -> np.float32:
    left = np.ascontiguousarray(left, dtype=np.float32)
    right = np.ascontiguousarray(right, dtype=np.float32)
    return np.float32(lib().oracle_dot_product(left.ctypes.data, right.ctypes.data, left.size))


def gemv(type_tag: int, matrix: np.ndarray, rows: int, columns: int, x: np.ndarray,
         threads: int = 1) -> np.ndarray:
    matrix = np.ascontiguousarray(matrix).view(np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == columns
    assert matrix.size >= rows * row_bytes(type_tag, columns)
    y = np.empty(rows, dtype=np.float32)
    _check(lib().oracle_gemv(type_tag, matrix.ctypes.data, rows, columns, x.ctypes.data,
                             y.ctypes.data, threads))
    return y


def select_top_k(logits: np.ndarray, k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.empty(k, dtype=np.int64)
    val = np.empty(k, dtype=np.float32)
    lib().oracle_select_top_k(logits.ctypes.data, logits.size, k, idx.ctypes.data,
                              val.ctypes.data)
    return idx, val


def sigmoid(x: float) -> float:
    return lib().oracle_sigmoid(x)


def silu(x: float) -> float:
    return lib().oracle_silu(x)


def relu_squared(x: float) -> float:
    return lib().oracle_relu_squared(x)


@dataclass
class MoeResult:
    y: np.ndarray
    top_indices: np.ndarray
    top_weights: np.ndarray
    router_logits: np.ndarray


def moe_forward(layer, x: np.ndarray, threads: int = 1) -> MoeResult:
    """Run one MoE layer token by token.

    ``layer`` is any object with the attributes of ``llambda_amd.moe.MoeLayer``
    (variant, hidden, expert_count, top_k, expert_ffn, shared_ffn, router,
    shared_gate_inp, router_bias, expert_weights_scale, expert_weights_norm and
    the (type, bytes) pairs gate/up/down/shared_gate/shared_up/shared_down).
    """
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, layer.hidden)
    tokens = x.shape[0]
    keep = []

    def arr(a, dtype):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dtype)
        keep.append(a)
        return a.ctypes.data

    d = MoeDesc()
    d.variant = layer.variant
    d.hidden = layer.hidden
    d.expert_count = layer.expert_count
    d.top_k = layer.top_k
    d.expert_ffn = layer.expert_ffn
    d.shared_ffn = layer.shared_ffn
    d.router = arr(layer.router, np.float32)
    d.shared_gate_inp = arr(layer.shared_gate_inp, np.float32)
    d.router_bias = arr(layer.router_bias, np.float32)
    d.expert_weights_scale = layer.expert_weights_scale
    d.expert_weights_norm = int(layer.expert_weights_norm)
    for name in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down"):
        pair = getattr(layer, name)
        field = name if name.startswith("shared") else name + "_exps"
        if pair is None:
            setattr(d, name + "_type", 0)
            setattr(d, field, None)
        else:
            setattr(d, name + "_type", pair[0])
            setattr(d, field, arr(pair[1], np.uint8))
    latent_down = getattr(layer, "latent_down", None)
    latent_up = getattr(layer, "latent_up", None)
    if latent_down is not None:  # [Li][H]
        d.latent_in = np.asarray(latent_down[1]).size // row_bytes(latent_down[0], layer.hidden)
        d.latent_down_type = latent_down[0]
        d.latent_down = arr(latent_down[1], np.uint8)
    if latent_up is not None:  # [H][Lo]
        d.latent_out = columns_of(latent_up[0], np.asarray(latent_up[1]).size // layer.hidden)
        d.latent_up_type = latent_up[0]
        d.latent_up = arr(latent_up[1], np.uint8)
    y = np.empty_like(x)
    idx = np.empty((tokens, layer.top_k), dtype=np.int64)
    w = np.empty((tokens, layer.top_k), dtype=np.float32)
    logits = np.empty((tokens, layer.expert_count), dtype=np.float32)
    _check(lib().oracle_moe_forward(ctypes.byref(d), x.ctypes.data, y.ctypes.data, tokens,
                                    idx.ctypes.data, w.ctypes.data, logits.ctypes.data,
                                    threads))
    return MoeResult(y, idx, w, logits)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rms_norm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().oracle_rms_norm(x.ctypes.data, w.ctypes.data, x.size, eps, out.ctypes.data)
    return out


def rope_head(head, position: int, rope_dim: int, theta_base: float,
              factors: Optional[np.ndarray] = None) -> np.ndarray:
    out = _f32(head).copy()
    f = None if factors is None else _f32(factors)
    lib().oracle_rope_head(out.ctypes.data, out.size, position, rope_dim, theta_base,
                           _ptr(f), 0 if f is None else f.size)
    return out


def softmax(logits) -> np.ndarray:
    x = _f32(logits)
    out = np.empty_like(x)
    lib().oracle_softmax(x.ctypes.data, x.size, out.ctypes.data)
    return out


def attention(q, kcache, vcache, n: int) -> np.ndarray:
    """q [heads][D]; caches [kv_heads][cap][D]; slots 0..n-1."""
    q, kc, vc = _f32(q), _f32(kcache), _f32(vcache)
    heads, D = q.shape
    kv_heads, cap, _ = kc.shape
    out = np.empty_like(q)
    _check(lib().oracle_attention(q.ctypes.data, kc.ctypes.data, vc.ctypes.data, cap, n, heads,
                                  kv_heads, D, out.ctypes.data))
    return out


def llama_step(weights, kv: np.ndarray, token: int, position: int, threads: int = 1,
               return_hidden: bool = False):
    """One step of the Llama step function on host weights (an object with the
    attributes of llambda_amd.llama.LlamaWeights).  kv: float32
    [layers][2][kv_heads][cap][head_dim], updated in place (slot `position`).
    With return_hidden, (logits, the output rows' input rms-norm(x) * output_norm)."""
    c = weights.config
    assert kv.dtype == np.float32 and kv.flags["C_CONTIGUOUS"]
    cap = kv.shape[3]
    keep = []

    def vec(a):
        a = _f32(a)
        keep.append(a)
        return a.ctypes.data

    def ten(t):
        a = np.ascontiguousarray(t[1], dtype=np.uint8)
        keep.append(a)
        o = OTensor()
        o.type, o.data = t[0], a.ctypes.data
        return o

    layers = (LlamaLayerDesc * c.layer_count)()
    for i, L in enumerate(weights.layers):
        layers[i].attn_norm = vec(L.attn_norm)
        layers[i].attn_q, layers[i].attn_k = ten(L.attn_q), ten(L.attn_k)
        layers[i].attn_v, layers[i].attn_output = ten(L.attn_v), ten(L.attn_output)
        layers[i].ffn_norm = vec(L.ffn_norm)
        layers[i].ffn_gate, layers[i].ffn_up = ten(L.ffn_gate), ten(L.ffn_up)
        layers[i].ffn_down = ten(L.ffn_down)
    d = LlamaDesc()
    d.hidden, d.layer_count, d.heads, d.kv_heads = c.hidden, c.layer_count, c.head_count, c.kv_head_count
    d.ffn, d.vocab, d.rope_dim = c.ffn, c.vocab, c.rope_dimension
    d.norm_eps, d.rope_base = c.norm_epsilon, c.rope_base
    if weights.rope_factors is not None:
        d.rope_factors = vec(weights.rope_factors)
        d.rope_factor_count = len(weights.rope_factors)
    d.token_embd, d.output = ten(weights.token_embd), ten(weights.output)
    d.output_norm = vec(weights.output_norm)
    d.layers = layers
    logits = np.empty(c.vocab, dtype=np.float32)
    hidden = np.empty(c.hidden, dtype=np.float32)
    _check(lib().oracle_llama_step_hidden(ctypes.byref(d), kv.ctypes.data, cap, token, position,
                                          logits.ctypes.data, hidden.ctypes.data, threads))
    return (logits, hidden) if return_hidden else logits


def repetition_penalty(logits, history, penalty: float) -> np.ndarray:
    out = _f32(logits).copy()
    h = np.ascontiguousarray(history, dtype=np.int64)
    _check(lib().oracle_repetition_penalty(out.ctypes.data, out.size, h.ctypes.data, h.size,
                                           penalty))
    return out


def top_k(logits, k: int) -> np.ndarray:
    out = _f32(logits).copy()
    _check(lib().oracle_top_k(out.ctypes.data, out.size, k))
    return out


def top_p(logits, p: float, temperature: float = 1.0) -> np.ndarray:
    out = _f32(logits).copy()
    _check(lib().oracle_top_p(out.ctypes.data, out.size, p, temperature))
    return out


def sample_from_probabilities(probs, roll: float) -> int:
    p = _f32(probs)
    return int(lib().oracle_sample_from_probabilities(p.ctypes.data, p.size, roll))


def sample_token(logits, *, history=None, repetition_penalty: float = 1.15, top_k: int = 40,
                 top_p: float = 0.95, temperature: float = 1.0, random_value: float) -> int:
    """sample-token-id-from-logits (llambda.lisp:1272-1317) on a copy of logits;
    top_k=None -> 40 and top_p=None -> 0.95 as the reference defaults them."""
    x = _f32(logits).copy()
    h = np.ascontiguousarray(history if history is not None else [], dtype=np.int64)
    tok = ctypes.c_int64()
    _check(lib().oracle_sample_token(x.ctypes.data, x.size, h.ctypes.data, h.size,
                                     repetition_penalty, 40 if top_k is None else top_k,
                                     0.95 if top_p is None else top_p, temperature,
                                     random_value, ctypes.byref(tok)))
    return tok.value
