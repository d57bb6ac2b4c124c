"""Device-resident Llama-layout decode token: host side of the llama session.

Mirrors the reference's ``make-llama-step-function`` (llambda.lisp:6294-6441):
the model hyper-parameters ``load-llama-model`` reads (llambda.lisp:6269-6292),
the tensors a step touches (``token_embd``, per layer ``attn_norm``,
``attn_q/k/v``, ``attn_output``, ``ffn_norm``, ``ffn_gate/up/down``, then
``output_norm`` and ``output``; ``rope_freqs`` when present) and the step
itself, ``(token-id position) -> logits``.  The whole step runs on the
device through ``llambda_hip_llama_session_*`` (include/llambda_hip.h); there
is no host fallback.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from . import ggml, native, synthetic

Tensor = Tuple[int, np.ndarray]  # (GGML type tag, packed bytes)


@dataclass
class LlamaConfig:
    """llama.* GGUF metadata (llambda.lisp:6269-6292) plus the cache size."""
    hidden: int
    layer_count: int
    head_count: int
    kv_head_count: int
    ffn: int
    vocab: int
    rope_dimension: int
    norm_epsilon: float = 1.0e-5
    rope_base: float = 500000.0
    context: int = 4352

    @property
    def head_dim(self) -> int:
        return self.hidden // self.head_count


LLAMA31_8B = LlamaConfig(hidden=4096, layer_count=32, head_count=32, kv_head_count=8, ffn=14336,
                         vocab=128256, rope_dimension=128)


@dataclass
class LlamaLayerWeights:
    attn_norm: np.ndarray
    attn_q: Tensor
    attn_k: Tensor
    attn_v: Tensor
    attn_output: Tensor
    ffn_norm: np.ndarray
    ffn_gate: Tensor
    ffn_up: Tensor
    ffn_down: Tensor


@dataclass
class LlamaWeights:
    config: LlamaConfig
    token_embd: Tensor
    output: Tensor
    output_norm: np.ndarray
    rope_factors: Optional[np.ndarray]
    layers: List[LlamaLayerWeights] = field(default_factory=list)


def llama31_rope_factors(head_dim: int, base: float = 500000.0, factor: float = 8.0,
                         low_freq_factor: float = 1.0, high_freq_factor: float = 4.0,
                         original_context: int = 8192) -> np.ndarray:
    """rope_freqs.weight of a Llama-3.1 model: the published Llama-3.1 RoPE
    scaling (wavelengths above original_context / low_freq_factor divided by
    `factor`, below original_context / high_freq_factor kept, a smooth blend
    between), as one factor per rotary pair."""
    low_wavelen = original_context / low_freq_factor
    high_wavelen = original_context / high_freq_factor
    out = []
    for i in range(0, head_dim, 2):
        freq = 1.0 / base ** (i / head_dim)
        wavelen = 2.0 * math.pi / freq
        if wavelen < high_wavelen:
            out.append(1.0)
        elif wavelen > low_wavelen:
            out.append(factor)
        else:
            smooth = (original_context / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
            out.append(1.0 / ((1.0 - smooth) / factor + smooth))
    return np.asarray(out, dtype=np.float32)


def _norm(rng: np.random.Generator, n: int) -> np.ndarray:
    return rng.uniform(0.5, 1.5, size=n).astype(np.float32)


def synthetic_llama(rng: np.random.Generator, config: LlamaConfig, *,
                    attn_v_type: int = ggml.Q6_K, ffn_down_type: int = ggml.Q6_K,
                    default_type: int = ggml.Q4_K, output_type: int = ggml.Q6_K,
                    rope_factors: bool = True) -> LlamaWeights:
    """Random-init weights of the given layout in host memory, Q4_K_M mix by
    default (attn_v and ffn_down Q6_K, the rest Q4_K; output Q6_K); norm
    weights ~ U[0.5, 1.5]."""
    c = config
    H, D = c.hidden, c.head_dim
    gen = synthetic.GENERATORS

    def t(type_tag, rows, cols):
        return (type_tag, gen[type_tag](rng, rows, cols))

    layers = []
    for _ in range(c.layer_count):
        layers.append(LlamaLayerWeights(
            attn_norm=_norm(rng, H),
            attn_q=t(default_type, c.head_count * D, H),
            attn_k=t(default_type, c.kv_head_count * D, H),
            attn_v=t(attn_v_type, c.kv_head_count * D, H),
            attn_output=t(default_type, H, c.head_count * D),
            ffn_norm=_norm(rng, H),
            ffn_gate=t(default_type, c.ffn, H),
            ffn_up=t(default_type, c.ffn, H),
            ffn_down=t(ffn_down_type, H, c.ffn)))
    return LlamaWeights(
        config=c,
        token_embd=t(default_type, c.vocab, H),
        output=t(output_type, c.vocab, H),
        output_norm=_norm(rng, H),
        rope_factors=llama31_rope_factors(D, c.rope_base) if rope_factors else None,
        layers=layers)


@dataclass
class DeviceTensor:
    """A packed tensor already in device memory (pointer and size)."""
    type: int
    ptr: int
    nbytes: int
    owner: object = None  # keeps the allocation alive


def synthetic_llama_device(seed: int, config: LlamaConfig, rng: np.random.Generator):
    """The same layout as ``synthetic_llama`` with the packed tensors drawn on
    the device (torch's generator) -- for full-size models, whose 5 GB of
    blocks would take minutes to draw on the host.  Norms and rope factors
    stay host arrays.  Returns a LlamaWeights whose tensors are DeviceTensor."""
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    c = config
    H, D = c.hidden, c.head_dim

    def d16(nb):
        return (torch.rand((nb, 1), device="cuda", generator=gen) * 9e-4 + 1e-4).half()

    def t(type_tag, rows, cols):
        nb = rows * (cols // 256)
        bb = ggml.block_bytes(type_tag)
        blocks = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device="cuda", generator=gen)
        if type_tag == ggml.Q4_K:
            blocks[:, 0:2] = d16(nb).view(torch.uint8)
            blocks[:, 2:4] = d16(nb).view(torch.uint8)
        elif type_tag == ggml.Q6_K:
            blocks[:, 192:208] = torch.randint(-64, 64, (nb, 16), dtype=torch.int8, device="cuda",
                                               generator=gen).view(torch.uint8)
            blocks[:, 208:210] = d16(nb).view(torch.uint8)
        else:
            raise ValueError("device synthesis covers Q4_K and Q6_K")
        return DeviceTensor(type_tag, blocks.data_ptr(), nb * bb, blocks)

    layers = []
    for _ in range(c.layer_count):
        layers.append(LlamaLayerWeights(
            attn_norm=_norm(rng, H),
            attn_q=t(ggml.Q4_K, c.head_count * D, H),
            attn_k=t(ggml.Q4_K, c.kv_head_count * D, H),
            attn_v=t(ggml.Q6_K, c.kv_head_count * D, H),
            attn_output=t(ggml.Q4_K, H, c.head_count * D),
            ffn_norm=_norm(rng, H),
            ffn_gate=t(ggml.Q4_K, c.ffn, H),
            ffn_up=t(ggml.Q4_K, c.ffn, H),
            ffn_down=t(ggml.Q6_K, H, c.ffn)))
    return LlamaWeights(config=c, token_embd=t(ggml.Q4_K, c.vocab, H),
                        output=t(ggml.Q6_K, c.vocab, H), output_norm=_norm(rng, H),
                        rope_factors=llama31_rope_factors(D, c.rope_base), layers=layers)


def _type(t) -> int:
    return t.type if isinstance(t, DeviceTensor) else t[0]


def _nbytes(t) -> int:
    return t.nbytes if isinstance(t, DeviceTensor) else t[1].nbytes


def weight_bytes(w: LlamaWeights) -> int:
    """Packed bytes one step reads: every layer matrix, the output rows and
    one embedding row."""
    nbytes = _nbytes
    total = nbytes(w.output) + ggml.row_bytes(_type(w.token_embd), w.config.hidden)
    for L in w.layers:
        for t in (L.attn_q, L.attn_k, L.attn_v, L.attn_output, L.ffn_gate, L.ffn_up, L.ffn_down):
            total += nbytes(t)
    return total


class LlamaError(RuntimeError):
    pass


def _check(status: int, what: str) -> None:
    if status != 0:
        raise LlamaError(f"{what}: {native.last_error()}")


class HipLlamaSession:
    """The model on the device with a zeroed fp32 KV cache of `context` slots
    per layer (llambda_hip_llama_session_*)."""

    def __init__(self, weights: LlamaWeights, context: Optional[int] = None):
        L = native.lib()
        c = weights.config
        self.config = c
        self.context = context or c.context
        keep = []

        def ref(t):
            r = native.TensorRef()
            if isinstance(t, DeviceTensor):
                r.type, r.data, r.bytes = t.type, t.ptr, t.nbytes
            else:
                a = np.ascontiguousarray(t[1], dtype=np.uint8)
                keep.append(a)
                r.type, r.data, r.bytes = t[0], a.ctypes.data, a.nbytes
            return r

        def vec(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            return a.ctypes.data

        on_device = isinstance(weights.output, DeviceTensor)
        layers = (native.LlamaLayer * c.layer_count)()
        for i, lw in enumerate(weights.layers):
            layers[i].attn_norm = vec(lw.attn_norm)
            layers[i].attn_q = ref(lw.attn_q)
            layers[i].attn_k = ref(lw.attn_k)
            layers[i].attn_v = ref(lw.attn_v)
            layers[i].attn_output = ref(lw.attn_output)
            layers[i].ffn_norm = vec(lw.ffn_norm)
            layers[i].ffn_gate = ref(lw.ffn_gate)
            layers[i].ffn_up = ref(lw.ffn_up)
            layers[i].ffn_down = ref(lw.ffn_down)
        d = native.LlamaDesc()
        d.hidden, d.layer_count, d.head_count = c.hidden, c.layer_count, c.head_count
        d.kv_head_count, d.ffn, d.vocab = c.kv_head_count, c.ffn, c.vocab
        d.rope_dimension = c.rope_dimension
        d.norm_epsilon, d.rope_base = c.norm_epsilon, c.rope_base
        if weights.rope_factors is not None:
            d.rope_factors = vec(weights.rope_factors)
            d.rope_factor_count = len(weights.rope_factors)
        d.context = self.context
        d.weights_on_device = int(on_device)
        d.token_embd = ref(weights.token_embd)
        d.output = ref(weights.output)
        d.output_norm = vec(weights.output_norm)
        d.layers = layers
        handle = ctypes.c_void_p()
        _check(L.llambda_hip_llama_session_create(ctypes.byref(d), ctypes.byref(handle)),
               "llama session")
        self._h = handle
        del keep

    def close(self) -> None:
        if getattr(self, "_h", None):
            native.lib().llambda_hip_llama_session_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    def step(self, token: int, position: int) -> np.ndarray:
        """logits[vocab] of one decode step (synchronous)."""
        out = np.empty(self.config.vocab, dtype=np.float32)
        _check(native.lib().llambda_hip_llama_session_step(self._h, token, position,
                                                           out.ctypes.data, out.size), "llama step")
        return out

    def step_device(self, token: int, position: int, logits_ptr: int = 0, stream: int = 0,
                    graph: bool = True) -> None:
        """Enqueue one step; logits_ptr = 0 writes the session's own buffer."""
        _check(native.lib().llambda_hip_llama_session_step_device(
            self._h, token, position, logits_ptr or None, stream or None, int(graph)),
            "llama step")

    def logits(self) -> np.ndarray:
        """The session's own logits buffer (after step_device with logits_ptr=0)."""
        out = np.empty(self.config.vocab, dtype=np.float32)
        _check(native.lib().llambda_hip_llama_session_logits(self._h, out.ctypes.data, out.size),
               "llama logits")
        return out

    def sync(self, stream: int = 0) -> None:
        _check(native.lib().llambda_hip_llama_session_sync(self._h, stream or None), "llama sync")

    def write_kv(self, layer: int, first: int, keys: np.ndarray, values: np.ndarray) -> None:
        """Cache slots [first, first + count) of `layer` from host arrays
        [kv_heads][count][head_dim] float32."""
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        values = np.ascontiguousarray(values, dtype=np.float32)
        assert keys.shape == values.shape and keys.shape[0] == self.config.kv_head_count
        _check(native.lib().llambda_hip_llama_session_write_kv(
            self._h, layer, first, keys.shape[1], keys.ctypes.data, values.ctypes.data, 0),
            "write_kv")

    def write_kv_device(self, layer: int, first: int, count: int, keys_ptr: int,
                        values_ptr: int) -> None:
        """As write_kv from device memory [kv_heads][count][head_dim]."""
        _check(native.lib().llambda_hip_llama_session_write_kv(
            self._h, layer, first, count, keys_ptr, values_ptr, 1), "write_kv")

    def read_kv(self, layer: int, first: int, count: int):
        shape = (self.config.kv_head_count, count, self.config.head_dim)
        k = np.empty(shape, dtype=np.float32)
        v = np.empty(shape, dtype=np.float32)
        _check(native.lib().llambda_hip_llama_session_read_kv(self._h, layer, first, count,
                                                              k.ctypes.data, v.ctypes.data),
               "read_kv")
        return k, v
