"""Routed-MoE layer sessions on the HIP backend.

A ``MoeLayer`` holds the tensors one layer of qwen3next-moe-into
(llambda.lisp:5321-5426) or nemotron-h-moe-ffn-into (llambda.lisp:5827-5949)
reads; ``HipMoeSession`` uploads them once and runs the whole feed-forward
(router, top-k, gating, experts, combine) on the device for a batch of
tokens.  In the reference the routed experts bypass the accelerator store
(llambda.lisp:4951-4971); this session is the per-layer hook, bound by layer
index in the model's MoE-layer table (projection.register_model_accelerator_
moe_layer), apart from the tensor-indexed 2-D projections, so the router
tensor blk.N.ffn_gate_inp.weight keeps its own 2-D binding.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np

from . import ggml, native, synthetic
from .hip_backend import HipBackendError, _check

QWEN3NEXT = 0
NEMOTRON_H = 1

Packed = Tuple[int, np.ndarray]  # (GGML type tag, bytes)


@dataclass
class MoeLayer:
    variant: int
    hidden: int
    expert_count: int
    top_k: int
    expert_ffn: int
    shared_ffn: int
    router: np.ndarray                        # F32 [E][H]   ffn_gate_inp
    up: Packed                                # [E*F][H]      ffn_up_exps
    down: Packed                              # [E*H][F]      ffn_down_exps
    gate: Optional[Packed] = None             # [E*F][H]      ffn_gate_exps (qwen3next)
    shared_gate_inp: Optional[np.ndarray] = None  # F32 [H]  ffn_gate_inp_shexp (qwen3next)
    router_bias: Optional[np.ndarray] = None  # F32 [E]       exp_probs_b.bias (nemotron)
    expert_weights_scale: float = 1.0
    expert_weights_norm: bool = False
    shared_gate: Optional[Packed] = None      # [Fs][H]       ffn_gate_shexp (qwen3next)
    shared_up: Optional[Packed] = None        # [Fs][H]       ffn_up_shexp
    shared_down: Optional[Packed] = None      # [H][Fs]       ffn_down_shexp
    latent_down: Optional[Packed] = None      # [Li][H]       ffn_latent_down (nemotron)
    latent_up: Optional[Packed] = None        # [H][Lo]       ffn_latent_up (nemotron)
    layer_index: Optional[int] = None         # blk.N, for the reference's error texts

    @property
    def latent_in(self) -> int:
        """Li: rows of ffn_latent_down (0 without it)."""
        if self.latent_down is None:
            return 0
        return self.latent_down[1].size // ggml.row_bytes(self.latent_down[0], self.hidden)

    @property
    def latent_out(self) -> int:
        """Lo: columns of ffn_latent_up (0 without it)."""
        if self.latent_up is None:
            return 0
        t, data = self.latent_up
        return data.size // self.hidden // ggml.block_bytes(t) * ggml.block_elements(t)

    def weight_bytes(self) -> int:
        """Packed bytes of every tensor the layer can read."""
        n = self.router.nbytes
        for t in (self.gate, self.up, self.down, self.shared_gate, self.shared_up, self.shared_down,
                  self.latent_down, self.latent_up):
            if t is not None:
                n += t[1].nbytes
        for v in (self.shared_gate_inp, self.router_bias):
            if v is not None:
                n += v.nbytes
        return n

    def expert_bytes(self) -> int:
        """Packed bytes of one routed expert (gate + up + down)."""
        din, dout = self.latent_in or self.hidden, self.latent_out or self.hidden
        per = ggml.row_bytes(self.up[0], din) * self.expert_ffn
        if self.gate is not None:
            per += ggml.row_bytes(self.gate[0], self.hidden) * self.expert_ffn
        per += ggml.row_bytes(self.down[0], self.expert_ffn) * dout
        return per

    def flops_per_token(self) -> int:
        """2 x the multiply-adds of one token: the router (and the shared-expert
        gate row), k routed experts (gate, up and down rows), the shared expert."""
        H, F, Fs = self.hidden, self.expert_ffn, self.shared_ffn
        din, dout = self.latent_in or H, self.latent_out or H
        per_expert = (2 if self.gate is not None else 1) * F * din + F * dout
        shared = ((3 if self.shared_gate is not None else 2) * Fs * H) if Fs else 0
        router = self.expert_count * H + (H if self.shared_gate_inp is not None else 0)
        latent = (self.latent_in + self.latent_out) * H
        return 2 * (self.top_k * per_expert + shared + router + latent)

    def shared_bytes(self) -> int:
        if not self.shared_ffn:
            return 0
        n = ggml.row_bytes(self.shared_up[0], self.hidden) * self.shared_ffn
        if self.shared_gate is not None:
            n += ggml.row_bytes(self.shared_gate[0], self.hidden) * self.shared_ffn
        n += ggml.row_bytes(self.shared_down[0], self.shared_ffn) * self.hidden
        if self.shared_gate_inp is not None:
            n += self.shared_gate_inp.nbytes
        return n


class MoeLayerInputError(RuntimeError):
    """The reference's own error for a token (status -2 from the library):
    a non-positive top-k weight sum (llambda.lisp:5373-5375, 5903-5905) or
    fewer than k selectable router logits.  Deliberately not a
    HipBackendError: the backend's error predicate does not select it, so
    the runtime fallback re-signals it and the layer stays on the device,
    as the reference's CPU body signals it for that call alone."""


def _check_moe(status: int, what: str, layer_index: Optional[int]) -> None:
    if status == native.INPUT_ERROR:
        text = native.last_error()
        if layer_index is not None:
            # the reference's texts name the layer: "<variant> layer N router ..."
            text = text.replace(" layer router ", f" layer {layer_index} router ", 1)
        raise MoeLayerInputError(text)
    _check(status, what)


class HipMoeSession:
    def __init__(self, layer: MoeLayer):
        self.layer = layer
        keep = []

        def arr(a, dtype):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return a.ctypes.data

        d = native.MoeDesc()
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
        d.expert_weights_norm = int(bool(layer.expert_weights_norm))
        for name, field in (("gate", "gate_exps"), ("up", "up_exps"), ("down", "down_exps"),
                            ("shared_gate", "shared_gate"), ("shared_up", "shared_up"),
                            ("shared_down", "shared_down"), ("latent_down", "latent_down"),
                            ("latent_up", "latent_up")):
            pair = getattr(layer, name)
            if pair is not None:
                setattr(d, name + "_type", pair[0])
                setattr(d, field, arr(pair[1], np.uint8))
        d.latent_in = layer.latent_in
        d.latent_out = layer.latent_out
        handle = ctypes.c_void_p()
        _check(native.lib().llambda_hip_moe_session_create(ctypes.byref(d), ctypes.byref(handle)),
               "HIP MoE session creation")
        self.pointer = handle.value

    def close(self) -> None:
        if self.pointer:
            native.lib().llambda_hip_moe_session_destroy(self.pointer)
            self.pointer = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    def _live(self):
        if not self.pointer:
            raise HipBackendError("HIP MoE session is closed.")
        return self.pointer

    @property
    def hidden_size(self) -> int:
        return native.lib().llambda_hip_moe_session_hidden_size(self.pointer)

    @property
    def expert_count(self) -> int:
        return native.lib().llambda_hip_moe_session_expert_count(self.pointer)

    def run_into(self, dest: np.ndarray, vector: np.ndarray) -> np.ndarray:
        """One token, the shape of the reference's MoE functions: dest[H] =
        the layer's FFN output for vector[H] (before the residual add)."""
        for a, what in ((dest, "destination"), (vector, "input")):
            if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
                raise HipBackendError(f"HIP MoE {what} must be a contiguous float32 array.")
        _check_moe(native.lib().llambda_hip_moe_session_run(
            self._live(), vector.ctypes.data, vector.size, dest.ctypes.data, dest.size, 1,
            None, None, None), "HIP MoE run", self.layer.layer_index)
        return dest

    def run(self, x: np.ndarray, with_routing: bool = False):
        """FFN output (before the residual) for x [tokens][H]; with_routing also
        returns (top_indices, top_weights, router_logits)."""
        L = self.layer
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, L.hidden)
        tokens = x.shape[0]
        y = np.empty_like(x)
        idx = w = logits = None
        if with_routing:
            idx = np.empty((tokens, L.top_k), dtype=np.int64)
            w = np.empty((tokens, L.top_k), dtype=np.float32)
            logits = np.empty((tokens, L.expert_count), dtype=np.float32)
        _check_moe(native.lib().llambda_hip_moe_session_run(
            self._live(), x.ctypes.data, x.size, y.ctypes.data, y.size, tokens,
            idx.ctypes.data if idx is not None else None,
            w.ctypes.data if w is not None else None,
            logits.ctypes.data if logits is not None else None), "HIP MoE run",
            self.layer.layer_index)
        return (y, idx, w, logits) if with_routing else y

    def run_device(self, x_ptr: int, y_ptr: int, tokens: int, stream: int = 0) -> None:
        _check(native.lib().llambda_hip_moe_session_run_device(self._live(), x_ptr, y_ptr, tokens,
                                                               stream or None),
               "HIP MoE device run")

    def sync(self, stream: int = 0) -> None:
        _check_moe(native.lib().llambda_hip_moe_session_sync(self._live(), stream or None),
                   "HIP MoE sync", self.layer.layer_index)


def moe_layer_from_model(model, layer_index: int, variant: int, *, expert_used_count: int,
                         expert_weights_scale: float = 1.0,
                         expert_weights_norm: bool = False) -> MoeLayer:
    """The tensors of layer `layer_index` as the reference's MoE functions look
    them up (blk.N.<name>.weight, llambda.lisp:5321-5426, 5827-5949), from a
    projection.ProjectionModel; k = min(E, expert_used_count)."""
    def info(name, required=False):
        suffix = ".bias" if name == "exp_probs_b" else ".weight"
        return model.tensor_info(f"blk.{layer_index}.{name}{suffix}", required=required)

    def packed(name, required=False):
        t = info(name, required)
        return (t.type_tag, t.data) if t is not None else None

    def vector(name, required=False):
        t = info(name, required)
        if t is None:
            return None
        if t.type_tag != ggml.F32:
            raise HipBackendError(f"blk.{layer_index}.{name} must be F32")
        return np.ascontiguousarray(t.data).view(np.float32)

    router = info("ffn_gate_inp", required=True)
    if router.type_tag != ggml.F32:
        raise HipBackendError(f"blk.{layer_index}.ffn_gate_inp must be F32")
    up = info("ffn_up_exps", required=True)
    shared_up = info("ffn_up_shexp")
    E, H = router.rows, router.columns
    return MoeLayer(
        variant=variant, hidden=H, expert_count=E, top_k=min(E, expert_used_count),
        expert_ffn=up.rows, shared_ffn=shared_up.rows if shared_up is not None else 0,
        router=np.ascontiguousarray(router.data).view(np.float32).reshape(E, H),
        up=(up.type_tag, up.data), down=packed("ffn_down_exps", True),
        gate=packed("ffn_gate_exps", variant == QWEN3NEXT),
        shared_gate_inp=vector("ffn_gate_inp_shexp") if variant == QWEN3NEXT else None,
        router_bias=vector("exp_probs_b", True) if variant == NEMOTRON_H else None,
        expert_weights_scale=expert_weights_scale if variant == NEMOTRON_H else 1.0,
        expert_weights_norm=expert_weights_norm if variant == NEMOTRON_H else True,
        shared_gate=packed("ffn_gate_shexp"), shared_up=packed("ffn_up_shexp"),
        shared_down=packed("ffn_down_shexp"),
        latent_down=packed("ffn_latent_down") if variant == NEMOTRON_H else None,
        latent_up=packed("ffn_latent_up") if variant == NEMOTRON_H else None,
        layer_index=layer_index)


def select_top_k(logits: np.ndarray, k: int):
    """Device top-k of each row of logits [batch][n] (select-top-k-logits-into)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None, :]
    batch, n = logits.shape
    idx = np.empty((batch, k), dtype=np.int64)
    val = np.empty((batch, k), dtype=np.float32)
    _check(native.lib().llambda_hip_select_top_k(logits.ctypes.data, n, k, batch, idx.ctypes.data,
                                                 val.ctypes.data), "HIP top-k")
    return idx, val


# ------------------------------------------------------------ synthetic layers

def synthetic_qwen3next(rng: np.random.Generator, *, hidden=2048, experts=512, top_k=10, ffn=512,
                        shared_ffn=512, gate_type=ggml.Q4_K, down_type=ggml.Q6_K,
                        router_std=0.02) -> MoeLayer:
    """A Qwen3Next-shaped layer: gate/up Q4_K, down Q6_K, router F32 ~ N(0, 0.02)."""
    gen = synthetic.packed
    return MoeLayer(
        variant=QWEN3NEXT, hidden=hidden, expert_count=experts, top_k=top_k, expert_ffn=ffn,
        shared_ffn=shared_ffn,
        router=rng.normal(0.0, router_std, size=(experts, hidden)).astype(np.float32),
        gate=(gate_type, gen(gate_type, rng, experts * ffn, hidden)),
        up=(gate_type, gen(gate_type, rng, experts * ffn, hidden)),
        down=(down_type, gen(down_type, rng, experts * hidden, ffn)),
        shared_gate_inp=(rng.normal(0.0, router_std, size=hidden).astype(np.float32)
                         if shared_ffn else None),
        shared_gate=(gate_type, gen(gate_type, rng, shared_ffn, hidden)) if shared_ffn else None,
        shared_up=(gate_type, gen(gate_type, rng, shared_ffn, hidden)) if shared_ffn else None,
        shared_down=(down_type, gen(down_type, rng, hidden, shared_ffn)) if shared_ffn else None,
    )


def zipf_bias(rng: np.random.Generator, experts: int, s: float = 1.1, c: float = 0.5) -> np.ndarray:
    """Per-expert router bias b_e = c * log(p_e) for Zipf(s) probabilities over a
    random permutation of expert ranks."""
    ranks = rng.permutation(experts) + 1
    p = ranks.astype(np.float64) ** (-s)
    p /= p.sum()
    return (c * np.log(p)).astype(np.float32)


def synthetic_nemotron_h(rng: np.random.Generator, *, hidden=2688, experts=128, top_k=6, ffn=1856,
                         shared_ffn=3712, expert_type=ggml.Q5_0, down_type=ggml.Q5_0,
                         router_std=0.02, zipf_s=1.1, zipf_c=0.5, weights_scale=1.0,
                         weights_norm=True, latent_in=0, latent_out=0,
                         latent_type=ggml.Q8_0) -> MoeLayer:
    """A Nemotron-H-MoE-shaped layer: relu^2 experts, biased sigmoid routing.
    latent_in > 0 adds ffn_latent_down [latent_in][hidden] (the routed
    experts' input is then latent_in wide), latent_out > 0 adds
    ffn_latent_up [hidden][latent_out] (their weighted sum is latent_out
    wide), both of latent_type."""
    gen = synthetic.packed
    din = latent_in or hidden
    dout = latent_out or hidden
    return MoeLayer(
        variant=NEMOTRON_H, hidden=hidden, expert_count=experts, top_k=top_k, expert_ffn=ffn,
        shared_ffn=shared_ffn,
        router=rng.normal(0.0, router_std, size=(experts, hidden)).astype(np.float32),
        router_bias=zipf_bias(rng, experts, zipf_s, zipf_c),
        expert_weights_scale=weights_scale, expert_weights_norm=weights_norm,
        up=(expert_type, gen(expert_type, rng, experts * ffn, din)),
        down=(down_type, gen(down_type, rng, experts * dout, ffn)),
        shared_up=(expert_type, gen(expert_type, rng, shared_ffn, hidden)) if shared_ffn else None,
        shared_down=(down_type, gen(down_type, rng, hidden, shared_ffn)) if shared_ffn else None,
        latent_down=(latent_type, gen(latent_type, rng, latent_in, hidden)) if latent_in else None,
        latent_up=(latent_type, gen(latent_type, rng, hidden, latent_out)) if latent_out else None,
    )
