"""Token sampling on the device: the host side of llambda_hip_sampler_*.

Mirrors the reference's ``sample-token-id-from-logits`` (llambda.lisp:1272-1317)
keyword for keyword -- history, repetition-penalty (1.15), top-k (40, NIL ->
40), top-p (0.95, NIL -> 0.95), temperature (1.0) and an explicit
random-value in [0, 1) -- and its argument errors.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np

from . import native

DEFAULT_TOP_K = 40      # llambda.lisp:32
DEFAULT_TOP_P = 0.95    # llambda.lisp:33


class SamplingError(RuntimeError):
    pass


def _params(history, repetition_penalty, top_k, top_p, temperature, random_value, keep):
    p = native.Sampling()
    if history is not None and len(history):
        h = np.ascontiguousarray(history, dtype=np.int64)
        keep.append(h)
        p.history, p.history_count = h.ctypes.data, h.size
    p.repetition_penalty = repetition_penalty
    p.top_k = DEFAULT_TOP_K if top_k is None else int(top_k)
    p.top_p = DEFAULT_TOP_P if top_p is None else float(top_p)
    p.temperature = temperature
    p.random_value = random_value
    return p


class HipSampler:
    """Device scratch for logits rows of up to `vocab` entries."""

    def __init__(self, vocab: int):
        handle = ctypes.c_void_p()
        if native.lib().llambda_hip_sampler_create(vocab, ctypes.byref(handle)) != 0:
            raise SamplingError(native.last_error())
        self._h = handle
        self.vocab = vocab

    def close(self) -> None:
        if getattr(self, "_h", None):
            native.lib().llambda_hip_sampler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    def sample(self, logits, *, random_value: float, history: Optional[Sequence[int]] = None,
               repetition_penalty: float = 1.15, top_k: Optional[int] = DEFAULT_TOP_K,
               top_p: Optional[float] = DEFAULT_TOP_P, temperature: float = 1.0,
               device_count: Optional[int] = None) -> int:
        """logits: a host array, or a device pointer (int) with device_count
        entries.  The logits are not modified."""
        keep = []
        p = _params(history, repetition_penalty, top_k, top_p, temperature, random_value, keep)
        tok = ctypes.c_int64()
        if isinstance(logits, int):
            ptr, n, dev = logits, int(device_count), 1
        else:
            a = np.ascontiguousarray(logits, dtype=np.float32)
            keep.append(a)
            ptr, n, dev = a.ctypes.data, a.size, 0
        if native.lib().llambda_hip_sampler_sample(self._h, ptr, n, dev, ctypes.byref(p),
                                                   ctypes.byref(tok)) != 0:
            raise SamplingError(native.last_error())
        return tok.value

    def sample_session(self, session, *, random_value: float, history=None,
                       repetition_penalty: float = 1.15, top_k=DEFAULT_TOP_K,
                       top_p=DEFAULT_TOP_P, temperature: float = 1.0) -> int:
        """Sample from a HipLlamaSession's own logits (after step_device with
        logits_ptr=0)."""
        keep = []
        p = _params(history, repetition_penalty, top_k, top_p, temperature, random_value, keep)
        tok = ctypes.c_int64()
        if native.lib().llambda_hip_llama_session_sample(session._h, self._h, ctypes.byref(p),
                                                         ctypes.byref(tok)) != 0:
            raise SamplingError(native.last_error())
        return tok.value
