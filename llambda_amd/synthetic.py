"""Seeded synthetic GGUF-layout tensors for the benchmark workloads.

Distributions follow the workloads this backend is measured on:
  Q4_K: fp16 d, dmin ~ U[1e-4, 1e-3]; 12 scale bytes uniform (16 independent
        6-bit fields); 128 nibble bytes uniform.
  Q6_K: ql, qh uniform bytes; 16 int8 scales ~ U{-64..63}; fp16 d ~ U[1e-4, 1e-3].
  Q5_0: fp16 d ~ U[1e-4, 1e-3]; high bits and nibbles uniform.
  Q8_0: fp16 d ~ U[1e-4, 1e-3]; 32 int8 uniform.
Every generator returns a flat uint8 array of rows * row_bytes bytes.
"""
from __future__ import annotations

import numpy as np

from . import ggml


def _d16(rng: np.random.Generator, n: int, lo: float = 1e-4, hi: float = 1e-3) -> np.ndarray:
    return rng.uniform(lo, hi, size=n).astype(np.float16).view(np.uint8).reshape(n, 2)


def q4_k(rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    nb = rows * (columns // 256)
    out = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    out[:, 0:2] = _d16(rng, nb)
    out[:, 2:4] = _d16(rng, nb)
    return out.reshape(-1)


def q6_k(rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    nb = rows * (columns // 256)
    out = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    out[:, 192:208] = rng.integers(-64, 64, size=(nb, 16), dtype=np.int8).view(np.uint8)
    out[:, 208:210] = _d16(rng, nb)
    return out.reshape(-1)


def q5_0(rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    nb = rows * (columns // 32)
    out = rng.integers(0, 256, size=(nb, 22), dtype=np.uint8)
    out[:, 0:2] = _d16(rng, nb)
    return out.reshape(-1)


def q8_0(rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    nb = rows * (columns // 32)
    out = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    out[:, 0:2] = _d16(rng, nb)
    return out.reshape(-1)


def f32(rng: np.random.Generator, rows: int, columns: int, std: float = 0.02) -> np.ndarray:
    return rng.normal(0.0, std, size=(rows, columns)).astype(np.float32).reshape(-1).view(np.uint8)


GENERATORS = {ggml.Q4_K: q4_k, ggml.Q6_K: q6_k, ggml.Q5_0: q5_0, ggml.Q8_0: q8_0, ggml.F32: f32}


def packed(type_tag: int, rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    ggml.tensor_byte_size(type_tag, columns)
    return GENERATORS[type_tag](rng, rows, columns)


def activations(rng: np.random.Generator, tokens: int, columns: int) -> np.ndarray:
    return rng.standard_normal(size=(tokens, columns)).astype(np.float32)


def reference_input(columns: int) -> np.ndarray:
    """The deterministic input of benchmark-gguf-projection-backends,
    x[i] = ((17 i + 11) mod 257) / 128 - 1 (llambda.lisp:4870-4874)."""
    i = np.arange(columns, dtype=np.int64)
    return (((i * 17 + 11) % 257) / 128.0 - 1.0).astype(np.float32)
