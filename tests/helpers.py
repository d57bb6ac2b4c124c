"""Shared test helpers: parity bounds and synthetic problems."""
from __future__ import annotations

import numpy as np

import oracle
from llambda_amd import ggml, synthetic

# per output row, max |y - y_ref| <= REL * sum_i |w_i * x_i|
# with w the exact dequantised weights (fp32 accumulation in another order).
REL = 1e-4


def abs_dot_bound(type_tag: int, packed: np.ndarray, rows: int, columns: int, x: np.ndarray,
                  chunk_rows: int = 8192) -> np.ndarray:
    """sum_i |w_i x_i| per row (float64), w from the oracle's dequantiser."""
    rb = ggml.row_bytes(type_tag, columns)
    ax = np.abs(x.astype(np.float64))
    out = np.empty(rows, dtype=np.float64)
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        if type_tag == ggml.F32:
            w = packed.view(np.float32).reshape(rows, columns)[r0:r1]
        else:
            w = oracle.dequantize(type_tag, packed[r0 * rb:r1 * rb], (r1 - r0) * columns)
            w = w.reshape(r1 - r0, columns)
        out[r0:r1] = np.abs(w).astype(np.float64) @ ax
    return out


def assert_within_bound(y: np.ndarray, y_ref: np.ndarray, bound: np.ndarray, what: str = ""):
    err = np.abs(y.astype(np.float64) - y_ref.astype(np.float64))
    limit = REL * bound
    bad = np.nonzero(~(err <= limit))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size} rows exceed 1e-4*sum|w*x| (first row {i}: |diff|={err[i]:.3e} "
            f"limit={limit[i]:.3e} gpu={y[i]!r} ref={y_ref[i]!r})")
    return float(np.max(err / np.maximum(bound, 1e-300))) if err.size else 0.0


def make_gemv(type_tag: int, rows: int, columns: int, seed: int):
    rng = np.random.default_rng(seed)
    w = synthetic.packed(type_tag, rng, rows, columns)
    x = synthetic.activations(rng, 1, columns)[0]
    return w, x


def routing_margin_ok(logits_ref: np.ndarray, k: int, bound: np.ndarray) -> np.ndarray:
    """Per token: True when the gap between every adjacent pair of the top k+1
    reference logits exceeds twice the router error bound, so the ordered
    selection is fixed by the reference arithmetic."""
    ok = np.empty(logits_ref.shape[0], dtype=bool)
    for t, row in enumerate(logits_ref):
        top = np.sort(row[np.isfinite(row)])[::-1][:k + 1]
        gaps = -np.diff(top)
        ok[t] = bool(np.all(gaps > 2 * bound[t]))
    return ok
