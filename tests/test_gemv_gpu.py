"""GPU parity of the dequant-fused GEMV against the oracle, through the C ABI.

Bound: per row, |y_gpu - y_oracle| <= 1e-4 * sum_i |w_i x_i| (exact w).
Dequantisation and the fp16-special rejection are checked bit-exactly.
"""
import os

import numpy as np
import pytest

import oracle
from llambda_amd import ggml, synthetic
from llambda_amd.hip_backend import (HipBackendError, make_hip_session, make_hip_session_packed,
                                     write_packed_projection)

from helpers import abs_dot_bound, assert_within_bound, make_gemv

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def check_gemv(type_tag, rows, columns, seed, x=None):
    w, x0 = make_gemv(type_tag, rows, columns, seed)
    x = x0 if x is None else x
    print(f"gemv type={ggml.NAMES[type_tag]} rows={rows} cols={columns} seed={seed}", flush=True)
    s = make_hip_session_packed(w, type_tag, rows, columns)
    try:
        y = np.empty(rows, dtype=np.float32)
        s.run_into(y, x)
    finally:
        s.close()
    y_ref = oracle.gemv(type_tag, w, rows, columns, x, threads=THREADS)
    bound = abs_dot_bound(type_tag, w, rows, columns, x)
    return assert_within_bound(y, y_ref, bound, f"{ggml.NAMES[type_tag]} {rows}x{columns}")


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_q4k_4096_square(hip, seed):
    check_gemv(ggml.Q4_K, 4096, 4096, seed)


def test_q4k_reference_input(hip):
    check_gemv(ggml.Q4_K, 4096, 4096, 7, x=synthetic.reference_input(4096))


def test_q6k_output_head(hip):
    check_gemv(ggml.Q6_K, 128256, 4096, 1)


@pytest.mark.parametrize("type_tag,rows,columns", [
    (ggml.Q4_K, 14336, 4096),   # ffn_gate / ffn_up
    (ggml.Q6_K, 4096, 14336),   # ffn_down
    (ggml.Q6_K, 1024, 4096),    # attn_v
    (ggml.Q4_K, 1024, 4096),    # attn_k
])
def test_llama_layer_shapes(hip, type_tag, rows, columns):
    check_gemv(type_tag, rows, columns, 11)


@pytest.mark.parametrize("type_tag", [ggml.Q4_K, ggml.Q6_K])
@pytest.mark.parametrize("rows", [1, 3, 95, 96, 97, 1000])
@pytest.mark.parametrize("columns", [256, 512, 768, 2816])
def test_small_shapes_kquants(hip, type_tag, rows, columns):
    check_gemv(type_tag, rows, columns, rows * 7 + columns)


@pytest.mark.parametrize("type_tag", [ggml.Q5_0, ggml.Q8_0, ggml.F32])
@pytest.mark.parametrize("rows,columns", [(1, 32), (7, 96), (130, 2688), (64, 1856), (33, 3712)])
def test_small_shapes_32blocks(hip, type_tag, rows, columns):
    check_gemv(type_tag, rows, columns, rows + columns)


@pytest.mark.parametrize("type_tag,columns", [(ggml.Q4_K, 768), (ggml.Q6_K, 768), (ggml.Q6_K, 1280),
                                              (ggml.Q5_0, 96), (ggml.Q8_0, 160)])
def test_dequantize_bit_exact(hip, type_tag, columns):
    rows = 37
    rng = np.random.default_rng(columns)
    w = synthetic.packed(type_tag, rng, rows, columns).reshape(rows * (columns // ggml.block_elements(type_tag)), -1)
    # spread the fp16 scale fields over normals, subnormals, zero and negatives
    d = rng.choice(np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x8001, 0xBC00, 0x7BFF, 0x0000, 0x8000],
                            dtype=np.uint16), size=w.shape[0])
    off = 208 if type_tag == ggml.Q6_K else 0
    w[:, off] = d & 0xFF
    w[:, off + 1] = d >> 8
    w = w.reshape(-1)
    s = make_hip_session_packed(w, type_tag, rows, columns)
    try:
        got = s.dequantize()
    finally:
        s.close()
    want = oracle.dequantize(type_tag, w, rows * columns).reshape(rows, columns)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("type_tag", [ggml.Q4_K, ggml.Q6_K, ggml.Q5_0])
def test_fp16_special_rejected(hip, type_tag):
    rows, columns = 4, 256
    w = synthetic.packed(type_tag, np.random.default_rng(5), rows, columns)
    off = 208 if type_tag == ggml.Q6_K else 0
    bb = ggml.block_bytes(type_tag)
    w = w.copy()
    blk = 2
    w[blk * bb + off] = 0x00
    w[blk * bb + off + 1] = 0x7C  # +inf
    with pytest.raises(HipBackendError, match="Unsupported fp16 special value"):
        make_hip_session_packed(w, type_tag, rows, columns)


def test_batch_matches_oracle(hip):
    """Every row of a multi-token run meets the bound against the oracle
    (batch runs use the token-tiled kernel, single runs the row-streaming one)."""
    rows, columns = 515, 2048
    rng = np.random.default_rng(3)
    for type_tag in (ggml.Q4_K, ggml.Q6_K, ggml.Q8_0):
        w = synthetic.packed(type_tag, rng, rows, columns)
        s = make_hip_session_packed(w, type_tag, rows, columns)
        try:
            for batch in (2, 3, 5, 9):
                x = synthetic.activations(rng, batch, columns)
                yb = np.empty((batch, rows), dtype=np.float32)
                s.run_batch_into(yb, x, batch)
                for t in range(batch):
                    y_ref = oracle.gemv(type_tag, w, rows, columns, x[t])
                    bound = abs_dot_bound(type_tag, w, rows, columns, x[t])
                    assert_within_bound(yb[t], y_ref, bound, f"batch {batch} token {t}")
        finally:
            s.close()


@pytest.mark.parametrize("type_tag", [ggml.Q6_K, ggml.Q4_K])
def test_tile_rounds_equal_the_short_launch_kernel(hip, type_tag):
    """A long launch (128256 rows x 4096: tile rounds, one contiguous DMA run
    per wave) and short launches over slices of the same rows (the per-wave
    chunk staging) compute each row with the same arithmetic in the same
    order: equal bit for bit, first, middle and last (partial) tiles."""
    rows, columns = 128256 - 7, 4096
    w, x = make_gemv(type_tag, rows, columns, 23)
    rb = ggml.row_bytes(type_tag, columns)
    s = make_hip_session_packed(w, type_tag, rows, columns)
    try:
        y = np.empty(rows, dtype=np.float32)
        s.run_into(y, x)
    finally:
        s.close()
    for first, count in ((0, 4096), (61440, 1000), (rows - 100, 100)):
        part = make_hip_session_packed(w[first * rb:(first + count) * rb], type_tag, count, columns)
        try:
            yp = np.empty(count, dtype=np.float32)
            part.run_into(yp, x)
        finally:
            part.close()
        assert np.array_equal(yp, y[first:first + count]), (first, count)


def test_scaling_is_exact(hip):
    """y(2x) = 2 y(x) bit for bit: power-of-two scaling commutes with every
    rounding, so any mismatch is a kernel bug."""
    rows, columns = 128256, 4096
    w, x = make_gemv(ggml.Q6_K, rows, columns, 21)
    s = make_hip_session_packed(w, ggml.Q6_K, rows, columns)
    try:
        y1 = np.empty(rows, dtype=np.float32)
        y2 = np.empty(rows, dtype=np.float32)
        s.run_into(y1, x)
        s.run_into(y2, (2 * x).astype(np.float32))
    finally:
        s.close()
    assert np.array_equal(y2, 2 * y1)


def test_packed_file_session(hip, tmp_path):
    rows, columns = 300, 512
    w, x = make_gemv(ggml.Q6_K, rows, columns, 4)
    path = str(tmp_path / "projection.onnx")
    write_packed_projection(path, ggml.Q6_K, rows, columns, w)
    s = make_hip_session(path, cache_directory=str(tmp_path), cache_key="k")
    try:
        assert s.input_element_count == columns and s.output_element_count == rows
        y = np.empty(rows, dtype=np.float32)
        s.run_into(y, x)
    finally:
        s.close()
    y_ref = oracle.gemv(ggml.Q6_K, w, rows, columns, x)
    assert_within_bound(y, y_ref, abs_dot_bound(ggml.Q6_K, w, rows, columns, x))


def test_count_mismatch_is_an_error(hip):
    rows, columns = 8, 256
    w, x = make_gemv(ggml.Q4_K, rows, columns, 1)
    s = make_hip_session_packed(w, ggml.Q4_K, rows, columns)
    try:
        with pytest.raises(HipBackendError, match="input element count"):
            s.run_into(np.empty(rows, dtype=np.float32), np.zeros(columns + 1, dtype=np.float32))
        with pytest.raises(HipBackendError, match="output element count"):
            s.run_into(np.empty(rows + 1, dtype=np.float32), x)
    finally:
        s.close()
