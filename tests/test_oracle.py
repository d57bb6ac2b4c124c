"""CPU tests that pin the oracle: the reference's known-answer tests, closed
forms, encoders written from the block layouts (round trips), and brute
force.  No GPU needed."""
import math

import numpy as np
import pytest

import oracle
from llambda_amd import ggml, synthetic

# ---------------------------------------------------------------- KATs

@pytest.mark.parametrize("name,type_tag", [("q4_k_dequantize", ggml.Q4_K),
                                           ("q6_k_dequantize", ggml.Q6_K)])
def test_reference_dequantize_kats(kats, name, type_tag):
    k = kats[name]
    block = np.frombuffer(bytes.fromhex(k["block_hex"]), dtype=np.uint8)
    w = oracle.dequantize(type_tag, block, 256)
    for start, end, value in k["expect_ranges"]:
        assert np.all(w[start:end] == np.float32(value)), (start, end)
    for i, value in k["expect_points"]:
        assert w[i] == np.float32(value)


def _sequential_dot(a, b):
    """dot-product (llambda.lisp:3491-3500): serial single-float sum."""
    s = np.float32(0.0)
    for x, y in zip(a.astype(np.float32), b.astype(np.float32)):
        s = np.float32(s + np.float32(x * y))
    return s


@pytest.mark.parametrize("name,type_tag,mod,off,div", [("q4_k_dot", ggml.Q4_K, 11, 5, 3.0),
                                                       ("q6_k_dot", ggml.Q6_K, 13, 6, 4.0)])
def test_reference_fused_dot_kats(kats, name, type_tag, mod, off, div):
    k = kats[name]
    block = np.frombuffer(bytes.fromhex(k["block_hex"]), dtype=np.uint8)
    v = np.array([np.float32(((i % mod) - off) / div) for i in range(256)], dtype=np.float32)
    expected = _sequential_dot(oracle.dequantize(type_tag, block, 256), v)
    got = oracle.dot_row(type_tag, block, v)
    assert abs(got - expected) < k["tolerance"]


def test_reference_silu_kat(kats):
    k = kats["silu"]
    assert abs(oracle.silu(k["x"]) - k["expect"]) < k["tolerance"]


# -------------------------------------------------------------- fp16

def test_fp16_all_patterns():
    bits = np.arange(65536, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    for b in range(65536):
        e = (b >> 10) & 31
        if e == 31:
            with pytest.raises(oracle.OracleError, match="Unsupported fp16 special value"):
                oracle.fp16_to_f32(b)
        else:
            got = np.float32(oracle.fp16_to_f32(b))
            assert got.view(np.uint32) == ref[b].view(np.uint32), hex(b)


# ------------------------------------------------- encoders (round trips)

def encode_scales_mins(scales, mins):
    """Pack 8 six-bit scales and mins into the 12 bytes of a Q4_K block:
    scales/mins 0..3 in the low 6 bits of bytes 0..3 / 4..7; scales/mins 4..7
    keep their low 4 bits in the low/high nibble of bytes 8..11 and their top
    2 bits in the top 2 bits of bytes 0..3 / 4..7."""
    b = [0] * 12
    for j in range(4):
        b[j] = (scales[j] & 63) | ((scales[j + 4] >> 4) << 6)
        b[j + 4] = (mins[j] & 63) | ((mins[j + 4] >> 4) << 6)
        b[j + 8] = (scales[j + 4] & 15) | ((mins[j + 4] & 15) << 4)
    return bytes(b)


def test_scale_min_round_trip():
    rng = np.random.default_rng(0)
    for _ in range(2000):
        sc = rng.integers(0, 64, size=8)
        mn = rng.integers(0, 64, size=8)
        packed = encode_scales_mins(sc, mn)
        for s in range(8):
            assert oracle.get_scale_min_k4(packed, s) == (sc[s], mn[s])


def encode_q4_k(d16, dmin16, scales, mins, q):
    """One Q4_K block from fields; q[256] in 0..15, element 64j + l (l < 32)
    is the low nibble of qs[32j + l], element 64j + 32 + l the high nibble."""
    qs = bytearray(128)
    for j in range(4):
        for l in range(32):
            qs[32 * j + l] = q[64 * j + l] | (q[64 * j + 32 + l] << 4)
    return (np.array([d16, dmin16], dtype="<u2").tobytes() + encode_scales_mins(scales, mins)
            + bytes(qs))


def test_q4_k_layout_from_fields():
    rng = np.random.default_rng(1)
    for _ in range(50):
        d = np.float16(rng.uniform(-2, 2))
        dmin = np.float16(rng.uniform(-2, 2))
        sc = rng.integers(0, 64, size=8)
        mn = rng.integers(0, 64, size=8)
        q = rng.integers(0, 16, size=256)
        blk = np.frombuffer(encode_q4_k(d.view(np.uint16), dmin.view(np.uint16), sc, mn, q),
                            dtype=np.uint8)
        w = oracle.dequantize(ggml.Q4_K, blk, 256)
        df, dminf = np.float32(d), np.float32(dmin)
        for e in range(256):
            s = e // 32
            want = np.float32(np.float32(np.float32(df * np.float32(sc[s])) * np.float32(q[e]))
                              - np.float32(dminf * np.float32(mn[s])))
            assert w[e].view(np.uint32) == want.view(np.uint32), e


def encode_q6_k(q, scales, d16):
    """One Q6_K block from q[256] in 0..63 (stored value q + 32 offset is
    applied by the decoder) and 16 int8 scales.  Element 128h + 32k + l:
    low 4 bits in ql[64h + l + 32*(k & 1)] (low nibble for k < 2, high for
    k >= 2), top 2 bits at bit 2k of qh[32h + l]."""
    ql = bytearray(128)
    qh = bytearray(64)
    for h in range(2):
        for k in range(4):
            for l in range(32):
                v = int(q[128 * h + 32 * k + l])
                idx = 64 * h + l + 32 * (k & 1)
                ql[idx] |= (v & 15) << (4 if k >= 2 else 0)
                qh[32 * h + l] |= (v >> 4) << (2 * k)
    return bytes(ql) + bytes(qh) + np.asarray(scales, dtype=np.int8).tobytes() + \
        np.array([d16], dtype="<u2").tobytes()


def test_q6_k_layout_from_fields():
    rng = np.random.default_rng(2)
    for _ in range(50):
        q = rng.integers(0, 64, size=256)
        sc = rng.integers(-128, 128, size=16)
        d = np.float16(rng.uniform(-1, 1))
        blk = np.frombuffer(encode_q6_k(q, sc, d.view(np.uint16)), dtype=np.uint8)
        w = oracle.dequantize(ggml.Q6_K, blk, 256)
        for e in range(256):
            h, k, l = e // 128, (e % 128) // 32, e % 32
            scale = sc[8 * h + l // 16 + 2 * k]
            want = np.float32(np.float32(np.float32(d) * np.float32(scale)) * np.float32(q[e] - 32))
            assert w[e].view(np.uint32) == want.view(np.uint32), e


def test_q5_0_and_q8_0_layout_from_fields():
    rng = np.random.default_rng(3)
    for _ in range(50):
        d = np.float16(rng.uniform(-1, 1))
        q5 = rng.integers(-16, 16, size=32)
        u = q5 + 16
        qh = 0
        qs = bytearray(16)
        for i in range(16):
            qs[i] = (u[i] & 15) | ((u[16 + i] & 15) << 4)
            qh |= ((u[i] >> 4) & 1) << i
            qh |= ((u[16 + i] >> 4) & 1) << (16 + i)
        blk = np.frombuffer(np.array([d.view(np.uint16)], dtype="<u2").tobytes()
                            + np.array([qh], dtype="<u4").tobytes() + bytes(qs), dtype=np.uint8)
        w = oracle.dequantize(ggml.Q5_0, blk, 32)
        assert np.array_equal(w, (np.float32(d) * q5.astype(np.float32)).astype(np.float32))
        q8 = rng.integers(-128, 128, size=32)
        blk8 = np.frombuffer(np.array([d.view(np.uint16)], dtype="<u2").tobytes()
                             + q8.astype(np.int8).tobytes(), dtype=np.uint8)
        w8 = oracle.dequantize(ggml.Q8_0, blk8, 32)
        assert np.array_equal(w8, (np.float32(d) * q8.astype(np.float32)).astype(np.float32))


# ------------------------------------------------------- fused dots, GEMV

@pytest.mark.parametrize("type_tag", [ggml.Q4_K, ggml.Q6_K, ggml.Q5_0, ggml.Q8_0])
def test_fused_dot_vs_float64(type_tag):
    rng = np.random.default_rng(type_tag)
    columns = 1024
    for _ in range(20):
        row = synthetic.packed(type_tag, rng, 1, columns)
        x = synthetic.activations(rng, 1, columns)[0]
        w = oracle.dequantize(type_tag, row, columns).astype(np.float64)
        exact = float(w @ x.astype(np.float64))
        bound = float(np.abs(w) @ np.abs(x.astype(np.float64)))
        got = oracle.dot_row(type_tag, row, x)
        # fp32 accumulation of 1024 terms: far inside 1e-5 of sum|w x|
        assert abs(got - exact) <= 1e-5 * bound


def test_f32_dot_is_serial_sum():
    rng = np.random.default_rng(4)
    a = rng.normal(size=777).astype(np.float32)
    b = rng.normal(size=777).astype(np.float32)
    want = _sequential_dot(b, a)
    assert oracle.dot_row(ggml.F32, a.view(np.uint8), b) == want
    assert oracle.dot_product(a, b) == _sequential_dot(a, b)


@pytest.mark.parametrize("type_tag", [ggml.Q4_K, ggml.Q6_K])
def test_gemv_thread_count_invariant(type_tag):
    rng = np.random.default_rng(5)
    rows, columns = 517, 512
    w = synthetic.packed(type_tag, rng, rows, columns)
    x = synthetic.activations(rng, 1, columns)[0]
    y1 = oracle.gemv(type_tag, w, rows, columns, x, threads=1)
    y7 = oracle.gemv(type_tag, w, rows, columns, x, threads=7)
    rb = ggml.row_bytes(type_tag, columns)
    assert np.array_equal(y1, y7)
    for r in (0, 95, 96, 516):
        assert y1[r] == np.float32(oracle.dot_row(type_tag, w[r * rb:(r + 1) * rb], x))


def test_row_bytes_errors():
    assert oracle.row_bytes(ggml.Q4_K, 4096) == 16 * 144
    assert oracle.row_bytes(ggml.Q6_K, 512) == 420
    with pytest.raises(oracle.OracleError, match="not a multiple of block size"):
        oracle.row_bytes(ggml.Q4_K, 2688)


# ----------------------------------------------------------- routing

def _stable_topk(row, k):
    valid = [i for i in range(row.size) if row[i] > np.float32(-3.4028235e38)]
    valid.sort(key=lambda i: (-float(row[i]), i))
    sel = valid[:k]
    idx = np.array(sel + [-1] * (k - len(sel)), dtype=np.int64)
    val = np.array([row[i] for i in sel] + [np.float32(-3.4028235e38)] * (k - len(sel)),
                   dtype=np.float32)
    return idx, val


def test_select_top_k_matches_stable_sort():
    rng = np.random.default_rng(6)
    for trial in range(300):
        n = int(rng.integers(1, 80))
        k = int(rng.integers(1, n + 1))
        row = rng.integers(-3, 4, size=n).astype(np.float32)  # many ties
        if trial % 3 == 0:
            row[rng.integers(0, n, size=max(1, n // 5))] = np.nan
        if trial % 5 == 0:
            row[rng.integers(0, n, size=max(1, n // 5))] = -np.inf
        if trial % 7 == 0:
            row[:] = np.float32(-3.4028235e38)
        idx, val = oracle.select_top_k(row, k)
        ridx, rval = _stable_topk(row, k)
        assert np.array_equal(idx, ridx), (row, k)
        assert np.array_equal(val.view(np.uint32), rval.view(np.uint32))


def test_activations_closed_forms():
    for x in np.linspace(-30, 30, 601).astype(np.float32):
        e = np.float32(math.exp(-float(x)))
        assert oracle.sigmoid(float(x)) == np.float32(1.0 / (1.0 + float(e)))
        assert oracle.silu(float(x)) == np.float32(float(x) / (1.0 + float(e)))
        r = max(np.float32(0), x)
        assert oracle.relu_squared(float(x)) == np.float32(r * r)
        assert abs(oracle.sigmoid(float(x)) - 1 / (1 + math.exp(-float(x)))) <= 2e-7
