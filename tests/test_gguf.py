"""The bounded GGUF parser (llambda_hip_gguf_*) against the reference's own
parser tests (tests.lisp:1512-1710, 1856-1935: byte-for-byte the same
fixtures), its error texts for malformed input, and writer round trips."""
import struct

import numpy as np
import pytest

from llambda_amd import ggml
from llambda_amd.gguf import (ARRAY, F32, STRING, U32, GgufError, GgufFile, load_llama,
                              read_gguf_header, save_llama, write_gguf)
from llambda_amd.llama import LlamaConfig, synthetic_llama


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


def string(s):
    b = s.encode()
    return u64(len(b)) + b


def header(tensors, kvs):
    return b"GGUF" + u32(3) + u64(tensors) + u64(kvs)


def write(tmp_path, name, data):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_read_gguf_header(tmp_path):
    # tests.lisp:1512-1546
    path = write(tmp_path, "h.gguf", header(17, 9))
    assert read_gguf_header(path) == {"magic": "GGUF", "version": 3, "tensor_count": 17,
                                      "metadata_kv_count": 9, "header_size": 24}
    with pytest.raises(GgufError, match="cannot fit"):  # the full parse is bounded
        GgufFile(path)
    with pytest.raises(GgufError, match="exceeds mapped file length"):
        read_gguf_header(write(tmp_path, "short.gguf", b"GGUF"))
    path = write(tmp_path, "h0.gguf", header(0, 0))
    with GgufFile(path) as f:
        assert (f.version, f.tensor_count, f.kv_count) == (3, 0, 0)


@pytest.mark.parametrize("name,data,text", [
    # tests.lisp:1548-1642
    ("header", b"GGUF", "exceeds mapped file length"),
    ("metadata-string", header(0, 1) + u64(1024) + b"\0" * 5, "exceeds mapped file length"),
    ("dimensions", header(1, 0) + string("x") + u32(5) + b"\0" * 20, "invalid dimension count"),
    ("tensor-data", header(1, 0) + string("x") + u32(1) + u64(1) + u32(0) + u64(0),
     "exceeds mapped file length"),
])
def test_malformed_gguf_input_is_bounded(tmp_path, name, data, text):
    if name == "tensor-data":
        data += b"\0" * ((-len(data)) % 32)
    with pytest.raises(GgufError, match=text):
        GgufFile(write(tmp_path, name + ".gguf", data))


@pytest.mark.parametrize("data,text", [
    (b"GGUX" + u32(3) + u64(0) + u64(0), "Invalid GGUF magic"),
    (b"", "exceeds mapped file length 0"),
    (header(0, 1) + string("a") + u32(9) + u32(9) + u64(1), "Nested GGUF metadata arrays"),
    (header(0, 1) + string("a") + u32(9) + u32(4) + u64(2 ** 40), "cannot fit"),
    (header(0, 1) + string("a") + u32(13), "Unsupported GGUF metadata value type"),
    (header(0, 1) + string("general.alignment") + u32(4) + u32(24),
     "alignment must be a positive power of two"),
    (header(2 ** 50, 0), "GGUF tensor info count"),
    (header(1, 0) + string("x") + u32(1) + u64(0) + u32(0) + u64(0), "non-positive dimensions"),
    (header(1, 0) + string("x") + u32(1) + u64(100) + u32(12) + u64(0),
     "not a multiple of block size 256"),
])
def test_more_malformed_input(tmp_path, data, text):
    with pytest.raises(GgufError, match=text):
        GgufFile(write(tmp_path, "m.gguf", data))


def test_read_gguf_kv_pairs(tmp_path):
    # tests.lisp:1644-1709
    data = header(0, 4)
    data += string("general.architecture") + u32(8) + string("llama")
    data += string("llama.block_count") + u32(4) + u32(32)
    data += string("general.add_bos_token") + u32(7) + b"\x01"
    data += string("test.array") + u32(9) + u32(4) + u64(2) + u32(7) + u32(8)
    with GgufFile(write(tmp_path, "kv.gguf", data)) as f:
        assert f.kv_pairs == [("general.architecture", "llama"), ("llama.block_count", 32),
                              ("general.add_bos_token", True), ("test.array", [7, 8])]


def test_read_gguf_tensor_infos_and_load_tensors(tmp_path):
    # tests.lisp:1856-1935
    data = header(2, 1) + string("general.alignment") + u32(4) + u32(32)
    data += string("tensor.f32") + u32(2) + u64(2) + u64(2) + u32(0) + u64(0)
    data += string("tensor.f16") + u32(1) + u64(2) + u32(1) + u64(16)
    data += b"\0" * ((-len(data)) % 32)
    data += struct.pack("<4f", 1.0, 2.0, 3.5, -4.0) + struct.pack("<2H", 0x3C00, 0xC000)
    with GgufFile(write(tmp_path, "t.gguf", data)) as f:
        assert len(f.tensor_infos) == 2
        t32, t16 = f.tensor_info("tensor.f32"), f.tensor_info("tensor.f16")
        assert t32["dimensions"] == [2, 2] and t32["type_name"] == "f32"
        assert t32["element_count"] == 4 and t32["byte_size"] == 16
        assert t16["dimensions"] == [2] and t16["type_name"] == "f16" and t16["offset"] == 16
        assert t16["data_offset"] == f.data_start + 16
        assert np.array_equal(f.tensor_f32("tensor.f32"), [1.0, 2.0, 3.5, -4.0])
        assert np.array_equal(f.tensor_bytes("tensor.f16").view(np.float16), [1.0, -2.0])


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(3)
    from llambda_amd import synthetic
    q4 = synthetic.q4_k(rng, 4, 512)
    q6 = synthetic.q6_k(rng, 3, 256)
    f32 = rng.normal(size=7).astype(np.float32)
    path = str(tmp_path / "w.gguf")
    write_gguf(path, [("a.u32", U32, 5), ("a.str", "héllo"), ("a.bool", True), ("a.f", F32, 0.5),
                      ("a.arr", ARRAY, (STRING, ["x", "yz"]))],
               [("q4", ggml.Q4_K, [512, 4], q4), ("q6", ggml.Q6_K, [256, 3], q6),
                ("f", ggml.F32, [7], f32)], alignment=64)
    with GgufFile(path) as f:
        assert f.alignment == 64 and f.data_start % 64 == 0
        assert f.kv["a.u32"] == 5 and f.kv["a.str"] == "héllo" and f.kv["a.bool"] is True
        assert f.kv["a.f"] == 0.5 and f.kv["a.arr"] == ["x", "yz"]
        assert np.array_equal(f.tensor_bytes("q4"), q4)
        assert np.array_equal(f.tensor_bytes("q6"), q6)
        assert np.array_equal(f.tensor_f32("f"), f32)
        for t in f.tensor_infos:
            assert t["data_offset"] % 64 == 0


def test_load_llama_round_trip(tmp_path):
    c = LlamaConfig(hidden=256, layer_count=2, head_count=2, kv_head_count=1, ffn=512, vocab=40,
                    rope_dimension=128, context=16)
    w = synthetic_llama(np.random.default_rng(4), c)
    path = str(tmp_path / "llama.gguf")
    save_llama(path, w)
    with GgufFile(path) as f:
        g = load_llama(f, context=16)
        # the epsilon is stored as F32, as GGUF files hold it
        assert g.config.norm_epsilon == float(np.float32(c.norm_epsilon))
        g.config.norm_epsilon = c.norm_epsilon
        assert g.config == c
        assert np.array_equal(g.token_embd[1], w.token_embd[1])
        assert np.array_equal(g.output[1], w.output[1]) and g.output[0] == w.output[0]
        assert np.array_equal(g.rope_factors, w.rope_factors)
        for a, b in zip(g.layers, w.layers):
            for name in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                         "ffn_down"):
                assert getattr(a, name)[0] == getattr(b, name)[0]
                assert np.array_equal(getattr(a, name)[1], getattr(b, name)[1])
            assert np.array_equal(a.attn_norm, b.attn_norm)
