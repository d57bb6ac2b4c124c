"""GGUF v3 files: the bounded parser over open/mmap (llambda_hip_gguf_*), a
writer, and the Llama loader on top of them.

``GgufFile`` mirrors the reference's read-gguf-header,
read-gguf-kv-pairs and read-gguf-tensor-infos (llambda.lisp:2047-2238):
metadata as (key, value) pairs in file order (arrays as lists, booleans as
True/False), tensor infos as dicts with the reference's plist keys
(name, dimension_count, dimensions, type_tag, type_name, offset,
element_count, byte_size, data_offset, data_end), and tensor bytes as
zero-copy numpy views of the mapping.  ``load_llama`` follows
load-llama-model (llambda.lisp:6269-6292).
"""
from __future__ import annotations

import ctypes
import struct
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import ggml, native

TYPE_NAMES = {0: "f32", 1: "f16", 6: "q5-0", 8: "q8-0", 30: "bf16", 12: "q4-k", 13: "q5-k",
              14: "q6-k"}

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)


class GgufError(RuntimeError):
    pass


def _check(status: int) -> None:
    if status != 0:
        raise GgufError(native.last_error())


class GgufFile:
    """A mapped GGUF file (read-only); close() unmaps it, invalidating the
    tensor views."""

    def __init__(self, path: str):
        L = native.lib()
        h = ctypes.c_void_p()
        _check(L.llambda_hip_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h
        v, tc, kc, al, ds = (ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(),
                             ctypes.c_uint64(), ctypes.c_uint64())
        _check(L.llambda_hip_gguf_header(h, ctypes.byref(v), ctypes.byref(tc), ctypes.byref(kc),
                                         ctypes.byref(al), ctypes.byref(ds)))
        self.version, self.tensor_count, self.kv_count = v.value, tc.value, kc.value
        self.alignment, self.data_start = al.value, ds.value
        size = ctypes.c_size_t()
        self._base = L.llambda_hip_gguf_mapping(h, ctypes.byref(size))
        self.size = size.value
        self.kv_pairs = [self._kv(i) for i in range(self.kv_count)]
        self.tensor_infos = [self._tensor(i) for i in range(self.tensor_count)]

    def close(self) -> None:
        if getattr(self, "_h", None):
            native.lib().llambda_hip_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _bytes(ptr: int, n: int) -> bytes:
        return ctypes.string_at(ptr, n) if n else b""

    def _value(self, v: native.GgufValue, index: int):
        t = v.type
        if t == STRING:
            return self._bytes(v.string, v.string_length).decode("utf-8", errors="replace")
        if t == BOOL:
            return bool(v.u)
        if t in (F32, F64):
            return float(v.f)
        if t in (U8, U16, U32, U64):
            return int(v.u)
        if t in (I8, I16, I32, I64):
            return int(v.i)
        if t == ARRAY:
            out = []
            e = native.GgufValue()
            for j in range(v.count):
                _check(native.lib().llambda_hip_gguf_kv_element(self._h, index, j,
                                                                ctypes.byref(e)))
                out.append(self._value(e, index))
            return out
        raise GgufError(f"Unsupported GGUF metadata value type: {t}.")

    def _kv(self, i: int):
        v = native.GgufValue()
        _check(native.lib().llambda_hip_gguf_kv(self._h, i, ctypes.byref(v)))
        key = self._bytes(v.key, v.key_length).decode("utf-8", errors="replace")
        return key, self._value(v, i)

    def _tensor(self, i: int) -> Dict:
        t = native.GgufTensor()
        _check(native.lib().llambda_hip_gguf_tensor_info(self._h, i, ctypes.byref(t)))
        dims = [int(t.dimensions[d]) for d in range(t.dimension_count)]
        byte_size = int(t.byte_size) if t.supported else None
        return {"name": self._bytes(t.name, t.name_length).decode("utf-8", errors="replace"),
                "dimension_count": int(t.dimension_count), "dimensions": dims,
                "type_tag": int(t.type),
                "type_name": TYPE_NAMES.get(int(t.type), f"type-{int(t.type)}"),
                "offset": int(t.offset), "element_count": int(t.element_count),
                "byte_size": byte_size, "data_offset": int(t.data_offset),
                "data_end": None if byte_size is None else int(t.data_offset) + byte_size}

    @property
    def kv(self) -> Dict:
        return dict(self.kv_pairs)

    def tensor_info(self, name: str) -> Optional[Dict]:
        for t in self.tensor_infos:
            if t["name"] == name:
                return t
        return None

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's packed bytes: a read-only view of the mapping."""
        t = self.tensor_info(name)
        if t is None:
            raise GgufError(f"Tensor {name!r} is not in the file.")
        if t["byte_size"] is None:
            raise GgufError(f"Tensor {name!r} has an unsupported type {t['type_tag']}.")
        buf = (ctypes.c_uint8 * t["byte_size"]).from_address(self._base + t["data_offset"])
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def tensor_f32(self, name: str) -> np.ndarray:
        t = self.tensor_info(name)
        if t is None or t["type_tag"] != ggml.F32:
            raise GgufError(f"Tensor {name!r} is not an F32 tensor.")
        return self.tensor_bytes(name).view(np.float32)


def read_gguf_header(path: str) -> Dict:
    """read-gguf-header (llambda.lisp:2047-2059) alone: the 24-byte header,
    without parsing the metadata or tensor infos."""
    with open(path, "rb") as fh:
        data = fh.read(24)
        fh.seek(0, 2)
        size = fh.tell()

    def need(off, n, what):
        if not (off <= size and n <= size - off):
            raise GgufError(f"{what} byte range [{off}, {off + n}) exceeds mapped file length "
                            f"{size}.")

    need(0, 4, "GGUF magic")
    if data[:4] != b"GGUF":
        raise GgufError(f"Invalid GGUF magic: {data[:4].decode('latin-1')!r}.")
    need(4, 4, "GGUF version")
    need(8, 8, "GGUF tensor count")
    need(16, 8, "GGUF metadata count")
    version, tensors, kvs = struct.unpack("<IQQ", data[4:24])
    return {"magic": "GGUF", "version": version, "tensor_count": tensors,
            "metadata_kv_count": kvs, "header_size": 24}


# ------------------------------------------------------------------ writer
def _pack_value(t: int, v) -> bytes:
    if t == STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_pack_value(et, x) for x in items)
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}[t]
    return struct.pack(fmt, int(v) if t not in (F32, F64) else float(v))


def _infer_type(v):
    if isinstance(v, bool):
        return BOOL, v
    if isinstance(v, int):
        return (U32, v) if 0 <= v < 2 ** 32 else (I64, v)
    if isinstance(v, float):
        return F32, v
    if isinstance(v, str):
        return STRING, v
    if isinstance(v, (list, tuple)):
        et = _infer_type(v[0])[0] if v else U32
        return ARRAY, (et, list(v))
    raise TypeError(f"cannot store {type(v).__name__} in GGUF metadata")


def write_gguf(path: str, kv: Sequence[Tuple], tensors: Sequence[Tuple], *,
               alignment: int = 32, version: int = 3) -> None:
    """Write a GGUF file.  kv: (key, value) or (key, gguf_type, value);
    tensors: (name, ggml_type, dimensions (GGUF order), bytes)."""
    meta = list(kv)
    if alignment != 32 and not any(m[0] == "general.alignment" for m in meta):
        meta.insert(0, ("general.alignment", U32, alignment))
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(meta))
    for m in meta:
        key, (t, v) = m[0], (m[1:] if len(m) == 3 else _infer_type(m[1]))
        out += _pack_value(STRING, key) + struct.pack("<I", t) + _pack_value(t, v)
    offset = 0
    placed = []
    for name, t, dims, data in tensors:
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        out += _pack_value(STRING, name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", t, offset)
        placed.append((offset, data))
        offset += (data.size + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    start = len(out)
    with open(path, "wb") as fh:
        fh.write(out)
        for off, data in placed:
            fh.seek(start + off)
            fh.write(data.tobytes())
        fh.truncate(start + offset)


# ------------------------------------------------------------------- llama
def save_llama(path: str, weights, *, alignment: int = 32) -> None:
    """A GGUF file of a LlamaWeights model (architecture llama)."""
    from .llama import LlamaWeights  # noqa: F401  (type of `weights`)
    c = weights.config
    kv = [("general.architecture", "llama"),
          ("llama.embedding_length", U32, c.hidden),
          ("llama.block_count", U32, c.layer_count),
          ("llama.attention.head_count", U32, c.head_count),
          ("llama.attention.head_count_kv", U32, c.kv_head_count),
          ("llama.feed_forward_length", U32, c.ffn),
          ("llama.attention.layer_norm_rms_epsilon", F32, c.norm_epsilon),
          ("llama.rope.freq_base", F32, c.rope_base),
          ("llama.rope.dimension_count", U32, c.rope_dimension)]
    H, D = c.hidden, c.head_dim
    tensors = [("token_embd.weight", weights.token_embd[0], [H, c.vocab], weights.token_embd[1])]
    for i, L in enumerate(weights.layers):
        p = f"blk.{i}."
        tensors += [
            (p + "attn_norm.weight", ggml.F32, [H], L.attn_norm),
            (p + "attn_q.weight", L.attn_q[0], [H, c.head_count * D], L.attn_q[1]),
            (p + "attn_k.weight", L.attn_k[0], [H, c.kv_head_count * D], L.attn_k[1]),
            (p + "attn_v.weight", L.attn_v[0], [H, c.kv_head_count * D], L.attn_v[1]),
            (p + "attn_output.weight", L.attn_output[0], [c.head_count * D, H],
             L.attn_output[1]),
            (p + "ffn_norm.weight", ggml.F32, [H], L.ffn_norm),
            (p + "ffn_gate.weight", L.ffn_gate[0], [H, c.ffn], L.ffn_gate[1]),
            (p + "ffn_up.weight", L.ffn_up[0], [H, c.ffn], L.ffn_up[1]),
            (p + "ffn_down.weight", L.ffn_down[0], [c.ffn, H], L.ffn_down[1])]
    tensors.append(("output_norm.weight", ggml.F32, [H], weights.output_norm))
    tensors.append(("output.weight", weights.output[0], [H, c.vocab], weights.output[1]))
    if weights.rope_factors is not None:
        tensors.append(("rope_freqs.weight", ggml.F32, [len(weights.rope_factors)],
                        weights.rope_factors))
    write_gguf(path, kv, tensors, alignment=alignment)


def load_llama(f: GgufFile, context: int = 4352):
    """LlamaWeights of an architecture-llama file (load-llama-model,
    llambda.lisp:6269-6292); the packed tensors are views of the mapping, so
    a HipLlamaSession uploads each of them once, straight from the file."""
    from .llama import LlamaConfig, LlamaLayerWeights, LlamaWeights
    kv = f.kv
    arch = kv.get("general.architecture")
    if arch != "llama":
        raise GgufError(f'LOAD-LLAMA-MODEL only supports general.architecture = "llama", got {arch!r}.')

    def req(key):
        if key not in kv:
            raise GgufError(f"GGUF metadata key {key!r} is missing.")
        return kv[key]

    c = LlamaConfig(hidden=req("llama.embedding_length"), layer_count=req("llama.block_count"),
                    head_count=req("llama.attention.head_count"),
                    kv_head_count=req("llama.attention.head_count_kv"),
                    ffn=req("llama.feed_forward_length"), vocab=0,
                    rope_dimension=req("llama.rope.dimension_count"),
                    norm_epsilon=float(req("llama.attention.layer_norm_rms_epsilon")),
                    rope_base=float(req("llama.rope.freq_base")), context=context)
    emb = f.tensor_info("token_embd.weight")
    if emb is None:
        raise GgufError("Tensor 'token_embd.weight' is not in the file.")
    c.vocab = emb["dimensions"][1]
    out_name = "output.weight" if f.tensor_info("output.weight") else "token_embd.weight"

    def q(name):
        return (f.tensor_info(name)["type_tag"] if f.tensor_info(name) else None,
                f.tensor_bytes(name))

    layers = []
    for i in range(c.layer_count):
        p = f"blk.{i}."
        layers.append(LlamaLayerWeights(
            attn_norm=f.tensor_f32(p + "attn_norm.weight"), attn_q=q(p + "attn_q.weight"),
            attn_k=q(p + "attn_k.weight"), attn_v=q(p + "attn_v.weight"),
            attn_output=q(p + "attn_output.weight"), ffn_norm=f.tensor_f32(p + "ffn_norm.weight"),
            ffn_gate=q(p + "ffn_gate.weight"), ffn_up=q(p + "ffn_up.weight"),
            ffn_down=q(p + "ffn_down.weight")))
    rope = f.tensor_f32("rope_freqs.weight") if f.tensor_info("rope_freqs.weight") else None
    return LlamaWeights(config=c, token_embd=q("token_embd.weight"), output=q(out_name),
                        output_norm=f.tensor_f32("output_norm.weight"), rope_factors=rope,
                        layers=layers)
