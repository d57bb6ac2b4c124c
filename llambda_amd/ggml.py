"""GGML type tags and block geometry as llambda reads them.

llambda.lisp:24-31 (type tags), 2126-2155 (ggml-type-block-size,
ggml-type-size, ggml-tensor-byte-size).
"""
from __future__ import annotations

F32 = 0
Q5_0 = 6
Q8_0 = 8
Q4_K = 12
Q6_K = 14

NAMES = {F32: "F32", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}

# (weights per block, bytes per block)
_GEOMETRY = {
    F32: (1, 4),
    Q5_0: (32, 22),    # fp16 d, u32 high bits, 16 B nibbles
    Q8_0: (32, 34),    # fp16 d, 32 x int8
    Q4_K: (256, 144),  # fp16 d, fp16 dmin, 12 B scales/mins, 128 B nibbles
    Q6_K: (256, 210),  # 128 B ql, 64 B qh, 16 x int8 scales, fp16 d
}


def block_elements(type_tag: int) -> int:
    try:
        return _GEOMETRY[type_tag][0]
    except KeyError:
        raise ValueError(f"Unsupported GGML tensor type tag {type_tag}.") from None


def block_bytes(type_tag: int) -> int:
    try:
        return _GEOMETRY[type_tag][1]
    except KeyError:
        raise ValueError(f"Unsupported GGML tensor type tag {type_tag}.") from None


def tensor_byte_size(type_tag: int, element_count: int) -> int:
    """ggml-tensor-byte-size: errors unless the count is a block multiple."""
    be = block_elements(type_tag)
    if element_count % be:
        raise ValueError(
            f"Tensor element count {element_count} is not a multiple of block size {be} "
            f"for type {NAMES.get(type_tag, type_tag)}.")
    return element_count // be * block_bytes(type_tag)


def row_bytes(type_tag: int, columns: int) -> int:
    return tensor_byte_size(type_tag, columns)
