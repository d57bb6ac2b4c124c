"""Write reference_kats.json: the known-answer blocks and expected values of
the reference's own tests for this path (tests.lisp), as data.

  dequantize-q4-k-m        tests.lisp:2386-2416
  dequantize-q6-k          tests.lisp:2418-2450
  load-gguf-tensor-quantized tests.lisp:2324-2367
  dot-product-with-q4-k-tensor-row tests.lisp:2257-2288
  dot-product-with-q6-k-tensor-row tests.lisp:2290-2322
  forward-primitives silu(2) tests.lisp:298-344
  forward-primitives rms-norm, apply-rope tests.lisp:305-344
  softmax of (2 1 0)        tests.lisp:1359-1361
  sampling-primitives       tests.lisp:1258-1375

The reference cannot run here (no Common Lisp implementation), so the blocks
are rebuilt from the byte assignments those tests make and the expected
values are the literals they assert.
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def q4k_block():
    b = bytearray(144)
    b[0], b[1], b[2], b[3] = 0x00, 0x3C, 0x00, 0x3C      # d = dmin = 1.0
    for i in range(4):
        b[4 + i] = 2          # scales 0..3
        b[8 + i] = 1          # mins 0..3
        b[12 + i] = 0x12      # low nibble: scales 4..7 = 2, high nibble: mins 4..7 = 1
    for i in range(128):
        b[16 + i] = 0x76      # low nibble 6, high nibble 7
    return bytes(b)


def q6k_block():
    b = bytearray(210)
    for i in range(32):
        b[i] = 0x31
        b[32 + i] = 0x42
        b[64 + i] = 0x31
        b[96 + i] = 0x42
    for i in range(64):
        b[128 + i] = 0xAA
    for i in range(16):
        b[192 + i] = 2
    b[208], b[209] = 0x00, 0x3C                            # d = 1.0
    return bytes(b)


def main():
    kats = {
        "source": "tests.lisp (llambda reference test suite)",
        "q4_k_dequantize": {
            "cite": "tests.lisp:2386-2416, 2324-2367",
            "block_hex": q4k_block().hex(),
            # (start, end, value) ranges the test asserts
            "expect_ranges": [[0, 32, 11.0], [32, 64, 13.0], [192, 224, 11.0], [224, 256, 13.0]],
            "expect_points": [[0, 11.0], [32, 13.0]],
        },
        "q6_k_dequantize": {
            "cite": "tests.lisp:2418-2450, 2324-2367",
            "block_hex": q6k_block().hex(),
            "expect_ranges": [[0, 32, 2.0], [32, 64, 4.0], [64, 96, 6.0], [96, 128, 8.0],
                              [128, 160, 2.0], [224, 256, 8.0]],
            "expect_points": [[0, 2.0], [96, 8.0]],
        },
        "q4_k_dot": {
            "cite": "tests.lisp:2257-2288",
            "block_hex": q4k_block().hex(),
            "activation": "((i mod 11) - 5) / 3",
            "tolerance": 1e-4,
        },
        "q6_k_dot": {
            "cite": "tests.lisp:2290-2322",
            "block_hex": q6k_block().hex(),
            "activation": "((i mod 13) - 6) / 4",
            "tolerance": 1e-4,
        },
        "silu": {"cite": "tests.lisp:298-344", "x": 2.0, "expect": 1.7615942, "tolerance": 1e-5},
        "rms_norm": {"cite": "tests.lisp:305-311, 323-328", "x": [3.0, 4.0], "weight": [1.0, 2.0],
                     "epsilon": 0.0, "expect": [0.84852815, 2.2627418], "tolerance": 1e-5},
        "rope": {"cite": "tests.lisp:338-344", "x": [1.0, 0.0, 5.0, 6.0], "position": 1,
                 "rope_dimension": 2, "theta_base": 10000.0,
                 "expect": ["cos 1", "sin 1", 5.0, 6.0], "tolerance": 1e-5},
        "softmax": {"cite": "tests.lisp:1359-1361", "x": [2.0, 1.0, 0.0],
                    "expect": "sums to 1 within 1e-5, strictly decreasing", "tolerance": 1e-5},
        "sampling": {
            "cite": "tests.lisp:1258-1375",
            "tolerance": 1e-5,
            "masked": -1.0e30,
            "temperature": {"x": [2.0, 1.0, -2.0], "t": 0.5, "expect": [4.0, 2.0, -4.0]},
            "repetition_penalty": {"x": [2.0, -3.0, 4.0, 1.0], "history": [2, 1, 2, 1],
                                   "penalty": 1.25, "expect": [2.0, -3.75, 3.2, 1.0]},
            "top_k": {"x": [0.5, 3.0, 2.0, 1.0, 2.0], "k": 2,
                      "expect": [-1.0e30, 3.0, 2.0, -1.0e30, 2.0]},
            "top_p": {"x": [3.0, 2.0, 1.0, -1.0e30], "p": 0.60, "t": 1.0,
                      "expect": [3.0, -1.0e30, -1.0e30, -1.0e30]},
            "probabilities": {"p": [0.7, 0.2, 0.1],
                              "draws": [[0.1, 0], [0.75, 1], [0.95, 2]]},
            # (logits, keyword arguments, random value, expected token)
            "tokens": [
                [[2.0, 1.95, 0.0], {"top_k": 0, "top_p": 1.0, "temperature": 1.0}, 0.45, 0],
                [[2.0, 1.95, 0.0], {"history": [0], "repetition_penalty": 1.15, "top_k": 0,
                                    "top_p": 1.0, "temperature": 1.0}, 0.45, 1],
                [[3.0, 2.9, 0.1], {"top_k": 2, "top_p": 1.0, "temperature": 1.0}, 0.9, 1],
                [[3.0, 2.0, 1.0], {"top_k": 0, "top_p": 0.60, "temperature": 1.0}, 0.95, 0],
                [[3.0, 1.0, 0.0], {"top_p": 1.0, "temperature": 1.0}, 0.1, 0],
                [[3.0, 1.0, 0.0], {"top_p": 1.0, "temperature": 1.0}, 0.9, 1],
            ],
            # pairs that must draw the same token: top-k nil = 40, top-p nil = 0.95
            "same": [
                [[float(v) for v in range(50, 0, -1)], {"top_k": None, "top_p": 1.0},
                 {"top_k": 40, "top_p": 1.0}, 0.9],
                [[3.0, 2.0, 1.0], {"top_k": 0, "top_p": None}, {"top_k": 0, "top_p": 0.95}, 0.9],
            ],
        },
    }
    with open(os.path.join(HERE, "reference_kats.json"), "w") as fh:
        json.dump(kats, fh, indent=1)
        fh.write("\n")


if __name__ == "__main__":
    main()
