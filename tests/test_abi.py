"""The C ABI library loads and exports every symbol include/llambda_hip.h
declares; host-only entry points behave without a GPU (no compute calls)."""
import ctypes
import hashlib
import os
import re

import numpy as np
import pytest

from llambda_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llambda_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llambda_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_lists_the_bound_functions():
    assert declared_functions() == sorted(native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(native.library_path())
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_versions_and_probe():
    L = native.lib()
    assert L.llambda_hip_bridge_version().startswith(b"llambda-hip")
    assert b"HIP runtime" in L.llambda_hip_runtime_version()
    assert L.llambda_hip_probe() in (0, 1)


@pytest.mark.parametrize("n", [0, 1, 55, 56, 63, 64, 65, 1000, 4096 + 17])
def test_sha256_matches_hashlib(n):
    data = bytes((i * 7 + 3) & 255 for i in range(n))
    buf = np.frombuffer(data, dtype=np.uint8) if n else np.zeros(1, dtype=np.uint8)
    out = ctypes.create_string_buffer(65)
    assert native.lib().llambda_hip_sha256(buf.ctypes.data, n, out, 65) == 0
    assert out.value.decode() == hashlib.sha256(data).hexdigest()


def test_sha256_rejects_short_output():
    out = ctypes.create_string_buffer(64)
    assert native.lib().llambda_hip_sha256(None, 0, out, 64) == -1
    assert "65" in native.last_error()


def test_null_arguments_fail_with_last_error():
    L = native.lib()
    assert L.llambda_hip_session_run(None, None, 0, None, 0) == -1
    assert "null session" in native.last_error()
    assert L.llambda_hip_session_input_element_count(None) == 0
    assert L.llambda_hip_session_output_element_count(None) == 0
    assert L.llambda_hip_moe_session_hidden_size(None) == 0
    L.llambda_hip_session_destroy(None)
    L.llambda_hip_moe_session_destroy(None)
    assert L.llambda_hip_session_create(None, None, None, None) == -1
    assert "null result" in native.last_error()
    # the error is cleared by the next successful call
    out = ctypes.create_string_buffer(65)
    assert L.llambda_hip_sha256(None, 0, out, 65) == 0
    assert native.last_error() == ""


def test_session_create_rejects_bad_files(tmp_path):
    L = native.lib()
    handle = ctypes.c_void_p()
    p = tmp_path / "junk.bin"
    p.write_bytes(b"not a projection at all, definitely longer than forty bytes")
    assert L.llambda_hip_session_create(str(p).encode(), None, None, ctypes.byref(handle)) == -1
    assert "bad magic" in native.last_error()
    assert handle.value is None
    assert L.llambda_hip_session_create(str(tmp_path / "absent").encode(), None, None,
                                        ctypes.byref(handle)) == -1
    assert "cannot open" in native.last_error()


def test_packed_create_validates_geometry():
    L = native.lib()
    handle = ctypes.c_void_p()
    buf = np.zeros(144 * 3, dtype=np.uint8)
    # 2688 columns is not a Q4_K block multiple (ggml-tensor-byte-size)
    assert L.llambda_hip_session_create_packed(buf.ctypes.data, buf.size, 12, 1, 2688,
                                               ctypes.byref(handle)) == -1
    assert "not a multiple of block size 256" in native.last_error()
    assert L.llambda_hip_session_create_packed(buf.ctypes.data, buf.size, 12, 2, 256,
                                               ctypes.byref(handle)) == -1
    assert "do not hold" in native.last_error()
    assert L.llambda_hip_session_create_packed(buf.ctypes.data, buf.size, 99, 3, 256,
                                               ctypes.byref(handle)) == -1
    assert "unsupported GGML tensor type" in native.last_error()


def test_moe_session_checks_latent_projections():
    """nemotron-h-moe-ffn-into's optional ffn_latent_down / ffn_latent_up
    (llambda.lisp:5845-5864, 5883-5887, 5933-5938): the layer reads them with
    their widths (rows of ffn_latent_down, columns of ffn_latent_up), and
    session creation refuses inconsistent descriptions before any device
    work."""
    import dataclasses

    from llambda_amd import ggml, projection, synthetic
    from llambda_amd.hip_backend import HipBackendError
    from llambda_amd.moe import NEMOTRON_H, HipMoeSession, moe_layer_from_model

    rng = np.random.default_rng(3)
    H, E, F, Li, Lo = 256, 8, 64, 128, 96
    t = projection.TensorInfo
    names = {
        "ffn_gate_inp.weight": (ggml.F32, (H, E), synthetic.f32(rng, E, H)),
        "exp_probs_b.bias": (ggml.F32, (E,), synthetic.f32(rng, 1, E)),
        "ffn_up_exps.weight": (ggml.Q8_0, (Li, F, E), synthetic.q8_0(rng, E * F, Li)),
        "ffn_down_exps.weight": (ggml.Q8_0, (F, Lo, E), synthetic.q8_0(rng, E * Lo, F)),
        "ffn_latent_down.weight": (ggml.Q8_0, (H, Li), synthetic.q8_0(rng, Li, H)),
        "ffn_latent_up.weight": (ggml.Q8_0, (Lo, H), synthetic.q8_0(rng, H, Lo)),
    }
    model = projection.ProjectionModel([t(f"blk.0.{n}", ty, dims, data)
                                        for n, (ty, dims, data) in names.items()], layer_count=1)
    layer = moe_layer_from_model(model, 0, NEMOTRON_H, expert_used_count=2)
    assert (layer.latent_in, layer.latent_out) == (Li, Lo)
    assert (layer.hidden, layer.expert_count, layer.top_k, layer.expert_ffn) == (H, E, 2, F)
    # Li must be a multiple of 32 (the experts' up rows are Li wide)
    odd = dataclasses.replace(layer, latent_down=(ggml.F32, synthetic.f32(rng, 100, H)))
    assert odd.latent_in == 100
    with pytest.raises(HipBackendError, match="ffn_latent_down needs its row count"):
        HipMoeSession(odd)
    # a Qwen3Next layer has no latent projections
    qwen = dataclasses.replace(layer, variant=0)
    with pytest.raises(HipBackendError, match="belong to Nemotron-H"):
        HipMoeSession(qwen)