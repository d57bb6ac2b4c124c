"""The real :hip descriptor through the reference's store protocol, on the
GPU: try-enable -> exporter -> content-addressed cache file -> session_create
-> gguf-model-matrix-vector-multiply-into, and a HIP error raised by the C
ABI itself falling back to the CPU kernel (llambda.lisp:3160-3208,
3039-3094, 4660-4741); then the routed-MoE layer hook the same way.  The
CPU kernel at the bottom of every chain is the oracle."""
import os
import warnings

import numpy as np
import pytest

import oracle
from llambda_amd import accelerator as acc
from llambda_amd import ggml, native, projection, synthetic
from llambda_amd.hip_backend import PACKED_MAGIC, make_hip_session_packed, register_hip_backend
from llambda_amd.moe import (NEMOTRON_H, QWEN3NEXT, HipMoeSession, MoeLayerInputError,
                             moe_layer_from_model, synthetic_nemotron_h, synthetic_qwen3next)

from helpers import REL, abs_dot_bound, assert_within_bound
from test_moe_gpu import _shared_weights, output_bounds

pytestmark = pytest.mark.gpu


def oracle_cpu(dest, tensor, vector):
    dest[:] = oracle.gemv(tensor.type_tag, tensor.data, tensor.rows, tensor.columns, vector)
    return dest


@pytest.fixture
def hip_backend(hip):
    register_hip_backend()
    yield acc.find_accelerator_backend("hip")
    acc.unregister_accelerator_backend("hip")


def test_hip_descriptor_through_the_store(hip_backend, tmp_path):
    rng = np.random.default_rng(31)
    H, F = 1024, 768
    shapes = {"attn_q": (ggml.Q4_K, H, H), "attn_v": (ggml.Q6_K, 256, H),
              "ffn_down": (ggml.Q6_K, H, F)}
    tensors = [projection.TensorInfo(f"blk.0.{n}.weight", t, (cols, rows),
                                     synthetic.packed(t, rng, rows, cols))
               for n, (t, rows, cols) in shapes.items()]
    model = projection.ProjectionModel(tensors, layer_count=1, architecture="llama",
                                       cpu_matrix_vector=oracle_cpu)
    cache = str(tmp_path / "cache")
    roles = ("attention-query", "attention-value", "ffn-down")
    assert projection.try_enable_model_accelerator_projections(
        model, "hip", layer_indices=[0], projection_roles=roles, cache_directory=cache) is True
    for name, info in model.tensors.items():
        path, _, key = projection.model_accelerator_projection_cache_pathnames(
            model, "hip", name, cache)
        with open(path, "rb") as fh:
            assert fh.read(8) == PACKED_MAGIC
        assert f"-weights-packed-ggml-ggml-{info.type_tag}-" in key
        x = synthetic.activations(rng, 1, info.columns)[0]
        y = projection.matrix_vector_multiply(model, name, x)
        assert_within_bound(y, oracle.gemv(info.type_tag, info.data, info.rows, info.columns, x),
                            abs_dot_bound(info.type_tag, info.data, info.rows, info.columns, x),
                            name)
    # a second model over the same bytes reuses the cache files
    again = projection.ProjectionModel(tensors, layer_count=1, cpu_matrix_vector=oracle_cpu)
    _, _, reused = projection.ensure_model_accelerator_projection(
        again, "hip", "blk.0.attn_q.weight", cache_directory=cache)
    assert reused is True
    projection.clear_model_accelerator_projections(again)

    # a HIP error from the C ABI: the bound session now points at a session of
    # another column count, so llambda_hip_session_run refuses the input count;
    # the store warns, unregisters the binding and runs the CPU kernel
    name = "blk.0.ffn_down.weight"
    info = model.tensors[name]
    bound = projection.model_accelerator_session(model, "hip", name)
    other = make_hip_session_packed(synthetic.packed(ggml.Q4_K, rng, H, 256), ggml.Q4_K, H, 256)
    own, bound.pointer = bound.pointer, other.pointer
    try:
        x = synthetic.activations(rng, 1, F)[0]
        with pytest.warns(UserWarning, match="input element count"):
            y = projection.matrix_vector_multiply(model, name, x)
        assert np.array_equal(y, oracle.gemv(info.type_tag, info.data, info.rows, info.columns, x))
        assert projection.model_accelerator_projection(model, "hip", name) is None
        assert bound.pointer is None  # the binding's session was closed
    finally:
        other.pointer = None  # closed through the binding
        native.lib().llambda_hip_session_destroy(own)
    # the other projections stay bound and keep running on the device
    assert projection.model_accelerator_projection(model, "hip", "blk.0.attn_q.weight")
    projection.clear_model_accelerator_projections(model)


def _moe_model(layer, index=0):
    """The layer's tensors under their GGUF names (dims = columns, rows[, experts])."""
    H, E, F, Fs = layer.hidden, layer.expert_count, layer.expert_ffn, layer.shared_ffn
    T = projection.TensorInfo
    p = f"blk.{index}."
    t = [T(p + "ffn_gate_inp.weight", ggml.F32, (H, E), layer.router.view(np.uint8).reshape(-1)),
         T(p + "ffn_up_exps.weight", layer.up[0], (H, F, E), layer.up[1]),
         T(p + "ffn_down_exps.weight", layer.down[0], (F, H, E), layer.down[1])]
    if layer.gate is not None:
        t.append(T(p + "ffn_gate_exps.weight", layer.gate[0], (H, F, E), layer.gate[1]))
    if layer.router_bias is not None:
        t.append(T(p + "exp_probs_b.bias", ggml.F32, (E,), layer.router_bias.view(np.uint8)))
    if Fs:
        if layer.shared_gate_inp is not None:
            t.append(T(p + "ffn_gate_inp_shexp.weight", ggml.F32, (H,),
                       layer.shared_gate_inp.view(np.uint8)))
        if layer.shared_gate is not None:
            t.append(T(p + "ffn_gate_shexp.weight", layer.shared_gate[0], (H, Fs),
                       layer.shared_gate[1]))
        t.append(T(p + "ffn_up_shexp.weight", layer.shared_up[0], (H, Fs), layer.shared_up[1]))
        t.append(T(p + "ffn_down_shexp.weight", layer.shared_down[0], (Fs, H),
                   layer.shared_down[1]))
    return projection.ProjectionModel(t, layer_count=index + 1, cpu_matrix_vector=oracle_cpu)


@pytest.mark.parametrize("variant", [QWEN3NEXT, NEMOTRON_H])
def test_moe_hook_on_the_device(hip_backend, variant):
    rng = np.random.default_rng(40 + variant)
    if variant == QWEN3NEXT:
        layer = synthetic_qwen3next(rng, hidden=512, experts=32, top_k=4, ffn=256, shared_ffn=256)
        knobs = dict(expert_used_count=4)
    else:
        layer = synthetic_nemotron_h(rng, hidden=512, experts=32, top_k=4, ffn=256,
                                     shared_ffn=256, weights_scale=1.5, weights_norm=True)
        knobs = dict(expert_used_count=4, expert_weights_scale=1.5, expert_weights_norm=True)
    model = _moe_model(layer)

    def make(m, i):
        return HipMoeSession(moe_layer_from_model(m, i, variant, **knobs))

    assert projection.try_enable_model_accelerator_moe_layers(model, "hip", [0], make) is True
    # the router tensor has no 2-D binding: the MoE session does not shadow it
    assert projection.model_accelerator_projection(model, "hip", "blk.0.ffn_gate_inp.weight") is None
    xs = synthetic.activations(rng, 6, layer.hidden)
    ref = oracle.moe_forward(layer, xs)
    S = output_bounds(layer, xs, ref.top_indices, ref.top_weights, _shared_weights(layer, xs))
    cpu_runs = []
    for t in range(xs.shape[0]):
        dest = np.empty(layer.hidden, dtype=np.float32)

        def cpu_body(t=t, dest=dest):
            cpu_runs.append(t)
            dest[:] = ref.y[t]
            return dest

        projection.moe_layer_into(dest, model, 0, xs[t], cpu_body)
        assert np.all(np.abs(dest.astype(np.float64) - ref.y[t]) <= REL * S[t]), t
    assert cpu_runs == []
    # a HIP error from the C ABI (the input's element count is not H):
    # warned, the layer's session unregistered, the CPU body runs
    dest = np.empty(layer.hidden, dtype=np.float32)

    def cpu_body_first():
        dest[:] = ref.y[0]
        return dest

    longer = np.concatenate([xs[0], np.zeros(1, np.float32)])
    with pytest.warns(UserWarning, match="element counts"):
        projection.moe_layer_into(dest, model, 0, longer, cpu_body_first)
    assert np.array_equal(dest, ref.y[0])
    assert not model.accelerator_moe_layers


def test_moe_hook_input_error_keeps_the_layer_on_the_device(hip_backend):
    """A token the reference itself rejects (NaN input: no selectable router
    logit, so a zero top-k weight sum) raises the reference's error for that call
    alone: no warning, the layer stays bound, and the next token runs on the
    device, not on the CPU body (llambda.lisp:4660-4676 re-signals any
    condition its backend's error predicate does not select)."""
    rng = np.random.default_rng(45)
    layer = synthetic_qwen3next(rng, hidden=512, experts=32, top_k=4, ffn=256, shared_ffn=256)
    model = _moe_model(layer, index=3)

    def make(m, i):
        return HipMoeSession(moe_layer_from_model(m, i, QWEN3NEXT, expert_used_count=4))

    assert projection.try_enable_model_accelerator_moe_layers(model, "hip", [3], make) is True
    cpu_runs = []

    def cpu_body():
        cpu_runs.append(1)
        raise AssertionError("the CPU body must not run")

    dest = np.empty(layer.hidden, dtype=np.float32)
    bad = np.full(layer.hidden, np.nan, dtype=np.float32)
    with warnings.catch_warnings():
        warnings.simplefilter("error")  # a warning would mean the layer was disabled
        with pytest.raises(MoeLayerInputError,
                           match=r"Qwen3Next layer 3 router produced non-positive top-k"):
            projection.moe_layer_into(dest, model, 3, bad, cpu_body)
    assert [p.backend.name for p in model.accelerator_moe_layers[3]] == ["hip"]
    x = synthetic.activations(rng, 1, layer.hidden)
    ref = oracle.moe_forward(layer, x)
    S = output_bounds(layer, x, ref.top_indices, ref.top_weights, _shared_weights(layer, x))
    projection.moe_layer_into(dest, model, 3, x[0], cpu_body)
    assert cpu_runs == []
    assert np.all(np.abs(dest.astype(np.float64) - ref.y[0]) <= REL * S[0])
    projection.clear_model_accelerator_projections(model)


def test_moe_hook_runs_a_latent_layer(hip_backend):
    """A Nemotron-H layer with ffn_latent_down / ffn_latent_up runs through the
    hook on the device (llambda.lisp:5845-5864, 5883-5887, 5933-5938): the
    session is bound, the CPU body never runs, and each token agrees with the
    oracle."""
    from test_moe_latent_gpu import absolute_layer
    rng = np.random.default_rng(44)
    layer = synthetic_nemotron_h(rng, hidden=256, experts=16, top_k=2, ffn=64, shared_ffn=64,
                                 expert_type=ggml.Q8_0, down_type=ggml.Q8_0, latent_in=128,
                                 latent_out=96, latent_type=ggml.Q5_0, router_std=0.05)
    model = _moe_model(layer)
    Li, Lo = layer.latent_in, layer.latent_out
    model.tensors["blk.0.ffn_up_exps.weight"] = projection.TensorInfo(
        "blk.0.ffn_up_exps.weight", layer.up[0], (Li, 64, 16), layer.up[1])
    model.tensors["blk.0.ffn_down_exps.weight"] = projection.TensorInfo(
        "blk.0.ffn_down_exps.weight", layer.down[0], (64, Lo, 16), layer.down[1])
    for name, pair, dims in (("ffn_latent_down", layer.latent_down, (256, Li)),
                             ("ffn_latent_up", layer.latent_up, (Lo, 256))):
        model.tensors[f"blk.0.{name}.weight"] = projection.TensorInfo(
            f"blk.0.{name}.weight", pair[0], dims, pair[1])

    def make(m, i):
        return HipMoeSession(moe_layer_from_model(m, i, NEMOTRON_H, expert_used_count=2))

    assert projection.try_enable_model_accelerator_moe_layers(model, "hip", [0], make) is True
    bound = model.accelerator_moe_layers[0][0].session.layer
    assert (bound.latent_in, bound.latent_out) == (Li, Lo)
    xs = synthetic.activations(rng, 3, layer.hidden)
    ref = oracle.moe_forward(layer, xs)
    A = absolute_layer(layer, xs, ref.top_indices, ref.top_weights)

    def cpu_body():
        raise AssertionError("the CPU body must not run")

    for t in range(xs.shape[0]):
        dest = np.empty(layer.hidden, dtype=np.float32)
        projection.moe_layer_into(dest, model, 0, xs[t], cpu_body)
        assert np.all(np.abs(dest.astype(np.float64) - ref.y[t]) <= REL * A[t]), t
    projection.clear_model_accelerator_projections(model)
