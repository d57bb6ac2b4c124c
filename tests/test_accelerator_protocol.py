"""The accelerator-backend protocol and the projection store, with fake
backends (the reference's own strategy: tests.lisp:131-176, 543-803).
CPU only."""
import threading
import time
import warnings

import numpy as np
import pytest

from llambda_amd import accelerator as acc
from llambda_amd import ggml, projection, synthetic
from llambda_amd.hip_backend import (HIP_BACKEND, PACKED_MAGIC, export_model_hip_projection,
                                     register_hip_backend)


class FakeAcceleratorError(RuntimeError):
    pass


def make_fake_backend(name, priority, run, close, available=lambda: True, make_session=None):
    def signal(fmt, *args):
        raise FakeAcceleratorError(fmt % args if args else fmt)

    return acc.AcceleratorBackend(
        name=name, display_name=name.upper(), priority=priority, initialization_priority=priority,
        load_function=lambda: True, available_p_function=available,
        runtime_version_function=lambda: "test-runtime",
        bridge_version_function=lambda: "test-bridge",
        make_session_function=make_session or (lambda path, **kw: name),
        close_session_function=close, run_session_function=run,
        session_input_element_count_function=lambda s: 1,
        session_output_element_count_function=lambda s: 1,
        error_p_function=lambda c: isinstance(c, FakeAcceleratorError),
        signal_error_function=signal,
        default_cache_directory_function=lambda: "/tmp",
        export_projection_function=lambda model, name, path, **kw: None,
        weight_format="float32",
        foreign_data_sha256_function=lambda ptr, n: "fake-foreign-sha256",
        byte_vector_sha256_function=lambda octets: "fake-byte-vector-sha256")


def one_weight_model():
    """A 1x1 F32 tensor holding 3.0; the CPU kernel gives 3 * x."""
    data = np.array([3.0], dtype=np.float32).view(np.uint8)
    info = projection.TensorInfo("test.weight", ggml.F32, (1, 1), data)

    def cpu(dest, tensor, vector):
        dest[0] = np.float32(tensor.data.view(np.float32)[0] * vector[0])
        return dest

    return projection.ProjectionModel([info], cpu_matrix_vector=cpu)


def test_protocol_priority_fallback_and_retirement(tmp_path):
    state = {"gpu_fails": False, "npu_fails": False, "available": True, "gpu_runs": 0,
             "npu_runs": 0}
    closed = []

    def run_gpu(dest, session, vector):
        state["gpu_runs"] += 1
        if state["gpu_fails"]:
            raise FakeAcceleratorError("simulated GPU failure")
        dest[0] = 10.0
        return dest

    def run_npu(dest, session, vector):
        state["npu_runs"] += 1
        if state["npu_fails"]:
            raise FakeAcceleratorError("simulated NPU failure")
        dest[0] = 20.0
        return dest

    gpu = make_fake_backend("fake-gpu", 1, run_gpu, closed.append,
                            available=lambda: state["available"])
    npu = make_fake_backend("fake-npu", 2, run_npu, closed.append)
    try:
        acc.register_accelerator_backend(gpu)
        acc.register_accelerator_backend(npu)
        with pytest.raises(ValueError):
            acc.register_accelerator_backend(gpu)
        names = [b.name for b in acc.ordered_accelerator_backends()]
        assert names.index("fake-gpu") < names.index("fake-npu")

        model = one_weight_model()
        x = np.array([2.0], dtype=np.float32)
        out = np.zeros(1, dtype=np.float32)
        projection.register_model_accelerator_projection(model, npu, "test.weight", "npu.onnx")
        projection.register_model_accelerator_projection(model, gpu, "test.weight", "gpu.onnx")
        ps = model.accelerator_projections["test.weight"]
        assert [p.backend for p in ps] == [gpu, npu]

        projection.matrix_vector_multiply_into(out, model, "test.weight", x)
        assert out[0] == 10.0 and state["gpu_runs"] == 1 and state["npu_runs"] == 0

        state["gpu_fails"] = True
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            projection.matrix_vector_multiply_into(out, model, "test.weight", x)
        assert out[0] == 20.0 and state["gpu_runs"] == 2 and state["npu_runs"] == 1
        assert "fake-gpu" in closed
        assert projection.model_accelerator_projection(model, gpu, "test.weight") is None

        state["npu_fails"] = True
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            projection.matrix_vector_multiply_into(out, model, "test.weight", x)
        assert out[0] == 6.0 and state["npu_runs"] == 2
        assert "fake-npu" in closed and not model.accelerator_projections

        _, path, reused = projection.ensure_model_accelerator_projection(
            model, gpu, "test.weight", cache_directory=str(tmp_path))
        assert path.endswith("projection.onnx") and reused is False
        assert projection.model_accelerator_projection(model, "fake-gpu", "test.weight")

        # retirement is deferred while inference contexts are active
        before = closed.count("fake-gpu")
        projection.acquire_model_inference_use(model)
        projection.acquire_model_inference_use(model)
        projection.unregister_model_accelerator_projection(model, "fake-gpu", "test.weight")
        assert closed.count("fake-gpu") == before
        projection.release_model_inference_use(model)
        assert closed.count("fake-gpu") == before
        projection.release_model_inference_use(model)
        assert closed.count("fake-gpu") == before + 1

        # setup fallback when the backend is unavailable
        state["available"] = False
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            assert projection.try_enable_model_accelerator_projections(
                model, gpu, ["test.weight"]) is None
        assert projection.clear_model_accelerator_projections(model) is model
    finally:
        acc.unregister_accelerator_backend("fake-gpu")
        acc.unregister_accelerator_backend("fake-npu")


def test_non_backend_errors_propagate():
    def run(dest, session, vector):
        raise KeyError("not a backend error")

    b = make_fake_backend("fake-x", 1, run, lambda s: None)
    acc.register_accelerator_backend(b, replace=True)
    try:
        model = one_weight_model()
        projection.register_model_accelerator_projection(model, b, "test.weight", "x")
        with pytest.raises(KeyError):
            projection.matrix_vector_multiply_into(np.zeros(1, np.float32), model, "test.weight",
                                                   np.ones(1, np.float32))
        assert projection.model_accelerator_projection(model, b, "test.weight") is not None
    finally:
        acc.unregister_accelerator_backend("fake-x")


def test_enable_rolls_back_on_failure():
    calls = []

    def make_session(path, **kw):
        calls.append(path)
        if len(calls) == 2:
            raise FakeAcceleratorError("second projection fails")
        return path

    closed = []
    b = make_fake_backend("fake-r", 1, lambda d, s, v: d, closed.append, make_session=make_session)
    acc.register_accelerator_backend(b, replace=True)
    try:
        data = np.array([1.0], dtype=np.float32).view(np.uint8)
        model = projection.ProjectionModel([projection.TensorInfo(n, ggml.F32, (1, 1), data)
                                            for n in ("a.weight", "b.weight")])
        with pytest.raises(FakeAcceleratorError):
            projection.enable_model_accelerator_projections(model, b, ["a.weight", "b.weight"],
                                                            cache_directory="/tmp/llambda-test")
        assert not model.accelerator_projections
        assert closed == [calls[0]]
    finally:
        acc.unregister_accelerator_backend("fake-r")


def test_session_runs_are_serialized():
    """One projection's runs never overlap (its run-mutex, tests.lisp:717-803)."""
    active = {"now": 0, "max": 0}
    lock = threading.Lock()

    def run(dest, session, vector):
        with lock:
            active["now"] += 1
            active["max"] = max(active["max"], active["now"])
        time.sleep(0.002)
        with lock:
            active["now"] -= 1
        dest[0] = 1.0
        return dest

    b = make_fake_backend("fake-s", 1, run, lambda s: None)
    acc.register_accelerator_backend(b, replace=True)
    try:
        model = one_weight_model()
        projection.register_model_accelerator_projection(model, b, "test.weight", "x")
        start = threading.Barrier(4)

        def worker():
            start.wait()
            for _ in range(20):
                projection.matrix_vector_multiply_into(np.zeros(1, np.float32), model,
                                                       "test.weight", np.ones(1, np.float32))

        threads = [threading.Thread(target=worker) for _ in range(4)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert active["max"] == 1
    finally:
        acc.unregister_accelerator_backend("fake-s")


def test_hip_descriptor_registers_before_gpu_and_npu():
    register_hip_backend()
    try:
        assert acc.find_accelerator_backend("hip") is HIP_BACKEND
        assert HIP_BACKEND.priority < 10 and HIP_BACKEND.weight_format == "packed-ggml"
        assert HIP_BACKEND.error_p_function(HIP_BACKEND_ERROR()) is True
        assert HIP_BACKEND.error_p_function(ValueError()) is False
    finally:
        acc.unregister_accelerator_backend("hip")


def HIP_BACKEND_ERROR():
    from llambda_amd.hip_backend import HipBackendError
    return HipBackendError("x")


def test_hip_exporter_writes_verbatim_blocks(tmp_path):
    rng = np.random.default_rng(0)
    data = synthetic.packed(ggml.Q6_K, rng, 5, 512)
    model = projection.ProjectionModel(
        [projection.TensorInfo("blk.0.ffn_down.weight", ggml.Q6_K, (512, 5), data)])
    path = str(tmp_path / "k" / "projection.onnx")
    export_model_hip_projection(model, "blk.0.ffn_down.weight", path)
    raw = open(path, "rb").read()
    assert raw[:8] == PACKED_MAGIC
    version, type_tag = np.frombuffer(raw[8:16], dtype="<u4")
    rows, cols, payload = np.frombuffer(raw[16:40], dtype="<u8")
    assert (version, type_tag, rows, cols, payload) == (1, ggml.Q6_K, 5, 512, data.size)
    assert raw[40:] == data.tobytes()


def test_cache_key_has_reference_fields():
    register_hip_backend()
    try:
        data = np.arange(16, dtype=np.float32).view(np.uint8)
        model = projection.ProjectionModel([projection.TensorInfo("t", ggml.F32, (4, 4), data)])
        path, root, key = projection.model_accelerator_projection_cache_pathnames(
            model, "hip", "t", "/tmp/cache")
        assert key.startswith("bridge-llambda-hip-0.1.0--gfx950--generator-none-ort-HIP-runtime")
        assert "-weights-packed-ggml-ggml-0-4-4-" in key
        import hashlib
        assert key.endswith(hashlib.sha256(data.tobytes()).hexdigest())
        assert path == f"/tmp/cache/{key}/projection.onnx" and root == "/tmp/cache"
    finally:
        acc.unregister_accelerator_backend("hip")


# ------------------------------------------------------------ MoE layer hook
# The routed-MoE layer sessions live in a table of their own, keyed by layer
# index; the reference's fallback rules apply to them as to projections
# (tests.lisp:543-715 for the projection case).

class FakeMoeSession:
    def __init__(self, name, hidden, experts, run):
        self.name, self.hidden_size, self.expert_count, self._run = name, hidden, experts, run
        self.closed = False

    def run_into(self, dest, vector):
        return self._run(self, dest, vector)

    def close(self):
        self.closed = True


def moe_model(hidden=4, experts=3, layers=2):
    """Router tensors blk.N.ffn_gate_inp.weight (F32 [experts][hidden])."""
    tensors = []
    for layer in range(layers):
        data = np.arange(experts * hidden, dtype=np.float32).view(np.uint8)
        tensors.append(projection.TensorInfo(f"blk.{layer}.ffn_gate_inp.weight", ggml.F32,
                                             (hidden, experts), data))

    def cpu(dest, tensor, vector):  # the router GEMV on the CPU
        w = tensor.data.view(np.float32).reshape(tensor.rows, tensor.columns)
        dest[:] = w @ vector
        return dest

    return projection.ProjectionModel(tensors, layer_count=layers, cpu_matrix_vector=cpu)


def test_moe_hook_priority_fallback_and_its_own_table():
    closed = []
    state = {"gpu_fails": False, "npu_fails": False}

    def runner(value, key):
        def run(session, dest, vector):
            if state[key]:
                raise FakeAcceleratorError(f"simulated {session.name} failure")
            dest[:] = value
            return dest
        return run

    gpu = make_fake_backend("fake-mgpu", 1, lambda d, s, v: d, lambda s: closed.append(s.name))
    npu = make_fake_backend("fake-mnpu", 2, lambda d, s, v: d, lambda s: closed.append(s.name))
    acc.register_accelerator_backend(gpu)
    acc.register_accelerator_backend(npu)
    try:
        model = moe_model()
        x = np.ones(4, dtype=np.float32)
        out = np.zeros(4, dtype=np.float32)
        cpu_calls = []

        def cpu_body():
            cpu_calls.append(1)
            out[:] = -1.0
            return out

        # no session bound: the CPU body
        projection.moe_layer_into(out, model, 0, x, cpu_body)
        assert out[0] == -1.0 and len(cpu_calls) == 1
        projection.register_model_accelerator_moe_layer(
            model, npu, 0, FakeMoeSession("npu0", 4, 3, runner(20.0, "npu_fails")))
        projection.register_model_accelerator_moe_layer(
            model, gpu, 0, FakeMoeSession("gpu0", 4, 3, runner(10.0, "gpu_fails")))
        assert [p.backend for p in model.accelerator_moe_layers[0]] == [gpu, npu]
        # the router keeps its own 2-D path: the MoE table is never consulted
        # for the tensor name, so its GEMV runs on the CPU kernel here
        assert not model.accelerator_projections
        logits = projection.matrix_vector_multiply(model, "blk.0.ffn_gate_inp.weight", x)
        assert np.array_equal(logits, np.array([6.0, 22.0, 38.0], dtype=np.float32))
        projection.moe_layer_into(out, model, 0, x, cpu_body)
        assert out[0] == 10.0 and len(cpu_calls) == 1
        # layer 1 has no session
        projection.moe_layer_into(out, model, 1, x, cpu_body)
        assert out[0] == -1.0 and len(cpu_calls) == 2
        # the first backend fails: warned, unregistered and closed; the next runs
        state["gpu_fails"] = True
        with pytest.warns(UserWarning, match="failed and was disabled"):
            projection.moe_layer_into(out, model, 0, x, cpu_body)
        assert out[0] == 20.0 and closed == ["gpu0"]
        assert projection.model_accelerator_moe_layer(model, gpu, 0) is None
        # all fail: the CPU body
        state["npu_fails"] = True
        with pytest.warns(UserWarning):
            projection.moe_layer_into(out, model, 0, x, cpu_body)
        assert out[0] == -1.0 and closed == ["gpu0", "npu0"] and not model.accelerator_moe_layers
        # retirement is deferred while inference is active; clear covers the table
        state["gpu_fails"] = False
        s = FakeMoeSession("gpu1", 4, 3, runner(10.0, "gpu_fails"))
        projection.register_model_accelerator_moe_layer(model, gpu, 1, s)
        projection.acquire_model_inference_use(model)
        projection.clear_model_accelerator_projections(model)
        assert not model.accelerator_moe_layers and closed == ["gpu0", "npu0"]
        projection.release_model_inference_use(model)
        assert closed == ["gpu0", "npu0", "gpu1"]
    finally:
        acc.unregister_accelerator_backend("fake-mgpu")
        acc.unregister_accelerator_backend("fake-mnpu")


def test_moe_hook_reraises_a_reference_input_error_and_keeps_the_layer():
    """An error that is not the backend's condition (the reference's own error
    for a token, e.g. moe.MoeLayerInputError) is re-signalled by the runtime
    fallback: no warning, nothing unregistered or closed, no CPU body, and
    the next token runs on the same session (llambda.lisp:4660-4676)."""
    from llambda_amd.moe import MoeLayerInputError
    closed = []
    state = {"bad": True}

    def run(session, dest, vector):
        if state["bad"]:
            raise MoeLayerInputError("Qwen3Next layer 0 router produced non-positive top-k "
                                     "weight sum.")
        dest[:] = 5.0
        return dest

    b = make_fake_backend("fake-minput", 1, lambda d, s, v: d, lambda s: closed.append(s.name))
    acc.register_accelerator_backend(b, replace=True)
    try:
        model = moe_model()
        projection.register_model_accelerator_moe_layer(model, b, 0,
                                                        FakeMoeSession("m0", 4, 3, run))
        out = np.zeros(4, dtype=np.float32)
        x = np.ones(4, dtype=np.float32)

        def cpu_body():
            raise AssertionError("the CPU body must not run")

        with warnings.catch_warnings():
            warnings.simplefilter("error")
            with pytest.raises(MoeLayerInputError, match="non-positive top-k weight sum"):
                projection.moe_layer_into(out, model, 0, x, cpu_body)
        assert closed == [] and projection.model_accelerator_moe_layer(model, b, 0) is not None
        state["bad"] = False
        projection.moe_layer_into(out, model, 0, x, cpu_body)
        assert out[0] == 5.0
    finally:
        acc.unregister_accelerator_backend("fake-minput")


def test_moe_hook_registration_checks_the_router_shape():
    closed = []
    b = make_fake_backend("fake-mreg", 1, lambda d, s, v: d, lambda s: closed.append(s.name))
    acc.register_accelerator_backend(b, replace=True)
    try:
        model = moe_model(hidden=4, experts=3)
        ok = lambda s, d, v: d  # noqa: E731
        with pytest.raises(ValueError, match="hidden size 5"):
            projection.register_model_accelerator_moe_layer(model, b, 0,
                                                            FakeMoeSession("h", 5, 3, ok))
        with pytest.raises(ValueError, match="expert count 4"):
            projection.register_model_accelerator_moe_layer(model, b, 0,
                                                            FakeMoeSession("e", 4, 4, ok))
        with pytest.raises(ValueError, match="invalid"):
            projection.register_model_accelerator_moe_layer(model, b, 7,
                                                            FakeMoeSession("l", 4, 3, ok))
        assert closed == ["h", "e", "l"]  # a refused session is closed
        projection.register_model_accelerator_moe_layer(model, b, 0, FakeMoeSession("a", 4, 3, ok))
        with pytest.raises(ValueError, match="already has"):
            projection.register_model_accelerator_moe_layer(model, b, 0,
                                                            FakeMoeSession("b", 4, 3, ok))
        assert closed == ["h", "e", "l", "b"] and not model.accelerator_projections
    finally:
        acc.unregister_accelerator_backend("fake-mreg")


def test_moe_hook_enable_rolls_back_and_falls_back():
    closed = []
    b = make_fake_backend("fake-men", 1, lambda d, s, v: d, lambda s: closed.append(s.name))
    acc.register_accelerator_backend(b, replace=True)
    try:
        model = moe_model(layers=3)
        made = []

        def make(model, layer):
            made.append(layer)
            if layer == 2:
                raise FakeAcceleratorError("layer 2 cannot be uploaded")
            return FakeMoeSession(f"s{layer}", 4, 3, lambda s, d, v: d)

        with pytest.warns(UserWarning, match="setup failed"):
            assert projection.try_enable_model_accelerator_moe_layers(model, b, [0, 1, 2],
                                                                      make) is None
        assert made == [0, 1, 2] and closed == ["s0", "s1"] and not model.accelerator_moe_layers
        assert projection.try_enable_model_accelerator_moe_layers(model, b, [0, 1], make) is True
        assert sorted(model.accelerator_moe_layers) == [0, 1]
    finally:
        acc.unregister_accelerator_backend("fake-men")


def test_hip_projection_runner_refuses_a_moe_session():
    from llambda_amd.hip_backend import HipBackendError, run_hip_session_into
    with pytest.raises(HipBackendError, match="not a 2-D projection session"):
        run_hip_session_into(np.zeros(4, np.float32), FakeMoeSession("m", 4, 3, None),
                             np.zeros(4, np.float32))
