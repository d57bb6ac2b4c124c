"""Tensor-indexed accelerator projection store with runtime fallback.

Mirrors the reference's binding store and its protocol (llambda.lisp):
  accelerator-projection            2356-2364
  register / unregister / clear     2672-2824 (copy-on-write tables)
  deferred retirement               2505-2549, 2662-2670
  cache key and paths               2954-3037
  ensure / enable (rollback)        3039-3094
  setup fallback / try-enable       3144-3208
  layer-role projection names       3256-3295
  run with runtime fallback         4660-4741
plus the one addition this backend needs: routed-MoE layer sessions, bound
per layer index in a table of their own (``accelerator_moe_layers``) and
tried first by the MoE functions (qwen3next-moe-into, llambda.lisp:5321;
nemotron-h-moe-ffn-into, 5827), falling back to their CPU body.  The
reference's routed experts never reach its store (4951-4971), and the
layer's router tensor, blk.N.ffn_gate_inp.weight, keeps its own 2-D binding.
The bottom of every fallback chain is the host's own CPU kernel
(%gguf-model-matrix-vector-multiply-into in the reference), which the host
supplies as ``ProjectionModel.cpu_matrix_vector``; this package has none.
"""
from __future__ import annotations

import os
import threading
import warnings
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import ggml
from .accelerator import (AcceleratorBackend, accelerator_backend_error_p,
                          resolve_accelerator_backend, signal_accelerator_backend_error)


@dataclass
class TensorInfo:
    """One GGUF tensor: dimensions are (columns, rows[, experts]) as in
    read-gguf-tensor-infos (llambda.lisp:2157-2238); ``data`` holds its bytes."""
    name: str
    type_tag: int
    dimensions: Tuple[int, ...]
    data: np.ndarray

    @property
    def columns(self) -> int:
        return self.dimensions[0]

    @property
    def rows(self) -> int:
        return self.dimensions[1] if len(self.dimensions) > 1 else 1

    @property
    def depth(self) -> int:
        return self.dimensions[2] if len(self.dimensions) > 2 else 1

    @property
    def byte_size(self) -> int:
        return self.rows * self.depth * ggml.row_bytes(self.type_tag, self.columns)


@dataclass
class AcceleratorProjection:
    """accelerator-projection (llambda.lisp:2356-2364)."""
    backend: AcceleratorBackend
    session: object
    run_mutex: threading.Lock = field(default_factory=threading.Lock)


CpuMatrixVector = Callable[[np.ndarray, "TensorInfo", np.ndarray], np.ndarray]


class ProjectionModel:
    """The parts of gguf-model (llambda.lisp:2366-2394) the projection path uses."""

    def __init__(self, tensors: Sequence[TensorInfo], *, layer_count: int = 0,
                 architecture: str = "", cpu_matrix_vector: Optional[CpuMatrixVector] = None):
        self.tensors: Dict[str, TensorInfo] = {t.name: t for t in tensors}
        self.layer_count = layer_count
        self.architecture = architecture
        self.cpu_matrix_vector = cpu_matrix_vector
        self.accelerator_projections: Dict[str, Tuple[AcceleratorProjection, ...]] = {}
        self.accelerator_moe_layers: Dict[int, Tuple[AcceleratorProjection, ...]] = {}
        self.retired: List[AcceleratorProjection] = []
        self.active_inference_count = 0
        self.runtime_mutex = threading.Lock()
        self.closed = False

    def tensor_info(self, name: str, required: bool = False) -> Optional[TensorInfo]:
        info = self.tensors.get(name)
        if required and info is None:
            raise KeyError(f"Model is missing required tensor {name!r}.")
        return info


# ------------------------------------------------------------ store edits

def model_accelerator_projection(model: ProjectionModel, backend, tensor_name: str):
    b = resolve_accelerator_backend(backend)
    for p in model.accelerator_projections.get(tensor_name, ()):
        if p.backend.name == b.name:
            return p
    return None


def model_accelerator_session(model: ProjectionModel, backend, tensor_name: str):
    p = model_accelerator_projection(model, backend, tensor_name)
    return p.session if p else None


def _close_projections(projections: List[AcceleratorProjection]) -> None:
    """close-retired-accelerator-projections (llambda.lisp:2517-2530)."""
    first = None
    for p in projections:
        try:
            p.backend.close_session_function(p.session)
        except Exception as exc:  # noqa: BLE001 - collected and re-raised below
            first = first or exc
    if first is not None:
        raise first


def _defer_or_collect(model: ProjectionModel, projections: List[AcceleratorProjection]):
    """defer-or-collect-accelerator-projections (llambda.lisp:2662-2670)."""
    if model.active_inference_count > 0:
        model.retired = projections + model.retired
        return []
    return projections


def register_model_accelerator_projection(model: ProjectionModel, backend, tensor_name: str,
                                          path: str, *, cache_directory=None, cache_key=None):
    """register-model-accelerator-projection (llambda.lisp:2672-2741)."""
    b = resolve_accelerator_backend(backend)
    info = model.tensor_info(tensor_name, required=True)
    session = b.make_session_function(path, cache_directory=cache_directory, cache_key=cache_key)
    try:
        if info.columns != b.session_input_element_count_function(session):
            raise ValueError(f"{b.display_name} input size does not match tensor {tensor_name!r}.")
        if info.rows != b.session_output_element_count_function(session):
            raise ValueError(f"{b.display_name} output size does not match tensor {tensor_name!r}.")
        with model.runtime_mutex:
            if model.closed:
                raise RuntimeError("REGISTER-MODEL-ACCELERATOR-PROJECTION on a closed model.")
            existing = model.accelerator_projections.get(tensor_name, ())
            if any(p.backend.name == b.name for p in existing):
                raise ValueError(f"Tensor {tensor_name!r} already has a {b.display_name} projection.")
            table = dict(model.accelerator_projections)
            table[tensor_name] = tuple(sorted(existing + (AcceleratorProjection(b, session),),
                                              key=lambda p: p.backend.priority))
            model.accelerator_projections = table
        session = None
    finally:
        if session is not None:
            b.close_session_function(session)
    return model


def unregister_model_accelerator_projection(model: ProjectionModel, backend, tensor_name: str):
    """unregister-model-accelerator-projection (llambda.lisp:2743-2789)."""
    b = resolve_accelerator_backend(backend)
    to_close: List[AcceleratorProjection] = []
    with model.runtime_mutex:
        existing = model.accelerator_projections.get(tensor_name, ())
        victim = next((p for p in existing if p.backend.name == b.name), None)
        if victim is not None:
            remaining = tuple(p for p in existing if p is not victim)
            table = dict(model.accelerator_projections)
            if remaining:
                table[tensor_name] = remaining
            else:
                table.pop(tensor_name, None)
            model.accelerator_projections = table
            to_close = _defer_or_collect(model, [victim])
    _close_projections(to_close)
    return model


def clear_model_accelerator_projections(model: ProjectionModel, backend=None):
    """clear-model-accelerator-projections (llambda.lisp:2791-2824)."""
    b = resolve_accelerator_backend(backend) if backend is not None else None
    with model.runtime_mutex:
        removed = []
        for attr in ("accelerator_projections", "accelerator_moe_layers"):
            table = {}
            for key, projections in getattr(model, attr).items():
                remaining = tuple(p for p in projections
                                  if b is not None and p.backend.name != b.name)
                removed.extend(p for p in projections if p not in remaining)
                if remaining:
                    table[key] = remaining
            setattr(model, attr, table)
        to_close = _defer_or_collect(model, removed)
    _close_projections(to_close)
    return model


def acquire_model_inference_use(model: ProjectionModel):
    """acquire-model-inference-use (llambda.lisp:2532-2537)."""
    with model.runtime_mutex:
        if model.closed:
            raise RuntimeError("INFERENCE on a closed model.")
        model.active_inference_count += 1
    return model


def release_model_inference_use(model: ProjectionModel):
    """release-model-inference-use (llambda.lisp:2539-2549)."""
    with model.runtime_mutex:
        model.active_inference_count -= 1
        if model.active_inference_count < 0:
            raise RuntimeError("Model inference use count became negative.")
        retired = []
        if model.active_inference_count == 0:
            retired, model.retired = model.retired, []
    _close_projections(retired)
    return model


# ------------------------------------------------------------ cache, setup

def _cache_component(value: str) -> str:
    """accelerator-cache-component (llambda.lisp:2969-2975)."""
    return "".join(c if (c.isalnum() or c in "-.") else "-" for c in value)


def model_accelerator_projection_cache_key(model: ProjectionModel, backend, tensor: TensorInfo,
                                           generator_path: Optional[str]) -> str:
    """model-accelerator-projection-cache-key (llambda.lisp:2977-2993)."""
    b = resolve_accelerator_backend(backend)
    if generator_path:
        with open(generator_path, "rb") as fh:
            generator_digest = b.byte_vector_sha256_function(fh.read())
    else:
        generator_digest = "none"
    data = np.ascontiguousarray(tensor.data).view(np.uint8)
    content = b.foreign_data_sha256_function(data.ctypes.data, tensor.byte_size)
    dims = "-".join(str(d) for d in tensor.dimensions)
    return (f"bridge-{_cache_component(b.bridge_version_function())}-generator-{generator_digest}"
            f"-ort-{_cache_component(b.runtime_version_function())}"
            f"-weights-{b.weight_format.lower()}-ggml-{tensor.type_tag}-{dims}-{content}")


def model_accelerator_projection_cache_pathnames(model, backend, tensor_name, cache_directory=None,
                                                 generator_path=None):
    """model-accelerator-projection-cache-pathnames (llambda.lisp:3003-3024):
    <root>/<cache-key>/projection.onnx (the file name is kept as an opaque
    name; the HIP backend writes its packed format there)."""
    b = resolve_accelerator_backend(backend)
    info = model.tensor_info(tensor_name, required=True)
    key = model_accelerator_projection_cache_key(model, b, info, generator_path)
    root = cache_directory or b.default_cache_directory_function()
    return os.path.join(root, key, "projection.onnx"), root, key


def ensure_model_accelerator_projection(model, backend, tensor_name, *, cache_directory=None,
                                        python_command=("python",), generator_path=None):
    """ensure-model-accelerator-projection (llambda.lisp:3039-3067)."""
    b = resolve_accelerator_backend(backend)
    if model_accelerator_projection(model, b, tensor_name):
        return model, None, True
    path, root, key = model_accelerator_projection_cache_pathnames(
        model, b, tensor_name, cache_directory, generator_path)
    reused = os.path.exists(path)
    if not reused:
        b.export_projection_function(model, tensor_name, path, python_command=python_command,
                                     generator_path=generator_path)
    register_model_accelerator_projection(model, b, tensor_name, path, cache_directory=root,
                                          cache_key=key)
    return model, path, reused


def enable_model_accelerator_projections(model, backend, tensor_names, *, cache_directory=None,
                                         python_command=("python",), generator_path=None):
    """enable-model-accelerator-projections (llambda.lisp:3069-3094): all or nothing."""
    b = resolve_accelerator_backend(backend)
    added, completed = [], False
    try:
        for name in tensor_names:
            if not model_accelerator_projection(model, b, name):
                ensure_model_accelerator_projection(model, b, name, cache_directory=cache_directory,
                                                    python_command=python_command,
                                                    generator_path=generator_path)
                added.append(name)
        completed = True
        return model
    finally:
        if not completed:
            for name in added:
                unregister_model_accelerator_projection(model, b, name)


PROJECTION_ROLE_SUFFIXES = {
    "attention-query": "attn_q.weight",
    "attention-key": "attn_k.weight",
    "attention-value": "attn_v.weight",
    "attention-output": "attn_output.weight",
    "ffn-gate": "ffn_gate.weight",
    "ffn-up": "ffn_up.weight",
    "ffn-down": "ffn_down.weight",
}


def model_accelerator_layer_projection_names(model, layer_indices, roles=tuple(PROJECTION_ROLE_SUFFIXES)):
    """model-accelerator-layer-projection-names (llambda.lisp:3265-3295)."""
    names = []
    for layer in layer_indices:
        if not (isinstance(layer, int) and 0 <= layer < model.layer_count):
            raise ValueError(f"Layer index {layer!r} is invalid for a {model.layer_count}-layer model.")
        for role in roles:
            suffix = PROJECTION_ROLE_SUFFIXES.get(role)
            if suffix is None:
                raise ValueError(f"Unknown accelerator projection role {role!r}.")
            name = f"blk.{layer}.{suffix}"
            if model.tensor_info(name) is None:
                raise ValueError(f"Model architecture {model.architecture} has no {role!r} "
                                 f"projection in layer {layer}.")
            names.append(name)
    return names


def call_with_accelerator_setup_fallback(backend, setup_function):
    """call-with-accelerator-setup-fallback (llambda.lisp:3144-3152)."""
    b = resolve_accelerator_backend(backend)
    try:
        return setup_function()
    except Exception as exc:  # noqa: BLE001 - the reference warns on any error
        warnings.warn(f"{b.display_name} setup failed; continuing with the next available "
                      f"backend: {exc}")
        return None


def try_enable_model_accelerator_projections(model, backend, tensor_names=(), *, layer_indices=None,
                                             projection_roles=tuple(PROJECTION_ROLE_SUFFIXES),
                                             cache_directory=None, python_command=("python",),
                                             generator_path=None):
    """try-enable-model-accelerator-projections (llambda.lisp:3160-3208)."""
    b = resolve_accelerator_backend(backend)

    def setup():
        names = list(dict.fromkeys(list(tensor_names) + (
            model_accelerator_layer_projection_names(model, layer_indices, projection_roles)
            if layer_indices else [])))
        if not names:
            signal_accelerator_backend_error(
                b, "%s acceleration was requested without any projections.", b.display_name)
        b.load_function()
        if not b.available_p_function():
            signal_accelerator_backend_error(b, "%s acceleration is unavailable.", b.display_name)
        enable_model_accelerator_projections(model, b, names, cache_directory=cache_directory,
                                             python_command=python_command,
                                             generator_path=generator_path)
        return True

    return call_with_accelerator_setup_fallback(b, setup)


# -------------------------------------------------------------- running

def call_with_accelerator_runtime_fallback(backend, accelerator_function, fallback_function,
                                           disable_function, tensor_name):
    """call-with-accelerator-runtime-fallback (llambda.lisp:4660-4676)."""
    b = resolve_accelerator_backend(backend)
    try:
        return accelerator_function()
    except Exception as exc:  # noqa: BLE001 - filtered by the backend's error predicate
        if not accelerator_backend_error_p(b, exc):
            raise
        disable_function()
        warnings.warn(f"{b.display_name} projection {tensor_name!r} failed and was disabled; "
                      f"using the next available backend: {exc}")
        return fallback_function()


def matrix_vector_multiply_into(dest: np.ndarray, model: ProjectionModel, tensor_name: str,
                                vector: np.ndarray) -> np.ndarray:
    """gguf-model-matrix-vector-multiply-into (llambda.lisp:4688-4741): run the
    tensor's bindings in priority order, each falling through to the next on
    its backend's error, and finally the host's CPU kernel."""
    projections = model.accelerator_projections.get(tensor_name)

    def run_on_cpu():
        info = model.tensor_info(tensor_name, required=True)
        if model.cpu_matrix_vector is None:
            raise RuntimeError(f"no CPU matrix-vector kernel configured for {tensor_name!r}")
        return model.cpu_matrix_vector(dest, info, vector)

    if not projections:
        return run_on_cpu()

    def run_projection_or_cpu(index: int):
        if index >= len(projections):
            return run_on_cpu()
        p = projections[index]

        def run():
            with p.run_mutex:
                return p.backend.run_session_function(dest, p.session, vector)

        return call_with_accelerator_runtime_fallback(
            p.backend, run, lambda: run_projection_or_cpu(index + 1),
            lambda: unregister_model_accelerator_projection(model, p.backend, tensor_name),
            tensor_name)

    return run_projection_or_cpu(0)


def matrix_vector_multiply(model: ProjectionModel, tensor_name: str, vector: np.ndarray) -> np.ndarray:
    """gguf-model-matrix-vector-multiply (llambda.lisp:4743-4750)."""
    info = model.tensor_info(tensor_name, required=True)
    return matrix_vector_multiply_into(np.empty(info.rows, dtype=np.float32), model, tensor_name,
                                       vector)


# ------------------------------------------------------- MoE layer hook

def model_accelerator_moe_layer(model: ProjectionModel, backend, layer_index: int):
    b = resolve_accelerator_backend(backend)
    for p in model.accelerator_moe_layers.get(layer_index, ()):
        if p.backend.name == b.name:
            return p
    return None


def register_model_accelerator_moe_layer(model: ProjectionModel, backend, layer_index: int,
                                         session):
    """Bind a routed-MoE layer session (an object with ``hidden_size``,
    ``expert_count``, ``run_into(dest, x)`` and ``close()``) to layer
    `layer_index`.  The check mirrors register-model-accelerator-projection's
    N x K check (llambda.lisp:2686-2703) for a layer: the session's hidden size
    must be the columns and its expert count the rows of the layer's router
    tensor blk.N.ffn_gate_inp.weight.  The table is copy-on-write like the
    projection table; the session is closed when registration fails.  No
    counterpart in the reference store (its routed experts bypass it,
    llambda.lisp:4951-4971)."""
    b = resolve_accelerator_backend(backend)
    try:
        if not (isinstance(layer_index, int) and 0 <= layer_index < max(model.layer_count, 1)):
            raise ValueError(f"Layer index {layer_index!r} is invalid for a "
                             f"{model.layer_count}-layer model.")
        router_name = f"blk.{layer_index}.ffn_gate_inp.weight"
        router = model.tensor_info(router_name, required=True)
        if session.hidden_size != router.columns:
            raise ValueError(f"{b.display_name} MoE session hidden size {session.hidden_size} does "
                             f"not match tensor {router_name!r} ({router.columns} columns).")
        if session.expert_count != router.rows:
            raise ValueError(f"{b.display_name} MoE session expert count {session.expert_count} "
                             f"does not match tensor {router_name!r} ({router.rows} rows).")
        with model.runtime_mutex:
            if model.closed:
                raise RuntimeError("REGISTER-MODEL-ACCELERATOR-MOE-LAYER on a closed model.")
            existing = model.accelerator_moe_layers.get(layer_index, ())
            if any(p.backend.name == b.name for p in existing):
                raise ValueError(f"Layer {layer_index} already has a {b.display_name} MoE session.")
            table = dict(model.accelerator_moe_layers)
            table[layer_index] = tuple(sorted(existing + (AcceleratorProjection(b, session),),
                                              key=lambda p: p.backend.priority))
            model.accelerator_moe_layers = table
        session = None
    finally:
        if session is not None:
            b.close_session_function(session)
    return model


def unregister_model_accelerator_moe_layer(model: ProjectionModel, backend, layer_index: int):
    """Remove the backend's MoE session of a layer; closed now, or when the
    model's active inferences end (as unregister-model-accelerator-projection,
    llambda.lisp:2743-2789)."""
    b = resolve_accelerator_backend(backend)
    to_close: List[AcceleratorProjection] = []
    with model.runtime_mutex:
        existing = model.accelerator_moe_layers.get(layer_index, ())
        victim = next((p for p in existing if p.backend.name == b.name), None)
        if victim is not None:
            remaining = tuple(p for p in existing if p is not victim)
            table = dict(model.accelerator_moe_layers)
            if remaining:
                table[layer_index] = remaining
            else:
                table.pop(layer_index, None)
            model.accelerator_moe_layers = table
            to_close = _defer_or_collect(model, [victim])
    _close_projections(to_close)
    return model


def try_enable_model_accelerator_moe_layers(model: ProjectionModel, backend, layer_indices,
                                            make_session):
    """Setup for the hook: load and probe the backend, then for each layer
    make_session(model, layer_index) and register it -- all or nothing, under
    the setup fallback (a failure warns, and the layers keep their CPU body),
    as try-enable-model-accelerator-projections (llambda.lisp:3160-3208)."""
    b = resolve_accelerator_backend(backend)

    def setup():
        layers = list(layer_indices)
        if not layers:
            signal_accelerator_backend_error(
                b, "%s MoE acceleration was requested without any layers.", b.display_name)
        b.load_function()
        if not b.available_p_function():
            signal_accelerator_backend_error(b, "%s acceleration is unavailable.", b.display_name)
        added, completed = [], False
        try:
            for layer in layers:
                if model_accelerator_moe_layer(model, b, layer) is None:
                    register_model_accelerator_moe_layer(model, b, layer, make_session(model, layer))
                    added.append(layer)
            completed = True
        finally:
            if not completed:
                for layer in added:
                    unregister_model_accelerator_moe_layer(model, b, layer)
        return True

    return call_with_accelerator_setup_fallback(b, setup)


def moe_layer_into(dest: np.ndarray, model: ProjectionModel, layer_index: int,
                   vector: np.ndarray, cpu_body: Callable[[], np.ndarray]) -> np.ndarray:
    """The hook at the top of qwen3next-moe-into / nemotron-h-moe-ffn-into:
    the layer's MoE sessions in priority order, each falling through to the
    next on its backend's error (and unregistered), then ``cpu_body`` -- the
    reference function's own body -- exactly as the projection path falls
    back (llambda.lisp:4660-4741)."""
    projections = model.accelerator_moe_layers.get(layer_index)
    if not projections:
        return cpu_body()
    name = f"blk.{layer_index} MoE layer"

    def run_or_next(index: int):
        if index >= len(projections):
            return cpu_body()
        p = projections[index]

        def run():
            with p.run_mutex:
                return p.session.run_into(dest, vector)

        return call_with_accelerator_runtime_fallback(
            p.backend, run, lambda: run_or_next(index + 1),
            lambda: unregister_model_accelerator_moe_layer(model, p.backend, layer_index), name)

    return run_or_next(0)
