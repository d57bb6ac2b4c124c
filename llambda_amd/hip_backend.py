"""The HIP (MI355X) accelerator backend: sessions over libllambda_hip.so and
the descriptor registered beside the reference's :gpu and :npu backends.

Lisp counterparts:
  make-/close-/run-*-session-into     llambda.lisp:260-358
  status -> condition mapping         llambda.lisp:256-258, 311-313
  descriptor registration             accelerators/directml.lisp:3-29
The backend consumes GGUF super-block bytes as they are (weight format
``packed-ggml``); its exporter writes them to the cache path in the
packed-projection format that llambda_hip_session_create reads.
"""
from __future__ import annotations

import ctypes
import os
import tempfile
from typing import Optional

import numpy as np

from . import ggml, native
from .accelerator import AcceleratorBackend, register_accelerator_backend


class HipBackendError(RuntimeError):
    """The backend's condition type; error-p selects exactly this class
    (the analogue of gpu-backend-error, accelerators/directml.lisp:20-21)."""


def signal_hip_backend_error(fmt: str, *args):
    raise HipBackendError(fmt % args if args else fmt)


def _check(status: int, what: str) -> None:
    if status != 0:
        raise HipBackendError(f"{what} failed: {native.last_error()}")


def load_hip_backend():
    """load-function: load the shared library (raises when it is missing)."""
    try:
        return native.lib()
    except (native.NativeLibraryMissing, OSError) as exc:
        raise HipBackendError(str(exc)) from exc


def hip_backend_available_p() -> bool:
    status = native.lib().llambda_hip_probe()
    if status < 0:
        raise HipBackendError(f"HIP probe failed: {native.last_error()}")
    return status == 1


def hip_runtime_version() -> str:
    return native.lib().llambda_hip_runtime_version().decode()


def hip_bridge_version() -> str:
    return native.lib().llambda_hip_bridge_version().decode()


def default_hip_cache_directory() -> str:
    base = os.environ.get("XDG_CACHE_HOME") or os.path.join(os.path.expanduser("~"), ".cache")
    return os.path.join(base, "llambda", "hip-cache")


def foreign_data_sha256(pointer: int, byte_size: int) -> str:
    out = ctypes.create_string_buffer(65)
    _check(native.lib().llambda_hip_sha256(pointer, byte_size, out, 65), "SHA-256")
    return out.value.decode("ascii")


def byte_vector_sha256(octets: bytes) -> str:
    buf = np.frombuffer(bytes(octets), dtype=np.uint8)
    return foreign_data_sha256(buf.ctypes.data if buf.size else None, buf.size)


# ------------------------------------------------------------------ sessions

class HipSession:
    """A projection session: one N x K packed tensor resident in HBM."""

    def __init__(self, pointer: int):
        self.pointer = pointer

    @property
    def input_element_count(self) -> int:
        return native.lib().llambda_hip_session_input_element_count(self.pointer)

    @property
    def output_element_count(self) -> int:
        return native.lib().llambda_hip_session_output_element_count(self.pointer)

    def close(self) -> None:
        """Idempotent, like close-gpu-session (llambda.lisp:327-332)."""
        if self.pointer:
            native.lib().llambda_hip_session_destroy(self.pointer)
            self.pointer = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    def _live(self):
        if not self.pointer:
            raise HipBackendError("HIP session is closed.")
        return self.pointer

    def run_into(self, dest: np.ndarray, vector: np.ndarray) -> np.ndarray:
        """run-gpu-session-into (llambda.lisp:334-358) for one token."""
        return self.run_batch_into(dest, vector, 1)

    def run_batch_into(self, dest: np.ndarray, inputs: np.ndarray, batch: int) -> np.ndarray:
        _require_f32(dest, "destination")
        _require_f32(inputs, "input")
        _check(native.lib().llambda_hip_session_run_batch(
            self._live(), inputs.ctypes.data, inputs.size, dest.ctypes.data, dest.size, batch),
            "HIP session run")
        return dest

    def run_device(self, input_ptr: int, output_ptr: int, batch: int = 1, stream: int = 0) -> None:
        _check(native.lib().llambda_hip_session_run_device(self._live(), input_ptr, output_ptr,
                                                           batch, stream or None),
               "HIP session device run")

    def dequantize(self) -> np.ndarray:
        out = np.empty(self.input_element_count * self.output_element_count, dtype=np.float32)
        _check(native.lib().llambda_hip_session_dequantize(self._live(), out.ctypes.data, out.size),
               "HIP session dequantize")
        return out.reshape(self.output_element_count, self.input_element_count)


def _require_f32(a: np.ndarray, what: str) -> None:
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous):
        raise HipBackendError(f"HIP session {what} must be a contiguous float32 array.")


def make_hip_session(model_path: str, *, cache_directory=None, cache_key=None) -> HipSession:
    """make-session-function: open a packed-projection file."""
    handle = ctypes.c_void_p()
    _check(native.lib().llambda_hip_session_create(
        os.fsencode(model_path), os.fsencode(cache_directory) if cache_directory else None,
        cache_key.encode() if cache_key else None, ctypes.byref(handle)),
        f"HIP session creation for {model_path}")
    return HipSession(handle.value)


def make_hip_session_packed(data: np.ndarray, type_tag: int, rows: int, columns: int) -> HipSession:
    """Upload a tensor straight from its bytes (no file)."""
    data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    handle = ctypes.c_void_p()
    _check(native.lib().llambda_hip_session_create_packed(
        data.ctypes.data, data.size, type_tag, rows, columns, ctypes.byref(handle)),
        "HIP session creation")
    return HipSession(handle.value)


def close_hip_session(session: Optional[HipSession]) -> None:
    if session is not None:
        session.close()


def run_hip_session_into(dest, session: HipSession, vector):
    """run-session-function: 2-D projection sessions only (a MoE layer session
    is bound in the MoE-layer table and run by the MoE hook)."""
    if not isinstance(session, HipSession):
        raise HipBackendError(f"{type(session).__name__} is not a 2-D projection session.")
    return session.run_into(dest, vector)


def hip_session_input_element_count(session: HipSession) -> int:
    return session.input_element_count


def hip_session_output_element_count(session: HipSession) -> int:
    return session.output_element_count


PACKED_MAGIC = b"LLHIPPRJ"
PACKED_VERSION = 1


def write_packed_projection(path: str, type_tag: int, rows: int, columns: int, data) -> None:
    """Write the packed-projection file atomically (the reference replaces
    cache files the same way, llambda.lisp:391-400)."""
    payload = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
    expected = rows * ggml.row_bytes(type_tag, columns)
    if payload.size != expected:
        raise HipBackendError(f"packed projection holds {payload.size} bytes, expected {expected}")
    directory = os.path.dirname(os.path.abspath(path))
    os.makedirs(directory, exist_ok=True)
    header = (PACKED_MAGIC + np.array([PACKED_VERSION, type_tag], dtype="<u4").tobytes()
              + np.array([rows, columns, payload.size], dtype="<u8").tobytes())
    fd, tmp = tempfile.mkstemp(dir=directory, suffix=".tmp")
    try:
        with os.fdopen(fd, "wb") as fh:
            fh.write(header)
            fh.write(memoryview(payload))
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise


def export_model_hip_projection(model, tensor_name: str, out_path: str, *, python_command=None,
                                generator_path=None) -> str:
    """export-projection-function: copy the tensor's GGUF bytes verbatim."""
    info = model.tensor_info(tensor_name, required=True)
    if len(info.dimensions) != 2:
        raise HipBackendError(f"Tensor {tensor_name!r} is not a two-dimensional projection.")
    write_packed_projection(out_path, info.type_tag, info.rows, info.columns, info.data)
    return out_path


HIP_BACKEND = AcceleratorBackend(
    name="hip",
    display_name="HIP",
    priority=5,                  # before :gpu (10) and :npu (20)
    initialization_priority=5,
    load_function=load_hip_backend,
    available_p_function=hip_backend_available_p,
    runtime_version_function=hip_runtime_version,
    bridge_version_function=hip_bridge_version,
    make_session_function=make_hip_session,
    close_session_function=close_hip_session,
    run_session_function=run_hip_session_into,
    session_input_element_count_function=hip_session_input_element_count,
    session_output_element_count_function=hip_session_output_element_count,
    error_p_function=lambda condition: isinstance(condition, HipBackendError),
    signal_error_function=signal_hip_backend_error,
    default_cache_directory_function=default_hip_cache_directory,
    export_projection_function=export_model_hip_projection,
    weight_format="packed-ggml",
    foreign_data_sha256_function=foreign_data_sha256,
    byte_vector_sha256_function=byte_vector_sha256,
)


def register_hip_backend():
    return register_accelerator_backend(HIP_BACKEND, replace=True)
