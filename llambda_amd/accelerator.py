"""The accelerator-backend descriptor protocol (accelerator.lisp:3-129).

An ``AcceleratorBackend`` is an immutable descriptor of 19 required slots,
registered by name; execution order is ascending ``priority``.  The HIP
backend (hip_backend.py) is one such descriptor, the way
accelerators/directml.lisp and accelerators/vitisai.lisp register theirs.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass, fields
from typing import Callable, Dict, List, Optional, Union


@dataclass(frozen=True)
class AcceleratorBackend:
    """make-accelerator-backend (accelerator.lisp:3-91); every slot is required."""
    name: str
    display_name: str
    priority: float
    initialization_priority: float
    load_function: Callable[[], object]
    available_p_function: Callable[[], bool]
    runtime_version_function: Callable[[], str]
    bridge_version_function: Callable[[], str]
    make_session_function: Callable[..., object]        # (model_path, *, cache_directory, cache_key)
    close_session_function: Callable[[object], None]
    run_session_function: Callable[[object, object, object], object]  # (dest, session, input)
    session_input_element_count_function: Callable[[object], int]
    session_output_element_count_function: Callable[[object], int]
    error_p_function: Callable[[BaseException], bool]
    signal_error_function: Callable[..., None]           # (fmt, *args) -> raises
    default_cache_directory_function: Callable[[], str]
    export_projection_function: Callable[..., object]   # (model, tensor_name, out_path, **kw)
    weight_format: str
    foreign_data_sha256_function: Callable[[object, int], str]
    byte_vector_sha256_function: Callable[[bytes], str]

    def __post_init__(self):
        for f in fields(self):
            if getattr(self, f.name) is None:
                raise ValueError(f"Accelerator backend {f.name.replace('_', ' ')} is required.")


_registry: Dict[str, AcceleratorBackend] = {}
_registry_lock = threading.Lock()


def register_accelerator_backend(backend: AcceleratorBackend, *, replace: bool = False):
    """register-accelerator-backend (accelerator.lisp:95-104)."""
    if not isinstance(backend, AcceleratorBackend):
        raise TypeError(f"Expected an accelerator backend descriptor, got {backend!r}.")
    with _registry_lock:
        if backend.name in _registry and not replace:
            raise ValueError(f"Accelerator backend {backend.name!r} is already registered.")
        _registry[backend.name] = backend
    return backend


def unregister_accelerator_backend(name: str) -> None:
    with _registry_lock:
        _registry.pop(name, None)


def find_accelerator_backend(name: Optional[str], required: bool = False):
    """find-accelerator-backend (accelerator.lisp:106-113)."""
    backend = _registry.get(name) if name else None
    if required and backend is None:
        known = ", ".join(repr(b.name) for b in ordered_accelerator_backends())
        raise ValueError(f"Unknown accelerator backend {name!r}. Registered backends: {known}.")
    return backend


def ordered_accelerator_backends() -> List[AcceleratorBackend]:
    """ordered-accelerator-backends (accelerator.lisp:115-120)."""
    with _registry_lock:
        backends = list(_registry.values())
    return sorted(backends, key=lambda b: b.priority)


def resolve_accelerator_backend(backend: Union[str, AcceleratorBackend]) -> AcceleratorBackend:
    """resolve-accelerator-backend (llambda.lisp:2631-2635)."""
    if isinstance(backend, AcceleratorBackend):
        return backend
    return find_accelerator_backend(backend, required=True)


def accelerator_backend_error_p(backend, condition: BaseException) -> bool:
    """accelerator-backend-error-p (accelerator.lisp:122-123)."""
    return bool(resolve_accelerator_backend(backend).error_p_function(condition))


def signal_accelerator_backend_error(backend, format_control: str, *args):
    """signal-accelerator-backend-error (accelerator.lisp:125-129)."""
    return resolve_accelerator_backend(backend).signal_error_function(format_control, *args)
