import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")
    # torch ships its own HIP runtime (libamdhip64.so, no soname) beside
    # /opt/rocm's (libamdhip64.so.7, which libllambda_hip.so names).  When
    # torch's is initialised first -- as bench.py does -- the library's HIP
    # calls resolve to that same runtime, so torch streams and device memory
    # can be handed to it; if the library initialised the device first,
    # torch would find none.  GPU tests that use torch need this order.
    try:
        import torch
    except ImportError:
        return
    if torch.cuda.is_available():
        torch.cuda.init()


@pytest.fixture(scope="session")
def hip():
    """The loaded HIP library; GPU tests fail loudly when it is missing."""
    from llambda_amd import native
    lib = native.lib()
    status = lib.llambda_hip_probe()
    assert status == 1, f"no usable gfx950 device (probe={status}): {native.last_error()}"
    return lib


@pytest.fixture(scope="session")
def kats():
    """Known answers of the reference's own tests (tests/golden/reference_kats.json)."""
    with open(os.path.join(ROOT, "tests", "golden", "reference_kats.json")) as fh:
        return json.load(fh)
