"""llambda_hip_smoke, the command-line check of one packed projection (the
counterpart of the reference's native/llambda_npu_smoke.cpp:41-151), and
llambda_hip_stream_read, the streaming-read ceiling bench.py reports."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from llambda_amd import ggml, native, synthetic

HERE = os.path.dirname(os.path.abspath(__file__))
SMOKE = os.path.join(os.path.dirname(HERE), "llambda_amd", "llambda_hip_smoke")


def _smoke(*args, timeout=60):
    return subprocess.run([SMOKE, *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                          text=True, timeout=timeout)


def test_smoke_cli_is_built_and_checks_its_arguments():
    assert os.access(SMOKE, os.X_OK), "build() writes llambda_amd/llambda_hip_smoke"
    r = _smoke()
    assert r.returncode == 2 and "usage: llambda_hip_smoke" in r.stderr
    r = _smoke("x.llhipprj", "-1", "1")
    assert r.returncode == 2 and "nonnegative" in r.stderr


@pytest.mark.gpu
def test_smoke_cli_runs_a_packed_projection(hip, tmp_path):
    from llambda_amd.hip_backend import make_hip_session_packed, write_packed_projection
    rng = np.random.default_rng(8)
    rows, cols = 1024, 2048
    w = synthetic.packed(ggml.Q4_K, rng, rows, cols)
    path = str(tmp_path / "blk.0.attn_q" / "projection.onnx")
    write_packed_projection(path, ggml.Q4_K, rows, cols, w)
    print("smoke CLI: Q4_K 1024x2048", flush=True)
    r = _smoke(path, "2", "5")
    assert r.returncode == 0, r.stderr
    m = re.search(r"^(HIP runtime .+) \((llambda-hip .+)\): (\d+) inputs -> (\d+) outputs; "
                  r"session = ([0-9.]+) ms; warm run = ([0-9.]+) ms; first output = (\S+)$",
                  r.stdout.strip())
    assert m, r.stdout
    assert (int(m.group(3)), int(m.group(4))) == (cols, rows)
    # the same call in this process: input 0.5 everywhere
    s = make_hip_session_packed(w, ggml.Q4_K, rows, cols)
    try:
        y = np.empty(rows, np.float32)
        s.run_into(y, np.full(cols, 0.5, np.float32))
    finally:
        s.close()
    assert np.float32(float(m.group(7))) == y[0]
    # a file that is not a packed projection: the library's error, status 1
    bad = tmp_path / "bad.onnx"
    bad.write_bytes(b"not a projection")
    r = _smoke(str(bad))
    assert r.returncode == 1 and "Session creation failed" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes", [16, 4096 * 1024, 10 * 1024 * 1024 + 48 * 16 + 16])
def test_stream_read_touches_every_byte(hip, nbytes):
    """The XOR of the wavefronts' words is the XOR of the whole buffer: every
    16-byte unit was read once (a skipped or repeated unit changes it)."""
    import torch
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2 ** 32, size=nbytes // 4, dtype=np.uint32)
    data = torch.from_numpy(host.view(np.int32)).cuda()
    out = torch.zeros(native.STREAM_READ_WORDS, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    print(f"stream_read {nbytes} bytes", flush=True)
    assert native.lib().llambda_hip_stream_read(data.data_ptr(), nbytes, out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)
    # unaligned or odd sizes are refused before anything is enqueued
    assert native.lib().llambda_hip_stream_read(data.data_ptr(), nbytes - 8 if nbytes > 16 else 8,
                                                out.data_ptr(), None) == -1
    assert "multiple of 16" in native.last_error()
