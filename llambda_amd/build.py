"""Build libllambda_hip.so in-tree (hipcc, gfx950) and the oracle (gcc).

``python -m llambda_amd.build`` or ``llambda_amd.build.build()``.  Objects go
to ``llambda_amd/_build/``; the shared library to
``llambda_amd/libllambda_hip.so``, and the command-line check
``llambda_amd/llambda_hip_smoke`` (linked against it) beside it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libllambda_hip.so")
SMOKE = os.path.join(HERE, "llambda_hip_smoke")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Device code: gfx950 only, packed-FP32 instructions disabled (they are
# emitted from ordinary float code otherwise).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the kernels scale and add them with
    # VALU instructions, which cannot read the accumulation registers
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall"]

HIP_SOURCES = ["gemv.hip", "gemv_mfma.hip", "moe.hip", "moe_mfma.hip", "decoder.hip", "sample.hip", "abi.hip"]
CXX_SOURCES = ["sha256.cpp", "gguf.cpp"]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is noise
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in line and line.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False, defines=(), obj_dir: str = OBJ, lib_path: str = LIB) -> str:
    """Compile every source and link the library; returns its path.
    ``defines`` are extra -D tuning constants (see gemv.hip)."""
    os.makedirs(obj_dir, exist_ok=True)
    jobs = []
    for src in HIP_SOURCES:
        obj = os.path.join(obj_dir, src + ".o")
        jobs.append([HIPCC, *HIP_FLAGS, *[f"-D{d}" for d in defines], "-c",
                     os.path.join(CSRC, src), "-o", obj])
    for src in CXX_SOURCES:
        obj = os.path.join(obj_dir, src + ".o")
        jobs.append(["g++", *CXX_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(4, len(jobs))) as pool:
        outs = list(pool.map(_run, jobs))
    if verbose:
        for o in outs:
            if o:
                print(o)
    objs = [os.path.join(obj_dir, s + ".o") for s in HIP_SOURCES + CXX_SOURCES]
    tmp = lib_path + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    shutil.move(tmp, lib_path)
    if lib_path == LIB:
        # the smoke CLI finds the library beside itself
        tmp = SMOKE + ".tmp"
        _run(["g++", *CXX_FLAGS, os.path.join(CSRC, "smoke.cpp"), "-o", tmp, f"-L{HERE}",
              "-lllambda_hip", "-Wl,-rpath,$ORIGIN"])
        shutil.move(tmp, SMOKE)
    return lib_path


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
