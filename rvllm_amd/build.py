"""Builds librvkv.so (HIP kernels + C ABI + host block manager) for gfx950,
and the benchmark's streaming-read probe as a separate librvkv_calib.so.

Run as ``python -m rvllm_amd.build``. hipcc cross-compiles for gfx950 on a
host without a GPU; the .so is written in-tree next to this file.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "librvkv.so")
CALIB_LIB = os.path.join(HERE, "librvkv_calib.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    os.path.join(HERE, "csrc", "rvkv.hip"),
    os.path.join(HERE, "csrc", "prefill.hip"),
    os.path.join(HERE, "csrc", "argmax.hip"),
    os.path.join(HERE, "csrc", "generic.hip"),
    os.path.join(HERE, "csrc", "block_manager.cpp"),
    os.path.join(HERE, "csrc", "scheduler.cpp"),
]

# Packed-FP32 instructions are kept out of generated code on purpose.
# Kernel-argument preload: a kernel's first six scalar or pointer arguments
# arrive in SGPRs (the decode kernels take the inputs of their start-up
# chain that way), so their first table read needs no argument load; on
# firmware without preload the code object's own prologue loads them.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=6",
    "-Wall", "-Wno-unused-result",
]


def build(verbose: bool = False) -> str:
    """Compiles every source into librvkv.so; returns its path."""
    objs = []
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    for src in SOURCES:
        obj = os.path.join(build_dir, os.path.basename(src) + ".o")
        if src.endswith(".hip"):
            cmd = [HIPCC, *HIP_FLAGS, "-c", src, "-o", obj]
        else:
            cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-c", src,
                   "-o", obj]
        _run(cmd, verbose)
        objs.append(obj)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp,
          *objs], verbose)
    os.replace(tmp, LIB)
    # The bench-only read probe: its own library, outside the product ABI.
    cobj = os.path.join(build_dir, "calib.hip.o")
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(HERE, "csrc", "calib.hip"),
          "-o", cobj], verbose)
    tmp = CALIB_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp,
          cobj], verbose)
    os.replace(tmp, CALIB_LIB)
    return LIB


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose=True))
