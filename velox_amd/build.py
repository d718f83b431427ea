"""Build libvelox_hip.so (gfx950) in-tree with hipcc.

Every translation unit is compiled in parallel (the .hip files by hipcc,
the host-only .cpp files by g++), then linked into velox_amd/libvelox_hip.so.
Packed-FP32 instruction selection is disabled (`-packed-fp32-ops`) for all
device code, and kernel-argument preloading is on (the leading scalar
arguments of a kernel arrive in SGPRs).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libvelox_hip.so")
SOURCES = ["qmm.hip", "attn.hip", "ops.hip", "engine.hip", "sched.cpp"]
ARCH = os.environ.get("VX_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-Wall", "-Wno-unused-function",
    "-Wno-unused-variable", "-Wno-unused-result",
    # gfx950 kernarg preload: a kernel's leading scalar arguments arrive in
    # SGPRs at wave launch instead of by a load from the argument block
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build velox_amd")
    return path


HOST_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-I", os.path.join(ROOT, "include"), "-Wall"]


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    if src.endswith(".cpp"):  # host-only code: no device pass
        cmd = [shutil.which("g++") or "g++", *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", out]
    else:
        cmd = [hipcc(), *FLAGS, "-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {src}:\n{r.stderr[-6000:]}")
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
