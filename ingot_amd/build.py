"""Builds libingot_rocm.so (gfx950) in-tree with hipcc.

Every source under ingot_amd/csrc is compiled to an object in parallel and
linked into ingot_amd/libingot_rocm.so. Run directly (``python
ingot_amd/build.py``) or through ``__graft_entry__.build()``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libingot_rocm.so")

ARCH = "gfx950"
# Packed-FP32 instructions are kept out of the generated code on purpose.
COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
SOURCES = ["gemm_bf16x2.hip", "gemm_bf16.hip", "gemm_f32.hip", "gemm_i8.hip", "gemm_mfma.hip", "gemv_bf16.hip", "gemv_i8g.hip", "qconv.hip", "elementwise.hip", "runtime.cpp", "ops.cpp", "graph.cpp"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return path


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON, "-c", os.path.join(CSRC, src), "-o", out]
    if src.endswith(".cpp"):
        cmd.insert(1, "-xhip")
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile {src} failed:\n{r.stderr}")
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    workers = min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    # A kernel whose host-side launch stub the compiler silently failed to emit
    # leaves an undefined symbol that a shared library links anyway.
    nm = shutil.which("nm")
    if nm:
        und = subprocess.run([nm, "-D", "--undefined-only", tmp], capture_output=True, text=True).stdout
        stubs = [ln for ln in und.splitlines() if "__device_stub__" in ln]
        if stubs:
            raise RuntimeError("link left kernel launch stubs undefined:\n" + "\n".join(stubs[:5]))
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
