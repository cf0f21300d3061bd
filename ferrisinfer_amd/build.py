"""Builds libferrisinfer_kernel.so (HIP, gfx950) in-tree with hipcc.

Run as ``python -m ferrisinfer_amd.build``; ``__graft_entry__.build()`` calls :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libferrisinfer_kernel.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

# Every translation unit of the library, host C++ and device HIP alike.
SOURCES = [
    "fi_context.cpp",
    "fi_attention.hip",
    "fi_prefill.hip",
    "fi_ops.hip",
    "fi_gemm.hip",
    "fi_gemm_packed.hip",
    "fi_gemm_bf16.hip",
    "fi_sample.hip",
    "fi_convert.hip",
]

# gfx950 only; packed-fp32 instructions are disabled (the compiler would otherwise form
# v_pk_* f32 ops from scalar code).
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP backend cannot be built")


RUNTIME_LIB = "libferrisinfer_runtime.so"
RUNTIME_PATH = os.path.join(PKG_DIR, RUNTIME_LIB)
RUNTIME_SOURCES = ["runtime/fr_model.cpp", "runtime/fr_scheduler.cpp", "runtime/fr_capi.cpp",
                   "runtime/fr_json.cpp", "runtime/fr_checkpoint.cpp"]


def build_runtime(verbose: bool = False) -> str:
    """Host runtime: plain C++17 (g++), linked against the kernel library's C ABI only."""
    srcs = [os.path.join(CSRC, s) for s in RUNTIME_SOURCES]
    tmp = RUNTIME_PATH + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-o", tmp, *srcs,
           "-L" + PKG_DIR, "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, cwd=PKG_DIR, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"g++ failed building {RUNTIME_LIB} (exit {res.returncode})")
    os.replace(tmp, RUNTIME_PATH)
    return RUNTIME_PATH


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, cwd=PKG_DIR, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {LIB_NAME} (exit {res.returncode})")
    os.replace(tmp, LIB_PATH)
    build_runtime(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
