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


OBJ_DIR = os.path.join(PKG_DIR, "_build")


def _compile(src: str, verbose: bool) -> str:
    """One translation unit to an object (its device code embedded) under _build/."""
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    cmd = [hipcc(), *flags, "-c", "-o", obj, src]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, cwd=PKG_DIR, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)} (exit {res.returncode})")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compiles every translation unit (in parallel, always from source) and links the
    kernel library, then the host runtime library."""
    from concurrent.futures import ThreadPoolExecutor

    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = jobs or max(1, min(len(srcs), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, cwd=PKG_DIR, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed linking {LIB_NAME} (exit {res.returncode})")
    os.replace(tmp, LIB_PATH)
    build_runtime(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
