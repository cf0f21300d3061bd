"""The C-ABI library loads and exports every symbol include/ferrisinfer_kernel.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ferrisinfer_kernel.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for required in ("fi_ctx_create", "fi_kv_append", "fi_attn_decode_paged", "fi_last_error"):
        assert required in syms


def test_library_exports_every_declared_symbol():
    from ferrisinfer_amd import kernel

    lib = ctypes.CDLL(kernel.library_path())
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_ctx_create_without_gpu_reports_unsupported():
    """With no device the backend reports 'unavailable' instead of failing obscurely
    (the reference degrades the same way, kernel/gpu/nvidia.rs:577-656)."""
    import torch

    if torch.cuda.is_available():
        return
    from ferrisinfer_amd import Context, FerrisError

    try:
        Context(0, use_torch_stream=False)
    except FerrisError as e:
        assert e.kind in ("Unsupported", "Runtime")
    else:
        raise AssertionError("context creation must fail without a GPU")


def test_packed_weight_sizes():
    """fi_weight_packed_floats (host arithmetic only): slabs of 16 * width columns, 64 * 4 *
    width floats per slab and 16-k step; width 32 is the 32-column layout, 512 floats per slab
    and step; other widths are refused."""
    from ferrisinfer_amd import kernel

    lib = ctypes.CDLL(kernel.library_path())
    out = ctypes.c_size_t()
    for k, n, pw, want in [(896, 1152, 1, 72 * 56 * 256), (896, 1152, 4, 18 * 56 * 1024),
                           (20, 37, 2, 2 * 2 * 512), (896, 1152, 32, 36 * 56 * 512),
                           (4864, 896, 32, 28 * 304 * 512), (36, 20, 32, 1 * 3 * 512)]:
        assert lib.fi_weight_packed_floats(k, n, pw, ctypes.byref(out)) == 0
        assert out.value == want, (k, n, pw)
    for pw in (0, 3, 8, 16):
        assert lib.fi_weight_packed_floats(64, 64, pw, ctypes.byref(out)) != 0


RUNTIME_HEADER = os.path.join(ROOT, "include", "ferrisinfer_runtime.h")


def test_runtime_library_exports_every_declared_symbol():
    from ferrisinfer_amd import runtime

    text = re.sub(r"/\*.*?\*/", "", open(RUNTIME_HEADER).read(), flags=re.S)
    syms = sorted(set(re.findall(r"\b(fr_[a-z0-9_]+)\s*\(", text)))
    assert "fr_execute_next_tick" in syms
    lib = ctypes.CDLL(runtime.LIB_PATH)
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
