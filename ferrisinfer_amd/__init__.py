"""ferrisinfer_amd — MI355X (gfx950) HIP backend of FerrisInfer's ragged-batch attention
hot path.

The compute lives in ``libferrisinfer_kernel.so`` (C ABI: include/ferrisinfer_kernel.h).
``ferrisinfer_amd.kernel`` binds it with ctypes; the host runtime (batch packing, block
pool, scheduler, session) sits above that boundary.
"""
from .kernel import DTYPE_BF16, DTYPE_F16, DTYPE_F32, Context, FerrisError, load  # noqa: F401

__all__ = ["Context", "FerrisError", "load", "DTYPE_F32", "DTYPE_BF16", "DTYPE_F16"]
