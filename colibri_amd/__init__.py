"""colibri_amd: gfx950 (MI355X) backend for colibri's quantized MoE expert path.

The product is libcoli_hip.so, a C-ABI shared library exporting the
`coli_cuda_*` function table that colibri's engine resolves by name
(c/backend_loader.c:1355-1400), plus a few `coli_hip_*` extensions
(include/coli_hip_ext.h). `backend` binds it with ctypes; there is no CPU
fallback: a missing library raises.
"""
from .backend import LIB_PATH, Backend, ColiHipMoeConfig, Session, declared_symbols  # noqa: F401

__all__ = ["LIB_PATH", "Backend", "ColiHipMoeConfig", "Session", "declared_symbols"]
