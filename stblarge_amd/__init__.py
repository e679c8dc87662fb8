"""stblarge_amd: an MI355X-native (gfx950) quantized expert-GEMV path with STBLarge's operator surface.

The computation lives in libstbl_amd.so (hand-written HIP kernels behind a C ABI, include/stbl_amd.h);
this package binds it with ctypes (_lib), wraps it for torch device tensors (ops), generates seeded
synthetic inputs (data) and builds the library (build).
"""

from . import _lib, data, ops  # noqa: F401

__all__ = ["_lib", "data", "ops"]
