"""MI355X logits-to-token stage: Python bindings of liblsamp.so (ctypes).

The kernels live in ../csrc (HIP, gfx950) behind the C ABI of
include/lsamp.h; this package loads that library and wraps it for torch
device tensors.  It has no fallback: if the library is not built every entry
point raises LibraryMissing.
"""
from . import _ffi  # noqa: F401
