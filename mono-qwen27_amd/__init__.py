"""mono27q: MI355X-native quantized matvec path of mono27b (eramax/mono-qwen27).

The product is libm27q.so (hand-written gfx950 HIP kernels behind the C ABI in
include/m27q.h); this package holds its sources (csrc/), its build (Makefile)
and a ctypes binding (m27q) for Python callers.
"""
from . import m27q  # noqa: F401

__all__ = ["m27q"]
