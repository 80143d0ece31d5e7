"""MI355X-native paged KV-cache hot path of MiniCPM5-5080Fast.

The product is libminicpm_native.so (HIP kernels for gfx950 + C++ host
runtime) behind the C ABI declared in include/minicpm_runtime.h and
include/mc_kv.h. This package is the Python host mirror of that ABI:
`kv` follows the reference launcher interface (native/kernels/sm120/kernels.h).
Import it as importlib.import_module("minicpm5-5080fast_amd").
"""
from . import _native, kv  # noqa: F401
from ._native import McError, lib  # noqa: F401

__all__ = ["kv", "lib", "McError"]
