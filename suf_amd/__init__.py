"""suf_amd: MI355X-native PFSS execution backend for SUF.

The product is the C-ABI shared library suf_amd/lib/libsuf_hip.so (declared
in include/suf_hip.h) with hand-written gfx950 HIP kernels; `native` binds it
with ctypes and `pfss` offers torch-tensor conveniences on top.
"""
from . import native  # noqa: F401

__all__ = ["native"]
