"""MI355X (gfx950) packed-weight hot path of ADI.

The product is libadi_hip.so (HIP kernels behind the C ABI in
include/adi_hip.h); `adi_amd.hip` binds it with ctypes and `adi_amd.build`
compiles it in-tree.
"""
__all__ = ["hip", "build", "synthetic"]
