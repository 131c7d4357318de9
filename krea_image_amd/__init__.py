"""krea_image_amd: MI355X (gfx950) drop-in for the DiT weight-GEMM hot path of shinoss/krea_image.

The product is libkh.so (HIP kernels + C ABI, include/kh.h); `krea_image_amd.kh` is its ctypes binding.
"""
from . import kh  # noqa: F401
