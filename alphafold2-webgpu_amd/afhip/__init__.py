"""afhip: MI355X (gfx950) kernels for alphafold2-webgpu's GEMM, triangle
multiplication and outer-product-mean path, behind the C ABI in
include/afhip.h. This package is the host-side mirror of the reference's
operator API; every computation runs in libafhip.so.
"""
from ._lib import AfhipError, AfhipUnavailable, RangeError  # noqa: F401

__all__ = ["AfhipError", "AfhipUnavailable", "RangeError"]
