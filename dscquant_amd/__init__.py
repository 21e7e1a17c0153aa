"""dscquant_amd: DSCQuant's W4A4 linear-layer path, native to MI355X (gfx950).

    dscquant_amd.w4a4            quantize / matmul / pack_weight (the reference
                                 extension's API, kernel/w4a4.cu:164-230)
    dscquant_amd.core.quantization   the reference's quantization primitives
    dscquant_amd.core.linear         QuantLinear with the integer W4A4 forward

The compute path is libdscq.so (hand-written HIP for gfx950, C ABI in
include/dscq.h), loaded through ctypes on torch's HIP runtime.
"""
from . import _lib, w4a4  # noqa: F401
from .core import linear, quantization  # noqa: F401

__version__ = "0.1.0"
