"""simdyolo_amd — MI355X (gfx950) forward-inference backend for SimdYolo.

The product is libsimdyolo_hip.so (C ABI, include/simdyolo_hip.h); this
package is its Python binding plus the seeded synthetic-model helpers.
"""
from . import _native
from ._native import (CONV_AUTO, CONV_DEPTHWISE, CONV_DIRECT, CONV_IGEMM, CONV_WINOGRAD, CONV_WINOGRAD2,
                      CONV_WINOGRAD3, SyError, Tensor)

__all__ = ["_native", "CONV_AUTO", "CONV_DEPTHWISE", "CONV_DIRECT", "CONV_IGEMM", "CONV_WINOGRAD", "CONV_WINOGRAD2",
           "CONV_WINOGRAD3", "SyError", "Tensor"]
