"""mold_amd — MI355X-native (gfx950) GGUF quantized-linear hot path for mold.

The product is libmoldq.so (HIP kernels behind the C ABI in include/moldq.h).
This package is the host-side mirror of candle's quantized API used by the
tests and the benchmark; see quantized.py and gguf.py.
"""
from ._lib import MoldqError, load  # noqa: F401
from .quantized import (ACT_GELU_TANH, ACT_NONE, Device, GgmlDType, Linear, Q8KActivations, QMatMul,  # noqa: F401
                        QTensor, QUANT_TYPES)

__all__ = ["MoldqError", "load", "Device", "GgmlDType", "Linear", "Q8KActivations", "QMatMul", "QTensor", "QUANT_TYPES",
           "ACT_NONE", "ACT_GELU_TANH"]
