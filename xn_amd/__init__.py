"""xn_amd: MI355X (gfx950) backend for xn's GGUF quantized matmul path.

The numerical work runs in libxnq.so (hand-written HIP kernels, C ABI in
include/xnq.h); this package is the host-side mirror of xn's quantized
tensor API (QTensor / QLinear / BackendQ) over that library.
"""
from ._lib import XnqError, load  # noqa: F401
from . import gguf  # noqa: F401
from .quantized import (  # noqa: F401
    DEVICE_DTYPES,
    GgmlDType,
    Q2kHip,
    Q3kHip,
    Q4kHip,
    Q5kHip,
    Q6kHip,
    Q40Hip,
    Q41Hip,
    Q50Hip,
    Q51Hip,
    Q80Hip,
    QLinear,
    QStorage,
    QTensor,
    vec_dot_type,
)

__all__ = [
    "XnqError", "load", "GgmlDType", "QTensor", "QStorage", "QLinear", "Q40Hip", "Q80Hip",
    "Q4kHip", "Q6kHip", "Q41Hip", "Q50Hip", "Q51Hip", "Q2kHip", "Q3kHip", "Q5kHip", "DEVICE_DTYPES", "vec_dot_type", "gguf",
]
