"""zero_amd: MI355X (gfx950) quantized-matmul hot path of silicatetech/zero.

Hand-written HIP kernels behind a C ABI (include/zero_gpu.h, built into
zero_amd/libzero_amd.so) replace the reference's AVX-512 GEMV kernels and
SMP row partitioning.  This package is the host-side mirror of the
reference's operator API over that ABI.
"""
from .ops import (  # noqa: F401
    VOCAB_SIZE_PADDED,
    VOCAB_SIZE_REAL,
    ArgmaxInPaddingRegion,
    Context,
    GgmlType,
    LinearDispatchError,
    LmHeadError,
    NonFiniteLogits,
    ZgError,
    tensor_bytes,
)
from .smodel import InvalidContainer, LoadError, MagicMismatch, SModel, UnsupportedFormat  # noqa: F401

__all__ = [
    "Context", "GgmlType", "LinearDispatchError", "LmHeadError", "NonFiniteLogits", "ArgmaxInPaddingRegion",
    "ZgError", "tensor_bytes", "VOCAB_SIZE_PADDED", "VOCAB_SIZE_REAL",
    "SModel", "LoadError", "MagicMismatch", "UnsupportedFormat", "InvalidContainer",
]
