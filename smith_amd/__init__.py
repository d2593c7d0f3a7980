"""smith_amd -- MI355X-native implementation of SMITH's quantized-weight
matmul path (quantizeQ4 / matmulQ4 / matmulQ8 and the GGUF decode that uses
them), behind the reference's own op names.

The compute path is libsmith.so (C ABI, include/smith.h) + the gfx950 code
object smith_kernels.hsaco; build both with `python -m smith_amd.build`.
Importing this package needs no GPU; the first GPU op creates the HIP
context and raises if there is no device (there is no CPU fallback).
"""
from .quantize import (GROUP_BYTES, GROUP_SIZE, Q8_BLOCK_BYTES, Q8_BLOCK_SIZE, QuantizedWeight, matmulQ4,
                       matmulQ8, quantizeQ4, quantizeQ8)
from .tensor import Tensor, create, ones, randn, tensor, to_array, zeros

toArray = to_array

__all__ = [
    "quantizeQ4", "matmulQ4", "matmulQ8", "quantizeQ8", "QuantizedWeight",
    "GROUP_SIZE", "GROUP_BYTES", "Q8_BLOCK_SIZE", "Q8_BLOCK_BYTES",
    "Tensor", "create", "tensor", "zeros", "ones", "randn", "to_array", "toArray",
]
