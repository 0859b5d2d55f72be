"""lisa_amd -- MI355X (gfx950) implementation of LISA's MLX affine quantized linear.

The product is ``liblisaq.so`` (hand-written HIP kernels + a C ABI,
``include/lisaq.h``).  This package is its Python host side: ``ops`` mirrors
the reference op surface, ``quant`` the engine's ``QuantizedLinear``,
``moe`` the generic ``SparseMoeBlock`` routed path, and ``loader`` the
safetensors weight upload with packed-layout validation.
"""
from ._lib import LisaqError  # noqa: F401

__version__ = "0.1.0"
