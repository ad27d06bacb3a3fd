"""Kernel-level entry points (reference: kernels/__init__.py:1-11)."""

from .attention import asymmetric_attention_scores
from .bit_ops import pack_bits, unpack_bits
from .quantize import lloyd_max_dequantize, lloyd_max_quantize

__all__ = [
    "pack_bits",
    "unpack_bits",
    "lloyd_max_quantize",
    "lloyd_max_dequantize",
    "asymmetric_attention_scores",
]
