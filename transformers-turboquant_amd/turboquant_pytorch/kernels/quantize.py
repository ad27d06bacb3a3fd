"""Lloyd-Max quantise/dequantise of rotated coordinates (reference: kernels/quantize.py).

The code of a coordinate y is #{j : boundaries[j] < y}, i.e.
``torch.searchsorted(boundaries, y)`` (side='left'), the rule of the
reference's packed fallback (quantize.py:334-337).
"""

from __future__ import annotations

import torch

from .._ops import ops
from .bit_ops import pack_bits, unpack_bits

__all__ = ["lloyd_max_quantize", "lloyd_max_dequantize"]


def lloyd_max_quantize(rotated: torch.Tensor, boundaries: torch.Tensor, b_eff: int) -> torch.Tensor:
    """f32 [N, d] -> packed uint8 [N, ceil(d*b_eff/8)] (quantize.py:201-247, :299-339)."""
    if not 1 <= b_eff <= 8:
        raise AssertionError(f"b_eff must be between 1 and 8, got {b_eff}")
    if boundaries.shape[0] != (1 << b_eff) - 1:
        raise AssertionError(
            f"Expected {(1 << b_eff) - 1} boundaries for b_eff={b_eff}, got {boundaries.shape[0]}")
    rotated = rotated.to(torch.float32)
    boundaries = boundaries.to(torch.float32).contiguous()
    n, d = rotated.shape
    if rotated.device.type == "cuda":
        return ops().quantize_pack(rotated, boundaries, b_eff)
    codes = torch.searchsorted(boundaries, rotated.reshape(-1).contiguous()).reshape(n, d)
    return pack_bits(codes.to(torch.int32), b_eff)


def lloyd_max_dequantize(packed: torch.Tensor, centroids: torch.Tensor, b: int, d: int) -> torch.Tensor:
    """Packed codes -> f16 [N, d] centroid values (quantize.py:249-290, :341-369)."""
    if not 1 <= b <= 8:
        raise AssertionError(f"b must be between 1 and 8, got {b}")
    centroids = centroids.to(torch.float16).contiguous()
    n = packed.shape[0]
    if packed.device.type == "cuda":
        return ops().dequantize(packed, centroids, b, d)
    return centroids[unpack_bits(packed, b, d).long()]
