"""Lloyd-Max quantise/dequantise of rotated coordinates (reference: kernels/quantize.py).

The code of a coordinate y is #{j : boundaries[j] < y}, i.e.
``torch.searchsorted(boundaries, y)`` (side='left'), the rule of the
reference's packed fallback (quantize.py:334-337).
"""

from __future__ import annotations

import torch

from .. import _native
from .bit_ops import _out_cols, pack_bits, unpack_bits

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
        rotated = rotated.contiguous()
        boundaries = boundaries.to(rotated.device)
        oc = _out_cols(d, b_eff)
        out = torch.empty(n, oc, dtype=torch.uint8, device=rotated.device)
        _native.check(_native.lib().tq_quantize_pack(
            rotated.data_ptr(), n, d, d, boundaries.data_ptr(), b_eff, out.data_ptr(), oc,
            _native.stream_of(out)), "lloyd_max_quantize")
        return out
    codes = torch.searchsorted(boundaries, rotated.reshape(-1).contiguous()).reshape(n, d)
    return pack_bits(codes.to(torch.int32), b_eff)


def lloyd_max_dequantize(packed: torch.Tensor, centroids: torch.Tensor, b: int, d: int) -> torch.Tensor:
    """Packed codes -> f16 [N, d] centroid values (quantize.py:249-290, :341-369)."""
    if not 1 <= b <= 8:
        raise AssertionError(f"b must be between 1 and 8, got {b}")
    centroids = centroids.to(torch.float16).contiguous()
    n = packed.shape[0]
    if packed.device.type == "cuda":
        packed = packed.contiguous()
        centroids = centroids.to(packed.device)
        out = torch.empty(n, d, dtype=torch.float16, device=packed.device)
        _native.check(_native.lib().tq_dequantize(
            packed.data_ptr(), n, d, packed.shape[1], centroids.data_ptr(), b, out.data_ptr(), d,
            _native.stream_of(out)), "lloyd_max_dequantize")
        return out
    return centroids[unpack_bits(packed, b, d).long()]
