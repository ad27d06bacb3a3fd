"""Bit packing of quantisation codes (reference: kernels/bit_ops.py).

Layout: code i of a row occupies bits [i*b, i*b + b), least-significant bit
first; bit k of the row is bit k%8 of byte k//8 (bit_ops.py:269-283).

GPU tensors go to the gfx950 library (``torch.ops.tq.pack_bits`` / ``unpack_bits`` over
``tq_pack_bits`` / ``tq_unpack_bits``);
CPU tensors use the vectorised torch formulation below.
"""

from __future__ import annotations

import math

import torch

from .._ops import ops

__all__ = ["pack_bits", "unpack_bits"]


def _out_cols(d: int, b: int) -> int:
    """Bytes holding d codes of b bits (bit_ops.py:162-164)."""
    return math.ceil(d * b / 8)


def _check_b(b: int) -> None:
    if not 1 <= b <= 8:
        raise AssertionError(f"b must be between 1 and 8, got {b}")


def _bits_to_bytes(bits: torch.Tensor, n_bytes: int) -> torch.Tensor:
    """[N, L] {0,1} -> uint8 [N, n_bytes], LSB-first."""
    n, length = bits.shape
    pad = n_bytes * 8 - length
    if pad:
        bits = torch.cat([bits, bits.new_zeros(n, pad)], dim=1)
    weights = (1 << torch.arange(8, dtype=torch.int32, device=bits.device))
    return (bits.view(n, n_bytes, 8).to(torch.int32) * weights).sum(-1).to(torch.uint8)


def _bytes_to_bits(packed: torch.Tensor, length: int) -> torch.Tensor:
    shifts = torch.arange(8, dtype=torch.int32, device=packed.device)
    bits = (packed.to(torch.int32).unsqueeze(-1) >> shifts) & 1
    return bits.reshape(packed.shape[0], -1)[:, :length]


def pack_bits(indices: torch.Tensor, b: int) -> torch.Tensor:
    """Pack int32 [N, d] codes into uint8 [N, ceil(d*b/8)] (bit_ops.py:173-204, :243-286)."""
    _check_b(b)
    if indices.dtype != torch.int32:
        indices = indices.to(torch.int32)
    n, d = indices.shape
    oc = _out_cols(d, b)
    if indices.device.type == "cuda":
        return ops().pack_bits(indices, b)
    shifts = torch.arange(b, dtype=torch.int32)
    bits = ((indices.unsqueeze(-1) >> shifts) & 1).reshape(n, d * b)
    return _bits_to_bytes(bits, oc)


def unpack_bits(packed: torch.Tensor, b: int, d: int) -> torch.Tensor:
    """uint8 [N, ceil(d*b/8)] -> int32 [N, d] (bit_ops.py:206-235, :288-326)."""
    _check_b(b)
    n = packed.shape[0]
    if packed.device.type == "cuda":
        return ops().unpack_bits(packed, b, d)
    bits = _bytes_to_bits(packed, d * b).view(n, d, b)
    weights = (1 << torch.arange(b, dtype=torch.int32))
    return (bits * weights).sum(-1).to(torch.int32)
