"""Asymmetric attention scores from packed keys (reference: kernels/attention.py).

    score(q, k) = vn_k <q_rot, C[codes_k]> + coeff * rn_k <S_eff q_rot, 2*sign_k - 1>

where q_rot = q Pi^T is the pre-rotated query and S_eff = S Pi^T, so that
<S_eff q_rot, .> = <S q, .> (attention.py:5-9, 424-461).
"""

from __future__ import annotations

import functools

import torch

from .. import _native
from ..codebook import split_f16
from .bit_ops import unpack_bits

__all__ = ["asymmetric_attention_scores"]


@functools.lru_cache(maxsize=None)
def _identity_split(d: int, device: str) -> torch.Tensor:
    return split_f16(torch.eye(d)).to(device)


def project_queries(q_rot: torch.Tensor, s_eff_f16: torch.Tensor) -> torch.Tensor:
    """f32 q_rot S_eff^T for f16 q_rot [B, H, S, d] on the GPU (attention.py:155-167, :453)."""
    B, H, S, d = q_rot.shape
    q_rot = q_rot.to(torch.float16)
    if q_rot.stride(-1) != 1:
        q_rot = q_rot.contiguous()
    rot_copy = torch.empty(B, H, S, d, dtype=torch.float16, device=q_rot.device)
    proj = torch.empty(B, H, S, d, dtype=torch.float32, device=q_rot.device)
    eye = _identity_split(d, str(q_rot.device))
    _native.check(_native.lib().tq_query_prep(
        q_rot.data_ptr(), _native.TQ_F16, B, H, S, d, q_rot.stride(0), q_rot.stride(1),
        q_rot.stride(2), eye.data_ptr(), s_eff_f16.data_ptr(), rot_copy.data_ptr(),
        proj.data_ptr(), _native.stream_of(q_rot)), "project_queries")
    return proj


def scores_from_prepared(q_rot16: torch.Tensor, q_proj32: torch.Tensor, codes: torch.Tensor,
                         signs: torch.Tensor, rn: torch.Tensor, vn: torch.Tensor,
                         centroids16: torch.Tensor, bits: int, coeff: float, hkv: int,
                         sk: int | None = None, kv_stride: int = 0) -> torch.Tensor:
    """Launch tq_attention_scores_kv.

    The key planes hold B*hkv head sequences of kv_stride rows each (kv_stride
    0: contiguous, B*hkv*Sk rows); the first sk rows of each are scored.
    """
    B, Hq, Sq, d = q_rot16.shape
    Sk = rn.numel() // (B * hkv) if sk is None else int(sk)
    out = torch.empty(B, Hq, Sq, Sk, dtype=torch.float32, device=q_rot16.device)
    _native.check(_native.lib().tq_attention_scores_kv(
        q_rot16.data_ptr(), q_proj32.data_ptr(), codes.data_ptr(), signs.data_ptr(),
        rn.data_ptr(), vn.data_ptr(), centroids16.data_ptr(), B, Hq, hkv, Sq, Sk, int(kv_stride), d,
        bits, float(coeff), out.data_ptr(), _native.stream_of(out)), "asymmetric_attention_scores")
    return out


def asymmetric_attention_scores(query: torch.Tensor, packed_key_indices: torch.Tensor,
                                packed_qjl_signs: torch.Tensor, residual_norms: torch.Tensor,
                                centroids: torch.Tensor, qjl_matrix: torch.Tensor,
                                vec_norms: torch.Tensor, b: int, coeff: float) -> torch.Tensor:
    """f32 [B, H, S_q, S_k] scores (attention.py:274-372 kernel path, :380-461 fallback).

    query: f16 [B, H, S_q, d], pre-rotated; packed_key_indices uint8
    [B, H, S_k, ceil(d*(b-1)/8)]; packed_qjl_signs uint8 [B, H, S_k, ceil(m/8)];
    residual_norms / vec_norms f16 [B, H, S_k]; centroids f16 [H, 2^(b-1)];
    qjl_matrix the effective QJL matrix S_eff f16 [m, d]; b total bits.
    """
    B, H, Sq, d = query.shape
    Sk = packed_key_indices.shape[2]
    m = qjl_matrix.shape[0]
    b_eff = b - 1
    if query.device.type == "cuda":
        if m != d:
            raise ValueError(f"GPU scores need a square QJL matrix (m == d); got m={m}, d={d}")
        dev = query.device
        q16 = query.to(torch.float16).contiguous()
        s_eff = qjl_matrix.to(dev, torch.float16).contiguous()
        q_proj = project_queries(q16, s_eff)
        codes = packed_key_indices.to(dev).contiguous()
        signs = packed_qjl_signs.to(dev).contiguous()
        rn = residual_norms.to(dev, torch.float16).contiguous()
        vn = vec_norms.to(dev, torch.float16).contiguous()
        cent = centroids.to(dev, torch.float16)
        if cent.dim() == 1:
            cent = cent.unsqueeze(0).expand(H, -1)
        if bool((cent == cent[:1]).all()):
            return scores_from_prepared(q16, q_proj, codes, signs, rn, vn, cent[0].contiguous(), b,
                                        coeff, H)
        # per-head codebooks: one launch per head
        outs = [scores_from_prepared(q16[:, h:h + 1].contiguous(), q_proj[:, h:h + 1].contiguous(),
                                     codes[:, h:h + 1].contiguous(), signs[:, h:h + 1].contiguous(),
                                     rn[:, h:h + 1].contiguous(), vn[:, h:h + 1].contiguous(),
                                     cent[h].contiguous(), b, coeff, 1) for h in range(H)]
        return torch.cat(outs, dim=1)

    # CPU tensors: the same estimator in f32 from the f16 inputs
    idx = unpack_bits(packed_key_indices.reshape(B * H * Sk, -1), b_eff, d).reshape(B, H, Sk, d)
    cent = centroids.float()
    if cent.dim() == 1:
        cent = cent.unsqueeze(0).expand(H, -1)
    heads = torch.arange(H).view(1, H, 1, 1)
    k_rot = cent[heads, idx.long()]
    q = query.float()
    t1 = torch.matmul(q, k_rot.transpose(-2, -1)) * vec_norms.float().unsqueeze(-2)
    bits = unpack_bits(packed_qjl_signs.reshape(B * H * Sk, -1), 1, m).reshape(B, H, Sk, m)
    pm = bits.float() * 2.0 - 1.0
    qp = torch.matmul(q, qjl_matrix.float().T)
    t2 = torch.matmul(qp, pm.transpose(-2, -1)) * (coeff * residual_norms.float().unsqueeze(-2))
    return t1 + t2
