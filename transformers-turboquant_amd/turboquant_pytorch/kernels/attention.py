"""Asymmetric attention scores from packed keys (reference: kernels/attention.py).

    score(q, k) = vn_k <q_rot, C[codes_k]> + coeff * rn_k <S_eff q_rot, 2*sign_k - 1>

where q_rot = q Pi^T is the pre-rotated query and S_eff = S Pi^T, so that
<S_eff q_rot, .> = <S q, .> (attention.py:5-9, 424-461).
"""

from __future__ import annotations

import functools

import torch

from .._ops import ops
from ..codebook import split_f16
from .bit_ops import unpack_bits

__all__ = ["asymmetric_attention_scores"]


@functools.lru_cache(maxsize=None)
def _identity_split(d: int, device: str) -> torch.Tensor:
    return split_f16(torch.eye(d)).to(device)


def project_queries(q_rot: torch.Tensor, s_eff_f16: torch.Tensor) -> torch.Tensor:
    """f32 q_rot S_eff^T for f16 q_rot [B, H, S, d] on the GPU (attention.py:155-167, :453)."""
    d = q_rot.shape[-1]
    eye = _identity_split(d, str(q_rot.device))
    _, proj = ops().query_prep(q_rot.to(torch.float16), eye, s_eff_f16)
    return proj


def scores_from_prepared(q_rot16: torch.Tensor, q_proj32: torch.Tensor, codes: torch.Tensor,
                         signs: torch.Tensor, rn: torch.Tensor, vn: torch.Tensor,
                         centroids16: torch.Tensor, bits: int, coeff: float, hkv: int,
                         sk: int | None = None, kv_stride: int = 0) -> torch.Tensor:
    """Launch tq_attention_scores_kv.

    The key planes hold B*hkv head sequences of kv_stride rows each (kv_stride
    0: contiguous, B*hkv*Sk rows); the first sk rows of each are scored.
    """
    B = q_rot16.shape[0]
    Sk = rn.numel() // (B * hkv) if sk is None else int(sk)
    return ops().scores(q_rot16, q_proj32, codes, signs, rn, vn, centroids16, bits, hkv, Sk, int(kv_stride),
                        float(coeff))


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
        dev = query.device
        q16 = query.to(torch.float16).contiguous()
        s_eff = qjl_matrix.to(dev, torch.float16).contiguous()
        codes = packed_key_indices.to(dev).contiguous()
        signs = packed_qjl_signs.to(dev).contiguous()
        rn = residual_norms.to(dev, torch.float16).contiguous()
        vn = vec_norms.to(dev, torch.float16).contiguous()
        cent = centroids.to(dev, torch.float16)
        if cent.dim() == 1:
            cent = cent.unsqueeze(0).expand(H, -1)
        if m != d and signs.shape[-1] != (m + 7) // 8:
            raise ValueError(f"packed_qjl_signs hold {signs.shape[-1]} bytes per key; m={m} needs {(m + 7) // 8}")
        # the kernels take a sign plane of d bits against a q_proj of d values; a QJL matrix of
        # m != d rows is scored as ceil(m / d) blocks of d rows (the last one zero-padded: a zero
        # q_proj value adds nothing for any sign bit), the first block with the codebook and the
        # others with a zero codebook (their term 1 is exactly 0), summed in f32
        blocks = []
        for r0 in range(0, m, d):
            rows = min(d, m - r0)
            s_blk = s_eff[r0:r0 + rows]
            sg = signs if m == d else signs[..., r0 // 8:(r0 + rows + 7) // 8]
            if rows < d:
                s_blk = torch.nn.functional.pad(s_blk, (0, 0, 0, d - rows))
                # bits past row m of the last byte meet zero q_proj values
                sg = torch.nn.functional.pad(sg, (0, d // 8 - sg.shape[-1]))
            blocks.append((project_queries(q16, s_blk.contiguous()), sg.contiguous(), r0 == 0))

        def score(cent_row, sl):
            out = None
            for q_proj, sg, first in blocks:
                c = cent_row if first else torch.zeros_like(cent_row)
                sc = scores_from_prepared(q16[:, sl].contiguous(), q_proj[:, sl].contiguous(),
                                          codes[:, sl].contiguous(), sg[:, sl].contiguous(),
                                          rn[:, sl].contiguous(), vn[:, sl].contiguous(), c, b, coeff,
                                          sl.stop - sl.start)
                out = sc if out is None else out.add_(sc)
            return out

        if bool((cent == cent[:1]).all()):
            return score(cent[0].contiguous(), slice(0, H))
        # per-head codebooks: one launch per head
        return torch.cat([score(cent[h].contiguous(), slice(h, h + 1)) for h in range(H)], dim=1)

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
