"""TurboQuant KV compressors (reference: src/turboquant_pytorch/compressors.py).

Keys: <q, k> ~ <q, k_mse> + ||r_k|| sqrt(pi/2)/m <S q, sign(S r_k)>, with
k_mse the Lloyd-Max reconstruction of the rotated key and r_k its residual.
Values: MSE-only Lloyd-Max codes of the rotated vector.

Tensors on a GPU are compressed by the gfx950 library into the reference's
packed format (``packed_key_indices``/``packed_qjl_signs``/``residual_norm``/
``vec_norms`` for keys, ``packed_indices``/``vec_norms`` for values).  Tensors on
the CPU get the reference's unpacked format (``k_mse``/``qjl_signs``/
``residual_norm`` and ``indices``/``vec_norms``).  The compressed dict is opaque
to callers; the methods dispatch on its keys (compressors.py:178, :301).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from ._ops import ops
from .codebook import codebook, gaussian_matrix, midpoints, random_rotation, split_f16
from .kernels.attention import scores_from_prepared

__all__ = ["TurboQuantCompressorV2", "TurboQuantCompressorMSE"]


@dataclass
class _DeviceTables:
    """Per-device operands of the HIP kernels, derived from the compressor's tensors."""
    key: tuple
    pi_split: torch.Tensor            # f16 [2, d, d]  split of Pi
    pit_split: torch.Tensor           # f16 [2, d, d]  split of Pi^T
    seff_split: torch.Tensor | None   # f16 [2, d, d]  split of the f32 S_eff = S Pi^T (keys)
    s_eff16: torch.Tensor | None      # f16 [d, d]     f16(S Pi^T) (keys)
    cent32: torch.Tensor              # f32 [2^b]
    cent16: torch.Tensor              # f16 [2^b]
    bounds32: torch.Tensor            # f32 [2^b - 1]


def _tables(comp, device: torch.device, with_qjl: bool) -> _DeviceTables:
    s = getattr(comp, "S", None) if with_qjl else None
    key = (str(device), id(comp.Pi), id(s), id(comp.centroids), id(comp.boundaries))
    cached = getattr(comp, "_dev_tables", None)
    if cached is not None and cached.key == key:
        return cached
    pi = comp.Pi.detach().to("cpu", torch.float32)
    cent = comp.centroids.detach().to("cpu", torch.float32)
    bounds = comp.boundaries.detach().to("cpu", torch.float32)
    seff_split = s_eff = None
    if s is not None:
        s32 = s.detach().to("cpu", torch.float32)
        s_eff32 = s32 @ pi.T  # compressors.py:189 forms S_eff as this f32 product
        seff_split = split_f16(s_eff32).to(device)
        s_eff = s_eff32.to(torch.float16).contiguous().to(device)
    t = _DeviceTables(
        key=key,
        pi_split=split_f16(pi).to(device),
        pit_split=split_f16(pi.T.contiguous()).to(device),
        seff_split=seff_split,
        s_eff16=s_eff,
        cent32=cent.contiguous().to(device),
        cent16=cent.to(torch.float16).contiguous().to(device),
        bounds32=bounds.contiguous().to(device),
    )
    comp._dev_tables = t
    return t


class TurboQuantCompressorV2:
    """Key compressor with the asymmetric (MSE + QJL) inner-product estimator.

    Attributes as in the reference (compressors.py:42-70): ``head_dim``,
    ``bits``, ``mse_bits = max(bits - 1, 1)``, ``device``, ``use_triton``,
    ``Pi`` (seeded Haar rotation), ``centroids`` / ``boundaries`` (Lloyd-Max,
    mse_bits), ``S`` (N(0,1) QJL matrix from seed + 10000), ``PiT``.
    ``use_triton`` is kept for API compatibility: GPU tensors always take the
    HIP kernels.
    """

    def __init__(self, head_dim: int, bits: int, seed: int, device: str = "cpu", use_triton: bool = True):
        self.head_dim = head_dim
        self.bits = bits
        self.seed = seed
        self.mse_bits = max(bits - 1, 1)
        self.device = device
        self.use_triton = use_triton
        self.Pi = random_rotation(head_dim, seed).to(device)
        cent = codebook(head_dim, self.mse_bits)
        self.centroids = cent.to(device)
        self.boundaries = midpoints(cent).to(device)
        self.S = gaussian_matrix(head_dim, seed + 10000).to(device)
        self.PiT = self.Pi.T.contiguous()

    # ------------------------------------------------------------------ compress
    @torch.no_grad()
    def compress(self, states: torch.Tensor) -> dict:
        """[B, H, S, D] -> compressed dict (compressors.py:99-161)."""
        B, H, S, D = states.shape
        if states.device.type == "cuda":
            return self._compress_gpu(states)
        return self._compress_cpu(states)

    def _compress_gpu(self, states: torch.Tensor, y_out=None, proj_out=None) -> dict:
        B, H, S, D = states.shape
        t = _tables(self, states.device, with_qjl=True)
        codes, signs, rn, vn = ops().compress_keys(states, t.pi_split, t.seff_split, t.cent32, t.bounds32,
                                                   self.mse_bits, y_out, proj_out)
        return {
            "packed_key_indices": codes,
            "packed_qjl_signs": signs,
            "residual_norm": rn,
            "vec_norms": vn,
            "shape": (B, H, S, D),
        }

    def _compress_cpu(self, states: torch.Tensor) -> dict:
        # reference PyTorch branch, compressors.py:104-112, :139-161
        B, H, S, D = states.shape
        x = states.reshape(-1, D).float()
        norms = torch.norm(x, dim=-1, keepdim=True)
        y = (x / (norms + 1e-8)) @ self.Pi.float().T
        cent = self.centroids.float()
        idx = (y.unsqueeze(-1) - cent).abs().argmin(dim=-1)
        k_mse = (cent[idx] @ self.Pi.float()) * norms
        resid = x - k_mse
        signs = torch.where(resid @ self.S.float().T >= 0, 1, -1).to(torch.int8)
        return {
            "k_mse": k_mse.to(torch.float16).reshape(B, H, S, D),
            "qjl_signs": signs.reshape(B, H, S, D),
            "residual_norm": torch.norm(resid, dim=-1).to(torch.float16).reshape(B, H, S),
            "shape": (B, H, S, D),
        }

    # ------------------------------------------------------------------ scores
    @torch.no_grad()
    def asymmetric_attention_scores(self, queries: torch.Tensor, compressed: dict) -> torch.Tensor:
        """<Q, K> from compressed K: f32 [B, Hq, S_q, S_k] (compressors.py:164-224).

        Hq may be a multiple of the compressed head count (grouped-query
        attention): query head h reads compressed head h // (Hq / Hkv).
        """
        B, Hq, Sq, D = queries.shape
        _, Hk, Sk, _ = compressed["shape"]
        if "packed_key_indices" in compressed:
            if queries.device.type != "cuda":
                raise ValueError("packed key planes live on the GPU; pass GPU queries")
            if Hq % Hk:
                raise ValueError(f"query heads {Hq} not a multiple of compressed heads {Hk}")
            q_rot, q_proj = self.prepare_queries(queries)
            t = _tables(self, queries.device, with_qjl=True)
            coeff = math.sqrt(math.pi / 2) / self.S.shape[0]
            return scores_from_prepared(
                q_rot, q_proj, compressed["packed_key_indices"], compressed["packed_qjl_signs"],
                compressed["residual_norm"], compressed["vec_norms"], t.cent16, self.mse_bits + 1,
                coeff, Hk, Sk, int(compressed.get("kv_stride", Sk)))
        # reference PyTorch branch (compressors.py:201-224)
        k_mse = compressed["k_mse"].float()
        signs = compressed["qjl_signs"].float()
        rnorm = compressed["residual_norm"].float()
        if Hq != Hk:
            g = Hq // Hk
            k_mse = k_mse.repeat_interleave(g, dim=1)
            signs = signs.repeat_interleave(g, dim=1)
            rnorm = rnorm.repeat_interleave(g, dim=1)
        q = queries.float()
        m = self.S.shape[0]
        term1 = torch.matmul(q, k_mse.transpose(-2, -1))
        qjl = torch.matmul(torch.matmul(q, self.S.float().T), signs.transpose(-2, -1))
        return term1 + (math.sqrt(math.pi / 2) / m) * qjl * rnorm.unsqueeze(-2)

    def prepare_queries(self, queries: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """GPU q_rot = f16(q Pi^T) (f16 [B, Hq, S_q, D]) and q_proj = q_rot S_eff^T (f32, the
        reference's fp32 projection, kernels/attention.py:158-167, :453)."""
        t = _tables(self, queries.device, with_qjl=True)
        return ops().query_prep(queries, t.pi_split, t.s_eff16)


class TurboQuantCompressorMSE:
    """Value compressor: MSE-only Lloyd-Max codes of the rotated vector.

    Attributes as in the reference (compressors.py:230-246): ``head_dim``,
    ``bits``, ``device``, ``use_triton``, ``Pi``, ``centroids``, ``boundaries``.
    """

    def __init__(self, head_dim: int, bits: int, seed: int, device: str = "cpu", use_triton: bool = True):
        self.head_dim = head_dim
        self.bits = bits
        self.seed = seed
        self.device = device
        self.use_triton = use_triton
        self.Pi = random_rotation(head_dim, seed).to(device)
        cent = codebook(head_dim, bits)
        self.centroids = cent.to(device)
        self.boundaries = midpoints(cent).to(device)

    @torch.no_grad()
    def compress(self, states: torch.Tensor) -> dict:
        """[B, H, S, D] -> compressed dict (compressors.py:271-294)."""
        B, H, S, D = states.shape
        if states.device.type == "cuda":
            return self._compress_gpu(states)
        x = states.reshape(-1, D).float()
        norms = torch.norm(x, dim=-1, keepdim=True)
        y = (x / (norms + 1e-8)) @ self.Pi.float().T
        idx = (y.unsqueeze(-1) - self.centroids.float()).abs().argmin(dim=-1).to(torch.uint8)
        return {"indices": idx, "vec_norms": norms.squeeze(-1).to(torch.float16), "shape": (B, H, S, D)}

    def _compress_gpu(self, states: torch.Tensor, y_out=None) -> dict:
        B, H, S, D = states.shape
        t = _tables(self, states.device, with_qjl=False)
        codes, vn = ops().compress_values(states, t.pi_split, t.bounds32, self.bits, y_out)
        return {"packed_indices": codes, "vec_norms": vn, "shape": (B, H, S, D)}

    @torch.no_grad()
    def decompress(self, compressed: dict) -> torch.Tensor:
        """Compressed dict -> f32 [B, H, S, D] = (C[codes] Pi) * vn (compressors.py:297-317)."""
        B, H, S, D = compressed["shape"]
        n = B * H * S
        if "packed_indices" in compressed:
            packed = compressed["packed_indices"]
            if packed.device.type != "cuda":
                raise ValueError("packed value planes live on the GPU")
            t = _tables(self, packed.device, with_qjl=False)
            return ops().decompress_values(packed, compressed["vec_norms"], t.pit_split, t.cent32, self.bits,
                                           [B, H, S, D])
        idx = compressed["indices"].long()
        rec = self.centroids.float()[idx] @ self.Pi.float()
        return (rec * compressed["vec_norms"].float().unsqueeze(-1)).reshape(B, H, S, D)
