"""Fused compressed-domain attention: the family forward tail in one HIP kernel.

Reference equivalent (families/qwen2.py:105-117; llama.py, deepseek.py and
gpt2.py repeat it):

    scores  = key_compressor.asymmetric_attention_scores(q, compress(k)) / sqrt(d)
    scores += attention_mask                      (if a mask is given)
    weights = softmax(scores.float())
    out     = weights @ val_compressor.decompress(compress(v))

Here the scores never reach memory: tq_attention_fwd streams the packed key and
value planes once per block of query rows, runs an online softmax in f32, and
accumulates P.V in the value compressor's rotated domain, applying Pi_v once
per output row.  Grouped-query attention is served without expanding K/V.
Few-query (decode) shapes take a split-K path whose partial results live in a
workspace that the op allocates from torch (tq_attention_workspace_size bytes), or
in the library's own scratch array (split_k="static").

A compressed dict may carry ``kv_stride``: its planes then hold ``kv_stride``
positions per (batch, kv head) of which the first ``shape[2]`` are attended
(the layout of :class:`transformers_turboquant.cache.TurboQuantCache`).
"""

from __future__ import annotations

import math

import torch

from ._ops import ops
from .compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2, _tables

__all__ = ["compressed_attention", "attention_from_prepared"]


def compressed_attention(queries: torch.Tensor, key_compressor: TurboQuantCompressorV2,
                         val_compressor: TurboQuantCompressorMSE, compressed_k: dict,
                         compressed_v: dict, attention_mask: torch.Tensor | None = None,
                         causal: bool = False, scale: float | None = None,
                         out_dtype: torch.dtype | None = None, split_k: bool | str = True) -> torch.Tensor:
    """Attention output [B, S_q, Hq, D] (heads already interleaved for o_proj).

    queries [B, Hq, S_q, D] (any strides with unit stride on D) on the GPU;
    compressed_k / compressed_v the packed dicts of [B, Hkv, S_k, D] keys and
    values; attention_mask an additive mask broadcastable to [B, Hq, S_q, S_k];
    causal drops keys j > i + S_k - S_q inside the kernel; split_k=False keeps
    few-query shapes on the tiled kernel instead of the split-K decode kernels, and
    split_k="static" runs the split-K kernels with their partials in the library's
    per-GPU scratch array (tq_attention_fwd_kv_noalloc: no allocation at all; calls
    that overlap on one GPU race).
    """
    if "packed_key_indices" not in compressed_k or "packed_indices" not in compressed_v:
        raise ValueError("compressed_attention needs the packed (GPU) formats")
    q_rot, q_proj = key_compressor.prepare_queries(queries)
    out_dtype = out_dtype or queries.dtype
    return attention_from_prepared(q_rot, q_proj, key_compressor, val_compressor, compressed_k,
                                   compressed_v, attention_mask, causal, scale, out_dtype, split_k)


def attention_from_prepared(q_rot: torch.Tensor, q_proj: torch.Tensor,
                            key_compressor: TurboQuantCompressorV2,
                            val_compressor: TurboQuantCompressorMSE, compressed_k: dict,
                            compressed_v: dict, attention_mask: torch.Tensor | None = None,
                            causal: bool = False, scale: float | None = None,
                            out_dtype: torch.dtype = torch.float32, split_k: bool | str = True) -> torch.Tensor:
    """The tq::attention op (tq_attention_fwd_kv) on queries already prepared by prepare_queries()."""
    B, Hq, Sq, D = q_rot.shape
    _, Hkv, Sk, _ = compressed_k["shape"]
    kv_stride = int(compressed_k.get("kv_stride", Sk))
    if int(compressed_v.get("kv_stride", Sk)) != kv_stride:
        raise ValueError("compressed key and value planes must share their kv_stride")
    dev = q_rot.device
    tk = _tables(key_compressor, dev, with_qjl=True)
    tv = _tables(val_compressor, dev, with_qjl=False)
    if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        out_dtype = torch.float32
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    coeff = math.sqrt(math.pi / 2) / key_compressor.S.shape[0]
    bits = key_compressor.mse_bits + 1
    mask = None
    if attention_mask is not None:
        mask = attention_mask.to(dev, torch.float32)
    mode = {"static": 2, True: 1, False: 0}[split_k]
    return ops().attention(
        q_rot, q_proj, compressed_k["packed_key_indices"], compressed_k["packed_qjl_signs"],
        compressed_k["residual_norm"], compressed_k["vec_norms"], tk.cent16, bits,
        compressed_v["packed_indices"], compressed_v["vec_norms"], tv.cent32, val_compressor.bits,
        tv.pit_split, Hkv, Sk, kv_stride, float(coeff), float(scale), bool(causal), mask, out_dtype, mode)
