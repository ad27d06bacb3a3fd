"""The compressed-attention tail shared by every family forward().

Reference steps (families/qwen2.py:100-117, gpt2.py:89-110): compress K and V,
estimate scores from compressed K, divide by sqrt(d), add the mask if given,
softmax in f32 cast to the model dtype, multiply by decompressed V.

On the GPU the tail is one tq_attention_fwd launch over Hkv compressed heads
(no repeat_interleave; query head h reads kv head h // G).  The materialised
path (HIP scores + HIP decompress, softmax/dropout in torch) is used only when
attention weights are requested or attention dropout is active.  On the CPU
the reference's own sequence runs on its unpacked format.

With a ``TurboQuantCache`` as the decoder's cache only the new tokens are
compressed (appended to the cache) and attention runs over every cached
position; any other transformers cache keeps the uncompressed K/V (its own
``update``), which are compressed whole on every step.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from turboquant_pytorch.fused import compressed_attention

from ..cache import TurboQuantCache


def additive_mask(mask: torch.Tensor | None, dtype=torch.float32) -> torch.Tensor | None:
    if mask is None:
        return None
    if mask.dtype == torch.bool:  # True = attend
        return torch.where(mask, torch.zeros((), dtype=dtype, device=mask.device),
                           torch.full((), torch.finfo(dtype).min, dtype=dtype, device=mask.device))
    return mask


def causal_mask(sq: int, sk: int, device, dtype=torch.float32) -> torch.Tensor:
    i = torch.arange(sq, device=device).unsqueeze(1) + (sk - sq)
    j = torch.arange(sk, device=device).unsqueeze(0)
    return torch.where(j <= i, torch.zeros((), dtype=dtype, device=device),
                       torch.full((), torch.finfo(dtype).min, dtype=dtype, device=device))


def want_causal(module, attention_mask) -> bool:
    """Causal masking inside the kernel: only with causal_mode "auto" and no mask passed."""
    mode = getattr(module, "causal_mode", False)
    return attention_mask is None and mode == "auto" and getattr(module, "is_causal", True)


def attention_tail(module, q, k, v, attention_mask, output_attentions: bool = False, dropout=None, cache=None):
    """q [B, Hq, T, D], k/v [B, Hkv, T_new, D] -> (attn [B, T, Hq*D] in q.dtype, weights or None).

    cache: the decoder's past_key_values (None without caching)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    group = Hq // Hkv
    mask = additive_mask(attention_mask)
    causal = want_causal(module, attention_mask)
    drop_active = dropout is not None and module.training and dropout.p > 0
    kc, vc = module.key_compressor, module.val_compressor

    fused = q.device.type == "cuda" and not output_attentions and not drop_active
    cached = None  # (compressed keys, compressed values) of every cached position
    if isinstance(cache, TurboQuantCache):
        if fused:
            # one operator call: one launch compresses the new keys / values into the cache and
            # prepares the queries, then the attention over every cached position
            out = cache.append_attend(module.layer_idx, kc, vc, k, v, q, attention_mask=mask, causal=causal,
                                      scale=1.0 / math.sqrt(D), out_dtype=q.dtype)
            return out.reshape(B, T, Hq * D), None
        cached = cache.append(module.layer_idx, kc, vc, k, v)
        lay = cache.layer(module.layer_idx)
    elif cache is not None:
        k, v = cache.update(k, v, module.layer_idx)
    S = cached[0]["shape"][2] if cached is not None else k.shape[2]

    if fused:
        ck, cv = kc.compress(k), vc.compress(v)
        out = compressed_attention(q, kc, vc, ck, cv, attention_mask=mask, causal=causal,
                                   scale=1.0 / math.sqrt(D), out_dtype=q.dtype)
        return out.reshape(B, T, Hq * D), None

    if q.device.type == "cuda":
        ck, cv = lay.compact() if cached is not None else (kc.compress(k), vc.compress(v))
        scores = kc.asymmetric_attention_scores(q, ck)
        values = vc.decompress(cv)
        if group > 1:
            values = values.repeat_interleave(group, dim=1)
    elif cached is not None:
        # unpacked CPU dicts of Hkv heads; per-row compression makes them equal to the
        # compression of the repeated heads
        scores = kc.asymmetric_attention_scores(q, cached[0])
        values = vc.decompress(cached[1])
        if group > 1:
            values = values.repeat_interleave(group, dim=1)
    else:
        if group > 1:
            k = k.repeat_interleave(group, dim=1)
            v = v.repeat_interleave(group, dim=1)
        scores = kc.asymmetric_attention_scores(q, kc.compress(k))
        values = vc.decompress(vc.compress(v))
    scores = scores / math.sqrt(D)
    if mask is not None:
        scores = scores + mask
    elif causal:
        scores = scores + causal_mask(T, S, scores.device)
    weights = F.softmax(scores.float(), dim=-1).to(q.dtype)
    if dropout is not None:
        weights = dropout(weights)
    out = torch.matmul(weights, values.to(q.dtype))
    return out.transpose(1, 2).reshape(B, T, Hq * D), (weights if output_attentions else None)


def move_compressors(module, fn):
    """Apply a Module._apply move to the compressors' tensors, keeping their f32 dtype."""
    for comp in (module.key_compressor, module.val_compressor):
        for attr in ("Pi", "PiT", "S", "centroids", "boundaries"):
            t = getattr(comp, attr, None)
            if t is None:
                continue
            dev = fn(torch.empty(0, device=t.device)).device
            setattr(comp, attr, t.to(dev))
        comp.device = str(comp.Pi.device)
