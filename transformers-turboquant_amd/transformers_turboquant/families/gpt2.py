"""GPT-2 family (reference: families/gpt2.py:17-119)."""

from __future__ import annotations

import torch.nn as nn

from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

from ..base import TurboQuantAttentionBase
from ..registry import register_family
from ._tail import attention_tail, move_compressors


@register_family("gpt2")
class TurboQuantGPT2Attention(TurboQuantAttentionBase):
    """Replacement for GPT2Attention: fused c_attn projection, compressed K/V."""

    ATTENTION_CLASS_NAMES = ("GPT2Attention",)

    @classmethod
    def from_original(cls, original: nn.Module, key_compressor: TurboQuantCompressorV2,
                      val_compressor: TurboQuantCompressorMSE) -> "TurboQuantGPT2Attention":
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        obj.c_attn = original.c_attn
        obj.c_proj = original.c_proj
        obj.attn_dropout = original.attn_dropout
        obj.resid_dropout = original.resid_dropout
        obj.embed_dim = original.embed_dim
        obj.num_heads = original.num_heads
        obj.head_dim = original.head_dim
        obj.is_causal = getattr(original, "is_causal", True)
        obj.layer_idx = getattr(original, "layer_idx", None)
        obj.key_compressor = key_compressor
        obj.val_compressor = val_compressor
        obj.causal_mode = False
        return obj

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse=recurse)
        move_compressors(self, fn)
        return self

    def forward(self, hidden_states, past_key_values=None, attention_mask=None, head_mask=None,
                encoder_hidden_states=None, encoder_attention_mask=None, use_cache=False,
                output_attentions=False, **kwargs):
        B, T, _ = hidden_states.shape
        q, k, v = self.c_attn(hidden_states).split(self.embed_dim, dim=2)
        q = q.view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        k = k.view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        v = v.view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        attn, weights = attention_tail(self, q, k, v, attention_mask, output_attentions,
                                       dropout=self.attn_dropout, cache=past_key_values)
        attn = self.resid_dropout(self.c_proj(attn))
        return attn, weights
