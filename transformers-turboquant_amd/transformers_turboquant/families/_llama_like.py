"""Shared body of the rotary-embedding, grouped-query families (llama, qwen2, deepseek).

The reference wrappers (families/llama.py:18-122, qwen2.py:18-125,
deepseek.py:22-125) read num_heads / num_key_value_heads / hidden_size from
the module and return three values; transformers 5.x modules carry neither
attribute and their decoder layers unpack two.  Here head counts come from the
module's config and forward returns (attn_output, attn_weights).
"""

from __future__ import annotations

import torch.nn as nn

from ..base import TurboQuantAttentionBase
from ._tail import attention_tail, move_compressors


class LlamaLikeAttention(TurboQuantAttentionBase):
    apply_rotary = None  # set by each family: transformers' apply_rotary_pos_emb

    @classmethod
    def from_original(cls, original: nn.Module, key_compressor, val_compressor):
        for attr in ("q_proj", "k_proj", "v_proj", "o_proj"):
            if not hasattr(original, attr):
                raise NotImplementedError(
                    f"{type(original).__name__} has no {attr}; only q/k/v/o-projection attention "
                    "is supported (multi-head latent attention is not)")
        cfg = getattr(original, "config", None)
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        obj.q_proj, obj.k_proj = original.q_proj, original.k_proj
        obj.v_proj, obj.o_proj = original.v_proj, original.o_proj
        obj.head_dim = original.head_dim
        obj.num_heads = getattr(original, "num_heads", None) or cfg.num_attention_heads
        obj.num_key_value_heads = (getattr(original, "num_key_value_heads", None)
                                   or getattr(cfg, "num_key_value_heads", None) or obj.num_heads)
        obj.num_key_value_groups = obj.num_heads // obj.num_key_value_heads
        obj.hidden_size = getattr(original, "hidden_size", None) or cfg.hidden_size
        obj.layer_idx = getattr(original, "layer_idx", None)
        obj.is_causal = getattr(original, "is_causal", True)
        obj.key_compressor = key_compressor
        obj.val_compressor = val_compressor
        obj.causal_mode = False
        return obj

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse=recurse)
        move_compressors(self, fn)
        return self

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                past_key_values=None, cache_position=None, output_attentions=False, **kwargs):
        B, T, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(B, T, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(B, T, self.num_key_value_heads, self.head_dim).transpose(1, 2)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            q, k = type(self).apply_rotary(q, k, cos, sin)
        attn, weights = attention_tail(self, q, k, v, attention_mask, output_attentions, cache=past_key_values)
        return self.o_proj(attn), weights
