"""Qwen2 family (reference: families/qwen2.py:18-125)."""

from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

from ..registry import register_family
from ._llama_like import LlamaLikeAttention


@register_family("qwen2")
class TurboQuantQwen2Attention(LlamaLikeAttention):
    ATTENTION_CLASS_NAMES = ("Qwen2Attention", "Qwen2SdpaAttention", "Qwen2FlashAttention2")
    apply_rotary = staticmethod(apply_rotary_pos_emb)
