"""LLaMA / Mistral family (reference: families/llama.py:18-122)."""

from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from ..registry import register_family
from ._llama_like import LlamaLikeAttention


@register_family("llama", "mistral")
class TurboQuantLlamaAttention(LlamaLikeAttention):
    ATTENTION_CLASS_NAMES = (
        "LlamaAttention", "LlamaSdpaAttention", "LlamaFlashAttention2",
        "MistralAttention", "MistralSdpaAttention", "MistralFlashAttention2",
    )
    apply_rotary = staticmethod(apply_rotary_pos_emb)
