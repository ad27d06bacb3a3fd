"""DeepSeek family (reference: families/deepseek.py:22-125).

DeepSeek-LLM checkpoints use model_type "llama" and take the llama family.
The native classes listed here must expose q/k/v/o projections; the
multi-head-latent-attention modules of V2/V3 do not and are refused.
"""

from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from ..registry import register_family
from ._llama_like import LlamaLikeAttention


@register_family("deepseek", "deepseek_v2", "deepseek_v3")
class TurboQuantDeepSeekAttention(LlamaLikeAttention):
    ATTENTION_CLASS_NAMES = (
        "DeepseekAttention", "DeepseekSdpaAttention", "DeepseekFlashAttention2",
        "DeepseekV2Attention", "DeepseekV3Attention",
    )
    apply_rotary = staticmethod(apply_rotary_pos_emb)
