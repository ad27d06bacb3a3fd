"""apply_turboquant: swap a model's attention modules (reference: transformers_turboquant/patch.py)."""

from __future__ import annotations

from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

from .registry import get_attention_class


def _head_dim(module, config) -> int:
    hd = getattr(module, "head_dim", None)
    if hd is not None:
        return int(hd)
    hidden = getattr(config, "hidden_size", getattr(config, "n_embd", None))
    heads = getattr(config, "num_attention_heads", getattr(config, "n_head", None))
    return hidden // heads


def apply_turboquant(model, bits: int = 3, seed: int = 42, use_triton: bool = True, causal=False):
    """Replace every attention module of *model* with its TurboQuant family (patch.py:13-82).

    Layer i (in ``named_modules()`` order) gets key seed ``seed + i`` and value
    seed ``seed + i + 10000``.  The model is changed in place, its
    ``config.use_cache`` is set to False (every forward recomputes the full
    sequence from compressed K/V), and the same object is returned.

    causal: False (default) reproduces the reference: the attention mask is
    added only when the decoder passes one (families/gpt2.py:99-101), so a
    decoder that passes none (transformers 5.x under SDPA without padding)
    attends to every position, as the reference does.  "auto" applies the
    module's own causal masking inside the kernel whenever no mask is passed.
    """
    family = get_attention_class(model.config.model_type)
    device = str(next(model.parameters()).device)
    i = 0
    for _, parent in list(model.named_modules()):
        for name, child in list(parent.named_children()):
            if type(child).__name__ not in family.ATTENTION_CLASS_NAMES:
                continue
            d = _head_dim(child, model.config)
            kc = TurboQuantCompressorV2(d, bits, seed=seed + i, device=device, use_triton=use_triton)
            vc = TurboQuantCompressorMSE(d, bits, seed=seed + i + 10000, device=device, use_triton=use_triton)
            new = family.from_original(child, kc, vc)
            new.causal_mode = causal
            setattr(parent, name, new)
            i += 1
    model.config.use_cache = False
    return model
