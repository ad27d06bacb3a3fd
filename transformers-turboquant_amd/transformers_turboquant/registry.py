"""model_type -> attention replacement class (reference: transformers_turboquant/registry.py)."""

from __future__ import annotations

from .base import TurboQuantAttentionBase

_REGISTRY: dict[str, type[TurboQuantAttentionBase]] = {}


class UnsupportedModelError(ValueError):
    """Raised when apply_turboquant meets a model_type with no registered family."""


def register_family(*model_types: str):
    """Class decorator registering an attention replacement for model_type strings
    (registry.py:12-25)::

        @register_family("llama", "mistral")
        class TurboQuantLlamaAttention(TurboQuantAttentionBase): ...
    """

    def decorator(cls: type[TurboQuantAttentionBase]) -> type[TurboQuantAttentionBase]:
        for name in model_types:
            _REGISTRY[name] = cls
        return cls

    return decorator


def get_attention_class(model_type: str) -> type[TurboQuantAttentionBase]:
    """Registered class for model_type; UnsupportedModelError otherwise (registry.py:28-38)."""
    cls = _REGISTRY.get(model_type)
    if cls is None:
        raise UnsupportedModelError(
            f"model_type={model_type!r} is not supported. Supported: {sorted(_REGISTRY)}. "
            f"To add support, implement TurboQuantAttentionBase in a new file and register it "
            f"with @register_family({model_type!r})."
        )
    return cls
