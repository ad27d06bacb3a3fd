"""Abstract attention replacement (reference: transformers_turboquant/base.py:14-39)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import ClassVar

import torch.nn as nn

from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2


class TurboQuantAttentionBase(ABC, nn.Module):
    """Base class of every TurboQuant attention replacement.

    A family declares the HuggingFace attention class names it replaces in
    ATTENTION_CLASS_NAMES, builds itself from an original module in
    from_original(), and runs compressed attention in forward().
    """

    ATTENTION_CLASS_NAMES: ClassVar[tuple[str, ...]]

    @classmethod
    @abstractmethod
    def from_original(cls, original: nn.Module, key_compressor: TurboQuantCompressorV2,
                      val_compressor: TurboQuantCompressorMSE) -> "TurboQuantAttentionBase":
        """Take over the original module's projections and keep the compressors."""

    @abstractmethod
    def forward(self, hidden_states, **kwargs):
        """Compressed attention forward pass."""
