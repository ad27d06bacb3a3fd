"""MI355X-native TurboQuant KV-cache compression (gfx950 HIP kernels behind a C ABI).

Public objects keep the reference's names (src/turboquant_pytorch/__init__.py:3).
"""

from .compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
from .fused import compressed_attention

__all__ = ["TurboQuantCompressorV2", "TurboQuantCompressorMSE", "compressed_attention"]
