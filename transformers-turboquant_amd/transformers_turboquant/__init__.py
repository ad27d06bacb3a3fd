"""HuggingFace integration of the MI355X TurboQuant path (reference: transformers_turboquant/__init__.py)."""

from . import families  # noqa: F401  (registers the built-in families)
from .cache import TurboQuantCache
from .patch import apply_turboquant

__version__ = "0.1.0"
__all__ = ["apply_turboquant", "TurboQuantCache"]
