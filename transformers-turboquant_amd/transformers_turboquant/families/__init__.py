"""Built-in attention families; importing registers them (reference: families/__init__.py:3)."""

from . import deepseek, gpt2, llama, qwen2  # noqa: F401
