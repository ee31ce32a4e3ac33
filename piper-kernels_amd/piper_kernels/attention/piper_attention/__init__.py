"""Piper Attention on MI355X."""

from .dispatch import piper_attention

__all__ = ["piper_attention"]
