"""SageAttention2++ on MI355X."""

from .dispatch import sage_attention_2pp

__all__ = ["sage_attention_2pp"]
