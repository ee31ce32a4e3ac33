"""MI355X-native Piper Attention and SageAttention2++ forward (gfx950 HIP kernels behind a C ABI).

Drop-in for the public operators of jumbledpoophj/piper-kernels
(``src/piper_kernels/__init__.py:3-6``): ``from piper_kernels import piper_attention,
sage_attention_2pp``.
"""

from .attention.piper_attention import piper_attention
from .attention.sage_attention_2pp import sage_attention_2pp

__all__ = ["piper_attention", "sage_attention_2pp"]
