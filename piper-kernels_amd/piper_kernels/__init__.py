"""MI355X-native Piper Attention forward (gfx950 HIP kernels behind a C ABI).

Drop-in for the public operator of jumbledpoophj/piper-kernels
(``src/piper_kernels/__init__.py:3-6``): ``from piper_kernels import piper_attention``.
"""

from .attention.piper_attention import piper_attention

__all__ = ["piper_attention"]
