"""MI355X (gfx950) GQA flash-attention forward.

Drop-in for reference gqa_kernels/__init__.py:1-4: same import path and the
same public function, ``gqa_flash_attn(q, k, v, causal=True)``.
"""
from .dispatch import gqa_flash_attn

__all__ = ["gqa_flash_attn"]
__version__ = "0.1.0"
