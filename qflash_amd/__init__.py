"""qflash_amd - integer-only FlashAttention on MI355X (gfx950), drop-in for qflash.

Public API (same names as EfficientCompLab/qflash, qflash/__init__.py:1-4):
``qflash`` (``qflash.forward``, ``qflash.kernel``), ``QAttention``,
``QWindowAttention``, ``patch_attention``.
"""
from .kernel import qflash
from .attention import QAttention, QWindowAttention, patch_attention

__all__ = ["qflash", "QAttention", "QWindowAttention", "patch_attention"]
