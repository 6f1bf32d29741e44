"""MI355X-native (gfx950) VMonarch attention hot path.

Public API identical to the reference package `video_monarch_attention` (its __init__.py:1-4):
VMonarchAttention, vmonarch_attention, flash_entropy_attention.
"""
from .kernel import flash_entropy_attention
from .vmonarch import VMonarchAttention, vmonarch_attention

__all__ = ["VMonarchAttention", "vmonarch_attention", "flash_entropy_attention"]
