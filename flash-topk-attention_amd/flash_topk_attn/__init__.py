"""MI355X (gfx950) V1 compatibility layer of flash-topk-attention.

Drop-in for the reference's V1 package ``flash_topk_attn``
(flash_topk_attn/__init__.py:1-4): ``flash_topk_score`` (top-k block scoring,
optionally with the dense attention output and its backward),
``build_qblock_topk_indices`` (exact per-q-block union) and
``flash_topk_attn`` (attention over the union).  Every kernel is the HIP code
of ``flash_topk_attn_v2`` (libfta_gfx950.so): scoring and selection, the union
builder, and the block-sparse attention forward and backward, which with every
block selected is dense attention.
"""

from .attention import build_qblock_topk_indices, flash_topk_attn
from .scoring import FlashPureScoringFunction, FlashScoringFunction, flash_topk_score

__all__ = [
    "flash_topk_score",
    "flash_topk_attn",
    "build_qblock_topk_indices",
    "FlashScoringFunction",
    "FlashPureScoringFunction",
]
