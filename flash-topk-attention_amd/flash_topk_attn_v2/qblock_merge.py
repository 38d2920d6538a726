"""Q-block merge: aggregate per-query top-k into per-q-block top-k (HIP, gfx950).

Mirrors flash_topk_attn_v2/qblock_merge.py:85-155 (reference).  Unlike the
reference kernel (shared-memory float atomics), the scatter-add runs in a fixed
(query row, slot) order, so merged scores and indices are deterministic; ties
in the merged score go to the lower block index.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def flash_qblock_merge(
    topk_indices: torch.Tensor,
    topk_scores: torch.Tensor,
    q_block_size: int,
    qblock_topk: int,
    num_score_blocks: int,
    counts_out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Merge per-query top-k into per-q-block top-k via scatter-add + sort.

    Args:
        topk_indices: ``[B, H, N, M_out]`` int32, ``-1`` for padding.
        topk_scores: ``[B, H, N, M_out]`` float32 (avg scores).
        q_block_size: Number of queries per q-block.
        qblock_topk: Number of top blocks to keep per q-block.
        num_score_blocks: Total number of KV score blocks (M_total).
        counts_out: optional ``[B, H, QM]`` int32 tensor receiving the number of
            valid merged entries per q-block.

    Returns:
        ``merged_indices [B, H, QM, qblock_topk]`` int32 (``-1`` padding) and
        ``merged_scores [B, H, QM, qblock_topk]`` float32 (``0`` padding).
    """
    if topk_indices.ndim != 4:
        raise ValueError("topk_indices must be [B, H, N, M_out]")
    if topk_scores.ndim != 4:
        raise ValueError("topk_scores must be [B, H, N, M_out]")
    if topk_indices.device.type != "cuda":
        raise ValueError("flash_qblock_merge requires CUDA tensors")

    B, H, N, M_out = topk_indices.shape
    if N % q_block_size != 0:
        raise ValueError(
            f"N ({N}) must be divisible by q_block_size ({q_block_size})"
        )
    if num_score_blocks <= 0:
        raise ValueError("num_score_blocks must be positive")
    if num_score_blocks > 4096:
        raise NotImplementedError(
            f"num_score_blocks={num_score_blocks} exceeds CUDA block sort "
            f"limit 4096"
        )
    if qblock_topk <= 0:
        raise ValueError("qblock_topk must be positive")

    QM = N // q_block_size
    idx = topk_indices.to(torch.int32).contiguous()
    scr = topk_scores.float().contiguous()
    merged = torch.empty(B, H, QM, qblock_topk, device=idx.device, dtype=torch.int32)
    mscores = torch.empty(B, H, QM, qblock_topk, device=idx.device, dtype=torch.float32)
    rc = _lib.lib().fta_qblock_merge(
        _lib.ptr(idx), _lib.ptr(scr), B * H * QM, q_block_size, M_out, num_score_blocks, qblock_topk,
        _lib.ptr(merged), _lib.ptr(mscores), _lib.ptr(counts_out), _lib.stream_ptr(idx.device),
    )
    _lib.check(rc, "flash_qblock_merge")
    return merged, mscores


__all__ = ["flash_qblock_merge"]
