"""Top-k block selection from per-query block scores (HIP, gfx950).

Mirrors flash_topk_attn_v2/topk_select.py (reference, :185-311): same
signature, validation and outputs.  One kernel serves every M <= 4096; the
``backend`` argument is accepted for API compatibility ("auto", "triton",
"cuda" all run the HIP kernel) and keeps the reference's argument errors.
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import _lib


def _next_power_of_2(x: int) -> int:
    if x <= 1:
        return 1
    return 1 << (x - 1).bit_length()


def flash_topk_select(
    block_scores: torch.Tensor,
    threshold: float,
    max_topk: int,
    score_block_size: int,
    padding: Tuple[int, int] = (0, 0),
    backend: str = "auto",
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Sort block scores by avg, cumsum raw scores, and truncate at threshold.

    Returns ``(topk_indices int32, topk_raw_scores f32, topk_avg_scores f32)``,
    each ``[B, H, N, M_OUT]`` with ``M_OUT = min(max_topk, M)`` (``M`` if
    ``max_topk == 0``).  Ties in the average score go to the lower block index;
    the cumulative sum is a sequential fp32 sum of ``avg * valid_count``.
    """
    if block_scores.ndim != 4:
        raise ValueError("block_scores must be [B, H, N, M]")
    if block_scores.device.type != "cuda":
        raise ValueError("flash_topk_select requires CUDA tensor")
    if block_scores.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("block_scores must be float16/bfloat16/float32")

    B, H, N, M = block_scores.shape
    if M <= 0:
        raise ValueError("M must be positive")
    if score_block_size <= 0:
        raise ValueError("score_block_size must be positive")

    pad_head, pad_tail = padding
    if pad_head < 0 or pad_tail < 0:
        raise ValueError("padding must be non-negative (pad_head, pad_tail)")
    if pad_head >= score_block_size or pad_tail >= score_block_size:
        raise ValueError(
            f"padding ({pad_head}, {pad_tail}) must each be < score_block_size "
            f"({score_block_size})"
        )
    if max_topk < 0:
        raise ValueError("max_topk must be >= 0")

    m_pad = _next_power_of_2(M)
    if backend == "triton":
        if m_pad > 512:
            raise ValueError(
                f"Triton backend requires M_PAD <= 512, got M={M} (M_PAD={m_pad})"
            )
    elif backend == "cuda":
        if M > 4096:
            raise NotImplementedError(f"CUDA backend requires M <= 4096, got M={M}")
    elif backend != "auto":
        raise ValueError(
            f"backend must be 'auto', 'triton', or 'cuda', got '{backend}'"
        )
    if M > 4096:
        raise NotImplementedError(f"M={M} exceeds block sort limit 4096")

    m_out = min(max_topk, M) if max_topk > 0 else M
    scores = block_scores if block_scores.dtype == torch.float32 else block_scores.float()
    rows = B * H * N
    if scores.stride(3) != 1 or scores.stride(2) * N != scores.stride(1) or scores.stride(1) * H != scores.stride(0):
        scores = scores.contiguous()
    idx = torch.empty(B, H, N, m_out, device=scores.device, dtype=torch.int32)
    raw = torch.empty(B, H, N, m_out, device=scores.device, dtype=torch.float32)
    avg = torch.empty(B, H, N, m_out, device=scores.device, dtype=torch.float32)
    rc = _lib.lib().fta_topk_select(
        _lib.ptr(scores), rows, M, scores.stride(2), scores.stride(3), max_topk, score_block_size,
        pad_head, pad_tail, float(threshold), _lib.ptr(idx), _lib.ptr(raw), _lib.ptr(avg),
        _lib.stream_ptr(scores.device),
    )
    _lib.check(rc, "flash_topk_select")
    return idx, raw, avg


__all__ = ["flash_topk_select"]
