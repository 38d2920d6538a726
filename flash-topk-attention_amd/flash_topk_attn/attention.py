"""V1 q-block union and attention (reference: flash_topk_attn/attention.py).

``build_qblock_topk_indices`` is the exact union of the per-query top-k block
ids of each q-block, sorted ascending (attention.py:23-138), built by the HIP
kernel ``fta_qblock_union``.  ``flash_topk_attn`` (attention.py:423-568) is
attention of every query of a q-block over the tokens of its union; it runs
on the block-sparse attention kernels of the V2 path, which treat the merged
ids as a set (ids past ``counts`` are masked to -1 first), so the output is
also differentiable in q, k and v.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from flash_topk_attn_v2 import _lib
from flash_topk_attn_v2.sparse_attn import flash_sparse_attn

_UNION_MAX = 8192  # largest q_block_size * K row the union kernel holds in LDS
_MAX_SUB_QBLOCK = 64  # largest q-block of the sparse attention kernels


def _next_power_of_2(x: int) -> int:
    if x <= 0:
        return 1
    return 1 << (x - 1).bit_length()


def build_qblock_topk_indices(
    topk_indices: torch.Tensor,
    q_block_size: int,
    q_padding: Tuple[int, int] = (0, 0),
) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """Sorted unique block ids per q-block (flash_topk_attn/attention.py:70-138).

    Args:
        topk_indices: ``[B, H, N, KQ]`` int32 or int64; ``-1`` marks empty slots.
        q_block_size: queries per q-block.
        q_padding: virtual ``(q_pad_head, q_pad_tail)``.

    Returns:
        ``merged_indices [B, H, QM, S_MAX]`` int32 (ascending ids, then -1),
        ``counts [B, H, QM]`` int32 and ``S_MAX = next_pow2(q_block_size * KQ)``.
    """
    B, H, N, KQ = topk_indices.shape
    q_pad_head, q_pad_tail = q_padding
    if q_pad_head >= q_block_size:
        raise ValueError(
            f"q_pad_head={q_pad_head} must be < q_block_size={q_block_size}; "
            "virtual padding should only complete partial blocks, not create new ones."
        )
    if q_pad_tail >= q_block_size:
        raise ValueError(
            f"q_pad_tail={q_pad_tail} must be < q_block_size={q_block_size}; "
            "virtual padding should only complete partial blocks, not create new ones."
        )
    if q_pad_head < 0 or q_pad_tail < 0:
        raise ValueError("q_padding must be non-negative")
    n_q_padded = q_pad_head + N + q_pad_tail
    if n_q_padded % q_block_size != 0:
        raise AssertionError(f"N_Q_PADDED={n_q_padded} must be divisible by q_block_size={q_block_size}")
    QM = n_q_padded // q_block_size
    s_max = _next_power_of_2(q_block_size * KQ)
    if s_max > _UNION_MAX:
        raise NotImplementedError(f"q_block_size * KQ = {q_block_size * KQ} exceeds the union limit {_UNION_MAX}")
    device = topk_indices.device
    merged = torch.empty(B, H, QM, s_max, device=device, dtype=torch.int32)
    counts = torch.empty(B, H, QM, device=device, dtype=torch.int32)
    if merged.numel() == 0:
        return merged, counts, s_max
    if device.type != "cuda":
        raise ValueError("build_qblock_topk_indices requires CUDA tensors")
    ids = topk_indices.to(torch.int32).contiguous()
    rc = _lib.lib().fta_qblock_union(
        _lib.ptr(ids), B * H, N, KQ, q_block_size, q_pad_head, q_pad_tail, s_max,
        _lib.ptr(merged), _lib.ptr(counts), _lib.stream_ptr(device),
    )
    _lib.check(rc, "build_qblock_topk_indices")
    return merged, counts, s_max


def _split_qblocks(merged, q_block_size, q_pad_head, N):
    """Re-express q-blocks larger than the kernels' 64 as sub-blocks of
    ``gs`` (the largest divisor of q_block_size <= 64) that share their parent's
    merged row; sub-blocks wholly inside the head padding are dropped."""
    gs = max(d for d in range(1, _MAX_SUB_QBLOCK + 1) if q_block_size % d == 0)
    r = q_block_size // gs
    a, ph = divmod(q_pad_head, gs)
    n_sub = (ph + N + gs - 1) // gs
    parent = (torch.arange(n_sub, device=merged.device) + a) // r
    return merged.index_select(2, parent).contiguous(), gs, (ph, n_sub * gs - ph - N)


def flash_topk_attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    merged_indices: torch.Tensor,
    counts: torch.Tensor,
    num_heads: int,
    q_block_size: int,
    kv_block_size: int,
    scale: Optional[float] = None,
    num_kv_heads: Optional[int] = None,
    kv_padding: Tuple[int, int] = (0, 0),
    q_padding: Tuple[int, int] = (0, 0),
    S_MAX: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention over the exact per-q-block union (flash_topk_attn/attention.py:423-568).

    Args:
        q, k, v: ``[B, N, C]``, ``C = num_heads * D``.
        merged_indices: ``[B, H_BI, QM, S_MAX]`` from ``build_qblock_topk_indices``;
            ``H_BI`` is 1 (one list for every head) or ``num_heads``.
        counts: ``[B, H_BI, QM]``: only the first ``min(count, S_MAX)`` ids are used.
        num_heads, q_block_size, kv_block_size: as in the reference.
        scale: softmax scale, default ``1 / sqrt(D)``.
        num_kv_heads: grouped-query attention when smaller than ``num_heads``
            (an extension: the reference V1 raises NotImplementedError).
        kv_padding, q_padding: virtual ``(pad_head, pad_tail)``.
        S_MAX: ids read per q-block; default ``merged_indices.shape[-1]``.

    Returns:
        ``o [B, N, C]`` (q's dtype), ``lse [B, H, N]`` float32 natural log;
        a q-block with no token gives o = 0, lse = -inf.
    """
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("flash_topk_attn requires CUDA tensors")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("q must be float16, bfloat16, or float32")
    B, N, C = q.shape
    H = num_heads
    D = C // H
    Q_BS, KV_BS = q_block_size, kv_block_size
    if C != H * D:
        raise ValueError(f"C ({C}) must be divisible by num_heads ({H})")

    kv_pad_head, kv_pad_tail = kv_padding
    q_pad_head, q_pad_tail = q_padding
    if kv_pad_head >= KV_BS:
        raise ValueError(
            f"kv_pad_head={kv_pad_head} must be < kv_block_size={KV_BS}; "
            "virtual padding should only complete partial blocks, not create new ones."
        )
    if kv_pad_tail >= KV_BS:
        raise ValueError(
            f"kv_pad_tail={kv_pad_tail} must be < kv_block_size={KV_BS}; "
            "virtual padding should only complete partial blocks, not create new ones."
        )
    if q_pad_head >= Q_BS:
        raise ValueError(
            f"q_pad_head={q_pad_head} must be < q_block_size={Q_BS}; "
            "virtual padding should only complete partial blocks, not create new ones."
        )
    if q_pad_tail >= Q_BS:
        raise ValueError(
            f"q_pad_tail={q_pad_tail} must be < q_block_size={Q_BS}; "
            "virtual padding should only complete partial blocks, not create new ones."
        )
    n_kv_padded = kv_pad_head + N + kv_pad_tail
    n_q_padded = q_pad_head + N + q_pad_tail
    if n_kv_padded % KV_BS != 0:
        need = KV_BS - (n_kv_padded % KV_BS)
        raise ValueError(
            f"N_KV_PADDED={n_kv_padded} must be divisible by kv_block_size={KV_BS}; "
            f"add {need} tokens of KV padding or adjust kv_block_size."
        )
    if n_q_padded % Q_BS != 0:
        need = Q_BS - (n_q_padded % Q_BS)
        raise ValueError(
            f"N_Q_PADDED={n_q_padded} must be divisible by q_block_size={Q_BS}; "
            f"add {need} tokens of Q padding or adjust q_block_size."
        )
    QM = n_q_padded // Q_BS

    merged = merged_indices.to(torch.int32)
    cnt = counts.to(torch.int32)
    H_BI = merged.shape[1]
    if H_BI not in (1, H):
        raise ValueError(f"merged_indices dim 1 ({H_BI}) must be 1 or num_heads ({H})")
    if merged.shape[2] != QM:
        raise ValueError(f"merged_indices dim 2 ({merged.shape[2]}) must equal QM = {QM}")
    if S_MAX is None:
        S_MAX = merged.shape[-1]
    W = max(1, min(int(S_MAX), merged.shape[-1]))
    # ids at positions >= min(count, S_MAX) are not part of the union
    live = torch.arange(W, device=merged.device, dtype=torch.int32) < cnt.clamp(max=W).unsqueeze(-1)
    merged = torch.where(live, merged[..., :W], torch.full_like(merged[..., :W], -1))
    if H_BI == 1 and H > 1:
        merged = merged.expand(B, H, QM, W)
    merged = merged.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    g, qpad = Q_BS, (q_pad_head, q_pad_tail)
    if Q_BS > _MAX_SUB_QBLOCK:
        merged, g, qpad = _split_qblocks(merged, Q_BS, q_pad_head, N)
    return flash_sparse_attn(q, k, v, merged, num_heads=H, q_block_size=g, kv_block_size=KV_BS, scale=scale,
                             q_padding=qpad, kv_padding=(kv_pad_head, kv_pad_tail), num_kv_heads=num_kv_heads)


__all__ = ["build_qblock_topk_indices", "flash_topk_attn"]
