"""MI355X (gfx950) flash-topk-attention V2 hot path.

Drop-in for the public API of the reference package ``flash_topk_attn_v2``
(flash_topk_attn_v2/__init__.py:16-176): ``flash_topk_score``,
``build_qblock_topk_indices`` and ``flash_topk_attn`` (differentiable), with
the same signatures, argument checks and return conventions.  All compute runs
in hand-written HIP kernels (libfta_gfx950.so, C ABI in include/fta.h).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from . import _lib
from .block_score import _parse_block_score_args, _prepare_qk, flash_block_score
from .qblock_merge import flash_qblock_merge
from .sparse_attn import FlashSparseAttnFunc, flash_sparse_attn
from .sparse_attn_bwd import flash_build_reverse_indices, flash_sort_by_count, preprocess_delta
from .topk_select import flash_topk_select


def flash_topk_score(
    q: torch.Tensor,
    k: torch.Tensor,
    num_heads: Optional[int] = None,
    score_block_size: int = 64,
    topk: int = 16,
    padding: Tuple[int, int] = (0, 0),
    threshold: float = 1.0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Block-level top-k scoring (reference: flash_topk_attn_v2/__init__.py:16-54).

    Returns ``(topk_indices int32, topk_raw_scores f32, topk_avg_scores f32)``,
    each ``[B, H, N, min(topk, M)]`` (``M`` when ``topk == 0``).  Scoring and
    selection run in one C call: the normalised ``[B, H, N, M]`` scores are
    never formed; for b = 64 or 128, D <= 128 and topk <= 32 the selector reads the
    scorer's candidate streams (bounded workspace), otherwise its per-block
    log2-sums.
    """
    input_4d = q.ndim == 4
    if input_4d:
        _, head_count, _, _ = q.shape
        if num_heads is not None and num_heads != head_count:
            raise ValueError(f"num_heads ({num_heads}) != q.shape[1] ({head_count})")
        num_heads = head_count
    else:
        if q.ndim != 3:
            raise ValueError("q must be 3D [B, N, C] or 4D [B, H, N, D]")
        if num_heads is None:
            raise ValueError("num_heads is required for 3D [B, N, C] input")

    parsed = _parse_block_score_args(q, k, num_heads, score_block_size, padding)
    input_4d, B, H, N, D, C, n_padded, pad_head, pad_tail = parsed
    M = n_padded // score_block_size
    if topk < 0:
        raise ValueError("max_topk must be >= 0")
    if M > 4096:
        raise NotImplementedError(f"M={M} exceeds block sort limit 4096")
    m_out = min(topk, M) if topk > 0 else M
    qq, kk, qs, ks, Dp = _prepare_qk(q, k, input_4d, H, D)
    dev = q.device
    idx = torch.empty(B, H, N, m_out, device=dev, dtype=torch.int32)
    raw = torch.empty(B, H, N, m_out, device=dev, dtype=torch.float32)
    avg = torch.empty(B, H, N, m_out, device=dev, dtype=torch.float32)
    L = _lib.lib()
    ws = _lib.workspace(L.fta_topk_score_workspace_size_ex(B, H, N, Dp, score_block_size, pad_head, pad_tail, topk),
                        dev)
    rc = L.fta_topk_score(
        _lib.ptr(qq), _lib.ptr(kk), _lib.dtype_code(qq.dtype), B, H, N, Dp, _lib.i64arr(qs), _lib.i64arr(ks),
        score_block_size, pad_head, pad_tail, float(D ** -0.5), topk, float(threshold),
        _lib.ptr(idx), _lib.ptr(raw), _lib.ptr(avg), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev),
    )
    _lib.check(rc, "flash_topk_score")
    # every id is < M <= 4096: build_qblock_topk_indices need not read the max back
    # (recorded with the tensor's version counter, so an in-place change through a
    # torch op voids it; writes that bypass the version counter -- through
    # ``.data``, numpy or DLPack views -- are not seen, and ids >= M written that
    # way would be dropped by the merge instead of raising as the reference does)
    idx._fta_id_bound = (M, idx._version)
    return idx, raw, avg


def build_qblock_topk_indices(
    topk_indices: torch.Tensor,
    q_block_size: int,
    q_padding: Tuple[int, int] = (0, 0),
    topk_scores: Optional[torch.Tensor] = None,
    qblock_topk: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """Per-q-block merged indices (reference: flash_topk_attn_v2/__init__.py:57-133).

    Returns ``(merged_indices [B, H, QM, W] int32, counts [B, H, QM] int32, W)``.
    """
    if topk_indices.ndim != 4:
        raise ValueError("topk_indices must be [B, H, N, K]")

    _, _, sequence_length, topk_width = topk_indices.shape
    q_pad_head, q_pad_tail = q_padding
    device = topk_indices.device

    if q_pad_head < 0 or q_pad_tail < 0:
        raise ValueError("q_padding must be non-negative")
    if q_pad_head >= q_block_size:
        raise ValueError(f"q_pad_head={q_pad_head} must be < q_block_size={q_block_size}")
    if q_pad_tail >= q_block_size:
        raise ValueError(f"q_pad_tail={q_pad_tail} must be < q_block_size={q_block_size}")

    padded_sequence_length = q_pad_head + sequence_length + q_pad_tail
    if padded_sequence_length % q_block_size != 0:
        raise ValueError(
            f"q_pad_head + N + q_pad_tail = {padded_sequence_length} must be divisible "
            f"by q_block_size ({q_block_size})"
        )

    indices_int = topk_indices.to(torch.int32).contiguous()
    if q_pad_head > 0 or q_pad_tail > 0:
        indices_int = F.pad(indices_int, (0, 0, q_pad_head, q_pad_tail), value=-1)

    if qblock_topk is None:
        qblock_topk = q_block_size * topk_width

    if topk_scores is not None:
        scores_float = topk_scores.float().contiguous()
        if q_pad_head > 0 or q_pad_tail > 0:
            scores_float = F.pad(scores_float, (0, 0, q_pad_head, q_pad_tail), value=0.0)
    else:
        scores_float = (indices_int >= 0).to(torch.float32)

    B, H = indices_int.shape[:2]
    QM = padded_sequence_length // q_block_size
    counts = torch.empty(B, H, QM, device=device, dtype=torch.int32)
    if indices_int.numel() == 0:
        merged_indices, _ = flash_qblock_merge(indices_int, scores_float, q_block_size=q_block_size,
                                               qblock_topk=qblock_topk, num_score_blocks=1, counts_out=counts)
        return merged_indices, counts, merged_indices.shape[-1]
    if qblock_topk <= 0:
        raise ValueError("qblock_topk must be positive")
    if indices_int.device.type != "cuda":
        raise ValueError("flash_qblock_merge requires CUDA tensors")

    merged_indices = torch.empty(B, H, QM, qblock_topk, device=device, dtype=torch.int32)
    merged_scores = torch.empty(B, H, QM, qblock_topk, device=device, dtype=torch.float32)
    bound = getattr(topk_indices, "_fta_id_bound", None)
    if bound is not None and bound[0] <= 4096 and bound[1] == topk_indices._version:
        # produced by flash_topk_score with M <= 4096 blocks: every id is below M,
        # so num_score_blocks = M keeps exactly the ids that max id + 1 keeps, and
        # neither the device max nor a host wait is needed
        rc = _lib.lib().fta_qblock_merge(
            _lib.ptr(indices_int), _lib.ptr(scores_float), B * H * QM, q_block_size, topk_width,
            int(bound[0]), qblock_topk, _lib.ptr(merged_indices), _lib.ptr(merged_scores), _lib.ptr(counts),
            _lib.stream_ptr(device),
        )
        _lib.check(rc, "flash_qblock_merge")
        return merged_indices, counts, merged_indices.shape[-1]
    # num_score_blocks = max id + 1, as in the reference (:101-105).  The max is
    # taken on the device and read by the merge kernel, and the host reads it
    # (to report ids past the 4096-block limit) only after the merge is queued,
    # so the GPU does not idle through the host round trip.
    max_id = indices_int.max().reshape(1)
    rc = _lib.lib().fta_qblock_merge_maxid(
        _lib.ptr(indices_int), _lib.ptr(scores_float), B * H * QM, q_block_size, topk_width,
        _lib.ptr(max_id), qblock_topk, _lib.ptr(merged_indices), _lib.ptr(merged_scores), _lib.ptr(counts),
        _lib.stream_ptr(device),
    )
    _lib.check(rc, "flash_qblock_merge")
    num_score_blocks = int(max_id.item()) + 1
    if num_score_blocks > 4096:
        raise NotImplementedError(
            f"num_score_blocks={num_score_blocks} exceeds CUDA block sort limit 4096"
        )
    max_merged_width = merged_indices.shape[-1]
    return merged_indices, counts, max_merged_width


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
    """Sparse attention over merged KV block indices
    (reference: flash_topk_attn_v2/__init__.py:136-169).  ``counts`` and
    ``S_MAX`` are accepted and ignored, as in the reference.

    ``num_kv_heads`` < ``num_heads`` runs grouped-query attention (k, v with
    ``num_kv_heads`` heads, ``num_heads`` a multiple of it).  This extends the
    reference, which raises NotImplementedError for it (:153-156).
    """
    del counts, S_MAX

    return flash_sparse_attn(
        q,
        k,
        v,
        merged_indices,
        num_heads=num_heads,
        q_block_size=q_block_size,
        kv_block_size=kv_block_size,
        scale=scale,
        q_padding=q_padding,
        kv_padding=kv_padding,
        num_kv_heads=num_kv_heads,
    )


__all__ = [
    "flash_topk_score",
    "build_qblock_topk_indices",
    "flash_topk_attn",
    "flash_block_score",
    "flash_topk_select",
    "flash_qblock_merge",
    "flash_sparse_attn",
    "FlashSparseAttnFunc",
    "preprocess_delta",
    "flash_build_reverse_indices",
    "flash_sort_by_count",
]
