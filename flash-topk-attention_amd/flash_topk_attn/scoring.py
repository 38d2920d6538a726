"""V1 ``flash_topk_score`` (reference: flash_topk_attn/scoring.py:1080-1357).

The reference runs one Triton kernel that computes dense attention and keeps
a streaming top-k pool of block scores.  Here the two outputs come from the
HIP kernels of the V2 path:

* top-k block scores: the fused scoring + selection of ``flash_topk_score``
  (V2) with no threshold cut, so exactly ``min(topk, M)`` blocks are kept in
  descending order (ties to the lower block index).  The V1 score of a block
  is its softmax mass, divided by the block's valid token count when virtual
  padding is used (scoring.py:1440-1449): V2's ``raw`` and ``avg`` outputs.
* ``o``: block-sparse attention with every KV block selected for every
  q-block, i.e. dense attention, and its backward (dQ, dK, dV).
"""

from __future__ import annotations

import math
import warnings
from typing import Optional, Tuple

import torch

from flash_topk_attn_v2 import flash_topk_score as _v2_topk_score
from flash_topk_attn_v2.sparse_attn import _sparse_attn_fwd
from flash_topk_attn_v2.sparse_attn_bwd import preprocess_delta, sparse_attn_bwd

_DENSE_BLOCK = 64  # q-block and KV-block size of the dense attention pass
_dense_cache: dict = {}


def _check_score_args(B, N, C, H, score_block_size, topk, padding):
    """Argument rules and messages of FlashScoringFunction.forward
    (flash_topk_attn/scoring.py:1085-1116)."""
    if C % H != 0:
        raise ValueError(f"C ({C}) must be divisible by num_heads ({H})")
    if score_block_size < 1:
        raise ValueError("score_block_size must be >= 1")
    pad_head, pad_tail = padding
    if pad_head < 0 or pad_tail < 0:
        raise ValueError("padding must be non-negative (pad_head, pad_tail)")
    if pad_head >= score_block_size or pad_tail >= score_block_size:
        raise ValueError(
            f"padding ({pad_head}, {pad_tail}) must each be < score_block_size ({score_block_size})"
        )
    n_padded = pad_head + N + pad_tail
    if n_padded % score_block_size != 0:
        need = score_block_size - (n_padded % score_block_size)
        raise ValueError(
            f"pad_head + N + pad_tail = {n_padded} must be divisible by "
            f"score_block_size ({score_block_size}). Try padding=(0, {pad_tail + need})."
        )
    num_blocks = n_padded // score_block_size
    if topk > num_blocks:
        raise ValueError(f"topk ({topk}) > num_blocks ({num_blocks})")
    if topk < 0:
        raise ValueError(f"topk ({topk}) must be >= 0")
    return num_blocks


def _topk_blocks(q, k, H, score_block_size, topk, padding):
    """``(indices int32, scores f32)`` ``[B, H, N, min(topk, M)]``."""
    B, N, C = q.shape
    if topk == 0:
        e = torch.empty(B, H, N, 0, device=q.device)
        return e.to(torch.int32), e.float()
    with torch.no_grad():
        idx, raw, avg = _v2_topk_score(q.detach(), k.detach(), H, score_block_size, topk, tuple(padding),
                                       math.inf)
    return idx, (raw if tuple(padding) == (0, 0) else avg)


def _dense_merged(B, H, N, device):
    """Every KV block for every q-block: ``[B, H, QM, M]`` int32 (cached)."""
    nb = (N + _DENSE_BLOCK - 1) // _DENSE_BLOCK
    key = (B, H, nb, str(device))
    m = _dense_cache.get(key)
    if m is None:
        m = torch.arange(nb, device=device, dtype=torch.int32).expand(B, H, nb, nb).contiguous()
        _dense_cache.clear()
        _dense_cache[key] = m
    pad = nb * _DENSE_BLOCK - N
    return m, (0, pad)


class FlashScoringFunction(torch.autograd.Function):
    """Top-k block scores plus the dense attention output, differentiable in
    ``q``, ``k``, ``v`` through ``o`` (flash_topk_attn/scoring.py:1080-1211)."""

    @staticmethod
    def forward(ctx, q, k, v, num_heads, score_block_size, topk, padding: Tuple[int, int]):
        B, N, C = q.shape
        H = num_heads
        if tuple(k.shape) != (B, N, C) or tuple(v.shape) != (B, N, C):
            raise ValueError("q, k, v must all be [B, N, C]")
        _check_score_args(B, N, C, H, score_block_size, topk, padding)
        D = C // H
        if D % 16 != 0 or D > 256:
            raise ValueError(f"D ({D}) must be a positive multiple of 16 and <= 256 for the attention output")
        idx, scores = _topk_blocks(q, k, H, score_block_size, topk, padding)
        orig_dtype = q.dtype
        qa, ka, va = (t.bfloat16() if orig_dtype == torch.float32 else t for t in (q, k, v))
        qa, ka, va = (t.contiguous() for t in (qa, ka, va))
        merged, pad = _dense_merged(B, H, N, q.device)
        scale = D ** -0.5
        o, lse = _sparse_attn_fwd(qa, ka, va, merged, H, _DENSE_BLOCK, _DENSE_BLOCK, scale, pad, pad, H)
        ctx.save_for_backward(qa, ka, va, o, merged, lse)
        ctx.num_heads = H
        ctx.pad = pad
        ctx.scale = scale
        ctx.orig_dtype = orig_dtype
        ctx.mark_non_differentiable(idx, scores)
        return o.to(orig_dtype), idx, scores

    @staticmethod
    def backward(ctx, grad_o, grad_topk_indices, grad_topk_scores):
        if grad_topk_scores is not None and grad_topk_scores.abs().sum() > 0:
            warnings.warn("topk_scores gradients are not implemented, ignoring...", UserWarning)
        q, k, v, o, merged, lse = ctx.saved_tensors
        do = grad_o.to(o.dtype).contiguous()
        delta = preprocess_delta(o, do, ctx.num_heads)
        dq, dk, dv = sparse_attn_bwd(q, k, v, o, do, lse, merged, ctx.num_heads, _DENSE_BLOCK, _DENSE_BLOCK,
                                     ctx.scale, ctx.pad, ctx.pad, delta=delta)
        od = ctx.orig_dtype
        return dq.to(od), dk.to(od), dv.to(od), None, None, None, None


class FlashPureScoringFunction(torch.autograd.Function):
    """Top-k block scores only (flash_topk_attn/scoring.py:1214-1286)."""

    @staticmethod
    def forward(_ctx, q, k, num_heads, score_block_size, topk, padding: Tuple[int, int]):
        B, N, C = q.shape
        if tuple(k.shape) != (B, N, C):
            raise ValueError("q and k must both be [B, N, C]")
        _check_score_args(B, N, C, num_heads, score_block_size, topk, padding)
        return _topk_blocks(q, k, num_heads, score_block_size, topk, padding)

    @staticmethod
    def backward(ctx, grad_topk_indices, grad_topk_scores):
        raise NotImplementedError("flash_topk_score_only does not support backward")


def flash_topk_score(
    q: torch.Tensor,
    k: torch.Tensor,
    v: Optional[torch.Tensor] = None,
    num_heads: Optional[int] = None,
    score_block_size: int = 64,
    topk: int = 16,
    padding: Tuple[int, int] = (0, 0),
    score_only: bool = False,
    backend: str = "triton",
):
    """Dense attention with top-k block scoring (flash_topk_attn/scoring.py:1289-1357).

    Args:
        q, k, v: ``[B, N, C]`` (``C = num_heads * D``) or ``[B, H, N, D]``;
            ``v`` is required unless ``score_only``.
        num_heads: required for 3D input; inferred from ``q.shape[1]`` for 4D.
        score_block_size: tokens per score block (any positive integer).
        topk: blocks to keep per query (``<= M``).
        padding: virtual ``(pad_head, pad_tail)`` of the score blocks.
        score_only: skip the attention output (no ``v`` needed).
        backend: ``"triton"`` (the reference's name, kept for drop-in use) or
            ``"hip"``; both run the HIP kernels.

    Returns:
        ``(o, topk_indices, topk_scores)``, or ``(topk_indices, topk_scores)``
        with ``score_only``.  ``o`` has q's layout and dtype; indices are int32
        and scores float32, ``[B, H, N, min(topk, M)]``.
    """
    if backend not in ("triton", "hip"):
        raise ValueError(f"unsupported backend: {backend!r}, must be 'triton'")
    if not score_only and v is None:
        raise ValueError("v is required when score_only=False")

    input_4d = q.ndim == 4
    if input_4d:
        B, H, N, D = q.shape
        if num_heads is not None and num_heads != H:
            raise ValueError(f"num_heads ({num_heads}) != q.shape[1] ({H})")
        num_heads = H
        C = H * D
        q = q.transpose(1, 2).reshape(B, N, C).contiguous()
        k = k.transpose(1, 2).reshape(B, N, C).contiguous()
        if not score_only:
            if v.shape != (B, H, N, D):
                raise ValueError("q, k, v must all be [B, H, N, D] for 4D input")
            v = v.transpose(1, 2).reshape(B, N, C).contiguous()
    else:
        if q.ndim != 3:
            raise ValueError("q must be 3D [B, N, C] or 4D [B, H, N, D]")
        if num_heads is None:
            raise ValueError("num_heads is required for 3D [B, N, C] input")

    if score_only:
        return FlashPureScoringFunction.apply(q, k, num_heads, score_block_size, topk, padding)
    o, topk_indices, topk_scores = FlashScoringFunction.apply(q, k, v, num_heads, score_block_size, topk, padding)
    if input_4d:
        B, N, C = o.shape
        H = num_heads
        o = o.view(B, N, H, C // H).transpose(1, 2).contiguous()
    return o, topk_indices, topk_scores


__all__ = ["flash_topk_score", "FlashScoringFunction", "FlashPureScoringFunction"]
