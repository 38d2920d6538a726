"""Per-query per-score-block softmax probability mass (HIP, gfx950).

Mirrors flash_topk_attn_v2/block_score.py (reference): same signature,
validation and error texts (:369-451).  The reference dispatches to CUDA or
Triton by head dim; here one MFMA kernel covers every D (zero-extended to the
next of 32/64/96/128/160/256 on load, never copied).
"""

from __future__ import annotations

from typing import Tuple

import torch
import torch.nn.functional as F

from . import _lib


def _parse_block_score_args(q, k, num_heads, score_block_size, padding):
    """Argument checks of the reference (block_score.py:369-414)."""
    if q.device.type != "cuda":
        raise ValueError("flash_block_score requires CUDA tensors")

    input_4d = q.ndim == 4
    if input_4d:
        B, H, N, D = q.shape
        if num_heads != H:
            raise ValueError(f"num_heads ({num_heads}) != q.shape[1] ({H})")
        C = H * D
    else:
        if q.ndim != 3:
            raise ValueError("q must be 3D [B, N, C] or 4D [B, H, N, D]")
        B, N, C = q.shape

    H = num_heads
    D = C // H
    pad_head, pad_tail = padding
    if pad_head < 0 or pad_tail < 0:
        raise ValueError("padding must be non-negative (pad_head, pad_tail)")
    if pad_head >= score_block_size or pad_tail >= score_block_size:
        raise ValueError(
            f"padding ({pad_head}, {pad_tail}) must each be < score_block_size "
            f"({score_block_size})"
        )
    n_padded = pad_head + N + pad_tail
    if n_padded % score_block_size != 0:
        need = score_block_size - (n_padded % score_block_size)
        raise ValueError(
            f"pad_head + N + pad_tail = {n_padded} must be divisible by "
            f"score_block_size ({score_block_size}). Try padding=(0, {pad_tail + need})."
        )

    if input_4d:
        if k.shape != (B, H, N, D):
            raise ValueError(f"k shape {k.shape} != {(B, H, N, D)}")
    else:
        if k.shape != (B, N, C):
            raise ValueError(f"k shape {k.shape} != {(B, N, C)}")
    if C % H != 0:
        raise ValueError(f"C={C} not divisible by num_heads={H}")

    if q.dtype != k.dtype:
        raise ValueError(f"q.dtype ({q.dtype}) != k.dtype ({k.dtype})")

    return input_4d, B, H, N, D, C, n_padded, pad_head, pad_tail


def _prepare_qk(q, k, input_4d, H, D):
    """fp32 -> bf16 (as the reference, block_score_cuda.py:115-121); pad D to a
    multiple of 8 when needed; return tensors + [B][N][H][D] strides."""
    if q.dtype == torch.float32:
        q = q.to(torch.bfloat16)
        k = k.to(torch.bfloat16)
    elif q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("q must be float16, bfloat16, or float32")
    layout = "bhnd" if input_4d else "bnc"
    Dp = D
    if D % 8 != 0:
        Dp = (D + 7) // 8 * 8
        if input_4d:
            q = F.pad(q, (0, Dp - D))
            k = F.pad(k, (0, Dp - D))
        else:
            B, N, _ = q.shape
            q = F.pad(q.view(B, N, H, D), (0, Dp - D)).reshape(B, N, H * Dp)
            k = F.pad(k.reshape(B, N, H, D), (0, Dp - D)).reshape(B, N, H * Dp)
    q, qs = _lib.token_view(q, layout, H)
    k, ks = _lib.token_view(k, layout, H)
    return q, k, qs, ks, Dp


def flash_block_score(
    q: torch.Tensor,
    k: torch.Tensor,
    num_heads: int,
    score_block_size: int,
    padding: Tuple[int, int] = (0, 0),
) -> torch.Tensor:
    """Fused block-wise attention mass per query and score block.

    Args:
        q: ``[B, N, C]`` or ``[B, H, N, D]`` (float16, bfloat16, or float32).
        k: Same shape, layout, and dtype as ``q``.
        num_heads: Must equal ``H`` when ``q`` is 4D.
        score_block_size: Logical KV tokens per score block (any positive integer).
        padding: Virtual padding ``(pad_head, pad_tail)``, each strictly less than
            ``score_block_size``.

    Returns:
        ``[B, H, N, M]`` float32, ``M = (pad_head + N + pad_tail) // score_block_size``;
        each row over ``M`` sums to 1.
    """
    parsed = _parse_block_score_args(q, k, num_heads, score_block_size, padding)
    input_4d, B, H, N, D, C, n_padded, pad_head, pad_tail = parsed
    M = n_padded // score_block_size
    qq, kk, qs, ks, Dp = _prepare_qk(q, k, input_4d, H, D)
    out = torch.empty(B, H, N, M, device=q.device, dtype=torch.float32)
    L = _lib.lib()
    ws = _lib.workspace(L.fta_block_score_workspace_size(B, H, N, M), q.device)
    rc = L.fta_block_score(
        _lib.ptr(qq), _lib.ptr(kk), _lib.dtype_code(qq.dtype), B, H, N, Dp,
        _lib.i64arr(qs), _lib.i64arr(ks), score_block_size, pad_head, pad_tail,
        float(D ** -0.5), _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(q.device),
    )
    _lib.check(rc, "flash_block_score")
    return out


__all__ = ["flash_block_score"]
