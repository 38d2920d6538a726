"""Block-sparse attention over merged KV-block indices (HIP, gfx950).

Mirrors flash_topk_attn_v2/sparse_attn.py (reference): ``flash_sparse_attn``
(:227-392) with the same signature, validation and outputs, and the autograd
function ``FlashSparseAttnFunc`` (:130-224).  The kernels handle any N, head
dim up to 256 (multiple of 16) and virtual padding directly, so the reference's
physical N / D padding copies are not needed.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib
from .sparse_attn_bwd import preprocess_delta, sparse_attn_bwd


def _sparse_attn_fwd(q, k, v, merged, H, g, kvb, scale, q_padding, kv_padding, Hk):
    B, N, C = q.shape
    D = C // H
    dev = q.device
    qq, qs = _lib.token_view(q, "bnc", H)
    kk, ks = _lib.token_view(k, "bnc", Hk)
    vv, vs = _lib.token_view(v, "bnc", Hk)
    o = torch.empty(B, N, C, device=dev, dtype=q.dtype)
    lse = torch.empty(B, H, N, device=dev, dtype=torch.float32)
    QM, W = merged.shape[2], merged.shape[3]
    L = _lib.lib()
    geo = (B, H, N, D, g, kvb, q_padding[0], q_padding[1], kv_padding[0], kv_padding[1])
    ws = _lib.workspace(L.fta_sparse_attn_fwd_workspace_size(*geo), dev)
    rc = L.fta_sparse_attn_fwd_gqa(
        _lib.ptr(qq), _lib.i64arr(qs), _lib.ptr(kk), _lib.i64arr(ks), _lib.ptr(vv), _lib.i64arr(vs),
        _lib.dtype_code(q.dtype), B, H, Hk, N, D, _lib.ptr(merged), QM, W, g, kvb,
        q_padding[0], q_padding[1], kv_padding[0], kv_padding[1], float(scale),
        _lib.ptr(o), _lib.i64arr([N * C, D, C]), _lib.ptr(lse), _lib.ptr(ws), ws.numel(),
        _lib.stream_ptr(dev),
    )
    _lib.check(rc, "flash_sparse_attn")
    return o, lse


class _SparseAttnGQAFunc(torch.autograd.Function):
    """Autograd function behind ``flash_sparse_attn``: HIP forward, HIP dQ / dK /
    dV backward, virtual paddings passed through, optional grouped K/V heads."""

    @staticmethod
    def forward(ctx, q, k, v, merged_indices, num_heads, q_block_size, kv_block_size,
                softmax_scale, q_padding, kv_padding, num_kv_heads=None):
        Hk = num_heads if num_kv_heads is None else num_kv_heads
        o, lse = _sparse_attn_fwd(q, k, v, merged_indices, num_heads, q_block_size, kv_block_size,
                                  softmax_scale, q_padding, kv_padding, Hk)
        ctx.num_kv_heads = Hk
        ctx.save_for_backward(q, k, v, o, merged_indices, lse)
        ctx.num_heads = num_heads
        ctx.q_block_size = q_block_size
        ctx.kv_block_size = kv_block_size
        ctx.softmax_scale = softmax_scale
        ctx.q_padding = q_padding
        ctx.kv_padding = kv_padding
        ctx.mark_non_differentiable(lse)
        return o, lse

    @staticmethod
    def backward(ctx, grad_output, _grad_lse):
        q, k, v, o, merged, lse = ctx.saved_tensors
        delta = preprocess_delta(o, grad_output, ctx.num_heads)
        dq, dk, dv = sparse_attn_bwd(
            q, k, v, o, grad_output, lse, merged, ctx.num_heads, ctx.q_block_size, ctx.kv_block_size,
            ctx.softmax_scale, ctx.q_padding, ctx.kv_padding, delta=delta, num_kv_heads=ctx.num_kv_heads,
        )
        return dq, dk, dv, None, None, None, None, None, None, None, None


def _apply_counts(merged: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
    """The list each q-block of the reference's kernel walks, with -1 after it.

    The reference (csrc/sparse_attn_kernel.cu:57-86) sorts rows of at most 512
    slots ascending with -1 mapped to INT_MAX and walks the first ``count``
    sorted ids; wider rows are walked unsorted for ``count`` slots.  Positions
    at or past ``count`` become -1 here; the kernels skip -1 entries, and a
    row with ``count <= 0`` has no entries (o = 0, lse = -inf).
    """
    W = merged.shape[-1]
    cnt = counts.to(device=merged.device, dtype=torch.int64).reshape(*merged.shape[:-1], 1)
    if W <= 512:
        key = torch.where(merged >= 0, merged, torch.full_like(merged, torch.iinfo(torch.int32).max))
        merged = torch.sort(key, dim=-1).values
        merged = torch.where(merged == torch.iinfo(torch.int32).max, torch.full_like(merged, -1), merged)
    pos = torch.arange(W, device=merged.device, dtype=torch.int64)
    return torch.where(pos < cnt, merged, torch.full_like(merged, -1)).contiguous()


class FlashSparseAttnFunc(torch.autograd.Function):
    """Autograd function with the reference's call contract
    (flash_topk_attn_v2/sparse_attn.py:130-224):

    ``FlashSparseAttnFunc.apply(q, k, v, merged_indices, counts, num_heads,
    q_block_size, kv_block_size, qblock_topk, softmax_scale, q_pad_head,
    kv_pad_head, N_real, num_kv_blocks)`` with q, k, v ``[B, N_phys, C]``
    (rows past ``N_real`` are physical padding and are not read) returns
    ``(output [B, N_real, C], softmax_max, softmax_lse)``, each ``[B, H, N_real]``
    fp32.  The kernels produce the full natural-log lse in one value, so
    ``softmax_max`` is 0 and ``softmax_lse`` is the lse: their sum is the
    reference's lse (sparse_attn.py:391).  The virtual tail paddings follow
    from the shapes, as in the reference's kernels: q tail =
    QM * q_block_size - q_pad_head - N_real, kv tail = num_kv_blocks *
    kv_block_size - kv_pad_head - N_real.  ``counts`` selects the blocks a
    q-block attends to as the reference's kernel does
    (csrc/sparse_attn_kernel.cu:39-86, :201): rows of at most 512 slots keep
    the ``counts`` smallest valid ids (the row sorted ascending, -1 entries
    last), wider rows their first ``counts`` slots; ``counts <= 0`` gives
    o = 0 and lse = -inf.  Counts that equal the number of valid entries (what
    ``build_qblock_topk_indices`` returns) keep every listed block.
    Gradients are ``[B, N_phys, C]`` with zero rows past ``N_real``.
    """

    @staticmethod
    def forward(ctx, q, k, v, merged_indices, counts, num_heads, q_block_size, kv_block_size, qblock_topk,
                softmax_scale, q_pad_head, kv_pad_head, N_real, num_kv_blocks):
        del qblock_topk
        B, N_phys, C = q.shape
        N = int(N_real)
        if N <= 0 or N > N_phys:
            raise ValueError(f"N_real={N_real} must be in [1, N_phys={N_phys}]")
        QM = merged_indices.shape[2]
        q_padding = (int(q_pad_head), QM * q_block_size - int(q_pad_head) - N)
        kv_padding = (int(kv_pad_head), int(num_kv_blocks) * kv_block_size - int(kv_pad_head) - N)
        if q_padding[1] < 0 or kv_padding[1] < 0:
            raise ValueError("merged_indices / num_kv_blocks do not cover N_real with the given head paddings")
        merged = _apply_counts(merged_indices.to(torch.int32), counts)
        qs, ks, vs = q[:, :N], k[:, :N], v[:, :N]
        o, lse = _sparse_attn_fwd(qs, ks, vs, merged, num_heads, q_block_size, kv_block_size,
                                  float(softmax_scale), q_padding, kv_padding, num_heads)
        softmax_max = torch.zeros_like(lse)
        ctx.save_for_backward(q, k, v, o, merged, lse)
        ctx.num_heads = num_heads
        ctx.q_block_size = q_block_size
        ctx.kv_block_size = kv_block_size
        ctx.softmax_scale = float(softmax_scale)
        ctx.q_padding = q_padding
        ctx.kv_padding = kv_padding
        ctx.N_real = N
        ctx.mark_non_differentiable(softmax_max, lse)
        return o, softmax_max, lse

    @staticmethod
    def backward(ctx, grad_output, _grad_sm, _grad_sl):
        q, k, v, o, merged, lse = ctx.saved_tensors
        N = ctx.N_real
        B, N_phys, C = q.shape
        H = ctx.num_heads
        delta = preprocess_delta(o, grad_output, H)
        dq, dk, dv = sparse_attn_bwd(
            q[:, :N], k[:, :N], v[:, :N], o, grad_output, lse, merged, H, ctx.q_block_size, ctx.kv_block_size,
            ctx.softmax_scale, ctx.q_padding, ctx.kv_padding, delta=delta,
        )
        if N_phys > N:
            grads = []
            for g in (dq, dk, dv):
                full = g.new_zeros(B, N_phys, C)
                full[:, :N] = g
                grads.append(full)
            dq, dk, dv = grads
        return (dq, dk, dv, None, None, None, None, None, None, None, None, None, None, None)


def flash_sparse_attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    merged_indices: torch.Tensor,
    num_heads: int,
    q_block_size: int,
    kv_block_size: int,
    scale: Optional[float] = None,
    q_padding: Tuple[int, int] = (0, 0),
    kv_padding: Tuple[int, int] = (0, 0),
    num_kv_heads: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block-sparse attention forward (differentiable in q, k, v).

    Args:
        q, k, v: ``[B, N, C]``, ``C = num_heads * D`` (float16, bfloat16, float32).
        merged_indices: ``[B, H, QM, qblock_topk]`` int32, ``-1`` padding,
            ``QM = (q_pad_head + N + q_pad_tail) // q_block_size``.
        num_heads: Number of attention heads.
        q_block_size: Query block size (1 to 64).
        kv_block_size: KV block size (any positive integer).
        scale: Softmax scale, default ``1 / sqrt(D)``.
        q_padding, kv_padding: virtual ``(pad_head, pad_tail)``.
        num_kv_heads: K/V heads for grouped-query attention (``k``, ``v`` are
            ``[B, N, num_kv_heads * D]``; query head ``h`` uses K/V head
            ``h // (num_heads // num_kv_heads)``).  Default: ``num_heads``.
            An extension: the reference has no GQA.

    Returns:
        ``(output [B, N, C] same dtype as q, lse [B, H, N] float32 natural log)``.
    """
    if q.ndim != 3:
        raise ValueError("q must be [B, N, C]")
    if q.device.type != "cuda":
        raise ValueError("flash_sparse_attn requires CUDA tensors")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("q must be float16, bfloat16, or float32")

    orig_dtype = q.dtype
    if orig_dtype == torch.float32:
        q = q.bfloat16()
        k = k.bfloat16()
        v = v.bfloat16()

    B, N, C = q.shape
    H = num_heads
    D = C // H

    if C != H * D:
        raise ValueError(f"C ({C}) must be divisible by num_heads ({H})")
    Hk = H if num_kv_heads is None else int(num_kv_heads)
    if Hk <= 0 or H % Hk != 0:
        raise ValueError(f"num_heads ({H}) must be a positive multiple of num_kv_heads ({Hk})")
    if tuple(k.shape) != (B, N, Hk * D) or tuple(v.shape) != (B, N, Hk * D):
        raise ValueError(f"k and v must be [B, N, num_kv_heads * D] = {[B, N, Hk * D]}")
    if q_block_size <= 0 or q_block_size > 64:
        raise ValueError(f"q_block_size must be in (0, 64], got {q_block_size}")
    if kv_block_size <= 0:
        raise ValueError(f"kv_block_size must be positive, got {kv_block_size}")
    if merged_indices.ndim != 4:
        raise ValueError("merged_indices must be [B, H, QM, qblock_topk]")
    if merged_indices.dtype != torch.int32:
        raise ValueError("merged_indices must be int32")

    q_pad_head, q_pad_tail = q_padding
    kv_pad_head, kv_pad_tail = kv_padding
    if q_pad_head < 0 or q_pad_tail < 0:
        raise ValueError("q_padding values must be non-negative")
    if kv_pad_head < 0 or kv_pad_tail < 0:
        raise ValueError("kv_padding values must be non-negative")
    if q_pad_head >= q_block_size:
        raise ValueError(f"q_pad_head={q_pad_head} must be < q_block_size={q_block_size}")
    if q_pad_tail >= q_block_size:
        raise ValueError(f"q_pad_tail={q_pad_tail} must be < q_block_size={q_block_size}")
    if kv_pad_head >= kv_block_size:
        raise ValueError(f"kv_pad_head={kv_pad_head} must be < kv_block_size={kv_block_size}")
    if kv_pad_tail >= kv_block_size:
        raise ValueError(f"kv_pad_tail={kv_pad_tail} must be < kv_block_size={kv_block_size}")

    n_q_padded = q_pad_head + N + q_pad_tail
    n_kv_padded = kv_pad_head + N + kv_pad_tail
    if n_q_padded % q_block_size != 0:
        raise ValueError(
            f"q_pad_head + N + q_pad_tail = {n_q_padded} must be divisible "
            f"by q_block_size={q_block_size}"
        )
    if n_kv_padded % kv_block_size != 0:
        raise ValueError(
            f"kv_pad_head + N + kv_pad_tail = {n_kv_padded} must be "
            f"divisible by kv_block_size={kv_block_size}"
        )
    QM = n_q_padded // q_block_size
    if merged_indices.shape[2] != QM:
        raise ValueError(
            f"merged_indices dim 2 ({merged_indices.shape[2]}) must match "
            f"QM = (q_pad_head + N + q_pad_tail) // q_block_size = {QM}"
        )
    if D <= 0 or D % 16 != 0:
        raise ValueError(f"D ({D}) must be a positive multiple of 16")
    if D > 256:
        raise ValueError(f"D ({D}) must be <= 256")
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    merged = merged_indices.contiguous()
    output, lse = _SparseAttnGQAFunc.apply(
        q, k, v, merged, H, q_block_size, kv_block_size, float(scale),
        (q_pad_head, q_pad_tail), (kv_pad_head, kv_pad_tail), Hk,
    )
    if orig_dtype == torch.float32:
        output = output.float()
    return output, lse


__all__ = ["flash_sparse_attn", "FlashSparseAttnFunc"]
