"""Sparse attention backward helpers (HIP, gfx950).

Mirrors flash_topk_attn_v2/sparse_attn_bwd.py (preprocess_delta, :12-33),
build_reverse_indices_cuda.py:32-78 and sort_by_count_cuda.py:33-67 of the
reference, plus the dQ/dK/dV launch used by the autograd backward
(sparse_attn.py:163-224, sparse_attn_bwd_dq_cuda.py, sparse_attn_bwd_dkv_cuda.py).
Reverse lists are in ascending q-block order (deterministic).
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import _lib


def preprocess_delta(o: torch.Tensor, do: torch.Tensor, num_heads: int) -> torch.Tensor:
    """delta = rowwise dot(O, dO) in fp32, ``[B, H, N]``."""
    B, N, C = o.shape
    H = num_heads
    D = C // H
    if do.dtype != o.dtype:
        do = do.to(o.dtype)
    oo, os_ = _lib.token_view(o, "bnc", H)
    dd, ds_ = _lib.token_view(do, "bnc", H)
    delta = torch.empty(B, H, N, device=o.device, dtype=torch.float32)
    rc = _lib.lib().fta_preprocess_delta(
        _lib.ptr(oo), _lib.i64arr(os_), _lib.ptr(dd), _lib.i64arr(ds_), _lib.dtype_code(o.dtype),
        B, H, N, D, _lib.ptr(delta), _lib.stream_ptr(o.device),
    )
    _lib.check(rc, "preprocess_delta")
    return delta


def flash_build_reverse_indices(
    merged_indices: torch.Tensor,
    counts: torch.Tensor,
    num_kv_blocks: int,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """KV block -> q-block lists.

    Returns ``reverse_indices [B, H, M, QM]`` int32 (ascending q-block ids,
    ``-1`` padding), ``reverse_counts [B, H, M]`` int32 and
    ``sorted_kv_indices [B, H, M]`` int32 (stable descending by count).
    """
    B, H, QM, W = merged_indices.shape
    M = num_kv_blocks
    dev = merged_indices.device
    merged = merged_indices.to(torch.int32).contiguous()
    rev = torch.empty(B, H, M, QM, device=dev, dtype=torch.int32)
    cnt = torch.empty(B, H, M, device=dev, dtype=torch.int32)
    skv = torch.empty(B, H, M, device=dev, dtype=torch.int32)
    L = _lib.lib()
    ws = _lib.workspace(L.fta_build_reverse_indices_workspace_size(B, H, QM, M), dev)
    rc = L.fta_build_reverse_indices(
        _lib.ptr(merged), _lib.ptr(counts), B, H, QM, W, M, _lib.ptr(rev), _lib.ptr(cnt), _lib.ptr(skv),
        _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev),
    )
    _lib.check(rc, "flash_build_reverse_indices")
    return rev, cnt, skv


def flash_sort_by_count(
    reverse_counts: torch.Tensor,
    num_heads: int,
    num_kv_blocks: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Global stable descending sort of ``reverse_counts`` (``[B*H*M]`` outputs)."""
    flat = reverse_counts.reshape(-1).to(torch.int32).contiguous()
    n = flat.numel()
    sc = torch.empty(n, device=flat.device, dtype=torch.int32)
    sid = torch.empty(n, device=flat.device, dtype=torch.int32)
    rc = _lib.lib().fta_sort_by_count(_lib.ptr(flat), n, _lib.ptr(sc), _lib.ptr(sid), _lib.stream_ptr(flat.device))
    _lib.check(rc, "flash_sort_by_count")
    return sc, sid


def sparse_attn_bwd(
    q, k, v, o, do, lse, merged_indices, num_heads, q_block_size, kv_block_size, scale,
    q_padding=(0, 0), kv_padding=(0, 0), delta=None, num_kv_heads=None,
):
    """dQ ``[B, N, C]``, dK, dV ``[B, N, Hk * D]`` (dtype of q) for block-sparse
    attention; ``Hk = num_kv_heads`` (default ``num_heads``), and each K/V head's
    gradient sums over the query heads that share it.

    ``q, o, do`` are ``[B, N, C]``, ``k, v`` ``[B, N, Hk * D]`` bf16/fp16; ``lse``
    is the forward's natural-log ``[B, H, N]``.
    """
    B, N, C = q.shape
    H = num_heads
    D = C // H
    Hk = H if num_kv_heads is None else num_kv_heads
    dev = q.device
    if delta is None:
        delta = preprocess_delta(o, do, H)
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    qq, qs = _lib.token_view(q, "bnc", H)
    kk, ks = _lib.token_view(k, "bnc", Hk)
    vv, vs = _lib.token_view(v, "bnc", Hk)
    dd, dos = _lib.token_view(do, "bnc", H)
    merged = merged_indices.to(torch.int32).contiguous()
    QM, W = merged.shape[2], merged.shape[3]
    dq = torch.empty(B, N, C, device=dev, dtype=q.dtype)
    dk = torch.empty(B, N, Hk * D, device=dev, dtype=q.dtype)
    dv = torch.empty(B, N, Hk * D, device=dev, dtype=q.dtype)
    gs = [N * C, D, C]
    gk = [N * Hk * D, D, Hk * D]
    L = _lib.lib()
    geo = (B, H, N, D, q_block_size, kv_block_size, q_padding[0], q_padding[1], kv_padding[0], kv_padding[1])
    ws = _lib.workspace(L.fta_sparse_attn_bwd_workspace_size(*geo), dev)
    rc = L.fta_sparse_attn_bwd_gqa(
        _lib.ptr(qq), _lib.i64arr(qs), _lib.ptr(kk), _lib.i64arr(ks), _lib.ptr(vv), _lib.i64arr(vs),
        _lib.ptr(dd), _lib.i64arr(dos), _lib.dtype_code(q.dtype), B, H, Hk, N, D, _lib.ptr(merged), QM, W,
        q_block_size, kv_block_size, q_padding[0], q_padding[1], kv_padding[0], kv_padding[1], float(scale),
        _lib.ptr(lse.contiguous()), _lib.ptr(delta.contiguous()), _lib.ptr(dq), _lib.i64arr(gs), _lib.ptr(dk),
        _lib.i64arr(gk), _lib.ptr(dv), _lib.i64arr(gk), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev),
    )
    _lib.check(rc, "sparse_attn_bwd")
    return dq, dk, dv


__all__ = [
    "preprocess_delta",
    "flash_build_reverse_indices",
    "flash_sort_by_count",
    "sparse_attn_bwd",
]
