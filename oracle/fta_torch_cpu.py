"""PyTorch-CPU fp32 restatement of the V2 hot path (the CPU baseline).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
module; ``bench.py``'s ``cpu_baseline`` leg times it on the host cores and
``tests/test_oracle.py`` pins it against the numpy oracle (``fta_oracle``).

It computes what the reference's PyTorch (naive) path computes, per head, in
float32 torch ops on the CPU (paths relative to the reference repository,
``v2/`` = ``flash_topk_attn_v2/``):

* ``block_score``   v2/block_score.py:295-366 (softmax over all keys, sums per
                    score block), in row chunks;
* ``topk_select``   v2/topk_select.py:128-182 (avg = raw / valid count,
                    descending stable sort, fp32 cumulative sum of raw, cut at
                    the threshold, cap at top-k);
* ``qblock_merge``  v2/qblock_merge.py:27-82 (score-weighted union per q-block,
                    descending, truncated to W);
* ``sparse_attn_fwd_bwd``  v2/sparse_attn.py:24-127 and
                    v2/sparse_attn_bwd.py:111-294: softmax over each q-block's
                    listed KV tokens, o = P V, and dQ / dK / dV by autograd.

Only unpadded geometries (N a multiple of the block sizes) are handled: it is
the baseline for the benchmark workload, not a general oracle.
"""

from __future__ import annotations

from typing import Tuple

import torch


def block_score(q: torch.Tensor, k: torch.Tensor, b: int, chunk: int = 2048) -> torch.Tensor:
    """q, k [N, D] fp32 -> [N, M] block probabilities (softmax mass per block)."""
    N, D = q.shape
    M = N // b
    scale = D ** -0.5
    out = torch.empty(N, M, dtype=torch.float32)
    kt = k.t().contiguous()
    for r0 in range(0, N, chunk):
        s = (q[r0:r0 + chunk] @ kt) * scale
        p = torch.softmax(s, dim=-1)
        out[r0:r0 + chunk] = p.view(-1, M, b).sum(-1)
    return out


def topk_select(scores: torch.Tensor, threshold: float, topk: int, b: int
                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """[R, M] -> (idx int32, raw f32, avg f32) [R, min(topk, M)], -1 / 0 after the cut."""
    M = scores.shape[-1]
    m_out = min(topk, M) if topk > 0 else M
    avg = scores / float(b)
    sa, order = torch.sort(avg, dim=-1, descending=True, stable=True)
    sa, order = sa[:, :m_out], order[:, :m_out]
    raw = sa * float(b)
    cs = torch.cumsum(raw, dim=-1)
    exceed = cs >= threshold
    first = torch.where(exceed.any(-1), exceed.float().argmax(-1) + 1, torch.full_like(exceed[:, 0], m_out,
                                                                                          dtype=torch.long))
    keep = torch.arange(m_out).unsqueeze(0) < first.unsqueeze(1)
    idx = torch.where(keep, order, torch.full_like(order, -1)).to(torch.int32)
    return idx, torch.where(keep, raw, torch.zeros_like(raw)), torch.where(keep, sa, torch.zeros_like(sa))


def qblock_merge(idx: torch.Tensor, avg: torch.Tensor, g: int, W: int, M: int
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """idx / avg [N, K] -> (merged [QM, W] int32, counts [QM] int32)."""
    N, K = idx.shape
    QM = N // g
    acc = torch.zeros(QM, M, dtype=torch.float32)
    il = idx.long().view(QM, g * K)
    sc = avg.view(QM, g * K)
    valid = il >= 0
    acc.scatter_add_(1, torch.where(valid, il, torch.zeros_like(il)), torch.where(valid, sc, torch.zeros_like(sc)))
    vals, order = torch.sort(acc, dim=-1, descending=True, stable=True)
    w = min(W, M)
    merged = torch.full((QM, W), -1, dtype=torch.int32)
    merged[:, :w] = torch.where(vals[:, :w] > 0, order[:, :w], torch.full_like(order[:, :w], -1)).to(torch.int32)
    return merged, (merged >= 0).sum(-1).to(torch.int32)


def sparse_attn_fwd_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, do: torch.Tensor,
                        merged: torch.Tensor, g: int, b: int, group: int = 64
                        ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k, v, do [N, D] fp32, merged [QM, W] -> (o, lse, dq, dk, dv).

    Each q-block attends to the tokens of its listed KV blocks; q-blocks are
    processed ``group`` at a time with their lists padded to the longest (the
    padding masked to -inf), and the gradients come from autograd."""
    N, D = q.shape
    QM, W = merged.shape
    scale = D ** -0.5
    counts = (merged >= 0).sum(-1)
    ql, kl, vl = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    outs, lses = [], []
    for q0 in range(0, QM, group):
        q1 = min(QM, q0 + group)
        cmax = max(int(counts[q0:q1].max()), 1)
        ids = merged[q0:q1, :cmax].long()
        ok = ids >= 0
        tok = (torch.where(ok, ids, torch.zeros_like(ids)).unsqueeze(-1) * b + torch.arange(b)).view(q1 - q0, -1)
        tmask = ok.unsqueeze(-1).expand(-1, -1, b).reshape(q1 - q0, -1)
        kg, vg = kl[tok], vl[tok]                                    # [G, cmax*b, D]
        qb = ql[q0 * g:q1 * g].view(q1 - q0, g, D)
        s = torch.einsum("gqd,gkd->gqk", qb, kg) * scale
        s = s.masked_fill(~tmask.unsqueeze(1), float("-inf"))
        # an empty list (count 0) gives o = 0 and lse = -inf
        # (v2/csrc/sparse_attn_kernel.cu:39-54); its row runs on zeros
        empty = ~ok.any(-1)
        s = torch.where(empty.view(-1, 1, 1), torch.zeros_like(s), s)
        lse = torch.logsumexp(s, dim=-1)
        p = torch.exp(s - lse.unsqueeze(-1)) * (~empty).view(-1, 1, 1).float()
        outs.append(torch.einsum("gqk,gkd->gqd", p, vg).reshape(-1, D))
        lses.append(torch.where(empty.view(-1, 1), torch.full_like(lse, float("-inf")), lse).reshape(-1))
    o = torch.cat(outs)
    o.backward(do)
    return o.detach(), torch.cat(lses).detach(), ql.grad, kl.grad, vl.grad


def pipeline_head(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, do: torch.Tensor, b: int, topk: int,
                  threshold: float, g: int, W: int):
    """One head's score -> top-k -> merge -> sparse attention forward + backward.
    Returns (merged, counts, o, lse, dq, dk, dv)."""
    N = q.shape[0]
    sc = block_score(q, k, b)
    idx, raw, avg = topk_select(sc, threshold, topk, b)
    merged, counts = qblock_merge(idx, avg, g, W, N // b)
    o, lse, dq, dk, dv = sparse_attn_fwd_bwd(q, k, v, do, merged, g, b)
    return merged, counts, o, lse, dq, dk, dv
