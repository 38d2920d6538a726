"""CPU oracle for the flash-topk-attention V2 hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may use it, and only as the checker / CPU baseline.

This is a numpy restatement of the reference's naive semantics (paths are
relative to the reference repository root, ``v2/`` = ``flash_topk_attn_v2/``):

* ``block_score``          v2/block_score.py:295-366
* ``topk_select``          v2/topk_select.py:128-182, cut and valid-count rules
                           of v2/topk_select.py:66-123 and
                           v2/csrc/topk_select_kernel.cu:50-110
* ``qblock_merge``         v2/qblock_merge.py:27-82, pad/<=0 rules of
                           v2/csrc/qblock_merge_kernel.cu:36-89
* ``build_qblock_topk_indices``  v2/__init__.py:57-133
* ``sparse_attn``          v2/sparse_attn.py:24-127 (empty q-block semantics of
                           v2/csrc/sparse_attn_kernel.cu:39-54)
* ``preprocess_delta``     v2/sparse_attn_bwd.py:12-33
* ``build_reverse_indices`` v2/sparse_attn_bwd.py:36-76 (+ the argsort of
                           v2/csrc/build_reverse_indices_kernel.cu:29-62)
* ``sort_by_count``        v2/sparse_attn_bwd.py:79-108
* ``sparse_attn_bwd``      v2/sparse_attn_bwd.py:111-294

V1 compatibility layer (``v1/`` = ``flash_topk_attn/``):

* ``v1_qblock_union``      v1/attention.py:23-138 (sort, dedup, -1 fill)
* ``v1_topk_score``        v1/scoring.py:1360-1469 (naive: softmax block sums,
                           / valid count under padding, descending top-k; dense o)
* ``v1_sparse_attn``       v1/attention.py:423-568, 571-647 (ids limited to
                           ``counts``, one merged row shared by all heads when
                           ``merged.shape[1] == 1``)

Orders that the reference leaves implementation-defined are fixed here, and
the HIP kernels follow the same rules:

* top-k ties: descending average score, ties broken by the LOWER block index
  (CUB BlockRadixSort is stable, v2/csrc/topk_select_kernel.cu:62);
* top-k cumulative sum: sequential fp32 sum in sorted order of
  ``raw' = avg * valid_count`` (both reference kernels re-derive raw from avg:
  v2/topk_select.py:101, v2/csrc/topk_select_kernel.cu:80);
* merge sums: sequential fp32 sum in (query row, slot) order (the reference
  uses shared-memory float atomics, whose order is undefined);
* merge ties: descending merged score, ties broken by the lower block index;
* reverse lists: q-block ids in ascending order (the reference's atomic slot
  order is undefined).

Floating-point attention maths (block scores, o, lse, gradients) is computed
in float64 from the caller's (already bf16/fp16-rounded) inputs.

``round_p`` ("bf16" / "fp16") of ``sparse_attn`` and ``sparse_attn_bwd``
additionally rounds, to that 16-bit type with round-to-nearest-even, the
operands that the reference's kernels convert to the input element type
before a matrix product (P before P.V in the forward,
v2/csrc/sparse_attn_kernel.cu:207-310; P before P^T.dO and dS before dS.K /
dS^T.Q in the backward, v2/csrc/sparse_attn_bwd_dq_kernel.cu and
sparse_attn_bwd_dkv_kernel.cu), everything else staying float64.  The forward
rounds P relative to the row's final maximum (a kernel's online softmax
rounds it relative to a running maximum, so the forward mode models the
rounding, it does not replicate it bit for bit); the backward's P is
normalised by the forward's lse in every implementation, so its rounding
points are those of the kernels.
"""

from __future__ import annotations

import math
from typing import Iterable, Optional, Sequence, Tuple

import numpy as np

# --------------------------------------------------------------------------
# helpers
# --------------------------------------------------------------------------


def round_to(x: np.ndarray, kind: Optional[str]) -> np.ndarray:
    """x rounded to bfloat16 / float16 (round to nearest, ties to even), as
    float64; ``kind`` None or "f64" returns x unchanged ("f64" as the
    ``round_p`` of sparse_attn runs a kernel's schedule without rounding)."""
    if kind is None or kind == "f64":
        return x
    if kind == "fp16":  # from float32, as the kernels round their fp32 values
        with np.errstate(over="ignore"):
            return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float16).astype(np.float64)
    if kind != "bf16":
        raise ValueError(f"unknown rounding {kind!r}")
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float64).astype(np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    finite = np.isfinite(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(finite, r, u & 0xFFFF0000)
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def _to_bhnd(x: np.ndarray, num_heads: int) -> np.ndarray:
    """[B, N, C] -> [B, H, N, D] (float64 view/copy)."""
    B, N, C = x.shape
    D = C // num_heads
    return x.reshape(B, N, num_heads, D).transpose(0, 2, 1, 3).astype(np.float64)


def _from_bhnd(x: np.ndarray) -> np.ndarray:
    B, H, N, D = x.shape
    return x.transpose(0, 2, 1, 3).reshape(B, N, H * D)


def _logsumexp(s: np.ndarray, axis: int = -1) -> np.ndarray:
    m = np.max(s, axis=axis, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    with np.errstate(divide="ignore"):
        out = np.log(np.sum(np.exp(s - m_safe), axis=axis, keepdims=True)) + m_safe
    return np.squeeze(out, axis=axis)


# --------------------------------------------------------------------------
# scoring: v2/block_score.py:295-366
# --------------------------------------------------------------------------


def block_score(
    q: np.ndarray,
    k: np.ndarray,
    num_heads: Optional[int],
    score_block_size: int,
    padding: Tuple[int, int] = (0, 0),
    rows: Optional[np.ndarray] = None,
    chunk: int = 1024,
) -> np.ndarray:
    """Per-query softmax mass per virtual score block (float64).

    Follows v2/block_score.py:295-366: softmax over all N keys with scale
    D**-0.5, then sums over keys ``[max(0, m*b - pad_head), min(N, (m+1)*b - pad_head))``.

    ``q``/``k`` are ``[B, N, C]`` (needs ``num_heads``) or ``[B, H, N, D]``.
    ``rows`` optionally restricts the computation to those query indices
    (the maths is row-independent); the result is then ``[B, H, len(rows), M]``.
    """
    if q.ndim == 4:
        B, H, N, D = q.shape
        q4 = q.astype(np.float64)
        k4 = k.astype(np.float64)
    else:
        B, N, C = q.shape
        H = num_heads
        D = C // H
        q4 = _to_bhnd(q, H)
        k4 = _to_bhnd(k, H)
    pad_head, pad_tail = padding
    n_padded = pad_head + N + pad_tail
    assert n_padded % score_block_size == 0
    M = n_padded // score_block_size
    scale = D ** -0.5
    if rows is None:
        rows = np.arange(N)
    rows = np.asarray(rows)
    out = np.zeros((B, H, len(rows), M), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            kk = k4[b, h]
            for c0 in range(0, len(rows), chunk):
                r = rows[c0 : c0 + chunk]
                s = (q4[b, h, r] * scale) @ kk.T
                s = s - s.max(axis=-1, keepdims=True)
                p = np.exp(s)
                p /= p.sum(axis=-1, keepdims=True)
                # keys live at padded coordinates p = t + pad_head; padded slots hold 0
                p_pad = np.zeros((len(r), n_padded), dtype=np.float64)
                p_pad[:, pad_head : pad_head + N] = p
                out[b, h, c0 : c0 + chunk] = p_pad.reshape(len(r), M, score_block_size).sum(-1)
    return out


def valid_counts(M: int, score_block_size: int, padding: Tuple[int, int]) -> np.ndarray:
    """Valid tokens per score block (v2/topk_select.py:152-156)."""
    pad_head, pad_tail = padding
    vc = np.full((M,), float(score_block_size), dtype=np.float32)
    if pad_head > 0:
        vc[0] = float(score_block_size - pad_head)
    if pad_tail > 0:
        vc[-1] = float(score_block_size - pad_tail)
    return vc


# --------------------------------------------------------------------------
# top-k select: v2/topk_select.py:128-182 (+ kernel rules)
# --------------------------------------------------------------------------


def topk_select(
    block_scores: np.ndarray,
    threshold: float,
    max_topk: int,
    score_block_size: int,
    padding: Tuple[int, int] = (0, 0),
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Sort by avg = raw / valid_count (desc, ties -> lower index), cumulative
    fp32 sum of raw' = avg * valid_count in sorted order, keep through the first
    position whose cumsum >= threshold (else all), cap at M_OUT.

    All arithmetic is fp32 so that a kernel fed the same fp32 block scores must
    agree bit for bit.  Returns (indices int32, raw f32, avg f32), ``[..., M_OUT]``.
    """
    raw = np.asarray(block_scores, dtype=np.float32)
    M = raw.shape[-1]
    vc = valid_counts(M, score_block_size, padding)
    avg = (raw / vc).astype(np.float32)
    m_out = min(max_topk, M) if max_topk > 0 else M
    order = np.argsort(-avg, axis=-1, kind="stable")[..., :m_out]
    sorted_avg = np.take_along_axis(avg, order, axis=-1)
    sorted_raw = (sorted_avg * vc[order]).astype(np.float32)
    cs = np.cumsum(sorted_raw, axis=-1, dtype=np.float32)
    exceed = cs >= np.float32(threshold)
    has = exceed.any(axis=-1)
    first = np.argmax(exceed, axis=-1)
    cut = np.where(has, first + 1, m_out)
    keep = np.arange(m_out) < cut[..., None]
    idx = np.where(keep, order, -1).astype(np.int32)
    raw_o = np.where(keep, sorted_raw, np.float32(0)).astype(np.float32)
    avg_o = np.where(keep, sorted_avg, np.float32(0)).astype(np.float32)
    return idx, raw_o, avg_o


# --------------------------------------------------------------------------
# q-block merge: v2/qblock_merge.py:27-82, v2/__init__.py:57-133
# --------------------------------------------------------------------------


def qblock_merge(
    topk_indices: np.ndarray,
    topk_scores: np.ndarray,
    q_block_size: int,
    qblock_topk: int,
    num_score_blocks: int,
) -> Tuple[np.ndarray, np.ndarray]:
    """Scatter-add (sequential fp32, (row, slot) order), keep positive entries
    sorted by score desc (ties -> lower id), truncate to ``qblock_topk``."""
    B, H, N, K = topk_indices.shape
    assert N % q_block_size == 0
    QM = N // q_block_size
    S = B * H * QM
    idx = topk_indices.reshape(S, q_block_size * K).astype(np.int64)
    scr = np.asarray(topk_scores, dtype=np.float32).reshape(S, q_block_size * K)
    Mt = num_score_blocks
    valid = (idx >= 0) & (idx < Mt)
    acc = np.zeros((S, Mt), dtype=np.float32)
    sl = np.broadcast_to(np.arange(S)[:, None], idx.shape)
    flat = (sl * Mt + np.where(valid, idx, 0))[valid]
    np.add.at(acc.reshape(-1), flat, scr[valid])  # sequential, in (row, slot) order
    order = np.argsort(-acc, axis=-1, kind="stable")
    vals = np.take_along_axis(acc, order, axis=-1)
    W = qblock_topk
    out_idx = np.full((S, W), -1, dtype=np.int32)
    out_scr = np.zeros((S, W), dtype=np.float32)
    w = min(W, Mt)
    pos = vals[:, :w] > 0
    out_idx[:, :w] = np.where(pos, order[:, :w], -1)
    out_scr[:, :w] = np.where(pos, vals[:, :w], 0)
    return out_idx.reshape(B, H, QM, W), out_scr.reshape(B, H, QM, W)


def build_qblock_topk_indices(
    topk_indices: np.ndarray,
    q_block_size: int,
    q_padding: Tuple[int, int] = (0, 0),
    topk_scores: Optional[np.ndarray] = None,
    qblock_topk: Optional[int] = None,
) -> Tuple[np.ndarray, np.ndarray, int]:
    """v2/__init__.py:57-133: q padding with -1 / 0, default W = g*K, ones
    scores for valid ids, num_score_blocks = max id + 1, counts = #valid."""
    B, H, N, K = topk_indices.shape
    ph, pt = q_padding
    idx = np.asarray(topk_indices).astype(np.int32)
    idx = np.pad(idx, ((0, 0), (0, 0), (ph, pt), (0, 0)), constant_values=-1)
    if qblock_topk is None:
        qblock_topk = q_block_size * K
    valid = idx >= 0
    nsb = int(idx[valid].max()) + 1 if valid.any() else 1
    if topk_scores is not None:
        scr = np.pad(np.asarray(topk_scores, dtype=np.float32),
                     ((0, 0), (0, 0), (ph, pt), (0, 0)), constant_values=0.0)
    else:
        scr = valid.astype(np.float32)
    merged, _ = qblock_merge(idx, scr, q_block_size, qblock_topk, nsb)
    counts = (merged >= 0).sum(-1).astype(np.int32)
    return merged, counts, merged.shape[-1]


# --------------------------------------------------------------------------
# sparse attention forward: v2/sparse_attn.py:24-127
# --------------------------------------------------------------------------


def _valid_tokens(blocks: Iterable[int], N: int, kv_block_size: int, kv_pad_head: int) -> np.ndarray:
    valid = np.zeros(N, dtype=bool)
    for bid in blocks:
        s = int(bid) * kv_block_size - kv_pad_head
        e = s + kv_block_size
        s, e = max(0, s), min(N, e)
        if s < e:
            valid[s:e] = True
    return valid


def _chunk_starts(blocks: Iterable[int], N: int, kv_block_size: int, kv_pad_head: int) -> np.ndarray:
    """For the valid tokens of ``_valid_tokens`` (ascending), the index of the
    64-key chunk each belongs to: chunks are the ascending blocks split every 64
    keys from the block start (virtual padding included)."""
    ids = sorted(set(int(x) for x in blocks))
    out, c = [], 0
    for m in ids:
        s0 = m * kv_block_size - kv_pad_head
        for j in range(0, kv_block_size, 64):
            lo, hi = max(0, s0 + j), min(N, s0 + min(j + 64, kv_block_size))
            if hi > lo:
                out.extend([c] * (hi - lo))
            c += 1
    return np.asarray(out, dtype=np.int64)


def _online_pv(s: np.ndarray, v: np.ndarray, chunk: np.ndarray, c: float, round_p: str,
               anchor_slack: float) -> np.ndarray:
    """o = sum_j round(P_j) v_j / sum_j P_j with P anchored to a lazily updated
    running maximum per row (see sparse_attn); s are the unscaled scores."""
    acc, l, _ = _online_pv_part(s, v, chunk, c, round_p, anchor_slack)
    return acc / l[:, None]


def _online_pv_part(s: np.ndarray, v: np.ndarray, chunk: np.ndarray, c: float, round_p: str,
                    anchor_slack: float) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The unnormalised (sum_j round(P_j) v_j, sum_j P_j, final anchor m) of
    _online_pv."""
    rows = s.shape[0]
    m = np.full(rows, -np.inf)
    acc = np.zeros((rows, v.shape[1]))
    l = np.zeros(rows)
    for ch in np.unique(chunk):
        sel = chunk == ch
        sc = s[:, sel]
        mx = sc.max(-1)
        mn = np.maximum(m, mx)
        with np.errstate(invalid="ignore"):
            grow = (mn - m) * c > anchor_slack
        alpha = np.where(grow, np.exp2(np.where(grow, (m - mn) * c, 0.0)), 1.0)
        acc *= alpha[:, None]
        l *= alpha
        m = np.where(grow, mn, m)
        p = np.exp2(sc * c - np.where(np.isfinite(m), m * c, 0.0)[:, None])
        l += p.sum(-1)
        acc += round_to(p, round_p) @ v[sel]
    return acc, l, m


def _split_parts(merged_bh: np.ndarray, q_block_size: int, N: int, q_pad_head: int, Mkv: int, splits: int,
                 p0: int, wg_rows: int = 256, seg: int = 512) -> dict:
    """Part of each KV block in the split forward walk of the workgroup whose
    padded query rows start at p0 (fta_sparse_attn_fwd_splits > 1): the union
    of the blocks listed by the q-blocks with valid rows in [p0, p0 + wg_rows),
    ascending per segment of `seg` blocks, cut into `splits` contiguous ranges
    of union positions [U sp / splits, U (sp + 1) / splits)."""
    QM = merged_bh.shape[0]
    g = q_block_size
    pend = p0 + wg_rows
    union = set()
    for qb in range(p0 // g, min((pend - 1) // g, QM - 1) + 1):
        lo = max(qb * g, p0, q_pad_head)
        hi = min(qb * g + g, pend, q_pad_head + N)
        if lo >= hi:
            continue
        union.update(int(m) for m in merged_bh[qb] if 0 <= m < Mkv)
    part = {}
    for seg0 in range(0, Mkv, seg):
        lst = sorted(m for m in union if seg0 <= m < seg0 + seg)
        U = len(lst)
        for sp in range(splits):
            for pos in range((U * sp) // splits, (U * (sp + 1)) // splits):
                part[lst[pos]] = sp
    return part


def sparse_attn(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    merged_indices: np.ndarray,
    num_heads: int,
    q_block_size: int,
    kv_block_size: int,
    scale: Optional[float] = None,
    q_padding: Tuple[int, int] = (0, 0),
    kv_padding: Tuple[int, int] = (0, 0),
    qblocks: Optional[Sequence[Tuple[int, int, int]]] = None,
    round_p: Optional[str] = None,
    anchor_slack: float = 8.0,
    splits: int = 1,
) -> Tuple[np.ndarray, np.ndarray]:
    """o [B, N, C] float64 and natural-log lse [B, H, N] (−inf and o = 0 for
    rows with no candidate token).  ``qblocks`` restricts the computation to the
    listed (b, h, qm) triples; other rows are left at o = 0 / lse = NaN.

    ``round_p``: the online-softmax schedule of a kernel, with P rounded to that
    16-bit type before its product with V (the normaliser sums unrounded P).
    The q-block's selected KV blocks are walked in ascending order in chunks of
    64 keys (a block of more than 64 keys spans several chunks); each row keeps
    a running maximum m and P = 2^(c s - c m), c = scale * log2(e).  m is
    re-anchored to the row maximum seen so far when that exceeds it by more than
    ``anchor_slack`` in log2 units (this build's kernels: 8; 0 re-anchors
    whenever the maximum grows, as the reference's kernel does,
    v2/csrc/sparse_attn_kernel.cuh:145-160), and the accumulators are scaled by
    2^(c m_old - c m_new) then.  ``splits`` > 1 models this build's split
    forward (small grids, fta_sparse_attn_fwd_splits): each 256-row workgroup's
    union walk is cut into that many parts (_split_parts), each part runs the
    schedule above from its own anchor, and the parts are merged as
    o = sum_p acc_p 2^(c m_p - c m) / sum_p l_p 2^(c m_p - c m), m = max m_p."""
    B, N, C = q.shape
    H = num_heads
    D = C // H
    q4, k4, v4 = _to_bhnd(q, H), _to_bhnd(k, H), _to_bhnd(v, H)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ph = q_padding[0]
    kph = kv_padding[0]
    QM = merged_indices.shape[2]
    o = np.zeros((B, H, N, D), dtype=np.float64)
    lse = np.full((B, H, N), -np.inf if qblocks is None else np.nan, dtype=np.float64)
    if qblocks is None:
        qblocks = [(b, h, qm) for b in range(B) for h in range(H) for qm in range(QM)]
    for b, h, qm in qblocks:
        r0 = qm * q_block_size - ph
        rs, re = max(0, r0), min(N, r0 + q_block_size)
        if rs >= re:
            continue
        lse[b, h, rs:re] = -np.inf
        ids = merged_indices[b, h, qm]
        valid = _valid_tokens(ids[ids >= 0], N, kv_block_size, kph)
        if not valid.any():
            continue
        s = (q4[b, h, rs:re] * scale) @ k4[b, h, valid].T
        row_lse = _logsumexp(s)
        if round_p is None:
            p = np.exp(s - row_lse[:, None])
            o[b, h, rs:re] = p @ v4[b, h, valid]
        elif splits <= 1:
            o[b, h, rs:re] = _online_pv(s / scale, v4[b, h, valid], _chunk_starts(ids[ids >= 0], N, kv_block_size,
                                                                                    kph),
                                        scale * math.log2(math.e), round_p, anchor_slack)
        else:
            c = scale * math.log2(math.e)
            chunk = _chunk_starts(ids[ids >= 0], N, kv_block_size, kph)
            tok_blk = (np.nonzero(valid)[0] + kph) // kv_block_size
            Mkv = (kph + N + kv_padding[1]) // kv_block_size
            r = rs
            while r < re:  # rows of one workgroup share its parts
                p0 = ((r + ph) // 256) * 256
                r1 = min(re, p0 + 256 - ph)
                part = _split_parts(merged_indices[b, h], q_block_size, N, ph, Mkv, splits, p0)
                tp = np.array([part.get(int(m), -1) for m in tok_blk])
                rows = r1 - r
                acc = np.zeros((rows, D))
                lsum = np.zeros(rows)
                parts = []
                for sp in range(splits):
                    sel = tp == sp
                    if sel.any():
                        parts.append(_online_pv_part(s[r - rs:r1 - rs][:, sel] / scale, v4[b, h, valid][sel],
                                                     chunk[sel], c, round_p, anchor_slack))
                mm = np.max([np.where(l_ > 0, m_, -np.inf) for _, l_, m_ in parts], axis=0)
                for a_, l_, m_ in parts:
                    with np.errstate(invalid="ignore"):
                        w = np.where(l_ > 0, np.exp2(c * (m_ - mm)), 0.0)
                    acc += np.where(l_ > 0, w, 0.0)[:, None] * np.nan_to_num(a_)
                    lsum += np.where(l_ > 0, w * l_, 0.0)
                o[b, h, r:r1] = acc / lsum[:, None]
                r = r1
        lse[b, h, rs:re] = row_lse
    return _from_bhnd(o), lse


# --------------------------------------------------------------------------
# backward: v2/sparse_attn_bwd.py:12-294
# --------------------------------------------------------------------------


def preprocess_delta(o: np.ndarray, do: np.ndarray, num_heads: int) -> np.ndarray:
    """delta[b, h, n] = sum_d O * dO (v2/sparse_attn_bwd.py:12-33)."""
    return (_to_bhnd(o, num_heads) * _to_bhnd(do, num_heads)).sum(-1)


def build_reverse_indices(
    merged_indices: np.ndarray, counts: np.ndarray, num_kv_blocks: int
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """KV block -> ascending list of q-blocks that selected it
    (v2/sparse_attn_bwd.py:36-76), plus the per-(b, h) stable descending
    argsort of the reverse counts (v2/csrc/build_reverse_indices_kernel.cu:29-62)."""
    B, H, QM, W = merged_indices.shape
    M = num_kv_blocks
    rev = np.full((B, H, M, QM), -1, dtype=np.int32)
    cnt = np.zeros((B, H, M), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            sel = np.zeros((M, QM), dtype=bool)
            for qm in range(QM):
                ids = merged_indices[b, h, qm, : int(counts[b, h, qm])]
                ids = ids[(ids >= 0) & (ids < M)]
                sel[ids, qm] = True
            for m in range(M):
                qs = np.nonzero(sel[m])[0]
                rev[b, h, m, : len(qs)] = qs
                cnt[b, h, m] = len(qs)
    sorted_kv = np.argsort(-cnt, axis=-1, kind="stable").astype(np.int32)
    return rev, cnt, sorted_kv


def sort_by_count(reverse_counts: np.ndarray, num_heads: int, num_kv_blocks: int) -> Tuple[np.ndarray, np.ndarray]:
    """Global stable descending sort of reverse counts (v2/sparse_attn_bwd.py:79-108)."""
    flat = np.asarray(reverse_counts).reshape(-1)
    order = np.argsort(-flat.astype(np.int64), kind="stable")
    return flat[order].astype(np.int32), order.astype(np.int32)


def sparse_attn_bwd(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    do: np.ndarray,
    merged_indices: np.ndarray,
    num_heads: int,
    q_block_size: int,
    kv_block_size: int,
    scale: Optional[float] = None,
    q_padding: Tuple[int, int] = (0, 0),
    kv_padding: Tuple[int, int] = (0, 0),
    qblocks: Optional[Sequence[Tuple[int, int, int]]] = None,
    round_p: Optional[str] = None,
    lse: Optional[np.ndarray] = None,
    delta: Optional[np.ndarray] = None,
) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """dQ, dK, dV (float64, [B, N, C]) following bwd_dq_naive / bwd_dkv_naive
    (v2/sparse_attn_bwd.py:111-294): P = softmax over the q-block's candidate
    tokens, dP = dO V^T, delta = rowsum(dO * (P V)), dS = P (dP - delta),
    dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO.  ``qblocks`` restricts the
    sum to the listed (b, h, qm) triples (dK/dV then hold partial sums).

    ``lse`` [B, H, N] (natural log) replaces the row normaliser, so that
    P = exp(s - lse) as in the backward kernels, which read the forward's lse;
    ``delta`` [B, H, N] replaces rowsum(dO * (P V)) (the reference computes it
    from the forward's stored output, v2/sparse_attn.py:177).  ``round_p``
    rounds P before P^T dO and dS before dS K / dS^T Q."""
    B, N, C = q.shape
    H = num_heads
    D = C // H
    q4, k4, v4, do4 = _to_bhnd(q, H), _to_bhnd(k, H), _to_bhnd(v, H), _to_bhnd(do, H)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ph = q_padding[0]
    kph = kv_padding[0]
    QM = merged_indices.shape[2]
    dq = np.zeros_like(q4)
    dk = np.zeros_like(k4)
    dv = np.zeros_like(v4)
    if qblocks is None:
        qblocks = [(b, h, qm) for b in range(B) for h in range(H) for qm in range(QM)]
    for b, h, qm in qblocks:
        r0 = qm * q_block_size - ph
        rs, re = max(0, r0), min(N, r0 + q_block_size)
        if rs >= re:
            continue
        ids = merged_indices[b, h, qm]
        valid = _valid_tokens(ids[ids >= 0], N, kv_block_size, kph)
        if not valid.any():
            continue
        qq, dd = q4[b, h, rs:re], do4[b, h, rs:re]
        kk, vv = k4[b, h, valid], v4[b, h, valid]
        s = (qq * scale) @ kk.T
        norm = _logsumexp(s) if lse is None else np.asarray(lse[b, h, rs:re], dtype=np.float64)
        p = np.exp(s - norm[:, None])
        dp = dd @ vv.T
        if delta is None:
            dl = (dd * (p @ vv)).sum(-1, keepdims=True)
        else:
            dl = np.asarray(delta[b, h, rs:re], dtype=np.float64)[:, None]
        ds = p * (dp - dl)
        dsr = round_to(ds, round_p)
        dq[b, h, rs:re] += scale * dsr @ kk
        dk[b, h, valid] += scale * dsr.T @ qq
        dv[b, h, valid] += round_to(p, round_p).T @ dd
    return _from_bhnd(dq), _from_bhnd(dk), _from_bhnd(dv)


__all__ = [
    "block_score",
    "valid_counts",
    "topk_select",
    "qblock_merge",
    "build_qblock_topk_indices",
    "sparse_attn",
    "preprocess_delta",
    "build_reverse_indices",
    "sort_by_count",
    "sparse_attn_bwd",
]


# --------------------------------------------------------------------------
# V1 compatibility layer: v1/attention.py, v1/scoring.py
# --------------------------------------------------------------------------


def _next_pow2(x: int) -> int:
    return 1 if x <= 0 else 1 << (x - 1).bit_length()


def v1_qblock_union(
    topk_indices: np.ndarray, q_block_size: int, q_padding: Tuple[int, int] = (0, 0)
) -> Tuple[np.ndarray, np.ndarray, int]:
    """v1/attention.py:23-138: per q-block, the ascending unique non-negative
    ids of its rows' top-k entries (rows padded with -1), -1 filled to
    ``S_MAX = next_pow2(q_block_size * K)``; counts = number of ids."""
    B, H, N, K = topk_indices.shape
    ph, pt = q_padding
    idx = np.pad(np.asarray(topk_indices).astype(np.int64), ((0, 0), (0, 0), (ph, pt), (0, 0)), constant_values=-1)
    QM = (ph + N + pt) // q_block_size
    S = _next_pow2(q_block_size * K)
    merged = np.full((B, H, QM, S), -1, dtype=np.int32)
    counts = np.zeros((B, H, QM), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            for qm in range(QM):
                ids = idx[b, h, qm * q_block_size:(qm + 1) * q_block_size].reshape(-1)
                u = np.unique(ids[ids >= 0])
                merged[b, h, qm, :len(u)] = u
                counts[b, h, qm] = len(u)
    return merged, counts, S


def v1_topk_score(
    q: np.ndarray,
    k: np.ndarray,
    v: Optional[np.ndarray],
    num_heads: Optional[int],
    score_block_size: int,
    topk: int,
    padding: Tuple[int, int] = (0, 0),
) -> Tuple[Optional[np.ndarray], np.ndarray, np.ndarray]:
    """v1/scoring.py:1360-1469.  Block scores are the softmax mass per block
    (float64), divided by the block's valid token count when padding is used
    (the count rule of ``valid_counts``); the top ``min(topk, M)`` are returned
    in descending order, ties to the lower index.  With ``v``, also the dense
    attention output ``o`` ([B, N, C] float64; q/k/v 3D only)."""
    bs = block_score(q, k, num_heads, score_block_size, padding)
    M = bs.shape[-1]
    if padding != (0, 0):
        bs = bs / valid_counts(M, score_block_size, padding).astype(np.float64)
    kk = min(topk, M)
    order = np.argsort(-bs, axis=-1, kind="stable")[..., :kk]
    scores = np.take_along_axis(bs, order, axis=-1)
    o = None
    if v is not None:
        B, N, C = q.shape
        H = num_heads
        Dh = C // H
        q4, k4, v4 = _to_bhnd(q, H), _to_bhnd(k, H), _to_bhnd(v, H)
        s = np.einsum("bhqd,bhkd->bhqk", q4 * Dh ** -0.5, k4)
        p = np.exp(s - _logsumexp(s)[..., None])
        o = _from_bhnd(np.einsum("bhqk,bhkd->bhqd", p, v4))
    return o, order.astype(np.int32), scores


def v1_sparse_attn(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    merged_indices: np.ndarray,
    counts: np.ndarray,
    num_heads: int,
    q_block_size: int,
    kv_block_size: int,
    scale: Optional[float] = None,
    kv_padding: Tuple[int, int] = (0, 0),
    q_padding: Tuple[int, int] = (0, 0),
    S_MAX: Optional[int] = None,
) -> Tuple[np.ndarray, np.ndarray]:
    """v1/attention.py:423-647: softmax over the union of the first
    ``min(count, S_MAX)`` ids of each q-block (heads share row 0 when
    ``merged.shape[1] == 1``); o = 0, lse = -inf for empty q-blocks."""
    B, N, C = q.shape
    H = num_heads
    merged = np.asarray(merged_indices).astype(np.int64)
    if S_MAX is None:
        S_MAX = merged.shape[-1]
    W = min(S_MAX, merged.shape[-1])
    merged = merged[..., :W]
    cnt = np.minimum(np.asarray(counts).astype(np.int64), W)
    merged = np.where(np.arange(W) < cnt[..., None], merged, -1)
    if merged.shape[1] == 1:
        merged = np.broadcast_to(merged, (B, H) + merged.shape[2:])
    return sparse_attn(q, k, v, merged, H, q_block_size, kv_block_size, scale, q_padding, kv_padding)
