"""Pins the CPU oracle (oracle/fta_oracle.py) against independent checks.

The reference ships no tests, fixtures or golden vectors, so every oracle
function is pinned here by brute force on tiny inputs, by special cases that
reduce to a library routine (torch softmax / SDPA / autograd), and by
invariants.  Each check is chosen so that a plausible slip (wrong tie
direction, dropped padding term, transposed operand, off-by-one cut) fails.
"""

import math
from collections import Counter

import numpy as np
import pytest
import torch

import fta_oracle as O


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- block score


def _brute_block_score(q, k, H, b, padding):
    B, N, C = q.shape
    D = C // H
    ph, pt = padding
    M = (ph + N + pt) // b
    out = np.zeros((B, H, N, M))
    for bb in range(B):
        for h in range(H):
            for n in range(N):
                s = [sum(q[bb, n, h * D + d] * k[bb, t, h * D + d] for d in range(D)) / math.sqrt(D)
                     for t in range(N)]
                mx = max(s)
                e = [math.exp(x - mx) for x in s]
                tot = sum(e)
                for t in range(N):
                    out[bb, h, n, (t + ph) // b] += e[t] / tot
    return out


@pytest.mark.parametrize("padding", [(0, 2), (1, 1), (2, 0)])
def test_block_score_brute_force(padding):
    r = _rng(0)
    B, N, H, D, b = 1, 7, 2, 4, 3
    if (padding[0] + N + padding[1]) % b:
        pytest.skip("not divisible")
    q = r.standard_normal((B, N, H * D))
    k = r.standard_normal((B, N, H * D))
    got = O.block_score(q, k, H, b, padding)
    ref = _brute_block_score(q, k, H, b, padding)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-12)


def test_block_score_b1_is_softmax_and_4d_layout():
    r = _rng(1)
    B, N, H, D = 2, 16, 3, 8
    q = r.standard_normal((B, N, H * D)).astype(np.float32)
    k = r.standard_normal((B, N, H * D)).astype(np.float32)
    got = O.block_score(q, k, H, 1)
    qt = torch.from_numpy(q).double().view(B, N, H, D).transpose(1, 2)
    kt = torch.from_numpy(k).double().view(B, N, H, D).transpose(1, 2)
    ref = torch.softmax(qt @ kt.transpose(-1, -2) / math.sqrt(D), dim=-1).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-15)
    # 4D input [B, H, N, D] gives the same result
    got4 = O.block_score(qt.numpy(), kt.numpy(), None, 1)
    np.testing.assert_allclose(got4, got, rtol=1e-12)
    # row subset
    rows = np.array([3, 0, 15])
    np.testing.assert_allclose(O.block_score(q, k, H, 1, rows=rows), got[:, :, rows], rtol=1e-12)


# ---------------------------------------------------------------- top-k select


def _brute_topk(scores, thr, topk, b, padding):
    M = len(scores)
    ph, pt = padding
    vc = [float(b)] * M
    if ph:
        vc[0] = float(b - ph)
    if pt:
        vc[-1] = float(b - pt)
    avg = [np.float32(np.float32(s) / np.float32(c)) for s, c in zip(scores, vc)]
    order = sorted(range(M), key=lambda j: (-float(avg[j]), j))
    m_out = min(topk, M) if topk > 0 else M
    cs = np.float32(0)
    cut = m_out
    for p in range(m_out):
        cs = np.float32(cs + np.float32(avg[order[p]] * np.float32(vc[order[p]])))
        if cs >= np.float32(thr):
            cut = p + 1
            break
    idx = [order[p] if p < cut else -1 for p in range(m_out)]
    avg_o = [float(avg[order[p]]) if p < cut else 0.0 for p in range(m_out)]
    return idx, avg_o


@pytest.mark.parametrize("thr,topk,padding", [(1.0, 0, (0, 0)), (0.5, 4, (0, 0)), (0.9, 8, (3, 5)),
                                              (2.0, 6, (7, 0)), (0.0, 5, (0, 0))])
def test_topk_select_brute_force(thr, topk, padding):
    r = _rng(2)
    b, M = 8, 12
    raw = r.dirichlet(np.ones(M), size=(1, 2, 5)).astype(np.float32)
    idx, rw, av = O.topk_select(raw, thr, topk, b, padding)
    for h in range(2):
        for n in range(5):
            bi, ba = _brute_topk(raw[0, h, n], thr, topk, b, padding)
            assert list(idx[0, h, n]) == bi
            np.testing.assert_array_equal(av[0, h, n], np.float32(ba))


def test_topk_select_ties_go_to_lower_index():
    raw = np.array([[[[0.1, 0.3, 0.3, 0.1, 0.2]]]], dtype=np.float32)
    idx, _, _ = O.topk_select(raw, 2.0, 0, 4)
    assert idx[0, 0, 0].tolist() == [1, 2, 4, 0, 3]


def test_topk_select_partial_block_normalisation():
    # block 0 only holds 2 valid tokens: its average beats a larger raw score
    raw = np.array([[[[0.3, 0.4, 0.3]]]], dtype=np.float32)
    idx, rw, av = O.topk_select(raw, 0.5, 3, 4, (2, 0))
    assert idx[0, 0, 0].tolist() == [0, 1, -1]
    np.testing.assert_allclose(av[0, 0, 0, :2], [0.15, 0.1], rtol=1e-6)
    np.testing.assert_allclose(rw[0, 0, 0, :2], [0.3, 0.4], rtol=1e-6)


def test_topk_select_threshold_one_and_full_sort():
    r = _rng(3)
    raw = r.random((1, 1, 4, 9)).astype(np.float32)
    idx, _, av = O.topk_select(raw, 1e9, 0, 2)
    for n in range(4):
        assert idx[0, 0, n].tolist() == sorted(range(9), key=lambda j: (-raw[0, 0, n, j], j))
        assert np.all(np.diff(av[0, 0, n]) <= 0)


# ---------------------------------------------------------------- merge


def test_merge_ones_is_count_union():
    r = _rng(4)
    B, H, N, K, g, M = 1, 2, 16, 3, 4, 10
    idx = np.stack([r.permutation(M)[:K] for _ in range(B * H * N)]).reshape(B, H, N, K).astype(np.int32)
    idx[0, 0, 3, 2] = -1
    merged, counts, W = O.build_qblock_topk_indices(idx, g)
    assert W == g * K
    for h in range(H):
        for qm in range(N // g):
            c = Counter(int(x) for x in idx[0, h, qm * g:(qm + 1) * g].ravel() if x >= 0)
            exp = sorted(c, key=lambda j: (-c[j], j))
            got = merged[0, h, qm]
            assert got[: len(exp)].tolist() == exp
            assert np.all(got[len(exp):] == -1)
            assert counts[0, h, qm] == len(exp)


def test_merge_scores_truncation_and_padding():
    idx = np.array([[[[2, 0], [0, -1], [5, 2], [1, 3]]]], dtype=np.int32)
    scr = np.array([[[[0.5, 0.25], [0.25, 9.0], [0.125, 0.5], [0.0, 0.75]]]], dtype=np.float32)
    # q_padding=(1,1) with g=3: rows -> [-1, r0, r1 | r2, r3, -1]
    merged, counts, W = O.build_qblock_topk_indices(idx, 3, (1, 1), scr, qblock_topk=3)
    # q-block 0: {2:.5, 0:.25+.25=.5} -> tie -> 0 then 2 ; q-block 1: {5:.125, 2:.5, 1:0, 3:.75}
    assert merged[0, 0, 0].tolist() == [0, 2, -1]
    assert merged[0, 0, 1].tolist() == [3, 2, 5]
    assert counts[0, 0].tolist() == [2, 3]


def test_merge_sequential_fp32_order():
    # 1 + 1e-8 + 1e-8 ... in (row, slot) order loses the small terms in fp32
    idx = np.zeros((1, 1, 4, 1), dtype=np.int32)
    scr = np.array([1.0, 1e-8, 1e-8, 1e-8], dtype=np.float32).reshape(1, 1, 4, 1)
    _, ms = O.qblock_merge(idx, scr, 4, 1, 1)
    assert ms[0, 0, 0, 0] == np.float32(1.0)


# ---------------------------------------------------------------- attention fwd/bwd


def _torch_masked_dense(q, k, v, merged, H, g, b, scale, qpad, kvpad):
    """Independent torch restatement (v2/sparse_attn.py:395-485) with autograd."""
    B, N, C = q.shape
    D = C // H
    QM = merged.shape[2]
    mask = torch.zeros(B, H, N, N, dtype=torch.bool)
    for bb in range(B):
        for h in range(H):
            for qm in range(QM):
                r0 = qm * g - qpad[0]
                rs, re = max(0, r0), min(N, r0 + g)
                for bid in merged[bb, h, qm]:
                    if bid < 0:
                        continue
                    ks, ke = max(0, bid * b - kvpad[0]), min(N, bid * b - kvpad[0] + b)
                    if rs < re and ks < ke:
                        mask[bb, h, rs:re, ks:ke] = True
    qh = q.view(B, N, H, D).transpose(1, 2)
    kh = k.view(B, N, H, D).transpose(1, 2)
    vh = v.view(B, N, H, D).transpose(1, 2)
    s = (qh * scale) @ kh.transpose(-1, -2)
    s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, -1)
    p = torch.softmax(s, -1).nan_to_num(0.0)
    o = (p @ vh).transpose(1, 2).reshape(B, N, C)
    return o, lse


@pytest.mark.parametrize("g,b,qpad,kvpad", [(3, 6, (0, 0), (0, 0)), (4, 5, (1, 1), (2, 0)), (5, 4, (3, 4), (1, 1))])
def test_sparse_attn_fwd_bwd_vs_torch_autograd(g, b, qpad, kvpad):
    r = _rng(5)
    B, N, H, D = 2, 18, 2, 8
    if (qpad[0] + N + qpad[1]) % g or (kvpad[0] + N + kvpad[1]) % b:
        pytest.skip("bad padding")
    QM = (qpad[0] + N + qpad[1]) // g
    M = (kvpad[0] + N + kvpad[1]) // b
    merged = np.full((B, H, QM, 3), -1, dtype=np.int32)
    for bb in range(B):
        for h in range(H):
            for qm in range(QM):
                n = r.integers(0, 4)
                merged[bb, h, qm, :n] = r.permutation(M)[:n]
    q, k, v, do = (r.standard_normal((B, N, H * D)) for _ in range(4))
    scale = 0.3
    o, lse = O.sparse_attn(q, k, v, merged, H, g, b, scale, qpad, kvpad)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    ot, lset = _torch_masked_dense(qt, kt, vt, merged, H, g, b, scale, qpad, kvpad)
    np.testing.assert_allclose(o, ot.detach().numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_array_equal(np.isinf(lse), torch.isinf(lset).numpy())
    fin = np.isfinite(lse)
    np.testing.assert_allclose(lse[fin], lset.detach().numpy()[fin], rtol=1e-10)
    ot.backward(torch.tensor(do))
    dq, dk, dv = O.sparse_attn_bwd(q, k, v, do, merged, H, g, b, scale, qpad, kvpad)
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, kt.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-9, atol=1e-11)
    # delta = rowsum(O * dO)
    dl = O.preprocess_delta(o, do, H)
    np.testing.assert_allclose(dl, (ot.detach().numpy() * do).reshape(B, N, H, D).sum(-1).transpose(0, 2, 1))


def test_sparse_attn_all_blocks_is_dense_sdpa():
    r = _rng(6)
    B, N, H, D, g, b = 1, 32, 2, 16, 8, 8
    M, QM = N // b, N // g
    merged = np.tile(np.arange(M, dtype=np.int32)[::-1], (B, H, QM, 1))
    q, k, v = (r.standard_normal((B, N, H * D)).astype(np.float32) for _ in range(3))
    o, lse = O.sparse_attn(q, k, v, merged, H, g, b)
    th = [torch.from_numpy(x).double().view(B, N, H, D).transpose(1, 2) for x in (q, k, v)]
    ref = torch.nn.functional.scaled_dot_product_attention(*th).transpose(1, 2).reshape(B, N, H * D)
    np.testing.assert_allclose(o, ref.numpy(), rtol=1e-10, atol=1e-12)
    ref_lse = torch.logsumexp(th[0] @ th[1].transpose(-1, -2) / math.sqrt(D), -1)
    np.testing.assert_allclose(lse, ref_lse.numpy(), rtol=1e-12)


def test_empty_qblock_gives_zero_and_neg_inf():
    r = _rng(7)
    q, k, v = (r.standard_normal((1, 8, 4)) for _ in range(3))
    merged = np.full((1, 1, 2, 2), -1, dtype=np.int32)
    merged[0, 0, 1, 0] = 1
    o, lse = O.sparse_attn(q, k, v, merged, 1, 4, 4)
    assert np.all(o[0, :4] == 0) and np.all(np.isneginf(lse[0, 0, :4]))
    assert np.all(np.isfinite(lse[0, 0, 4:]))


# ---------------------------------------------------------------- reverse index / sort


def test_reverse_indices_brute_force():
    r = _rng(8)
    B, H, QM, W, M = 1, 3, 9, 4, 7
    merged = np.full((B, H, QM, W), -1, dtype=np.int32)
    counts = np.zeros((B, H, QM), dtype=np.int32)
    for h in range(H):
        for qm in range(QM):
            n = r.integers(0, W + 1)
            merged[0, h, qm, :n] = r.permutation(M)[:n]
            counts[0, h, qm] = n
    rev, cnt, skv = O.build_reverse_indices(merged, counts, M)
    for h in range(H):
        lists = {m: [] for m in range(M)}
        for qm in range(QM):
            for s in range(counts[0, h, qm]):
                lists[int(merged[0, h, qm, s])].append(qm)
        for m in range(M):
            assert rev[0, h, m, : cnt[0, h, m]].tolist() == sorted(lists[m])
            assert np.all(rev[0, h, m, cnt[0, h, m]:] == -1)
        assert skv[0, h].tolist() == sorted(range(M), key=lambda m: (-len(lists[m]), m))
    sc, sid = O.sort_by_count(cnt, H, M)
    flat = cnt.ravel().tolist()
    assert sid.tolist() == sorted(range(len(flat)), key=lambda i: (-flat[i], i))
    assert sc.tolist() == [flat[i] for i in sid]


# ---------------------------------------------------------------- V1 layer


def test_v1_union_brute_force():
    r = _rng(20)
    B, H, N, K, g, qpad = 2, 2, 37, 5, 8, (1, 2)
    ids = r.integers(-1, 12, (B, H, N, K))
    merged, counts, S = O.v1_qblock_union(ids, g, qpad)
    assert S == 64  # next_pow2(8 * 5)
    QM = (1 + N + 2) // g
    for b in range(B):
        for h in range(H):
            for qm in range(QM):
                want = set()
                for j in range(g):
                    n = qm * g + j - qpad[0]
                    if 0 <= n < N:
                        want |= {int(x) for x in ids[b, h, n] if x >= 0}
                row = merged[b, h, qm]
                assert counts[b, h, qm] == len(want)
                assert list(row[:len(want)]) == sorted(want)
                assert np.all(row[len(want):] == -1)


def test_v1_topk_score_is_sorted_block_mass_and_dense_o():
    r = _rng(21)
    B, N, H, D, b = 1, 24, 2, 8, 8
    q, k, v = (r.standard_normal((B, N, H * D)) for _ in range(3))
    o, idx, sc = O.v1_topk_score(q, k, v, H, b, 3)
    brute = _brute_block_score(q, k, H, b, (0, 0))
    # topk = M: every block, in descending mass, and the masses sum to 1
    np.testing.assert_allclose(sc.sum(-1), 1.0, rtol=1e-12)
    for bb in range(B):
        for h in range(H):
            for n in range(N):
                order = sorted(range(3), key=lambda m: (-brute[bb, h, n, m], m))
                assert list(idx[bb, h, n]) == order
                np.testing.assert_allclose(sc[bb, h, n], brute[bb, h, n, order], rtol=1e-10)
    th = [torch.from_numpy(x).view(B, N, H, D).transpose(1, 2) for x in (q, k, v)]
    ref = torch.nn.functional.scaled_dot_product_attention(*th).transpose(1, 2).reshape(B, N, H * D)
    np.testing.assert_allclose(o, ref.numpy(), rtol=1e-10, atol=1e-12)


def test_v1_topk_score_padding_divides_by_valid_count():
    r = _rng(22)
    B, N, H, D, b, pad = 1, 13, 1, 4, 8, (3, 0)
    q, k = (r.standard_normal((B, N, H * D)) for _ in range(2))
    _, idx, sc = O.v1_topk_score(q, k, None, H, b, 2, pad)
    brute = _brute_block_score(q, k, H, b, pad)
    per_tok = brute / np.array([5.0, 8.0])  # block 0 holds 8 - 3 real tokens
    for n in range(N):
        order = sorted(range(2), key=lambda m: (-per_tok[0, 0, n, m], m))
        assert list(idx[0, 0, n]) == order
        np.testing.assert_allclose(sc[0, 0, n], per_tok[0, 0, n, order], rtol=1e-10)


def test_v1_sparse_attn_counts_and_shared_heads():
    r = _rng(23)
    B, N, H, D, g, b = 1, 16, 2, 4, 8, 4
    q, k, v = (r.standard_normal((B, N, H * D)) for _ in range(3))
    merged = np.array([[[[0, 2, 3, -1], [1, 3, 0, 2]]]], dtype=np.int32)  # H_BI = 1
    counts = np.array([[[2, 4]]], dtype=np.int32)
    o, lse = O.v1_sparse_attn(q, k, v, merged, counts, H, g, b, S_MAX=3)
    # q-block 0 uses blocks {0, 2}; q-block 1 uses the first 3 ids {1, 3, 0}; both heads alike
    q4, k4, v4 = (x.reshape(B, N, H, D).transpose(0, 2, 1, 3) for x in (q, k, v))
    for h in range(H):
        for qm, blocks in ((0, [0, 2]), (1, [1, 3, 0])):
            toks = [t for m in blocks for t in range(m * b, m * b + b)]
            s = q4[0, h, qm * g:(qm + 1) * g] @ k4[0, h, toks].T / math.sqrt(D)
            p = np.exp(s - s.max(-1, keepdims=True))
            ref_lse = np.log(p.sum(-1)) + s.max(-1)
            ref_o = (p / p.sum(-1, keepdims=True)) @ v4[0, h, toks]
            np.testing.assert_allclose(lse[0, h, qm * g:(qm + 1) * g], ref_lse, rtol=1e-12)
            np.testing.assert_allclose(o.reshape(B, N, H, D)[0, qm * g:(qm + 1) * g, h], ref_o, rtol=1e-10)


# ---------------------------------------------------------- 16-bit rounding modes


def test_round_to_matches_torch_conversions():
    """bf16 / fp16 round-to-nearest-even from float32, as torch converts (an
    independent implementation), including ties, subnormals and overflow."""
    rng = _rng(40)
    x = rng.standard_normal(20000) * np.exp(rng.uniform(-40, 40, 20000))
    # exact ties between two bf16 / fp16 neighbours
    x = np.concatenate([x, [1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 1e-40, 7e4, -np.inf]])
    for kind, tdt in (("bf16", torch.bfloat16), ("fp16", torch.float16)):
        ref = torch.from_numpy(x).float().to(tdt).double().numpy()
        np.testing.assert_array_equal(O.round_to(x, kind), ref)
    assert O.round_to(np.array([1 + 2.0 ** -8]), "bf16")[0] == 1.0  # tie to even
    assert O.round_to(np.array([1 + 3 * 2.0 ** -8]), "bf16")[0] == 1 + 2.0 ** -6


@pytest.mark.parametrize("slack", [0.0, 8.0, 1e9])
def test_online_softmax_schedule_without_rounding_is_softmax(slack):
    """The forward rounding mode's online softmax (chunked, lazily re-anchored
    running maximum) equals softmax(s) V when nothing is rounded, for any
    chunking and anchor slack: a wrong rescale factor, sign or a dropped
    chunk fails this."""
    rng = _rng(41)
    R, T, D = 5, 300, 16
    s = rng.standard_normal((R, T)) * 6
    s[:, 150:] += 30  # a later chunk raises the maximum far beyond the slack
    v = rng.standard_normal((T, D))
    chunk = np.sort(rng.integers(0, 9, T))
    c = 0.7
    got = O._online_pv(s, v, chunk, c, None, slack)
    w = np.exp2(c * (s - s.max(-1, keepdims=True)))
    np.testing.assert_allclose(got, (w / w.sum(-1, keepdims=True)) @ v, rtol=1e-12, atol=1e-12)


def test_split_parts_partition_the_workgroup_union():
    """_split_parts (the split forward's parts): the parts of one workgroup
    cover exactly the union of the blocks listed by its q-blocks with valid
    rows, per 512-block segment in ascending order, in contiguous ranges whose
    sizes differ by at most one; q-blocks whose rows all lie in padding or in
    another workgroup add nothing."""
    rng = _rng(43)
    g, N, ph, Mkv = 48, 1000, 40, 1300
    QM = (ph + N + 8) // g
    merged = np.full((QM, 20), -1, dtype=np.int32)
    for qb in range(QM):
        n = int(rng.integers(0, 21))
        merged[qb, :n] = rng.permutation(Mkv)[:n]
    for splits in (2, 3, 4):
        for p0 in (0, 256, 768):
            part = O._split_parts(merged, g, N, ph, Mkv, splits, p0)
            want = set()
            for qb in range(QM):
                lo, hi = max(qb * g, p0, ph), min(qb * g + g, p0 + 256, ph + N)
                if lo < hi:
                    want.update(int(m) for m in merged[qb] if m >= 0)
            assert set(part) == want
            for seg0 in (0, 512, 1024):
                lst = sorted(m for m in want if seg0 <= m < seg0 + 512)
                sps = [part[m] for m in lst]
                assert sps == sorted(sps)  # contiguous, ascending
                sizes = [sps.count(sp) for sp in range(splits)]
                assert max(sizes) - min(sizes) <= 1 and sum(sizes) == len(lst)


@pytest.mark.parametrize("splits", [1, 2, 3, 4])
def test_split_schedule_without_rounding_is_softmax(splits):
    """The split forward's schedule (per-part anchors, then the merge of the
    parts' (acc, l, m)) equals the exact softmax(s) V when nothing is rounded,
    over several workgroups, padding and two 512-block segments (one-key KV
    blocks): a wrong part weight, sign or a dropped part fails this."""
    rng = _rng(44)
    B, N, H, D, g, b = 1, 600, 2, 16, 32, 1
    qpad, kvpad = (8, 24), (0, 0)
    QM = (qpad[0] + N + qpad[1]) // g
    merged = np.full((B, H, QM, 300), -1, dtype=np.int32)
    for h in range(H):
        for qm in range(QM):
            n = int(rng.integers(0, 301))
            merged[0, h, qm, :n] = rng.permutation(N)[:n]
    q = rng.standard_normal((B, N, H * D)) * 3
    k = rng.standard_normal((B, N, H * D))
    v = rng.standard_normal((B, N, H * D))
    o64, l64 = O.sparse_attn(q, k, v, merged, H, g, b, None, qpad, kvpad)
    os_, ls = O.sparse_attn(q, k, v, merged, H, g, b, None, qpad, kvpad, round_p="f64", splits=splits)
    np.testing.assert_allclose(os_, o64, rtol=1e-10, atol=1e-12)
    np.testing.assert_array_equal(ls, l64)
    if splits > 1:  # with bf16 P the split schedule rounds differently from the unsplit one
        ob1, _ = O.sparse_attn(q, k, v, merged, H, g, b, None, qpad, kvpad, round_p="bf16")
        obs, _ = O.sparse_attn(q, k, v, merged, H, g, b, None, qpad, kvpad, round_p="bf16", splits=splits)
        assert np.abs(obs - ob1).max() > 0
        assert np.abs(obs - o64).max() < 2e-2 and np.abs(ob1 - o64).max() < 2e-2


def test_rounding_modes_bound_and_exact_cases():
    """With every P exactly representable (all scores equal, so P = 1 / n after
    normalisation in the backward and 1 before it in the forward) the rounding
    modes equal the float64 oracle; in general they differ from it by at most
    the 16-bit rounding of P / dS (relative 2^-8 of bf16 per term)."""
    rng = _rng(42)
    B, N, H, D, g, b = 1, 128, 1, 16, 32, 64
    merged = np.array([[[[0, 1], [1, -1], [0, -1], [0, 1]]]], dtype=np.int32)
    q = np.zeros((B, N, H * D))
    k = rng.standard_normal((B, N, H * D))
    v = O.round_to(rng.standard_normal((B, N, H * D)), "bf16")
    do = O.round_to(rng.standard_normal((B, N, H * D)), "bf16")
    o64, l64 = O.sparse_attn(q, k, v, merged, H, g, b)
    orr, lr = O.sparse_attn(q, k, v, merged, H, g, b, round_p="bf16")
    np.testing.assert_allclose(orr, o64, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(lr, l64)
    # general inputs: |dV_r - dV| <= 2^-8 sum_q P |dO| (P rounded once per term)
    q = rng.standard_normal((B, N, H * D))
    o64, l64 = O.sparse_attn(q, k, v, merged, H, g, b)
    d64 = O.sparse_attn_bwd(q, k, v, do, merged, H, g, b)
    dr = O.sparse_attn_bwd(q, k, v, do, merged, H, g, b, round_p="bf16", lse=l64)
    absdo = np.abs(do)
    bound = np.zeros_like(d64[2])
    for qm in range(4):
        ids = merged[0, 0, qm]
        keys = np.concatenate([np.arange(m * b, (m + 1) * b) for m in ids[ids >= 0]])
        rows = slice(qm * g, (qm + 1) * g)
        s = (q[0, rows] / math.sqrt(D)) @ k[0, keys].T
        p = np.exp(s - l64[0, 0, rows][:, None])
        bound[0, keys] += 2.0 ** -8 * p.T @ absdo[0, rows]
    assert np.all(np.abs(dr[2] - d64[2]) <= bound + 1e-12)
    assert np.abs(dr[2] - d64[2]).max() > 0  # the mode does round
    # lse / delta passed in equal the ones the oracle derives itself
    dl = (do * o64).reshape(B, N, H, D).sum(-1).transpose(0, 2, 1)
    d2 = O.sparse_attn_bwd(q, k, v, do, merged, H, g, b, lse=l64, delta=dl)
    for a, c in zip(d2, d64):
        np.testing.assert_allclose(a, c, rtol=1e-10, atol=1e-10)


def test_check_topk_f64_rules():
    """The float64 top-k comparison used by the GPU tests accepts only near-ties
    (including one at the threshold crossing, which moves the cut) and
    near-threshold cuts."""
    from _helpers import check_topk_f64

    raw = np.array([[0.5, 0.3, 0.15, 0.05]])
    avg = raw.copy()
    assert check_topk_f64(np.array([[0, 1, 2, -1]]), avg, raw, 0.9, 4) == 0
    assert check_topk_f64(np.array([[0, 1, -1, -1]]), avg, raw, 0.9, 4) == 1  # cut early, 0.8 far from 0.9
    assert check_topk_f64(np.array([[1, 0, 2, -1]]), avg, raw, 0.9, 4) == 1  # swap with a 0.2 gap
    raw2 = np.array([[0.5, 0.4 - 1e-9, 0.1]])
    assert check_topk_f64(np.array([[0, 1, 2]]), raw2, raw2, 0.9, 3) == 0  # cum 0.9 - 1e-9: near the threshold
    raw3 = np.array([[0.4, 0.4 + 1e-9, 0.2]])
    assert check_topk_f64(np.array([[0, 1, 2]]), raw3, raw3, 1.0, 3) == 0  # near-tie swap
    # a near-tie where the sum crosses the threshold: either order is a valid
    # selection, and the cut follows the order (block 2: small edge block whose
    # average ties block 1's)
    raw4 = np.array([[0.45, 0.30, 0.012, 0.238]])
    avg4 = np.array([[0.45, 0.30, 0.30 + 1e-10, 0.238]])
    assert check_topk_f64(np.array([[0, 2, 1, -1]]), avg4, raw4, 0.5, 4) == 0  # 0.45, 0.462, 0.762
    assert check_topk_f64(np.array([[0, 1, -1, -1]]), avg4, raw4, 0.5, 4) == 0  # 0.45, 0.75
    assert check_topk_f64(np.array([[0, 2, 1, 3]]), avg4, raw4, 0.5, 4) == 1   # past the crossing
    assert check_topk_f64(np.array([[0, 2, -1, -1]]), avg4, raw4, 0.5, 4) == 1  # stops at 0.462
    # a block left out that ranks above the last one kept, a repeated block, -1 inside
    assert check_topk_f64(np.array([[0, 3, -1, -1]]), avg4, raw4, 0.5, 4) == 1
    assert check_topk_f64(np.array([[0, 0, -1, -1]]), avg4, raw4, 0.5, 4) == 1
    assert check_topk_f64(np.array([[0, -1, 1, -1]]), avg4, raw4, 0.5, 4) == 1
    # a full list (m_out = 2) may stop below the threshold
    assert check_topk_f64(np.array([[0, 1]]), avg4, raw4, 0.9, 2) == 0


def test_torch_cpu_baseline_matches_numpy_oracle():
    """The PyTorch-CPU fp32 pipeline that bench.py times as the CPU baseline
    (oracle/fta_torch_cpu.py) against the numpy oracle on the same inputs:
    block scores within fp32 rounding of the float64 ones; the top-k, fed the
    same fp32 scores, bit for bit; the merge, fed the same top-k, equal; o, lse
    and the gradients, given the same merged lists, within fp32 rounding."""
    import fta_torch_cpu as T

    N, D, b, topk, thr, g, W = 512, 64, 64, 4, 0.9, 32, 8
    gen = torch.Generator().manual_seed(5)
    q, k, v, do = (torch.randn(N, D, generator=gen) for _ in range(4))
    sc = T.block_score(q, k, b, chunk=128)
    ref = O.block_score(q.numpy()[None], k.numpy()[None], 1, b)[0, 0]
    np.testing.assert_allclose(sc.numpy(), ref, rtol=2e-5, atol=1e-7)
    idx, raw, avg = T.topk_select(sc, thr, topk, b)
    ri, rr, ra = O.topk_select(sc.numpy(), thr, topk, b)
    np.testing.assert_array_equal(idx.numpy(), ri)
    np.testing.assert_array_equal(avg.numpy(), ra)
    np.testing.assert_array_equal(raw.numpy(), rr)
    merged, counts = T.qblock_merge(idx, avg, g, W, N // b)
    rm, _ = O.qblock_merge(idx.numpy()[None, None], avg.numpy()[None, None], g, W, N // b)
    np.testing.assert_array_equal(merged.numpy(), rm[0, 0])
    np.testing.assert_array_equal(counts.numpy(), (rm[0, 0] >= 0).sum(-1))
    merged[3] = -1  # an empty q-block
    o, lse, dq, dk, dv = T.sparse_attn_fwd_bwd(q, k, v, do, merged, g, b, group=5)
    mm = merged.numpy()[None, None]
    ro, rl = O.sparse_attn(q.numpy()[None], k.numpy()[None], v.numpy()[None], mm, 1, g, b)
    np.testing.assert_allclose(o.numpy(), ro[0], rtol=1e-4, atol=1e-5)
    assert np.array_equal(np.isneginf(lse.numpy()), np.isneginf(rl[0, 0]))
    fin = np.isfinite(rl[0, 0])
    np.testing.assert_allclose(lse.numpy()[fin], rl[0, 0][fin], rtol=1e-5, atol=1e-5)
    grads = O.sparse_attn_bwd(q.numpy()[None], k.numpy()[None], v.numpy()[None], do.numpy()[None], mm, 1, g, b)
    for got, r in zip((dq, dk, dv), grads):
        np.testing.assert_allclose(got.numpy(), r[0], rtol=1e-4, atol=2e-5)
