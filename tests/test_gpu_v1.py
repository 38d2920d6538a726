"""GPU parity of the V1 compatibility layer (flash_topk_attn) against the CPU oracle.

Bars: union merged indices / counts bit-exact; top-k indices identical except
where the oracle's (float64) scores of the swapped blocks differ by < 1e-6;
scores within rtol 1e-4 (fp32 softmax sums vs float64); o, dQ, dK, dV within
atol 2e-3 + rtol 1e-2 (fp16/bf16), lse rtol 1e-4.
"""

import numpy as np
import pytest
import torch

import fta_oracle as O
from _helpers import assert_close_frac, assert_within, check_topk_gap, np32, rand, round_kind, say

pytestmark = pytest.mark.gpu

v1 = pytest.importorskip("flash_topk_attn")


def _rounded(x):
    return np32(x.bfloat16() if x.dtype == torch.float32 else x)


UNION_CASES = [
    # B, H, N, K, g, q_padding, id range, int64 input
    (1, 2, 1024, 16, 32, (0, 0), 16, False),
    (2, 3, 1000, 8, 16, (4, 4), 157, True),
    (1, 1, 300, 5, 7, (3, 5), 40, False),
    (1, 2, 4096, 16, 512, (0, 0), 64, False),   # g*K = 8192: the largest row
    (1, 2, 64, 0, 16, (0, 0), 1, False),        # K = 0: every q-block empty
    (1, 1, 40, 16, 64, (0, 24), 100000, False),  # ids far beyond any bitmap
    # LDS bitonic paths with several waves per workgroup; 3 heads x 5 q-blocks = 15
    # slices, a count that neither 4 nor 2 waves per workgroup divide (tail workgroup)
    (1, 3, 320, 16, 64, (0, 0), 700, False),    # g*K = 1024
    (1, 3, 640, 16, 128, (0, 0), 3000, False),  # g*K = 2048
    (1, 3, 640, 32, 128, (0, 0), 4096, False),  # g*K = 4096
    (1, 3, 600, 32, 128, (20, 20), 4000, True),  # g*K = 4096 with q padding
]


@pytest.mark.parametrize("case", UNION_CASES, ids=lambda c: f"N{c[2]}K{c[3]}g{c[4]}p{c[5][0]}-{c[5][1]}")
def test_union_bit_exact(case):
    B, H, N, K, g, qpad, idr, i64 = case
    say(f"[v1 union] {case}")
    gen = torch.Generator().manual_seed(7)
    ids = torch.randint(-1, idr, (B, H, N, K), generator=gen, dtype=torch.int64)
    t = ids.cuda() if i64 else ids.int().cuda()
    merged, counts, S = v1.build_qblock_topk_indices(t, g, qpad)
    torch.cuda.synchronize()
    rm, rc, rS = O.v1_qblock_union(ids.numpy(), g, qpad)
    assert S == rS and merged.dtype == torch.int32 and counts.dtype == torch.int32
    np.testing.assert_array_equal(merged.cpu().numpy(), rm)
    np.testing.assert_array_equal(counts.cpu().numpy(), rc)


SCORE_CASES = [
    # B, N, H, D, b, topk, padding, dtype, layout
    (1, 1024, 2, 64, 64, 16, (0, 0), torch.bfloat16, "bnc"),
    (1, 1000, 2, 128, 64, 8, (24, 0), torch.float16, "bnc"),
    (2, 640, 3, 128, 32, 16, (0, 0), torch.bfloat16, "bhnd"),
    (1, 300, 2, 64, 48, 7, (12, 24), torch.float16, "bnc"),
    (1, 256, 2, 64, 64, 4, (0, 0), torch.bfloat16, "bnc"),  # topk = M
]


def _score_inputs(case, seed, with_v):
    B, N, H, D, b, topk, pad, dt, layout = case
    shape = (B, H, N, D) if layout == "bhnd" else (B, N, H * D)
    q = rand(shape, seed, dt, "cuda")
    k = rand(shape, seed + 1, dt, "cuda")
    v = rand(shape, seed + 2, dt, "cuda") if with_v else None
    return q, k, v


def _check_topk(case, idx, scores, q, k):
    B, N, H, D, b, topk, pad, dt, layout = case
    _, ri, rs = O.v1_topk_score(np32(q), np32(k), None, H, b, topk, pad)
    assert idx.shape == ri.shape and idx.dtype == torch.int32 and scores.dtype == torch.float32
    # full-precision scores of every block, to judge near-ties
    full = O.block_score(np32(q), np32(k), H, b, pad)
    if pad != (0, 0):
        full = full / O.valid_counts(full.shape[-1], b, pad).astype(np.float64)
    bad, ndiff = check_topk_gap(idx.cpu().numpy(), full, ri)
    assert bad == 0, f"{bad} of {ndiff} differing indices have score gap >= 1e-6"
    gi = idx.cpu().numpy()
    got_at = np.take_along_axis(full, gi.astype(np.int64), axis=-1)
    np.testing.assert_allclose(scores.cpu().numpy(), got_at, rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(np.sort(scores.cpu().numpy(), axis=-1), np.sort(rs, axis=-1), rtol=1e-4, atol=1e-7)


@pytest.mark.parametrize("case", SCORE_CASES, ids=lambda c: f"N{c[1]}D{c[3]}b{c[4]}k{c[5]}{c[8]}")
def test_score_only_vs_oracle(case):
    B, N, H, D, b, topk, pad, dt, layout = case
    say(f"[v1 score_only] {case}")
    q, k, _ = _score_inputs(case, 50, False)
    nh = None if layout == "bhnd" else H
    idx, scores = v1.flash_topk_score(q, k, None, nh, b, topk, pad, score_only=True)
    torch.cuda.synchronize()
    _check_topk(case, idx, scores, q, k)


DENSE_CASES = [
    (1, 1024, 2, 64, 64, 16, (0, 0), torch.bfloat16, "bnc"),
    (1, 1000, 2, 128, 64, 8, (24, 0), torch.float16, "bnc"),
    (2, 300, 2, 64, 48, 4, (12, 24), torch.bfloat16, "bhnd"),
]


@pytest.mark.parametrize("case", DENSE_CASES, ids=lambda c: f"N{c[1]}D{c[3]}b{c[4]}{c[8]}")
def test_score_with_dense_output_and_backward(case):
    B, N, H, D, b, topk, pad, dt, layout = case
    say(f"[v1 score+o] {case}")
    q, k, v = _score_inputs(case, 60, True)
    for t in (q, k, v):
        t.requires_grad_(True)
    nh = None if layout == "bhnd" else H
    o, idx, scores = v1.flash_topk_score(q, k, v, nh, b, topk, pad)
    do = rand(tuple(o.shape), 98, o.dtype, "cuda")
    o.backward(do)
    torch.cuda.synchronize()
    assert o.dtype == dt and o.shape == q.shape
    _check_topk(case, idx, scores, q.detach(), k.detach())
    to3 = (lambda x: np.ascontiguousarray(np32(x).transpose(0, 2, 1, 3).reshape(B, N, H * D))) \
        if layout == "bhnd" else np32
    qn, kn, vn, don, on = (to3(t) for t in (q.detach(), k.detach(), v.detach(), do, o.detach()))
    ro, _, _ = O.v1_topk_score(qn, kn, vn, H, b, topk, pad)
    assert_close_frac(on, ro, atol=2e-3, rtol=1e-2, name="o vs f64")
    # dense = every 64-token KV block selected for every 64-query block; primary check:
    # the oracle with the kernels' 16-bit rounding points, every element within the bound
    nb = (N + 63) // 64
    merged = np.ascontiguousarray(np.broadcast_to(np.arange(nb, dtype=np.int32), (B, H, nb, nb)))
    pad64 = (0, nb * 64 - N)
    rk = round_kind(dt)
    rr, rl = O.sparse_attn(qn, kn, vn, merged, H, 64, 64, None, pad64, pad64, round_p=rk)
    assert_within(on, rr, name="o vs rounding oracle")
    from flash_topk_attn_v2.sparse_attn_bwd import preprocess_delta

    delta = preprocess_delta(torch.from_numpy(on).to(dt).cuda(), torch.from_numpy(don).to(dt).cuda(), H)
    kw = dict(round_p=rk, lse=rl, delta=delta.cpu().numpy().astype(np.float64))
    dq, dk, dv = O.sparse_attn_bwd(qn, kn, vn, don, merged, H, 64, 64, None, pad64, pad64, **kw)
    dq64, dk64, dv64 = O.sparse_attn_bwd(qn, kn, vn, don, merged, H, 64, 64, None, pad64, pad64)
    for name, got, ref, r64 in (("dq", q.grad, dq, dq64), ("dk", k.grad, dk, dk64), ("dv", v.grad, dv, dv64)):
        assert_within(to3(got), ref, name=f"{name} vs rounding oracle")
        # unscaled bound (the largest |gradient| is reported); the hard bound also allows
        # twice what the 16-bit rounding of P / dS moves each element
        say(f"{name} vs f64: max |ref| {np.abs(r64).max():.3f}")
        assert_close_frac(to3(got), r64, atol=2e-3, rtol=1e-2, name=f"{name} vs f64", min_frac=0.9995,
                          hard_atol=1e-2, slack=2 * np.abs(ref - r64))


ATTN_CASES = [
    # B, N, H, D, g, b, K, qpad, kvpad, H_BI, S_MAX, dtype
    (1, 1024, 2, 64, 32, 64, 4, (0, 0), (0, 0), 2, None, torch.bfloat16),
    (1, 1000, 2, 128, 16, 64, 3, (4, 4), (24, 0), 1, None, torch.float16),   # one list for every head
    (1, 700, 2, 64, 32, 32, 4, (0, 4), (0, 4), 2, 16, torch.bfloat16),      # S_MAX truncates the lists
    (1, 1000, 2, 64, 128, 64, 2, (20, 4), (0, 24), 2, None, torch.bfloat16),  # q-block > 64: sub-blocks
    (1, 1000, 2, 64, 128, 64, 2, (100, 52), (0, 24), 2, None, torch.bfloat16),  # head pad > sub-block
    (1, 600, 2, 64, 96, 64, 2, (30, 42), (0, 40), 1, None, torch.float16),    # 96 = 2 x 48, H_BI = 1
]


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: f"N{c[1]}g{c[4]}b{c[5]}H{c[9]}S{c[10]}")
def test_attn_over_union_vs_oracle(case):
    B, N, H, D, g, b, K, qpad, kvpad, HBI, smax, dt = case
    say(f"[v1 attn] {case}")
    M = (kvpad[0] + N + kvpad[1]) // b
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(-1, M, (B, HBI, N, K), generator=gen).int()
    merged, counts, S = v1.build_qblock_topk_indices(ids.cuda(), g, qpad)
    q = rand((B, N, H * D), 70, dt, "cuda")
    k = rand((B, N, H * D), 71, dt, "cuda")
    v = rand((B, N, H * D), 72, dt, "cuda")
    o, lse = v1.flash_topk_attn(q, k, v, merged, counts, H, g, b, None, None, kvpad, qpad, smax)
    torch.cuda.synchronize()
    ro, rl = O.v1_sparse_attn(np32(q), np32(k), np32(v), merged.cpu().numpy(), counts.cpu().numpy(), H, g, b,
                              None, kvpad, qpad, smax)
    assert o.dtype == dt
    assert_close_frac(np32(o), ro, atol=2e-3, rtol=1e-2, name="o vs f64")
    # primary: the V2 oracle with the kernels' rounding points on the lists the V1
    # semantics select (first min(count, S_MAX) ids, one list for every head when H_BI = 1);
    # a row's result depends only on its ascending block set, not on the q-block grouping
    mv = merged.cpu().numpy().copy()
    lim = counts.cpu().numpy() if smax is None else np.minimum(counts.cpu().numpy(), smax)
    mv[np.arange(mv.shape[-1]) >= lim[..., None]] = -1
    if mv.shape[1] == 1:
        mv = np.repeat(mv, H, axis=1)
    rr, _ = O.sparse_attn(np32(q), np32(k), np32(v), mv, H, g, b, None, qpad, kvpad, round_p=round_kind(dt))
    assert_within(np32(o), rr, name="o vs rounding oracle")
    l = lse.cpu().numpy()
    np.testing.assert_array_equal(np.isneginf(l), np.isneginf(rl))
    fin = np.isfinite(rl)
    np.testing.assert_allclose(l[fin], rl[fin], rtol=1e-4, atol=1e-4)


def test_attn_pipeline_from_v1_scores():
    """score_only -> union -> attention, as a V1 caller chains them."""
    B, N, H, D, b, g = 1, 512, 2, 64, 64, 32
    say("[v1 pipeline]")
    q = rand((B, N, H * D), 80, torch.bfloat16, "cuda")
    k = rand((B, N, H * D), 81, torch.bfloat16, "cuda")
    v = rand((B, N, H * D), 82, torch.bfloat16, "cuda")
    idx, _ = v1.flash_topk_score(q, k, None, H, b, 2, score_only=True)
    merged, counts, S = v1.build_qblock_topk_indices(idx, g)
    o, lse = v1.flash_topk_attn(q, k, v, merged, counts, H, g, b)
    torch.cuda.synchronize()
    rm, rc, _ = O.v1_qblock_union(idx.cpu().numpy(), g)
    np.testing.assert_array_equal(merged.cpu().numpy(), rm)
    ro, rl = O.v1_sparse_attn(np32(q), np32(k), np32(v), rm, rc, H, g, b)
    assert_close_frac(np32(o), ro, atol=2e-3, rtol=1e-2, name="o")
    np.testing.assert_allclose(lse.cpu().numpy(), rl, rtol=1e-4, atol=1e-4)
