"""Shared helpers for the GPU parity tests (test infrastructure)."""

import sys

import numpy as np
import torch


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rand(shape, seed, dtype, device, scale=1.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(device)


def np32(t):
    return t.detach().float().cpu().numpy()


def check_topk_gap(gpu_idx, ref_scores_avg, ref_idx, atol_gap=1e-6):
    """Indices must agree except where the oracle's avg scores of the two
    differing blocks are within ``atol_gap`` (ties / near ties)."""
    gi = np.asarray(gpu_idx)
    ri = np.asarray(ref_idx)
    diff = np.nonzero(gi != ri)
    bad = 0
    for pos in zip(*diff):
        row = pos[:-1]
        a, b = gi[pos], ri[pos]
        if a < 0 or b < 0:
            # cut position differs: only acceptable as a near-tie at the cut
            bad += 1
            continue
        gap = abs(ref_scores_avg[row + (a,)] - ref_scores_avg[row + (b,)])
        if gap > atol_gap:
            bad += 1
    return bad, len(diff[0])


def assert_close_frac(got, ref, atol, rtol, min_frac=0.9999, hard_atol=1e-2, name="", slack=None):
    """bf16/fp16 tolerance: |got - ref| <= atol + rtol*|ref| on at least
    ``min_frac`` of the elements (P is rounded to 16 bits before the P.V / dS.K
    products, as in the reference kernels, so isolated elements can exceed the
    per-element bound), and never more than ``hard_atol`` + rtol*|ref| (+ the
    per-element ``slack``, e.g. a multiple of what that 16-bit rounding moves
    the element by, for long sums of rounded terms)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, name
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    frac = ok.mean() if ok.size else 1.0
    assert frac >= min_frac, f"{name}: only {frac:.6f} of elements within atol={atol}, rtol={rtol}; max err {err.max()}"
    hard = hard_atol + rtol * np.abs(ref) + (0.0 if slack is None else np.asarray(slack, dtype=np.float64))
    bad = err > hard
    assert not bad.any(), f"{name}: max err {err.max()} beyond hard bound ({int(bad.sum())} elements)"


def assert_within(got, ref, atol=2e-3, rtol=1e-2, name=""):
    """The north-star bound on every element: |got - ref| <= atol + rtol |ref|."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, name
    err = np.abs(got - ref)
    lim = atol + rtol * np.abs(ref)
    bad = err > lim
    if bad.any():
        i = np.unravel_index(np.argmax(err / lim), err.shape)
        raise AssertionError(f"{name}: {int(bad.sum())} of {bad.size} elements beyond atol={atol} + rtol={rtol}|ref|; "
                             f"worst at {i}: got {got[i]} ref {ref[i]}")


def round_kind(dtype):
    """The 16-bit type the kernels compute in for inputs of `dtype` (fp32 runs in bf16)."""
    return "fp16" if dtype == torch.float16 else "bf16"


def check_topk_f64(gpu_idx, avg64, raw64, threshold, m_out, gap=1e-6):
    """GPU top-k rows against the selection on float64 scores.

    gpu_idx [R, m_out] (-1 after the cut), avg64 / raw64 [R, M] float64.  The
    float64 selection sorts by avg descending (ties to the lower index), keeps
    through the first position whose float64 cumulative raw sum reaches the
    threshold, capped at m_out.  A row may differ only (a) by blocks whose
    float64 averages lie within `gap` of each other (near-ties) or (b) in the
    cut, where the float64 cumulative sum at the shorter cut lies within `gap`
    of the threshold.  Returns the number of rows that differ otherwise."""
    gpu_idx = np.asarray(gpu_idx)
    R, M = avg64.shape
    bad = 0
    for r in range(R):
        order = np.lexsort((np.arange(M), -avg64[r]))
        cs = np.cumsum(raw64[r, order])
        hit = np.nonzero(cs >= threshold)[0]
        cut64 = min(int(hit[0]) + 1 if hit.size else M, m_out)
        g = gpu_idx[r]
        cutg = int((g >= 0).sum())
        if cutg != cut64:
            lo = min(cutg, cut64)
            if not (lo >= 1 and abs(cs[lo - 1] - threshold) < gap):
                bad += 1
                continue
        n = min(cutg, cut64)
        ref = order[:n]
        got = g[:n]
        if np.array_equal(ref, got):
            continue
        # near-ties: the sorted float64 averages of both lists agree within gap
        # position by position, and the lists hold the same blocks up to such swaps
        if not np.all(np.abs(avg64[r, ref] - avg64[r, got]) < gap):
            bad += 1
    return bad
