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
    per-element bound), and never more than ``hard_atol`` + rtol*|ref|.  Both
    bounds add the per-element ``slack`` when given: a multiple of what that
    16-bit rounding itself moves the element by, which long sums of rounded
    terms make larger than the fixed bounds."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, name
    err = np.abs(got - ref)
    extra = 0.0 if slack is None else np.asarray(slack, dtype=np.float64)
    ok = err <= atol + rtol * np.abs(ref) + extra
    frac = ok.mean() if ok.size else 1.0
    assert frac >= min_frac, f"{name}: only {frac:.6f} of elements within atol={atol}, rtol={rtol}; max err {err.max()}"
    hard = hard_atol + rtol * np.abs(ref) + extra
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
    threshold, capped at m_out.  A GPU row passes when it is that selection
    for some order of the blocks whose float64 averages lie within `gap` of
    each other (near-ties): its blocks are distinct, their averages do not
    rise by more than `gap` along the list, no block left out ranks more than
    `gap` above the last one kept, and the cut is where the float64
    cumulative sum taken in the GPU's order first reaches the threshold
    (within `gap`) or the list is full.  So a near-tie may swap two blocks,
    and when the swap falls where the sum crosses the threshold it may move
    the cut by that block.  Returns the number of rows that fail."""
    gpu_idx = np.asarray(gpu_idx)
    R, M = avg64.shape
    cap = min(m_out, M)
    bad = 0
    for r in range(R):
        g = gpu_idx[r]
        n = int((g >= 0).sum())
        lst = g[:n]
        if n == 0 or (g[n:] != -1).any() or len(set(lst.tolist())) != n or (lst >= M).any():
            bad += 1
            continue
        a = avg64[r, lst]
        if np.any(a[1:] > a[:-1] + gap):
            bad += 1
            continue
        out = np.ones(M, dtype=bool)
        out[lst] = False
        if out.any() and avg64[r, out].max() > a[-1] + gap:
            bad += 1
            continue
        cs = np.cumsum(raw64[r, lst])
        if n >= 2 and cs[-2] >= threshold + gap:  # the sum reached the threshold before the last block
            bad += 1
            continue
        if n < cap and cs[-1] < threshold - gap:  # stopped before reaching it, list not full
            bad += 1
    return bad
