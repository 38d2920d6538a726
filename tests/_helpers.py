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


def assert_close_frac(got, ref, atol, rtol, min_frac=0.9999, hard_atol=1e-2, name=""):
    """bf16/fp16 tolerance: |got - ref| <= atol + rtol*|ref| on at least
    ``min_frac`` of the elements (P is rounded to 16 bits before the P.V / dS.K
    products, as in the reference kernels, so isolated elements can exceed the
    per-element bound), and never more than ``hard_atol`` + rtol*|ref|."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, name
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    frac = ok.mean() if ok.size else 1.0
    assert frac >= min_frac, f"{name}: only {frac:.6f} of elements within atol={atol}, rtol={rtol}; max err {err.max()}"
    assert np.all(err <= hard_atol + rtol * np.abs(ref)), f"{name}: max err {err.max()} beyond hard bound"
