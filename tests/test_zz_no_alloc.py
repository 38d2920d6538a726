"""The allocation-free backward entry point (fta_sparse_attn_bwd_noalloc),
called through the C ABI, against fta_sparse_attn_bwd_gqa with a caller
workspace: dQ, dK and dV bit for bit, on two calls in a row (the second with a
smaller problem, so stale scratch contents from the first would show), then the
first problem again."""

import pytest
import torch

from _helpers import rand, say

pytestmark = pytest.mark.gpu


def _problem(dev, B, N, H, Hk, D, b, g, topk, seed):
    import flash_topk_attn_v2 as fta

    q = rand((B, N, H * D), seed, torch.bfloat16, dev)
    k = rand((B, N, Hk * D), seed + 1, torch.bfloat16, dev)
    v = rand((B, N, Hk * D), seed + 2, torch.bfloat16, dev)
    do = rand((B, N, H * D), seed + 3, torch.bfloat16, dev)
    kr = k.repeat_interleave(H // Hk, dim=2) if Hk != H else k
    idx, _, avg = fta.flash_topk_score(q, kr, H, b, topk, (0, 0), 1.0)
    merged, _, _ = fta.build_qblock_topk_indices(idx, g, (0, 0), avg, None)
    o, lse = fta.flash_topk_attn(q, k, v, merged, None, H, g, b, num_kv_heads=Hk)
    return dict(q=q, k=k, v=v, do=do, o=o, lse=lse, merged=merged, B=B, N=N, H=H, Hk=Hk, D=D, b=b, g=g)


def _with_workspace(p):
    from flash_topk_attn_v2.sparse_attn_bwd import sparse_attn_bwd

    return sparse_attn_bwd(p["q"], p["k"], p["v"], p["o"], p["do"], p["lse"], p["merged"], p["H"], p["g"],
                           p["b"], p["D"] ** -0.5, num_kv_heads=p["Hk"])


def _noalloc(p):
    from flash_topk_attn_v2 import _lib
    from flash_topk_attn_v2.sparse_attn_bwd import preprocess_delta

    B, N, H, Hk, D = p["B"], p["N"], p["H"], p["Hk"], p["D"]
    dev = p["q"].device
    delta = preprocess_delta(p["o"], p["do"], H)
    merged = p["merged"].to(torch.int32).contiguous()
    QM, W = merged.shape[2], merged.shape[3]
    dq = torch.empty(B, N, H * D, device=dev, dtype=torch.bfloat16)
    dk = torch.empty(B, N, Hk * D, device=dev, dtype=torch.bfloat16)
    dv = torch.empty(B, N, Hk * D, device=dev, dtype=torch.bfloat16)
    sq = [N * H * D, D, H * D]
    sk = [N * Hk * D, D, Hk * D]
    torch.cuda.synchronize()
    rc = _lib.lib().fta_sparse_attn_bwd_noalloc(
        _lib.ptr(p["q"]), _lib.i64arr(sq), _lib.ptr(p["k"]), _lib.i64arr(sk), _lib.ptr(p["v"]), _lib.i64arr(sk),
        _lib.ptr(p["do"]), _lib.i64arr(sq), _lib.DTYPE_BF16, B, H, Hk, N, D, _lib.ptr(merged), QM, W, p["g"],
        p["b"], 0, 0, 0, 0, float(D ** -0.5), _lib.ptr(p["lse"]), _lib.ptr(delta), _lib.ptr(dq), _lib.i64arr(sq),
        _lib.ptr(dk), _lib.i64arr(sk), _lib.ptr(dv), _lib.i64arr(sk), _lib.stream_ptr(dev),
    )
    _lib.check(rc, "sparse_attn_bwd_noalloc")
    return dq, dk, dv


def test_noalloc_bwd_matches_workspace_entry_point(gpu):
    big = dict(B=1, N=4096, H=4, Hk=4, D=128, b=64, g=32, topk=16, seed=101)
    small = dict(B=2, N=512, H=4, Hk=2, D=64, b=32, g=16, topk=4, seed=202)
    problems = [("big", _problem(gpu, **big)), ("small", _problem(gpu, **small))]
    problems.append(("big again", problems[0][1]))
    for name, p in problems:
        say(f"noalloc bwd: {name} B{p['B']} N{p['N']} H{p['H']} Hk{p['Hk']} D{p['D']} b{p['b']} g{p['g']}")
        ref = _with_workspace(p)
        got = _noalloc(p)
        torch.cuda.synchronize()
        for n, r, x in zip(("dq", "dk", "dv"), ref, got):
            assert torch.equal(r, x), f"{name}: {n} differs from the workspace entry point"


def test_noalloc_bwd_rejects_oversized_problem(gpu):
    from flash_topk_attn_v2 import _lib

    # lse in log2 units alone needs B*H*N*4 = 128 MiB > the 64 MiB array; rejected before any launch
    rc = _lib.lib().fta_sparse_attn_bwd_noalloc(
        None, None, None, None, None, None, None, None, _lib.DTYPE_BF16, 1, 32, 32, 1 << 20, 128, None,
        (1 << 20) // 32, 16, 32, 64, 0, 0, 0, 0, 0.1, None, None, None, None, None, None, None, None, None)
    assert rc == _lib.FTA_ERR_UNSUPPORTED
    assert b"FTA_NOALLOC_SCRATCH_BYTES" in _lib.lib().fta_last_error()
