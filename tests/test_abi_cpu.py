"""CPU-side checks of the boundary: the C-ABI library loads and exports every
symbol declared in include/fta.h; argument validation raises the reference's
exception types without touching the GPU."""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fta.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fta_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from flash_topk_attn_v2 import _lib

    so = ctypes.CDLL(_lib.LIB_PATH)
    names = _declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(so, n), n
    assert set(names) == set(_lib._SIGNATURES)


def test_error_path_returns_status_without_gpu():
    from flash_topk_attn_v2 import _lib

    L = _lib.lib()
    # invalid geometry is rejected before any launch
    rc = L.fta_topk_select(None, 1, 0, 0, 1, 16, 64, 0, 0, 1.0, None, None, None, None)
    assert rc == _lib.FTA_ERR_ARG
    assert b"M must be positive" in L.fta_last_error()
    rc = L.fta_qblock_merge(None, None, 1, 32, 16, 5000, 16, None, None, None, None)
    assert rc == _lib.FTA_ERR_UNSUPPORTED
    assert L.fta_sparse_attn_bwd_workspace_size(1, 1, 100, 64, 32, 64, 0, 0, 0, 0) == 0  # 100 % 32 != 0
    assert L.fta_sparse_attn_fwd_workspace_size(1, 2, 128, 64, 32, 64, 0, 0, 0, 0) == 768  # head work, placement and 64 partial counts per head
    # small grids split the forward's walks: 64 workgroups of 256 queries -> 4 parts,
    # whose (m, L) float2 and unnormalised O (64 columns) follow, 256-byte aligned
    assert L.fta_sparse_attn_fwd_splits(1, 8, 2048, 32, 64, 64, 0, 0, 0, 0) == 4
    assert L.fta_sparse_attn_fwd_workspace_size(1, 8, 2048, 32, 64, 64, 0, 0, 0, 0) == 2304 + 4 * 8 * 2048 * (8 + 256)
    assert L.fta_sparse_attn_fwd_splits(1, 32, 32768, 128, 32, 64, 0, 0, 0, 0) == 1  # 4096 workgroups
    assert L.fta_sparse_attn_fwd_splits(1, 8, 2048, 160, 64, 64, 0, 0, 0, 0) == 1    # D > 128: not pipelined
    assert L.fta_sparse_attn_fwd_splits(1, 2, 448, 64, 64, 64, 0, 0, 0, 0) == 1      # 7 KV blocks
    assert L.fta_sparse_attn_fwd_splits(1, 2, 100, 64, 32, 64, 0, 0, 0, 0) == 0      # invalid geometry
    # backward scratch = membership bitmap [B*H][M_kv][ceil(QM/32)] uint32, lse in log2
    # units [B*H][N] fp32, dK/dV launch order [B*H][M_kv] int32, head work and head
    # placement [B*H] int32 each, each region 256-byte aligned
    # plus the split parts of small grids, one region shared by dK/dV and then dQ:
    # dK/dV [2][parts][B*H][M_kv * 64][D] fp32 with up to 4 parts while fewer
    # workgroups than 512 (two per CU) run; dQ [parts][B*H][N][D] fp32 as for the
    # forward's split walks (fewer than 128 workgroups, at least 8 KV blocks).
    # B1 H2 N128 D64: 4 dK/dV workgroups, 4 parts; dQ not split (2 KV blocks)
    assert L.fta_sparse_attn_bwd_workspace_size(1, 2, 128, 64, 32, 64, 0, 0, 0, 0) == (
        256 + 1024 + 256 + 256 + 2 * 4 * 2 * 2 * 64 * 64 * 4)
    # B1 H8 N2048 D64: 256 dK/dV workgroups (2 parts) and 64 dQ workgroups (4 parts),
    # the same 16 MiB either way
    assert L.fta_sparse_attn_bwd_workspace_size(1, 8, 2048, 64, 64, 64, 0, 0, 0, 0) == (
        1024 + 8 * 2048 * 4 + 1024 + 256 + 4 * 8 * 2048 * 64 * 4)
    assert 4 * 8 * 2048 * 64 * 4 == 2 * 2 * 8 * 32 * 64 * 64 * 4
    # D 160 / 256 (register-staged dQ, 128-query workgroups): split while at most 128
    # workgroups run; the D = 256 dK/dV split while fewer than 256 (one per CU)
    bare = 1024 + 8 * 2048 * 4 + 1024 + 256
    assert L.fta_sparse_attn_bwd_workspace_size(1, 8, 2048, 256, 64, 64, 0, 0, 0, 0) == (
        bare + 2 * 8 * 2048 * 256 * 4)  # 128 dQ workgroups: 2 parts; 256 dK/dV workgroups: none
    assert L.fta_sparse_attn_bwd_workspace_size(1, 8, 4096, 256, 64, 64, 0, 0, 0, 0) == (
        8 * 64 * 2 * 4 + 8 * 4096 * 4 + 8 * 64 * 4 + 256)  # 256 dQ workgroups: no split parts
    assert L.fta_sparse_attn_bwd_workspace_size(1, 4, 1024, 160, 32, 64, 0, 0, 0, 0) == (
        256 + 4 * 1024 * 4 + 256 + 256 + 4 * 4 * 1024 * 160 * 4)  # 32 dQ workgroups: 4 parts
    # 4096 dQ workgroups at C3: no split parts
    assert L.fta_sparse_attn_bwd_workspace_size(1, 32, 32768, 128, 32, 64, 0, 0, 0, 0) == (
        32 * 512 * 32 * 4 + 32 * 32768 * 4 + 32 * 512 * 4 + 256)


def test_api_validation_matches_reference_errors():
    import flash_topk_attn_v2 as fta

    q = torch.zeros(1, 10, 4)
    with pytest.raises(ValueError, match="num_heads is required"):
        fta.flash_topk_score(q, q)
    with pytest.raises(ValueError, match="topk_indices must be"):
        fta.build_qblock_topk_indices(torch.zeros(2, 2, dtype=torch.int32), 4)
    with pytest.raises(ValueError, match="q_pad_head=4 must be < q_block_size=4"):
        fta.build_qblock_topk_indices(torch.zeros(1, 1, 8, 2, dtype=torch.int32), 4, (4, 0))
    # GQA is supported (an extension of the reference), so no NotImplementedError;
    # CPU tensors are rejected as for any other call
    with pytest.raises(ValueError, match="requires CUDA"):
        fta.flash_topk_attn(q, q, q, torch.zeros(1, 2, 3, 1, dtype=torch.int32), None, 2, 4, 4, num_kv_heads=1)
    with pytest.raises(ValueError, match="requires CUDA"):
        fta.flash_sparse_attn(q, q, q, torch.zeros(1, 1, 1, 1, dtype=torch.int32), 1, 4, 4)
    with pytest.raises(ValueError, match="requires CUDA"):
        fta.flash_block_score(q, q, 1, 5)


def test_gqa_head_count_checked_before_any_gpu_work():
    """fta_sparse_attn_{fwd,bwd}_gqa reject H not a multiple of Hk up front."""
    from flash_topk_attn_v2 import _lib

    L = _lib.lib()
    st = _lib.i64arr([0, 0, 0])
    rc = L.fta_sparse_attn_fwd_gqa(None, st, None, st, None, st, 0, 1, 6, 4, 64, 64, None, 2, 1, 32, 64,
                                   0, 0, 0, 0, 0.125, None, st, None, None, 0, None)
    assert rc == 1 and b"multiple of num_kv_heads" in L.fta_last_error()
    rc = L.fta_sparse_attn_bwd_gqa(None, st, None, st, None, st, None, st, 0, 1, 6, 0, 64, 64, None, 2, 1, 32, 64,
                                   0, 0, 0, 0, 0.125, None, None, None, st, None, st, None, st, None, 0, None)
    assert rc == 1 and b"multiple of num_kv_heads" in L.fta_last_error()


def test_v1_api_validation_without_gpu():
    import flash_topk_attn as v1

    q = torch.zeros(1, 100, 64)
    with pytest.raises(ValueError, match="unsupported backend"):
        v1.flash_topk_score(q, q, q, 1, backend="cuda")
    with pytest.raises(ValueError, match="v is required"):
        v1.flash_topk_score(q, q, None, 1)
    with pytest.raises(ValueError, match="num_heads is required"):
        v1.flash_topk_score(q, q, q)
    with pytest.raises(ValueError, match="must each be <"):
        v1.flash_topk_score(q, q, None, 1, 64, 1, (64, 0), score_only=True)
    with pytest.raises(ValueError, match="must be divisible"):
        v1.flash_topk_score(q, q, None, 1, 64, 1, (0, 0), score_only=True)
    with pytest.raises(ValueError, match=r"topk \(3\) > num_blocks \(2\)"):
        v1.flash_topk_score(q, q, None, 1, 64, 3, (0, 28), score_only=True)
    with pytest.raises(ValueError, match=r"num_heads \(3\) != q.shape\[1\] \(2\)"):
        v1.flash_topk_score(torch.zeros(1, 2, 8, 16), torch.zeros(1, 2, 8, 16), None, 3, score_only=True)
    ids = torch.zeros(1, 1, 100, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="q_pad_head=32 must be < q_block_size=32"):
        v1.build_qblock_topk_indices(ids, 32, (32, 0))
    with pytest.raises(AssertionError, match="must be divisible"):
        v1.build_qblock_topk_indices(ids, 32, (0, 0))
    with pytest.raises(NotImplementedError, match="union limit"):
        v1.build_qblock_topk_indices(torch.zeros(1, 1, 128, 256, dtype=torch.int32), 64)
    with pytest.raises(ValueError, match="requires CUDA"):
        v1.build_qblock_topk_indices(ids, 20, (0, 0))
    with pytest.raises(ValueError, match="requires CUDA"):
        v1.flash_topk_attn(q, q, q, ids, ids[..., 0], 1, 32, 64)
