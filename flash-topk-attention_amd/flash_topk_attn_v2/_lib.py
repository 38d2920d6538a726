"""ctypes binding of libfta_gfx950.so (the C ABI declared in include/fta.h).

The library is the only compute path: there is no CPU or PyTorch fallback.  If
the shared object is missing or a call fails, an exception is raised.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache
from typing import Sequence

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfta_gfx950.so")

FTA_OK = 0
FTA_ERR_ARG = 1
FTA_ERR_UNSUPPORTED = 2
FTA_ERR_HIP = 3
DTYPE_BF16 = 0
DTYPE_F16 = 1

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "fta_last_error": (ctypes.c_char_p, []),
    "fta_version": (_i, []),
    "fta_block_score_workspace_size": (_sz, [_i, _i, _i, _i]),
    "fta_block_score": (_i, [_p, _p, _i, _i, _i, _i, _i, _i64p, _i64p, _i, _i, _i, _f, _p, _p, _sz, _p]),
    "fta_block_score_lse": (_i, [_p, _p, _i, _i, _i, _i, _i, _i64p, _i64p, _i, _i, _i, _f, _p, _p, _p]),
    "fta_topk_select": (_i, [_p, _i64, _i, _i64, _i64, _i, _i, _i, _i, _f, _p, _p, _p, _p]),
    "fta_topk_score_workspace_size": (_sz, [_i, _i, _i, _i]),
    "fta_topk_score": (_i, [_p, _p, _i, _i, _i, _i, _i, _i64p, _i64p, _i, _i, _i, _f, _i, _f, _p, _p, _p, _p,
                            _sz, _p]),
    "fta_topk_score_candidates": (_i, [_p, _p, _i, _i, _i, _i, _i, _i64p, _i64p, _i, _i, _i, _f, _i, _p, _sz, _p]),
    "fta_topk_select_candidates": (_i, [_p, _p, _i, _i, _i, _i, _i, _i64p, _i64p, _i, _i, _i, _f, _i, _f, _p, _p,
                                        _p, _p, _sz, _p]),
    "fta_topk_score_workspace_size_ex": (_sz, [_i] * 8),
    "fta_topk_score_workspace_min": (_sz, [_i] * 8),
    "fta_qblock_merge": (_i, [_p, _p, _i64, _i, _i, _i, _i, _p, _p, _p, _p]),
    "fta_qblock_merge_maxid": (_i, [_p, _p, _i64, _i, _i, _p, _i, _p, _p, _p, _p]),
    "fta_qblock_union": (_i, [_p, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p]),
    "fta_build_reverse_indices_workspace_size": (_sz, [_i, _i, _i, _i]),
    "fta_build_reverse_indices": (_i, [_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _p, _sz, _p]),
    "fta_sort_by_count": (_i, [_p, _i64, _p, _p, _p]),
    "fta_sparse_attn_fwd_workspace_size": (_sz, [_i] * 10),
    "fta_sparse_attn_fwd_splits": (_i, [_i] * 10),
    "fta_sparse_attn_fwd": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _p, _i, _i, _i, _i, _i, _i,
                                 _i, _i, _f, _p, _i64p, _p, _p, _sz, _p]),
    "fta_sparse_attn_fwd_gqa": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _i, _p, _i, _i, _i, _i,
                                     _i, _i, _i, _i, _f, _p, _i64p, _p, _p, _sz, _p]),
    "fta_preprocess_delta": (_i, [_p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _p, _p]),
    "fta_sparse_attn_bwd_workspace_size": (_sz, [_i] * 10),
    "fta_sparse_attn_bwd": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _p, _i, _i, _i,
                                 _i, _i, _i, _i, _i, _f, _p, _p, _p, _i64p, _p, _i64p, _p, _i64p, _p, _sz, _p]),
    "fta_sparse_attn_bwd_gqa": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _i, _p, _i,
                                     _i, _i, _i, _i, _i, _i, _i, _f, _p, _p, _p, _i64p, _p, _i64p, _p, _i64p, _p,
                                     _sz, _p]),
    "fta_sparse_attn_bwd_dq": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _i, _p, _i, _i,
                                    _i, _i, _i, _i, _i, _i, _f, _p, _p, _p, _i64p, _p]),
    "fta_sparse_attn_bwd_dkv": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _i, _p, _i,
                                     _i, _i, _i, _i, _i, _i, _i, _f, _p, _p, _p, _i64p, _p, _i64p, _p, _sz, _p]),
    "fta_sparse_attn_bwd_noalloc": (_i, [_p, _i64p, _p, _i64p, _p, _i64p, _p, _i64p, _i, _i, _i, _i, _i, _i, _p,
                                         _i, _i, _i, _i, _i, _i, _i, _i, _f, _p, _p, _p, _i64p, _p, _i64p, _p,
                                         _i64p, _p]),
}


class FtaError(RuntimeError):
    """A libfta call failed (launch error or unsupported configuration)."""


@lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} not found: build it with `python flash-topk-attention_amd/build_lib.py` "
            "(hipcc --offload-arch=gfx950). There is no non-HIP fallback."
        )
    so = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(so, name)
        fn.restype = res
        fn.argtypes = args
    return so


def check(rc: int, what: str) -> None:
    if rc == FTA_OK:
        return
    msg = lib().fta_last_error().decode(errors="replace")
    if rc == FTA_ERR_ARG:
        raise ValueError(f"{what}: {msg}")
    if rc == FTA_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise FtaError(f"{what}: {msg}")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def i64arr(vals: Sequence[int]):
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float16:
        return DTYPE_F16
    raise ValueError(f"unsupported dtype {dt}; expected bfloat16 or float16")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def token_view(x: torch.Tensor, layout: str, num_heads: int):
    """Return (tensor, [stride_b, stride_h, stride_n]) addressing x as [B][N][H][D]
    with unit D stride and 16-byte aligned rows; copies only when needed.

    layout "bnc": x is [B, N, H*D]; layout "bhnd": x is [B, H, N, D].
    """

    def ok(t, strides):
        return (
            t.stride(-1) == 1
            and t.data_ptr() % 16 == 0
            and all(int(s) % 8 == 0 for s in strides)
        )

    if layout == "bnc":
        D = x.shape[2] // num_heads
        strides = [x.stride(0), D, x.stride(1)]
        if not ok(x, strides):
            x = x.contiguous()
            strides = [x.stride(0), D, x.stride(1)]
        return x, strides
    strides = [x.stride(0), x.stride(1), x.stride(2)]
    if not ok(x, strides):
        x = x.contiguous()
        strides = [x.stride(0), x.stride(1), x.stride(2)]
    return x, strides
