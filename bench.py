"""Benchmark: flash-topk-attention V2 hot path on one MI355X.

One step = flash_topk_score -> build_qblock_topk_indices -> flash_topk_attn
forward -> backward, on BASELINE config 3 (B=1, N=32768, H=32, D=128 bf16,
peaked synthetic attention, b=64, topk=16, threshold=0.9, g=32, W=256).
Prints one JSON line (driver contract).  Extra fields: the scoring kernel's
roofline (HIP events on the stream it runs on), `stage_roofline` (every stage
launched alone through its C entry point and timed with HIP events, with its
MFMA or HBM fraction of peak), `configs` (the same per-stage figures for the
C3-iid variant and configs C2, C4 and C5), the V1 rows, the reference's
published V2 shapes, and a CPU baseline (a PyTorch-CPU fp32 restatement of the
reference's path on two of the 32 heads, host cores).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-topk-attention_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


# HBM bytes per launch of the scoring kernel (candidate streams) on the default
# workload, from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of
# `bench.py --only scorer`, scaled by what the same counters read for a 128 MiB
# device copy (`--only copy`: FETCH_SIZE x2.0, WRITE_SIZE x1.0).  A PMC pass
# cannot run inside this process, so this is the last measured figure; it is
# refreshed whenever the kernel changes.
SCORE_FETCH_KIB, SCORE_WRITE_KIB = 6.517e5, 7.793e5
SCORE_TRAFFIC_BYTES = int((2.0 * SCORE_FETCH_KIB + 1.0 * SCORE_WRITE_KIB) * 1024)


def make_inputs(B, N, H, D, peaked, seed, dev, dtype=None, scale=1.0):
    """Synthetic q, k, v [B, N, H*D] generated in fp32 on the CPU (torch.Generator
    on the CPU, seeded), then cast and moved: the recipe the full-size parity
    tests use, so the timed data is the checked data.

    peaked=True is config 3: block centres c ~ N(0, 1) per 64-token block,
    k = 0.3 N(0, 1) + c[token // 64]; per 1024-query segment 8 block ids are
    drawn without replacement and each query takes one of them uniformly,
    q = 0.3 N(0, 1) + c[pick]; v ~ N(0, 1).  Otherwise q, k, v ~ scale * N(0, 1).
    """
    import torch

    dtype = dtype or torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(seed)
    C = H * D
    if not peaked:
        return tuple((torch.randn(B, N, C, generator=g) * scale).to(dtype).to(dev) for _ in range(3))
    b = 64
    M = N // b
    cent = torch.randn(B, M, C, generator=g)
    k = 0.3 * torch.randn(B, N, C, generator=g) + cent.repeat_interleave(b, dim=1)
    nseg = N // 1024
    choice = torch.stack([torch.randperm(M, generator=g)[:8] for _ in range(B * nseg)]).view(B, nseg, 8)
    pick_slot = torch.randint(0, 8, (B, N), generator=g)
    seg = torch.arange(N) // 1024
    pick = torch.gather(choice[:, seg, :], 2, pick_slot.unsqueeze(-1)).squeeze(-1)  # [B, N]
    q = 0.3 * torch.randn(B, N, C, generator=g) + torch.gather(cent, 1, pick.unsqueeze(-1).expand(B, N, C))
    v = torch.randn(B, N, C, generator=g)
    return tuple(x.to(dtype).to(dev) for x in (q, k, v))


def cpu_baseline(q, k, v, do, H, D, b, topk, thr, g, W, heads):
    """The reference algorithm's PyTorch path, restated in fp32 torch ops on the
    CPU (oracle/fta_torch_cpu.py), on heads 0 .. heads-1 of the workload at the
    full sequence length: score -> top-k -> merge -> sparse attention forward
    and autograd backward.  Work is counted as for the GPU value (2 N^2 D for
    the scores, 4 D P forward, 10 D P backward)."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fta_torch_cpu as T

    N = q.shape[1]
    secs, flops = 0.0, 0.0
    for h in range(heads):
        f = lambda t: t[0, :, h * D:(h + 1) * D].float().cpu().contiguous()
        qh, kh, vh, dh = f(q), f(k), f(v), f(do)
        t0 = time.perf_counter()
        merged, counts, *_ = T.pipeline_head(qh, kh, vh, dh, b, topk, thr, g, W)
        secs += time.perf_counter() - t0
        P = g * b * int(counts.sum())
        flops += 2.0 * N * N * D + 14.0 * D * P
    return {"value": flops / secs / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "host_cpus": os.cpu_count(), "kind": "port", "seconds": round(secs, 3),
            "full_config_seconds_extrapolated": round(secs * H / heads, 2),
            "sample": f"PyTorch-CPU fp32 restatement of the reference's path (oracle/fta_torch_cpu.py), "
                      f"{heads} of {H} heads at N={N} of the C3 workload (score+select+merge+fwd+bwd); "
                      f"full_config_seconds_extrapolated = seconds x {H}/{heads}"}


# V1 fused scoring rows of the reference's BENCHMARK.md (other hardware; D not
# stated there, 128 here): (B, N, H, b, topk, published "Scoring (ms)", its
# "FA2 (ms)" forward-only lower bound, line)
V1_ROWS = [(1, 32768, 4, 64, 64, 112.299, 18.524, 136), (1, 8192, 8, 128, 16, 3.759, 2.284, 108)]


def bench_v1(dev, stream):
    """V1 flash_topk_score (dense o + top-k block scores) forward, and forward
    + backward through o, at two rows of the reference's V1 benchmark, and the
    exact q-block union of the forward's top-k indices."""
    import torch

    import flash_topk_attn as v1

    D = 128
    res = []
    for B, N, H, b, topk, ref_ms, fa2_ms, line in V1_ROWS:
        gen = torch.Generator(device="cpu").manual_seed(9)
        q, k, v, do = (torch.randn(B, N, H * D, generator=gen).to(torch.bfloat16).to(dev) for _ in range(4))
        fw, fb = [], []
        for it in range(4):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            e[0].record(stream)
            with torch.no_grad():
                _, idx, _ = v1.flash_topk_score(q, k, v, H, b, topk)
            e[1].record(stream)
            ql, kl, vl = (t.detach().requires_grad_(True) for t in (q, k, v))
            o, _, _ = v1.flash_topk_score(ql, kl, vl, H, b, topk)
            o.backward(do)
            e[2].record(stream)
            torch.cuda.synchronize()
            if it:
                fw.append(e[0].elapsed_time(e[1]))
                fb.append(e[1].elapsed_time(e[2]))
        fms, fbms = sorted(fw)[1], sorted(fb)[1]
        # exact q-block union of those indices (q_block_size 32)
        ut = []
        for it in range(4):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            e[0].record(stream)
            v1.build_qblock_topk_indices(idx, 32)
            e[1].record(stream)
            torch.cuda.synchronize()
            if it:
                ut.append(e[0].elapsed_time(e[1]))
        f_fwd = 2.0 * B * H * N * N * D + 4.0 * B * H * N * N * D  # scoring QK^T + dense attention
        res.append({"config": f"B{B} N{N} H{H} D{D} b{b} topk{topk} bf16", "fwd_ms": round(fms, 3),
                    "fwd_tflops": round(f_fwd / fms / 1e9, 1), "fwd_bwd_ms": round(fbms, 3),
                    "union_g32_ms": round(sorted(ut)[1], 3),
                    "reference_published_ms_other_hw": ref_ms,
                    "reference_fa2_ms_other_hw": fa2_ms, "reference_source": f"BENCHMARK.md:{line}"})
        del q, k, v, do, ql, kl, vl, o, idx
    return res


# The reference's published V2 numbers (V2_BENCHMARK.md; bf16, threshold 1.0,
# q_block_size = score_block_size, qblock_topk = q_block_size * K).
# Forward rows, RTX 4090: (B, N, H, D, b, K, {stage: (published ms, line)}).
V2_FWD_ROWS = [
    (1, 2048, 32, 128, 64, 16, {"score": (0.68, 11), "attn_fwd": (1.24, 30)}),
    (1, 4096, 32, 128, 64, 16, {"score": (2.67, 12), "attn_fwd": (4.44, 31), "end_to_end": (7.26, 62)}),
    (1, 8192, 32, 128, 64, 16, {"score": (10.56, 13), "attn_fwd": (17.37, 32), "end_to_end": (28.15, 63)}),
    (1, 4096, 32, 128, 128, 16, {"score": (2.42, 14), "attn_fwd": (4.48, 33)}),
    (1, 4096, 32, 128, 64, 32, {"score": (2.69, 15), "attn_fwd": (4.53, 34), "end_to_end": (7.37, 64)}),
    (2, 4096, 32, 128, 64, 16, {"score": (5.28, 16), "attn_fwd": (8.95, 35), "end_to_end": (14.42, 65)}),
    (1, 2016, 32, 128, 48, 16, {"score": (0.98, 17), "attn_fwd": (1.98, 36)}),
    (1, 4032, 32, 128, 48, 16, {"score": (3.82, 18), "attn_fwd": (7.42, 37), "end_to_end": (11.25, 66)}),
    (1, 3008, 32, 128, 64, 16, {"score": (1.57, 19), "attn_fwd": (2.55, 38)}),
    (1, 5056, 32, 128, 64, 16, {"score": (4.63, 20), "attn_fwd": (6.70, 39), "end_to_end": (11.42, 67)}),
    (1, 4096, 4, 64, 64, 16, {"score": (0.28, 21), "attn_fwd": (0.38, 40)}),
    (1, 4096, 32, 64, 64, 16, {"score": (2.10, 22), "attn_fwd": (2.28, 41), "end_to_end": (4.47, 68)}),
]
# Sparse attention forward over D, RTX 3090: B1 H8 N2048 b64 K8: (D, published ms, line).
V2_ATTN_D_ROWS = [(32, 0.065, 49), (48, 0.140, 50), (64, 0.108, 51), (80, 0.203, 52), (96, 0.154, 53),
                  (128, 0.182, 54)]
# Backward (fwd + bwd minus fwd), RTX 3090, q and KV blocks of 64:
# (N, H, D, K, dtype, published ms, line).
V2_BWD_ROWS = (
    [(n, h, 128, 8, "bf16", ms, ln) for n, h, ms, ln in
     ((256, 8, 2.09, 78), (512, 8, 2.06, 79), (1024, 8, 1.93, 80), (2048, 8, 1.73, 81), (4096, 4, 1.96, 82),
      (8192, 2, 1.47, 83))]
    + [(2048, 8, 128, kk, "bf16", ms, ln) for kk, ms, ln in
       ((1, 1.99, 89), (2, 2.01, 90), (4, 1.95, 91), (8, 1.94, 92), (16, 1.91, 93), (32, 1.56, 94))]
    + [(2048, 8, d, 8, "bf16", ms, ln) for d, ms, ln in
       ((32, 2.03, 100), (48, 2.97, 101), (64, 2.04, 102), (80, 2.95, 103), (96, 1.20, 104), (128, 1.94, 105),
        (160, 1.88, 106), (256, 1.57, 107))]
    + [(2048, 8, 128, 8, dt, ms, ln) for dt, ms, ln in (("bf16", 1.76, 113), ("fp16", 1.95, 114))]
)


def _median_ms(fn, stream, reps=20, warmup=3):
    """Per-call GPU time of fn, timed the way the reference's V2 tables were
    (``triton.testing.do_bench``, V2_BENCHMARK.md:72): before every call a
    256 MB buffer is zeroed on the stream (the L2 / last-level cache starts
    cold, and the host queues the call while the GPU is still clearing, so its
    launch overhead is not timed), events bracket the call alone, and no call
    waits for the previous one.  Median over ``reps`` calls."""
    import torch

    flush = torch.empty(int(256e6 // 4), dtype=torch.int32, device="cuda")
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    # `stream` is the current stream: fn and the fill run on it
    for e0, e1 in ev:
        flush.zero_()
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    ts = sorted(e0.elapsed_time(e1) for e0, e1 in ev)
    del flush
    return ts[len(ts) // 2]


def bench_v2_rows(dev, stream):
    """Every shape of the reference's V2_BENCHMARK.md: flash_topk_score (scoring
    + top-k), flash_topk_attn forward given the merged indices, the end-to-end
    forward (score + merge + attention) and the backward (forward + backward
    minus forward, as the reference measures it); synthetic N(0, 1) inputs,
    timed as the reference's tables were (cold cache, calls queued back to
    back: `_median_ms`).  One entry per (shape, stage) with the published
    time and the GPU it was measured on."""
    import torch

    import flash_topk_attn_v2 as fta

    res = []

    def prepare(B, N, H, D, b, K, dtype=None):
        q, k, v = make_inputs(B, N, H, D, False, 11, dev, dtype=dtype)
        # q_block_size = score_block_size as the reference's tables state; its
        # flash_sparse_attn accepts q blocks of at most 64 (sparse_attn.py:279),
        # so the 128-token row uses 64
        g = min(b, 64)
        W = g * K
        idx, _, avg = fta.flash_topk_score(q, k, H, b, K, (0, 0), 1.0)
        merged, counts, _ = fta.build_qblock_topk_indices(idx, g, (0, 0), avg, W)
        return q, k, v, g, W, merged, counts

    def entry(cfg, stage, ms, flop, ref, hw):
        res.append({"config": cfg, "stage": stage, "ms": round(ms, 4),
                    "tflops": round(flop / ms / 1e9, 1) if flop else None, "reference_ms": ref[0],
                    "reference_hw": hw, "reference_source": f"V2_BENCHMARK.md:{ref[1]}"})

    with torch.no_grad():
        for B, N, H, D, b, K, refs in V2_FWD_ROWS:
            q, k, v, g, W, merged, counts = prepare(B, N, H, D, b, K)
            P = float(g * b * counts.sum().item())  # (query, key) pairs of the merged lists
            cfg = f"B{B} N{N} H{H} D{D} b{b} K{K} g{g} bf16"
            fns = {
                "score": (lambda: fta.flash_topk_score(q, k, H, b, K, (0, 0), 1.0), 2.0 * B * H * N * N * D),
                "attn_fwd": (lambda: fta.flash_topk_attn(q, k, v, merged, counts, H, g, b), 4.0 * D * P),
            }

            def e2e():
                i, _, a = fta.flash_topk_score(q, k, H, b, K, (0, 0), 1.0)
                m, c, _ = fta.build_qblock_topk_indices(i, g, (0, 0), a, W)
                return fta.flash_topk_attn(q, k, v, m, c, H, g, b)

            fns["end_to_end"] = (e2e, fns["score"][1] + fns["attn_fwd"][1])
            for stage, ref in refs.items():
                fn, flop = fns[stage]
                entry(cfg, stage, _median_ms(fn, stream), flop, ref, "RTX 4090")
            del q, k, v, merged, counts
        for D, ref_ms, line in V2_ATTN_D_ROWS:
            q, k, v, g, W, merged, counts = prepare(1, 2048, 8, D, 64, 8)
            P = float(g * 64 * counts.sum().item())
            ms = _median_ms(lambda: fta.flash_topk_attn(q, k, v, merged, counts, 8, g, 64), stream)
            entry(f"B1 N2048 H8 D{D} b64 K8 g64 bf16", "attn_fwd", ms, 4.0 * D * P, (ref_ms, line), "RTX 3090")
            del q, k, v, merged, counts
    for N, H, D, K, dt, ref_ms, line in V2_BWD_ROWS:
        dtype = torch.float16 if dt == "fp16" else torch.bfloat16
        q, k, v, g, W, merged, counts = prepare(1, N, H, D, 64, K, dtype)
        P = float(g * 64 * counts.sum().item())
        ql, kl, vl = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        do = torch.randn_like(q)

        def fwd():
            with torch.no_grad():
                return fta.flash_topk_attn(ql, kl, vl, merged, counts, H, g, 64)

        def fwd_bwd():
            for t in (ql, kl, vl):  # fresh gradients, not accumulated ones (do_bench's grad_to_none)
                t.grad = None
            o, _ = fta.flash_topk_attn(ql, kl, vl, merged, counts, H, g, 64)
            o.backward(do)

        ms = _median_ms(fwd_bwd, stream) - _median_ms(fwd, stream)
        entry(f"B1 N{N} H{H} D{D} b64 K{K} g64 {dt}", "attn_bwd", ms, 10.0 * D * P, (ref_ms, line), "RTX 3090")
        del q, k, v, ql, kl, vl, do, merged, counts
    return res


class Pipeline:
    """One configuration's inputs, indices and stage launchers (C ABI calls on
    the current stream), for per-stage HIP-event timing."""

    def __init__(self, dev, B, N, H, D, b, topk, thr, g, W, pad=(0, 0), qpad=(0, 0), peaked=False, seed=0,
                 dtype=None, scale=1.0, qkv=None):
        import torch

        import flash_topk_attn_v2 as fta
        from flash_topk_attn_v2 import _lib
        from flash_topk_attn_v2.sparse_attn_bwd import preprocess_delta

        self.torch, self.fta, self._lib, self.delta_fn = torch, fta, _lib, preprocess_delta
        self.dev, self.B, self.N, self.H, self.D, self.b = dev, B, N, H, D, b
        self.topk, self.thr, self.g, self.W, self.pad, self.qpad = topk, thr, g, W, pad, qpad
        self.dtype = dtype or torch.bfloat16
        self.q, self.k, self.v = qkv if qkv is not None else make_inputs(B, N, H, D, peaked, seed, dev, self.dtype,
                                                                           scale)
        gd = torch.Generator(device="cpu").manual_seed(seed + 7)
        self.do = torch.randn(B, N, H * D, generator=gd).to(self.dtype).to(dev)
        self.stream = torch.cuda.current_stream(dev)
        self.M = (pad[0] + N + pad[1]) // b
        self.idx, self.raw, self.avg = fta.flash_topk_score(self.q, self.k, H, b, topk, pad, thr)
        self.merged, self.counts, self.Wd = fta.build_qblock_topk_indices(self.idx, g, qpad, self.avg, W)
        self.QM = self.merged.shape[2]
        self.o, self.lse = fta.flash_topk_attn(self.q, self.k, self.v, self.merged, self.counts, H, g, b,
                                               None, None, pad, qpad)
        self.delta = preprocess_delta(self.o, self.do, H)
        L = _lib.lib()
        self.L = L
        self.st = _lib.i64arr([N * H * D, D, H * D])
        self.dt = _lib.dtype_code(self.dtype)
        m_out = topk if 0 < topk < self.M else self.M
        self.m_out = m_out
        self.ws_score = _lib.workspace(L.fta_topk_score_workspace_size_ex(B, H, N, D, b, pad[0], pad[1], topk), dev)
        geo = (B, H, N, D, g, b, qpad[0], qpad[1], pad[0], pad[1])
        self.ws_bwd = _lib.workspace(L.fta_sparse_attn_bwd_workspace_size(*geo), dev)
        self.dq, self.dk, self.dv = (torch.empty_like(self.q) for _ in range(3))
        self.streams_ok = b in (64, 128) and D in (64, 128) and m_out <= 32
        shp = (B, H, N, m_out)
        self.sel_out = (torch.empty(shp, dtype=torch.int32, device=dev), torch.empty(shp, device=dev),
                        torch.empty(shp, device=dev))
        if self.streams_ok:
            self.scorer()  # ws_score holds valid streams from here on (select_streams reads them)

    # --- stage launchers
    def score(self):
        self.fta.flash_topk_score(self.q, self.k, self.H, self.b, self.topk, self.pad, self.thr)

    def scorer(self):
        L, _lib = self.L, self._lib
        rc = L.fta_topk_score_candidates(self.q.data_ptr(), self.k.data_ptr(), self.dt, self.B, self.H, self.N,
                                         self.D, self.st, self.st, self.b, self.pad[0], self.pad[1], self.D ** -0.5,
                                         self.topk, self.ws_score.data_ptr(), self.ws_score.numel(),
                                         self.stream.cuda_stream)
        _lib.check(rc, "fta_topk_score_candidates")

    def select_streams(self):
        """The stream selector alone, over the streams the last scorer() call left."""
        L, _lib = self.L, self._lib
        rc = L.fta_topk_select_candidates(self.q.data_ptr(), self.k.data_ptr(), self.dt, self.B, self.H, self.N,
                                          self.D, self.st, self.st, self.b, self.pad[0], self.pad[1], self.D ** -0.5,
                                          self.topk, self.thr, self.sel_out[0].data_ptr(),
                                          self.sel_out[1].data_ptr(), self.sel_out[2].data_ptr(),
                                          self.ws_score.data_ptr(), self.ws_score.numel(), self.stream.cuda_stream)
        _lib.check(rc, "fta_topk_select_candidates")

    def merge(self):
        self.fta.build_qblock_topk_indices(self.idx, self.g, self.qpad, self.avg, self.W)

    def fwd(self):
        self.fta.flash_topk_attn(self.q, self.k, self.v, self.merged, self.counts, self.H, self.g, self.b,
                                 None, None, self.pad, self.qpad)

    def delta_stage(self):
        self.delta_fn(self.o, self.do, self.H)

    def _bwd_args(self):
        s = self.st
        return (self.q.data_ptr(), s, self.k.data_ptr(), s, self.v.data_ptr(), s, self.do.data_ptr(), s, self.dt,
                self.B, self.H, self.H, self.N, self.D, self.merged.data_ptr(), self.QM, self.merged.shape[3],
                self.g, self.b, self.qpad[0], self.qpad[1], self.pad[0], self.pad[1], self.D ** -0.5,
                self.lse.data_ptr(), self.delta.data_ptr())

    def dq_stage(self):
        rc = self.L.fta_sparse_attn_bwd_dq(*self._bwd_args(), self.dq.data_ptr(), self.st, self.stream.cuda_stream)
        self._lib.check(rc, "fta_sparse_attn_bwd_dq")

    def bwd_gqa_stage(self):
        """dK/dV then dQ through the combined entry (dQ reuses the dK/dV pass's head placement)."""
        rc = self.L.fta_sparse_attn_bwd_gqa(*self._bwd_args(), self.dq.data_ptr(), self.st, self.dk.data_ptr(),
                                            self.st, self.dv.data_ptr(), self.st, self.ws_bwd.data_ptr(),
                                            self.ws_bwd.numel(), self.stream.cuda_stream)
        self._lib.check(rc, "fta_sparse_attn_bwd_gqa")

    def dkv_stage(self):
        rc = self.L.fta_sparse_attn_bwd_dkv(*self._bwd_args(), self.dk.data_ptr(), self.st, self.dv.data_ptr(),
                                            self.st, self.ws_bwd.data_ptr(), self.ws_bwd.numel(),
                                            self.stream.cuda_stream)
        self._lib.check(rc, "fta_sparse_attn_bwd_dkv")

    # --- measurement
    def time(self, fn, reps=5):
        """Mean ms per call over `reps` back-to-back calls, HIP events on the stream."""
        torch = self.torch
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(self.stream)
        for _ in range(reps):
            fn()
        e1.record(self.stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def pairs(self):
        """P = sum over (b, h, q-block) of valid query rows x valid KV tokens of the listed blocks."""
        torch = self.torch
        N, g, b = self.N, self.g, self.b
        qs = torch.arange(self.QM, device=self.dev) * g - self.qpad[0]
        qvalid = (torch.clamp(qs + g, max=N) - torch.clamp(qs, min=0)).clamp(min=0).float()
        ks = torch.arange(self.M, device=self.dev) * b - self.pad[0]
        kvalid = (torch.clamp(ks + b, max=N) - torch.clamp(ks, min=0)).clamp(min=0).float()
        m = self.merged.long()
        tok = torch.where(m >= 0, kvalid[m.clamp(min=0)], torch.zeros((), device=self.dev)).sum(-1)  # [B,H,QM]
        return float((tok * qvalid).sum().item())

    def selector_bytes(self):
        """Bytes the stream selector moves: candidate entries read (8 B each), the
        row total and start bound (8 B per row) and the three outputs."""
        rows = self.B * self.H * self.N
        waves = self.B * self.H * ((self.N + 255) // 256) * 4
        cnt = self.ws_score[: waves * 4].view(self.torch.int32)  # per-wave entry counts lead the workspace
        return float(cnt.clamp(min=0).sum().item()) * 8 + rows * 8 + rows * self.m_out * 12

    def stream_stats(self):
        """Entries per query of the scorer's candidate streams, tiles sent to the
        fallback, and the stream workspace (after a scorer() + select_streams())."""
        waves = self.B * self.H * ((self.N + 255) // 256) * 4
        cnt = self.ws_score[: waves * 4].view(self.torch.int32)
        return {"entries_per_query": round(float(cnt.clamp(min=0).sum().item()) / (self.B * self.H * self.N), 2),
                "overflow_waves": int((cnt < 0).sum().item()), "workspace_bytes": int(self.ws_score.numel())}

    def stages(self, bwd=True, reps=5):
        """Per-stage ms and roofline fractions."""
        B, H, N, D, b, g = self.B, self.H, self.N, self.D, self.b, self.g
        P = self.pairs()
        r = {}
        f_score = 2.0 * B * H * N * N * D
        t_score = self.time(self.score, reps)
        r["score"] = {"ms": t_score, "tflops": f_score / t_score / 1e9}
        if self.streams_ok:
            t_k = self.time(self.scorer, reps)
            sel_ms = self.time(self.select_streams, reps)
            r["score_kernel"] = {"ms": t_k, "bound": "mfma", "tflops": f_score / t_k / 1e9,
                                 "frac": f_score / t_k / 1e9 / PEAK_BF16_TFLOPS}
            sb = self.selector_bytes()
            r["topk_select"] = {"ms": sel_ms, "bound": "hbm", "gbs": sb / sel_ms / 1e6,
                                "frac": sb / sel_ms / 1e6 / PEAK_HBM_GBS, "bytes": sb,
                                "note": "fta_topk_select_candidates alone over the scorer's streams"}
            r["streams"] = self.stream_stats()
        K = self.idx.shape[-1]
        mb = 2.0 * B * H * N * K * 4 + B * H * self.QM * (self.merged.shape[3] + 1) * 4
        t = self.time(self.merge, reps)
        r["merge"] = {"ms": t, "bound": "hbm", "gbs": mb / t / 1e6, "frac": mb / t / 1e6 / PEAK_HBM_GBS}
        t = self.time(self.fwd, reps)
        r["fwd"] = {"ms": t, "bound": "mfma", "tflops": 4 * D * P / t / 1e9,
                    "frac": 4 * D * P / t / 1e9 / PEAK_BF16_TFLOPS}
        r["P_pairs"] = P
        if bwd:
            db = 2.0 * B * N * H * D * 2 + B * H * N * 4
            t_d = self.time(self.delta_stage, reps)
            r["delta"] = {"ms": t_d, "bound": "hbm", "gbs": db / t_d / 1e6, "frac": db / t_d / 1e6 / PEAK_HBM_GBS}
            t_q = self.time(self.dq_stage, reps)
            r["dq"] = {"ms": t_q, "bound": "mfma", "tflops_executed_6DP": 6 * D * P / t_q / 1e9,
                       "frac": 6 * D * P / t_q / 1e9 / PEAK_BF16_TFLOPS}
            t_kv = self.time(self.dkv_stage, reps)
            r["dkv"] = {"ms": t_kv, "bound": "mfma", "tflops_executed_8DP": 8 * D * P / t_kv / 1e9,
                        "frac": 8 * D * P / t_kv / 1e9 / PEAK_BF16_TFLOPS,
                        "note": "includes the membership bitmap and log2-lse kernels"}
            r["dq"]["note"] = "dQ entry alone: natural head order (in the combined backward dQ runs in the head placement of the dK/dV pass)"
            t_b = t_d + self.time(self.bwd_gqa_stage, reps)
            r["bwd"] = {"ms": t_b, "tflops_10DP": 10 * D * P / t_b / 1e9,
                        "frac": 10 * D * P / t_b / 1e9 / PEAK_BF16_TFLOPS,
                        "note": "delta + the combined dK/dV + dQ entry"}
        return {k2: ({kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v2.items()}
                     if isinstance(v2, dict) else v2) for k2, v2 in r.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the C3-iid, C2, C4, C5 and V1 rows")
    ap.add_argument("--cpu-heads", type=int, default=2)
    ap.add_argument("--only", choices=["score", "scorer", "topk", "merge", "fwd", "bwd", "dq", "dkv", "copy", "v1",
                                       "v2"],
                    default=None, help="profiling aid: run one stage of the C3 step --steps times and exit")
    ap.add_argument("--iid", action="store_true",
                    help="with --only: the C3-iid variant (iid q/k/v, threshold 1.0, qblock_topk 512)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); every stage is per (b, h) "
              "and shards over heads with no communication, so N>1 is not measured here.", file=sys.stderr)
        sys.exit(2)

    import torch

    import flash_topk_attn_v2 as fta

    dev = torch.device("cuda:0")
    if args.only == "v1":  # the V1 benchmark rows alone (profiling aid)
        for _ in range(args.steps):
            bench_v1(dev, torch.cuda.current_stream(dev))
        torch.cuda.synchronize()
        print(json.dumps({"only": "v1", "steps": args.steps}), flush=True)
        return
    if args.only == "v2":  # the reference's V2 shapes alone
        print(json.dumps({"only": "v2", "rows": bench_v2_rows(dev, torch.cuda.current_stream(dev))}), flush=True)
        return
    B, N, H, D, b, topk, thr, g, W = 1, 32768, 32, 128, 64, 16, 0.9, 32, 256
    stream = torch.cuda.current_stream(dev)

    if args.only:
        if args.iid:
            pl = Pipeline(dev, B, N, H, D, b, topk, 1.0, g, 512, peaked=False, seed=3)
        else:
            pl = Pipeline(dev, B, N, H, D, b, topk, thr, g, W, peaked=True, seed=2)
        big = torch.empty(256 << 20, device=dev, dtype=torch.uint8)
        fn = {"score": pl.score, "scorer": pl.scorer, "topk": pl.select_streams, "merge": pl.merge, "fwd": pl.fwd,
              "dq": pl.dq_stage, "dkv": pl.dkv_stage,
              "bwd": lambda: (pl.delta_stage(), pl.dq_stage(), pl.dkv_stage()),
              "copy": lambda: big[: 128 << 20].copy_(big[128 << 20:])}[args.only]
        if args.only == "topk":
            pl.scorer()  # the streams the selector reads
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "steps": args.steps}), flush=True)
        return

    q, k, v = make_inputs(B, N, H, D, True, 2, dev)
    gd = torch.Generator(device="cpu").manual_seed(7)
    do = torch.randn(B, N, H * D, generator=gd).to(torch.bfloat16).to(dev)
    ql, kl, vl = (t.detach().requires_grad_(True) for t in (q, k, v))

    def step():
        ql.grad = kl.grad = vl.grad = None
        idx, raw, avg = fta.flash_topk_score(ql.detach(), kl.detach(), H, b, topk, (0, 0), thr)
        merged, counts, Wd = fta.build_qblock_topk_indices(idx, g, (0, 0), avg, W)
        o, lse = fta.flash_topk_attn(ql, kl, vl, merged, counts, H, g, b)
        o.backward(do)
        return counts

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        counts = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps

    P = g * b * float(counts.sum().item())
    f_score = 2.0 * B * H * N * N * D
    f_fwd, f_bwd = 4.0 * D * P, 10.0 * D * P
    flops = f_score + f_fwd + f_bwd
    value = flops / (ms * 1e-3) / 1e12

    # per-stage times and rooflines, each stage launched alone (HIP events on the stream)
    pl = Pipeline(dev, B, N, H, D, b, topk, thr, g, W, qkv=(q, k, v), seed=0)
    pl.do = do
    pl.delta = pl.delta_fn(pl.o, do, H)
    stages = pl.stages(bwd=True)
    # dominant kernel: the scoring kernel (candidate streams), 10 launches
    k_ms = pl.time(pl.scorer, reps=10)
    achieved = f_score / (k_ms * 1e-3) / 1e12

    out = {
        "metric": "score+attn fwd+bwd ms and TFLOP/s at N=32K,D=128 bf16; % of MFMA peak",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (BASELINE config 3: peaked block-centred q/k, iid v, CPU generator seed 2)",
        "config": {"workload": "C3 threshold: B1 N32768 H32 D128, b64 topk16 thr0.9 g32 W256; "
                               "score+merge+sparse fwd+bwd",
                   "global_batch": B, "seq_len": N, "heads": H, "head_dim": D, "parallelism": "none"},
        "flops": {"score": f_score, "fwd": f_fwd, "bwd_10DP": f_bwd, "P_pairs": P},
        "roofline": {"bound": "mfma", "kernel": "fta_block_score_lse_pipe_kernel (candidate streams)",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "kernel_ms": round(k_ms, 3),
                     "traffic": SCORE_TRAFFIC_BYTES,
                     "algorithmic_bytes": 2 * B * H * N * D * 2},
        "stage_roofline": stages,
    }
    del pl, ql, kl, vl
    torch.cuda.empty_cache()

    if not args.no_extra:
        extra = {}
        # C3-iid: the MFMA gate for the sparse forward / backward (threshold 1.0, W 512)
        pl = Pipeline(dev, B, N, H, D, b, topk, 1.0, g, 512, peaked=False, seed=3)
        extra["C3_iid"] = pl.stages(bwd=True, reps=3)
        extra["C3_iid"]["mean_count"] = float(pl.counts.float().mean().item())
        del pl
        torch.cuda.empty_cache()
        # C2: B2 N8192 H16 D64 fp16, top-16, g = 1 (W 16) and g = 32 (W 512), forward only
        for name, gg, ww in (("C2_g1", 1, 16), ("C2_g32", 32, 512)):
            pl = Pipeline(dev, 2, 8192, 16, 64, 64, 16, 1.0, gg, ww, peaked=False, seed=1, dtype=torch.float16)
            extra[name] = pl.stages(bwd=False)
            del pl
        # C4: virtual padding, B2 N10000 H12 D64 fp16, padding (24, 24), top-8, g 16, forward + backward
        pl = Pipeline(dev, 2, 10000, 12, 64, 64, 8, 1.0, 16, None, pad=(24, 24), peaked=False, seed=4,
                      dtype=torch.float16)
        extra["C4"] = pl.stages(bwd=True)
        del pl
        # C5: training, B1 N16384 H16 D128, q/k/v ~ N(0, 1) / sqrt(D); indices from layer 0 reused by 4 layers
        pl = Pipeline(dev, 1, 16384, 16, 128, 64, 16, 1.0, 32, 512, peaked=False, seed=5, scale=D ** -0.5)
        layers = []
        for layer in range(4):
            ql5, kl5, vl5 = (t.requires_grad_(True) for t in make_inputs(1, 16384, 16, 128, False, 50 + layer, dev,
                                                                          scale=D ** -0.5))
            e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            e[0].record(stream)
            o5, _ = fta.flash_topk_attn(ql5, kl5, vl5, pl.merged, pl.counts, 16, 32, 64)
            e[1].record(stream)
            o5.backward(pl.do)
            e[2].record(stream)
            torch.cuda.synchronize()
            layers.append((e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])))
        P5 = pl.pairs()
        fw5 = sum(x[0] for x in layers[1:]) / 3
        bw5 = sum(x[1] for x in layers[1:]) / 3
        extra["C5"] = {"score_merge": pl.stages(bwd=False), "layers": 4, "P_pairs": P5,
                       "fwd_ms_per_layer": round(fw5, 4), "bwd_ms_per_layer": round(bw5, 4),
                       "fwd_frac": round(4 * 128 * P5 / fw5 / 1e9 / PEAK_BF16_TFLOPS, 4),
                       "bwd_frac_10DP": round(10 * 128 * P5 / bw5 / 1e9 / PEAK_BF16_TFLOPS, 4)}
        del pl
        torch.cuda.empty_cache()
        out["configs"] = extra
        out["v1_score"] = bench_v1(dev, stream)
        out["v2_reference_rows"] = bench_v2_rows(dev, stream)

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(q, k, v, do, H, D, b, topk, thr, g, W, args.cpu_heads)

    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
