"""Benchmark: flash-topk-attention V2 hot path on one MI355X.

One step = flash_topk_score -> build_qblock_topk_indices -> flash_topk_attn
forward -> backward, on BASELINE config 3 (B=1, N=32768, H=32, D=128 bf16,
peaked synthetic attention, b=64, topk=16, threshold=0.9, g=32, W=256).
Prints one JSON line (driver contract).  Extra fields: per-stage ms, the
C3-iid variant's forward/backward throughput, the scoring kernel's roofline
(measured with HIP events on the stream it runs on) and a CPU baseline (the
numpy oracle on a bounded sample, host cores).
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


# HBM bytes per fta_block_score_lse launch on the default workload (pipelined
# kernel), from rocprofv3 --pmc FETCH_SIZE (6.544e5 KiB, x2.0) and WRITE_SIZE
# (2.102e6 KiB, x1.0); the factors are what the same counters read for a 128 MiB
# device copy (bench.py --only copy).  A PMC pass cannot run inside this process,
# so the figure is the last measured one and is refreshed with the kernel.
SCORE_TRAFFIC_BYTES = int((2.0 * 6.544e5 + 1.0 * 2.102e6) * 1024)


def make_inputs(B, N, H, D, peaked, seed, dev):
    import torch

    g = torch.Generator(device=dev).manual_seed(seed)
    C = H * D
    if not peaked:
        q, k, v = (torch.randn(B, N, C, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
        return q, k, v
    b = 64
    M = N // b
    cent = torch.randn(B, M, C, generator=g, device=dev)
    k = 0.3 * torch.randn(B, N, C, generator=g, device=dev) + cent.repeat_interleave(b, dim=1)
    nseg = N // 1024
    choice = torch.stack([torch.randperm(M, generator=g, device=dev)[:8] for _ in range(B * nseg)]).view(B, nseg, 8)
    pick_slot = torch.randint(0, 8, (B, N), generator=g, device=dev)
    seg = torch.arange(N, device=dev) // 1024
    pick = torch.gather(choice[:, seg, :], 2, pick_slot.unsqueeze(-1)).squeeze(-1)  # [B, N]
    q = 0.3 * torch.randn(B, N, C, generator=g, device=dev) + torch.gather(
        cent, 1, pick.unsqueeze(-1).expand(B, N, C))
    v = torch.randn(B, N, C, generator=g, device=dev)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def cpu_baseline(q, k, v, do, H, D, b, topk, thr, g, W, rows, heads):
    """Numpy oracle (oracle/fta_oracle.py) on heads 0 .. heads-1, first `rows` queries of each."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fta_oracle as O

    N = q.shape[1]
    secs, flops = 0.0, 0.0
    for h in range(heads):
        f = lambda t: t[:, :, h * D:(h + 1) * D].float().cpu().numpy()
        qn, kn, vn, dn = f(q), f(k), f(v), f(do)
        t0 = time.perf_counter()
        sc = O.block_score(qn, kn, 1, b, rows=np.arange(rows))
        idx, raw, avg = O.topk_select(sc.astype(np.float32), thr, topk, b)
        merged, counts, _ = O.build_qblock_topk_indices(idx, g, (0, 0), avg, W)
        qbl = [(0, 0, qm) for qm in range(rows // g)]
        full = np.full((1, 1, N // g, W), -1, dtype=np.int32)
        full[:, :, : rows // g] = merged
        O.sparse_attn(qn, kn, vn, full, 1, g, b, None, qblocks=qbl)
        O.sparse_attn_bwd(qn, kn, vn, dn, full, 1, g, b, None, qblocks=qbl)
        secs += time.perf_counter() - t0
        P = g * b * int(counts.sum())
        flops += 2.0 * rows * N * D + 14.0 * D * P
    try:  # threads of numpy's BLAS pool (the only multi-threaded part of the oracle)
        import threadpoolctl

        cores = max(int(i.get("num_threads", 1)) for i in threadpoolctl.threadpool_info()) or 1
    except Exception:
        cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": flops / secs / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "seconds": secs,
            "sample": f"numpy oracle, {heads} head(s) x {rows} queries of the C3 workload "
                      f"(score+select+merge+fwd+bwd), float64 BLAS"}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-iid", action="store_true")
    ap.add_argument("--no-v1", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=32768)
    ap.add_argument("--cpu-heads", type=int, default=2)
    ap.add_argument("--only", choices=["score", "topk", "merge", "fwd", "bwd", "copy", "v1"], default=None,
                    help="profiling aid: run one stage of the C3 step --steps times and exit")
    ap.add_argument("--iid", action="store_true",
                    help="with --only: the C3-iid variant (iid q/k/v, threshold 1.0, qblock_topk 512)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); every stage is per (b, h) "
              "and shards over heads with no communication, so N>1 is not measured here.", file=sys.stderr)
        sys.exit(2)

    import torch

    import flash_topk_attn_v2 as fta
    from flash_topk_attn_v2 import _lib

    dev = torch.device("cuda:0")
    if args.only == "v1":  # the V1 benchmark rows alone (profiling aid)
        for _ in range(args.steps):
            bench_v1(dev, torch.cuda.current_stream(dev))
        torch.cuda.synchronize()
        print(json.dumps({"only": "v1", "steps": args.steps}), flush=True)
        return
    B, N, H, D, b, topk, thr, g, W = 1, 32768, 32, 128, 64, 16, 0.9, 32, 256
    q, k, v = make_inputs(B, N, H, D, True, 2, dev)
    gd = torch.Generator(device=dev).manual_seed(7)
    do = torch.randn(B, N, H * D, generator=gd, device=dev).to(torch.bfloat16)
    ql, kl, vl = (t.detach().requires_grad_(True) for t in (q, k, v))

    stream = torch.cuda.current_stream(dev)

    def step(record=None):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)] if record is not None else None
        ql.grad = kl.grad = vl.grad = None
        if ev: ev[0].record(stream)
        idx, raw, avg = fta.flash_topk_score(ql.detach(), kl.detach(), H, b, topk, (0, 0), thr)
        if ev: ev[1].record(stream)
        merged, counts, Wd = fta.build_qblock_topk_indices(idx, g, (0, 0), avg, W)
        if ev: ev[2].record(stream)
        o, lse = fta.flash_topk_attn(ql, kl, vl, merged, counts, H, g, b)
        if ev: ev[3].record(stream)
        o.backward(do)
        if ev:
            ev[4].record(stream)
            record.append(ev)
        return counts

    if args.only:
        if args.iid:
            thr, W = 1.0, 512
            q, k, v = make_inputs(B, N, H, D, False, 3, dev)
            ql, kl, vl = (t.detach().requires_grad_(True) for t in (q, k, v))
        idx, raw, avg = fta.flash_topk_score(q, k, H, b, topk, (0, 0), thr)
        merged, counts, Wd = fta.build_qblock_topk_indices(idx, g, (0, 0), avg, W)
        o, lse = fta.flash_topk_attn(ql, kl, vl, merged, counts, H, g, b)
        M_ = N // b
        blk = torch.empty(B * H * M_ * N, device=dev, dtype=torch.float32)
        row = torch.empty(B * H * N, device=dev, dtype=torch.float32)
        sst = _lib.i64arr([N * H * D, D, H * D])
        big = torch.empty(256 << 20, device=dev, dtype=torch.uint8)
        for _ in range(args.steps):
            if args.only == "score":
                _lib.check(_lib.lib().fta_block_score_lse(q.data_ptr(), k.data_ptr(), 0, B, H, N, D, sst, sst, b, 0, 0,
                                                          D ** -0.5, blk.data_ptr(), row.data_ptr(),
                                                          stream.cuda_stream), "score")
            elif args.only == "topk":
                fta.flash_topk_score(q, k, H, b, topk, (0, 0), thr)
            elif args.only == "merge":
                fta.build_qblock_topk_indices(idx, g, (0, 0), avg, W)
            elif args.only == "fwd":
                fta.flash_topk_attn(q, k, v, merged, counts, H, g, b)
            elif args.only == "bwd":
                ql.grad = kl.grad = vl.grad = None
                o, lse = fta.flash_topk_attn(ql, kl, vl, merged, counts, H, g, b)
                o.backward(do)
            else:  # plain copy of 256 MiB: calibrates FETCH_SIZE / WRITE_SIZE
                big[: 128 << 20].copy_(big[128 << 20:])
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "steps": args.steps}), flush=True)
        return

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        counts = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps

    recs = []
    for _ in range(3):
        counts = step(recs)
    torch.cuda.synchronize()
    names = ["score", "merge", "fwd", "bwd"]
    stage = {n: sorted(r[i].elapsed_time(r[i + 1]) for r in recs)[1] for i, n in enumerate(names)}

    P = g * b * float(counts.sum().item())
    f_score = 2.0 * B * H * N * N * D
    f_fwd, f_bwd = 4.0 * D * P, 10.0 * D * P
    flops = f_score + f_fwd + f_bwd
    value = flops / (ms * 1e-3) / 1e12

    # dominant kernel: scoring stage 1 (fta_block_score_lse_kernel), timed alone
    M = N // b
    blk = torch.empty(B * H * M * N, device=dev, dtype=torch.float32)
    row = torch.empty(B * H * N, device=dev, dtype=torch.float32)
    qs = _lib.i64arr([N * H * D, D, H * D])
    L = _lib.lib()

    def score_lse():
        rc = L.fta_block_score_lse(q.data_ptr(), k.data_ptr(), 0, B, H, N, D, qs, qs, b, 0, 0, D ** -0.5,
                                   blk.data_ptr(), row.data_ptr(), stream.cuda_stream)
        _lib.check(rc, "fta_block_score_lse")

    score_lse()
    reps = 10
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        score_lse()
    e1.record(stream)
    torch.cuda.synchronize()
    k_ms = e0.elapsed_time(e1) / reps
    achieved = f_score / (k_ms * 1e-3) / 1e12
    del blk, row

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
        "data": "synthetic (BASELINE config 3: peaked block-centred q/k, iid v, seed 2)",
        "config": {"workload": "C3 threshold: B1 N32768 H32 D128, b64 topk16 thr0.9 g32 W256; "
                               "score+merge+sparse fwd+bwd",
                   "global_batch": B, "seq_len": N, "heads": H, "head_dim": D, "parallelism": "none"},
        "stage_ms": {k2: round(v2, 3) for k2, v2 in stage.items()},
        "flops": {"score": f_score, "fwd": f_fwd, "bwd_10DP": f_bwd, "P_pairs": P},
        "roofline": {"bound": "mfma", "kernel": "fta_block_score_lse_pipe_kernel", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "kernel_ms": round(k_ms, 3),
                     "traffic": SCORE_TRAFFIC_BYTES if (B, N, H, D, b) == (1, 32768, 32, 128, 64) else None,
                     "algorithmic_bytes": 2 * B * H * N * D * 2 + 4 * B * H * (M + 1) * N},
    }

    if not args.no_iid:
        # C3-iid variant (the MFMA gate for the sparse forward/backward)
        del ql, kl, vl
        torch.cuda.empty_cache()
        qi, ki, vi = make_inputs(B, N, H, D, False, 3, dev)
        idx, raw, avg = fta.flash_topk_score(qi, ki, H, b, topk, (0, 0), 1.0)
        merged, counts_i, _ = fta.build_qblock_topk_indices(idx, g, (0, 0), avg, 512)
        qi.requires_grad_(True)
        ki.requires_grad_(True)
        vi.requires_grad_(True)
        fw, bw = [], []
        for it in range(4):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            e[0].record(stream)
            o, lse = fta.flash_topk_attn(qi, ki, vi, merged, counts_i, H, g, b)
            e[1].record(stream)
            o.backward(do)
            e[2].record(stream)
            torch.cuda.synchronize()
            if it:
                fw.append(e[0].elapsed_time(e[1]))
                bw.append(e[1].elapsed_time(e[2]))
        Pi = g * b * float(counts_i.sum().item())
        fms, bms = sorted(fw)[1], sorted(bw)[1]
        out["c3_iid"] = {"fwd_ms": round(fms, 3), "bwd_ms": round(bms, 3),
                         "fwd_tflops": round(4 * D * Pi / fms / 1e9, 2),
                         "bwd_tflops_10DP": round(10 * D * Pi / bms / 1e9, 2),
                         "mean_count": Pi / (g * b * B * H * (N // g))}

    if not args.no_v1:
        out["v1_score"] = bench_v1(dev, stream)

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(q, k, v, do, H, D, b, topk, thr, g, W, args.cpu_rows, args.cpu_heads)

    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
