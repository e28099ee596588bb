#!/usr/bin/env python3
"""Headline benchmark of the retrieval hot path on one MI355X.

Workload (BASELINE.json configs[0] shape): q8 packed-candidate dot + top-10,
N = 65,536 candidates x D = 256 per query, one query per candidate set.  A
step scores `--sets` independent (query, candidate set) problems in one
fused launch sequence -- the reference's batched score layout
[Q,D] x [Q,N,D] (runtime/backend/tensor_ops.go:1511-1519) -- over distinct
candidate copies whose total (32 x 17 MB) exceeds the 256 MB MALL, so the
candidates stream from HBM.  Inputs are resident in HBM before timing.

Prints one JSON line.  `roofline` is measured live with HIP events around
every launch of the dominant kernel (q8_scan); `cpu_baseline` times the
CPU oracle's restatement of the reference host path (f32 dotRows +
full-sort topKTensor, one thread) on a bounded sample of the same problems.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
N, D, K = 65536, 256, 10


def c0_bytes_per_problem(n=N, d=D, k=K) -> int:
    # candidates (int8 codes + f32 scale) + f16 query + k (id, score) pairs
    return n * (d + 4) + 2 * d + k * 8


def cpu_baseline(codes, scales, queries, budget_s: float) -> dict:
    """Reference host path, restated by the CPU oracle (1 thread): the q8
    tensor's f32-backed values, f32 dotRows, full-sort topKTensor."""
    from oracle import oracle as orc

    sets = codes.shape[0]
    docs = [codes[s].astype(np.float32) * scales[s][:, None] for s in range(min(sets, 2))]
    qf = orc.f16_to_f32(queries)
    done = 0
    t0 = time.perf_counter()
    while True:
        s = done % len(docs)
        scores = orc.dot_rows(qf[s], docs[s])
        orc.topk(scores, K)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 4000:
            break
    return {
        "value": done * N / el,
        "unit": "candidates/s",
        "cores": 1,
        "kind": "port",
        "sample": "%d C0 problems (1 query x %d x %d), reference host path restated in C "
                  "(f32 dotRows + full-sort topKTensor), %.1f s" % (done, N, D, el),
    }


def profiled_traffic(name: str):
    """HBM bytes per launch measured by rocprofv3 PMC (FETCH_SIZE + WRITE_SIZE,
    copy-kernel calibrated) and recorded in the committed profile summary."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def copy_calibration(mib: int) -> int:
    """A plain copy kernel of known size: under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE per dispatch calibrate the counters (bytes read =
    bytes written = mib MiB per launch)."""
    import torch

    n = mib * 1024 * 1024 // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": n * 4, "launches": 10}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sets", type=int, default=32, help="C0 problems per step")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC scaling run)")
    args = ap.parse_args()
    if args.copy_calibration_mb:
        return copy_calibration(args.copy_calibration_mb)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (candidate rows "
              "would shard across GPUs with a KB-scale top-k merge; see DESIGN.md). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    from manta_amd import rocm, synth

    t_gen = time.perf_counter()
    queries, codes, scales = synth.config0(sets=args.sets)
    t_gen = time.perf_counter() - t_gen

    rt = rocm.Runtime(0)
    cands = rt.bind_q8(codes, scales)
    q_dev = rt.to_device(queries)
    ids = rt.empty((args.sets, K), np.int32)
    sc = rt.empty((args.sets, K), np.float32)
    out = (ids, sc, None)

    for _ in range(args.warmup):
        rt.score_topk(cands, "dot", q_dev, K, out=out)
    rt.synchronize()

    rt.set_timing(True)
    rt.timing(reset=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        rt.score_topk(cands, "dot", q_dev, K, out=out)
    rt.synchronize()
    elapsed = time.perf_counter() - t0
    scan_n, scan_ms = rt.timing("q8_scan")
    all_n, all_ms = rt.timing(None)
    rt.set_timing(False)

    ms_per_step = elapsed * 1000.0 / args.steps
    value = args.sets * N / (elapsed / args.steps)
    scan_avg_s = scan_ms / 1000.0 / max(scan_n, 1)
    bytes_per_launch = args.sets * c0_bytes_per_problem()
    achieved = bytes_per_launch / scan_avg_s / 1e9

    # single-query latency (one problem per call, back to back)
    q1 = rt.to_device(queries[:1])
    one = rt.bind_q8(codes[0], scales[0])
    ids1 = rt.empty((1, K), np.int32)
    for _ in range(5):
        rt.score_topk(one, "dot", q1, K, out=(ids1, None, None))
    rt.synchronize()
    reps = 200
    t1 = time.perf_counter()
    for _ in range(reps):
        rt.score_topk(one, "dot", q1, K, out=(ids1, None, None))
    rt.synchronize()
    single_us = (time.perf_counter() - t1) * 1e6 / reps

    line = {
        "metric": "candidates scored/sec (q8 dot + top-k, BASELINE config 0 shape)",
        "value": value,
        "unit": "candidates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8",
        "data": "synthetic (seeded generator, manta_amd/csrc/synth.cpp)",
        "config": {
            "workload": "c0_q8_dot_top10_batched",
            "n": N, "d": D, "k": K,
            "problems_per_step": args.sets,
            "layout": "[Q,D] x [Q,N,D]: one query per distinct 65536x256 q8 candidate set",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "q8_scan (manta::q8_scan_kernel<0,16,1>)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic("q8_scan_c0_batched.md") if args.sets == 32 else None,
            "traffic_source": "profiles/q8_scan_c0_batched.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
            "avg_launch_us": scan_avg_s * 1e6,
            "bytes_per_launch": bytes_per_launch,
        },
        "device_ms_per_step_all_kernels": all_ms / args.steps,
        "single_query_call_us": single_us,
        "hbm_fraction_of_step": bytes_per_launch / (ms_per_step / 1000.0) / 1e9 / HBM_PEAK_GBS,
        "gen_seconds": t_gen,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(codes, scales, queries, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    cands.close()
    one.close()
    rt.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
