#!/usr/bin/env python3
"""Benchmark of the retrieval hot path on one MI355X, every BASELINE config.

Headline (BASELINE.json configs[0] shape): q8 packed-candidate dot + top-10,
N = 65,536 candidates x D = 256 per query, one query per candidate set, with
BASELINE's quantized-query dot formula.  A step scores `--sets` independent
(query, candidate set) problems in one fused launch -- the reference's batched
score layout [Q,D] x [Q,N,D] (runtime/backend/tensor_ops.go:1511-1519) --
over distinct candidate copies whose total (32 x 17 MB) exceeds the 256 MB
MALL, so the candidates stream from HBM.  Inputs are resident in HBM before
timing.  The default run adds configs 1-4 under "configs": C1 the f16 embed,
C2 q4 cosine and C3 q8 l2 with the reference's own arithmetic (cosineRows /
l2DistanceRows, bit for bit), C4 the q8-projection embed then BASELINE's
quantized-query q8 dot.

Prints one JSON line.  Each `roofline` is measured live with HIP events around
every launch of the dominant kernel; each `cpu_baseline` times the CPU
oracle's restatement of the reference host path (f32-backed values, the
reference's score loops, full-sort topKTensor; one thread) on a bounded
sample of the same work, and `fair_cpu` the same work's quantized-query
scores on packed data with heap top-k on all host cores.
"""
from __future__ import annotations

import argparse
import math
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

N, D, K = 65536, 256, 10
# the per-config lines time at least this long (more steps than --steps when
# a step is short); the C0 headline times exactly --steps
MIN_TIMED_S = 0.02


def c0_bytes_per_problem(n=N, d=D, k=K) -> int:
    # candidates (int8 codes + f32 scale) + f16 query + k (id, score) pairs
    return n * (d + 4) + 2 * d + k * 8


def host_info() -> dict:
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "threads_used_fair": _fair_threads()}


def _fair_threads() -> int:
    # the GPU box grants 16 host cores to a one-GPU job
    return max(1, min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", "16") or 16)))


def _budget_loop(budget_s, fn, max_iter=10**6):
    done = 0
    t0 = time.perf_counter()
    while True:
        fn(done)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= max_iter:
            return done, el


def cpu_baseline(codes, scales, queries, budget_s: float) -> dict:
    """C0 reference host path, restated by the CPU oracle (1 thread): the q8
    tensor's f32-backed values, f32 dotRows, full-sort topKTensor."""
    from oracle import oracle as orc

    sets = codes.shape[0]
    docs = [orc.dequant_q8(codes[s], scales[s]) for s in range(min(sets, 2))]
    qf = orc.f16_to_f32(queries)

    def one(i):
        s = i % len(docs)
        orc.topk(orc.dot_rows(qf[s], docs[s]), K)

    done, el = _budget_loop(budget_s, one, 4000)
    return {
        "value": done * N / el,
        "unit": "candidates/s",
        "cores": 1,
        "kind": "port",
        "sample": "%d C0 problems (1 query x %d x %d), reference host path restated in C "
                  "(f32 dotRows + full-sort topKTensor), %.1f s" % (done, N, D, el),
    }


def fair_c0(codes, scales, queries, budget_s: float) -> dict:
    from oracle import oracle as orc

    nt = _fair_threads()
    done, el = _budget_loop(budget_s, lambda i: orc.fair_q8_topk("dot", queries[i % 2:i % 2 + 1], codes[i % 2],
                                                                  scales[i % 2], K, threads=nt), 20000)
    return {"value": done * N / el, "unit": "candidates/s", "cores": nt, "kind": "fair",
            "sample": "%d C0 problems, BASELINE's q8 dot on the int8 data, heap top-k, %d threads, %.1f s"
                      % (done, nt, el)}


def _ref_cpu(unit, per_item, budget_s, fn, label, total):
    """Time `fn(i)` (one item of the reference host path) for about budget_s
    and report the rate scaled to the config's unit."""
    done, el = _budget_loop(budget_s, fn, total)
    return {"value": done * per_item / el, "unit": unit, "cores": 1, "kind": "port",
            "sample": "%d of %d %s, %.1f s; reference host path restated in C, one thread" % (done, total, label, el)}
def profiled_traffic(name: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch (or per step) measured by rocprofv3 PMC
    (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated) and recorded in the
    committed profile summary."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        for line in open(path):
            if line.startswith(key + ":"):
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


HBM_PEAK = 8000.0          # GB/s
F16_PEAK = 2517.0          # dense f16 MFMA TFLOP/s
I8_PEAK = 5033.0           # dense i8 MFMA TOP/s
F32_PEAK = 157.3           # dense f32 MFMA TFLOP/s


def _timed(rt, fn, steps, warmup, families, min_warm_s=0.5, min_timed_s=0.0):
    """Run fn warmup times, then time exactly `steps` calls with no per-launch
    instrumentation: seconds per step on the host clock (synchronized on both
    sides) and device ms per step from two HIP events on the runtime's stream
    around the whole run.  Then run `steps` more calls with HIP events around
    every launch for the per-kernel breakdown: (launches per step, ms per
    launch, ms per step) of each family.  (Each event pair adds a few
    microseconds to a launch, which is why the timed run has none.)  The
    warmup runs at least
    min_warm_s seconds: the part's clocks take a few hundred milliseconds of
    load to settle, and steps timed before that read up to 15% slower.
    With min_timed_s > 0 the timed run takes at least that long (more steps
    than `steps` when a step is short), so the synchronize around it does
    not weigh on the per-step time; the count timed comes back last."""
    t_w = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - t_w < min_warm_s:
        fn()
        done += 1
        if done >= warmup:
            rt.synchronize()
    rt.synchronize()
    est = (time.perf_counter() - t_w) / max(done, 1)  # per step, synchronizes included (an upper bound)
    nt = steps
    if min_timed_s > 0.0 and est * steps < min_timed_s:
        nt = int(math.ceil(min_timed_s / est))
    t0 = time.perf_counter()
    rt.span(False)
    for _ in range(nt):
        fn()
    span_ms = rt.span(True)
    rt.synchronize()
    el = time.perf_counter() - t0
    rt.set_timing(True)
    rt.timing(reset=True)
    for _ in range(steps):
        fn()
    rt.synchronize()
    fam = {}
    for f in families:
        n, ms = rt.timing(f)
        # (launches per step, average ms per launch, total ms per step)
        fam[f] = (n / steps, ms / max(n, 1), ms / steps)
    rt.set_timing(False)
    rt.timing(reset=True)
    return el / nt, fam, span_ms / nt, nt


def _kernels(fam) -> dict:
    """Device time per step of each kernel family that ran."""
    return {f: {"launches_per_step": v[0], "us_per_step": v[2] * 1000.0} for f, v in fam.items() if v[0]}


def run_c1(rt, steps, warmup, cpu_s) -> dict:
    """Config 1: embed pipeline, f16, B=64, T=128, V=32000, D=E=384."""
    from manta_amd import synth

    tokens, mask, table, proj = synth.config1()
    b, t = tokens.shape
    d, e = proj.shape
    td, md, tbd, pd = (rt.to_device(x) for x in (tokens, mask, table, proj))
    out = rt.empty((b, e), np.uint16)
    step_s, fam, dev_ms, nt = _timed(rt, lambda: rt.embed_pooled(td, md, tbd, pd, out=out), steps, warmup,
                                     ["embed", "embed_transpose", "embed_finalize"], min_timed_s=MIN_TIMED_S)
    flops = 2.0 * b * t * d * e
    # one launch per step: the uninstrumented run's device time per step
    # bounds the kernel's (it adds only the gap between back-to-back
    # launches), while an event pair around a launch this short adds a tenth
    k_ms = fam["embed"][1]
    if fam["embed"][0] == 1.0 and not fam["embed_transpose"][0] and not fam["embed_finalize"][0]:
        k_ms = min(dev_ms, k_ms)
    achieved = flops / (k_ms / 1000.0) / 1e12
    return {
        "workload": "c1_embed_f16", "shape": {"b": b, "t": t, "vocab": table.shape[0], "d": d, "e": e},
        "value": b * t / step_s, "unit": "tokens/s", "ms_per_step": step_s * 1000.0, "timed_steps": nt,
        "device_ms_per_step": dev_ms,
        "roofline": {"bound": "mfma", "kernel": "embed_gemm7_kernel (f16 MFMA 32x32x16; 128 rows x 96 columns per "
                                                "workgroup, one round of loads: table rows gathered straight to "
                                                "registers, projection slice direct to LDS and read as stored through "
                                                "transpose reads; finalize fused)",
                     "achieved": achieved, "peak": F16_PEAK, "unit": "TFLOP/s", "frac": achieved / F16_PEAK,
                     "avg_launch_us": k_ms * 1000.0, "event_timed_launch_us": fam["embed"][1] * 1000.0,
                     "flops_per_launch": flops,
                     "bytes_per_launch": b * t * (4 + 4 + d * 2) + d * e * 2 + b * e * 2,
                     "traffic": profiled_traffic("embed_gemm7_c1_embed_f16.md"),
                     "traffic_source": "profiles/embed_gemm7_c1_embed_f16.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
                     "note": "flops counted over all B*T positions (masked ones included), as the reference computes them"},
        "finalize_us": fam["embed_finalize"][1] * 1000.0,
        "transpose_us": fam["embed_transpose"][1] * 1000.0,
        **c1_cpu(tokens, mask, table, proj, cpu_s),
    }


def c1_cpu(tokens, mask, table, proj, cpu_s) -> dict:
    if cpu_s <= 0:
        return {"cpu_baseline": None, "fair_cpu": None}
    from oracle import oracle as orc

    b, t = tokens.shape
    nt = _fair_threads()

    def one(i):
        j = (i * 4) % b
        orc.embed(tokens[j:j + 4], mask[j:j + 4], table, proj_f16=proj)

    cpu = _ref_cpu("tokens/s", 4 * t, cpu_s, one,
                   "batches of 4 sequences (gather, f32 sequential matmul, masked mean_pool, normalize)", b // 4)
    done, el = _budget_loop(cpu_s / 2, lambda i: orc.fair_embed(tokens, mask, table, proj_f16=proj, threads=nt), 200)
    fair = {"value": done * b * t / el, "unit": "tokens/s", "cores": nt, "kind": "fair",
            "sample": "%d full C1 batches, f32 embed pipeline over %d threads, %.1f s" % (done, nt, el)}
    return {"cpu_baseline": cpu, "fair_cpu": fair}


def run_c2(rt, steps, warmup, cpu_s) -> dict:
    """Config 2: batched q4 cosine + top-100, Q=256, N=1,048,576, D=384, with
    the reference's cosineRows on the dequantized candidates."""
    from manta_amd import synth

    queries, packed, scales = synth.config2()
    nq, d = queries.shape
    n = packed.shape[0]
    k = 100
    cands = rt.bind_q4(packed, scales, d)
    qd = rt.to_device(queries)
    ids = rt.empty((nq, k), np.int32)
    sc = rt.empty((nq, k), np.float32)
    fams = ["mq_scan", "mq_select", "q4_scan", "topk_merge", "query_encode", "ref_rescore", "ref_finish", "ref_scan"]
    step_s, fam, dev_ms, nt = _timed(rt, lambda: rt.score_topk(cands, "cosine", qd, k, out=(ids, sc, None)),
                                     steps, warmup, fams, min_timed_s=MIN_TIMED_S)
    # the presets' step after top-k: candidate ids, packed rows and scales of
    # the selected rows
    cid = rt.to_device(np.arange(n, dtype=np.int64) * 7 + 3)
    pack_s, pfam, _, _ = _timed(rt, lambda: rt.pack_candidates(cands, ids, cid), steps, warmup, ["pack_candidates"],
                                min_warm_s=0.1, min_timed_s=MIN_TIMED_S)
    pack_bytes = nq * k * (4 + 8 + d // 2 + d // 16 + 8 + d // 2 + d // 16)  # reads + writes
    dom = "mq_scan" if fam["mq_scan"][0] else "q4_scan"
    # the scan reads the q4 matrix's int8 shadow: 384 code bytes and one f32
    # scale per row (built once, on the first call)
    spitch = (d + 127) // 128 * 128
    nbytes = n * (spitch + 4)
    achieved = nbytes / (fam[dom][2] / 1000.0) / 1e9
    ops = 2.0 * nq * n * d
    cands.close()
    return {
        "workload": "c2_q4_cosine_top100", "shape": {"q": nq, "n": n, "d": d, "k": k},
        "semantics": "reference cosineRows on the dequantized q4 values (ids and scores bit-exact)",
        "value": nq * n / step_s, "unit": "candidates/s", "ms_per_step": step_s * 1000.0, "timed_steps": nt,
        "device_ms_per_step": dev_ms, "kernels": _kernels(fam),
        # The contraction is Q x N x D against f16 queries: priced at the f16
        # MFMA peak (the exact two-int8-digit split would execute twice the
        # ops at twice the rate, the same time).  The shadow scan runs it as
        # one int8 digit on each side, so its executed i8 ops are reported
        # against the i8 peak beside it, and its bytes against HBM.
        "roofline": {"bound": "mfma", "kernel": dom + " (mq8_scan_kernel on the int8 shadow)",
                     "achieved": ops / (fam[dom][2] / 1000.0) / 1e12, "peak": F16_PEAK, "unit": "TFLOP/s",
                     "frac": ops / (fam[dom][2] / 1000.0) / 1e12 / F16_PEAK,
                     "step_frac": ops / (dev_ms / 1000.0) / 1e12 / F16_PEAK,
                     "scan_us_per_step": fam[dom][2] * 1000.0, "ops_per_step": ops,
                     "executed_i8_frac": ops / (fam[dom][2] / 1000.0) / 1e12 / I8_PEAK,
                     "hbm_GB_s": achieved, "hbm_frac": achieved / HBM_PEAK, "shadow_bytes_per_step": nbytes,
                     "traffic": profiled_traffic("mq8_shadow_c2_q4_cosine_top100.md", "traffic_bytes_per_step"),
                     "traffic_source": "profiles/mq8_shadow_c2_q4_cosine_top100.md (rocprofv3 --pmc FETCH_SIZE, "
                                       "WRITE_SIZE; all scan passes of a step)",
                     "note": "all threshold passes of the scan together cover the N rows once; survivors are "
                             "rescored with the exact 16-bit-query q4 score in mq_select, and the best "
                             "k + k/16 with the reference arithmetic in ref_finish; step_frac prices the whole "
                             "step (scan, select, finish, encoding)"},
        "pack_candidates": {"us_per_call": pfam["pack_candidates"][1] * 1000.0, "rows": nq * k,
                            "bytes_per_call": pack_bytes,
                            "GB_s": pack_bytes / (pfam["pack_candidates"][1] / 1000.0) / 1e9},
        **c2_cpu(queries, packed, scales, k, cpu_s),
    }


def c2_cpu(queries, packed, scales, k, cpu_s) -> dict:
    if cpu_s <= 0:
        return {"cpu_baseline": None, "fair_cpu": None}
    from oracle import oracle as orc

    nq, d = queries.shape
    n = packed.shape[0]
    nt = _fair_threads()

    def one(i):
        orc.topk(orc.ref_score_q4("cosine", queries[i:i + 1], packed, scales, d), k)

    cpu = _ref_cpu("candidates/s", n, cpu_s, one, "queries (cosineRows over the dequantized q4 rows + "
                   "full-sort topKTensor)", nq)
    done, el = _budget_loop(cpu_s / 2, lambda i: orc.fair_q4_topk("cosine", queries[(8 * i) % nq:(8 * i) % nq + 8],
                                                                   packed, scales, d, k, threads=nt), nq // 8)
    fair = {"value": done * 8 * n / el, "unit": "candidates/s", "cores": nt, "kind": "fair",
            "sample": "%d batches of 8 queries, 16-bit-query q4 cosine on the nibbles, heap top-k, %d threads, "
                      "%.1f s" % (done, nt, el)}
    return {"cpu_baseline": cpu, "fair_cpu": fair}


def run_c3(rt, steps, warmup, cpu_s) -> dict:
    """Config 3: q8 l2_distance rerank, smallest-1000, Q=32, N=8,388,608,
    D=128, with the reference's l2DistanceRows on the dequantized rows."""
    from manta_amd import synth

    queries, codes, scales = synth.config3()
    nq, d = queries.shape
    n = codes.shape[0]
    k = 1000
    cands = rt.bind_q8(codes, scales)
    qd = rt.to_device(queries)
    ids = rt.empty((nq, k), np.int32)
    sc = rt.empty((nq, k), np.float32)
    fams = ["mq_scan", "mq_select", "q8_scan", "topk_merge", "query_encode", "ref_rescore", "ref_finish", "ref_scan"]
    step_s, fam, dev_ms, nt = _timed(rt, lambda: rt.score_topk(cands, "l2_distance", qd, k, smallest=True,
                                                               out=(ids, sc, None)), steps, warmup, fams,
                                     min_timed_s=MIN_TIMED_S)
    dom = "mq_scan" if fam["mq_scan"][0] else "q8_scan"
    nbytes = n * (d + 4) + nq * d * 2 + nq * k * 8
    achieved = nbytes / (fam[dom][2] / 1000.0) / 1e9
    cands.close()
    return {
        "workload": "c3_q8_l2_smallest1000", "shape": {"q": nq, "n": n, "d": d, "k": k},
        "semantics": "reference l2DistanceRows on the dequantized q8 values (ids and scores bit-exact)",
        "value": nq * n / step_s, "unit": "candidates/s", "ms_per_step": step_s * 1000.0, "timed_steps": nt,
        "device_ms_per_step": dev_ms, "kernels": _kernels(fam),
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK, "scan_us_per_step": fam[dom][2] * 1000.0,
                     "bytes_per_step": nbytes,
                     "traffic": profiled_traffic("mq_scan_c3_l2_smallest1000.md", "traffic_bytes_per_step"),
                     "traffic_source": "profiles/mq_scan_c3_l2_smallest1000.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
                     "step_frac": nbytes / (dev_ms / 1000.0) / 1e9 / HBM_PEAK,
                     "note": "all threshold passes of the scan together cover the N rows once; step_frac "
                             "prices the whole step (scan, select, finish)"},
        **c3_cpu(queries, codes, scales, k, cpu_s),
    }


def c3_cpu(queries, codes, scales, k, cpu_s) -> dict:
    if cpu_s <= 0:
        return {"cpu_baseline": None, "fair_cpu": None}
    from oracle import oracle as orc

    nq, d = queries.shape
    n = codes.shape[0]
    nt = _fair_threads()

    def one(i):
        orc.topk(orc.ref_score_q8("l2_distance", queries[i:i + 1], codes, scales), k, smallest=True)

    cpu = _ref_cpu("candidates/s", n, cpu_s, one, "queries (l2DistanceRows over the dequantized q8 rows + "
                   "full-sort smallest-k)", nq)
    done, el = _budget_loop(cpu_s / 2, lambda i: orc.fair_q8_topk("l2_distance", queries[(4 * i) % nq:(4 * i) % nq + 4],
                                                                   codes, scales, k, smallest=True, threads=nt), nq // 4)
    fair = {"value": done * 4 * n / el, "unit": "candidates/s", "cores": nt, "kind": "fair",
            "sample": "%d batches of 4 queries, 16-bit-query q8 l2 on the int8 rows, heap top-k, %d threads, "
                      "%.1f s" % (done, nt, el)}
    return {"cpu_baseline": cpu, "fair_cpu": fair}


def run_c4(rt, steps, warmup, cpu_s) -> dict:
    """Config 4: embed 1024x64 tokens with a q8 projection, then q8 dot
    top-50 of the 1024 embedded queries over 4,194,304 x 384 candidates, with
    BASELINE's quantized-query dot formula."""
    from manta_amd import synth

    tokens, mask, table, pcodes, cs, codes, scales = synth.config4()
    b, t = tokens.shape
    d = table.shape[1]
    e = pcodes.shape[1]
    n = codes.shape[0]
    k = 50
    cands = rt.bind_q8(codes, scales)
    td, md, tbd, pd, csd = (rt.to_device(x) for x in (tokens, mask, table, pcodes, cs))
    # the projection is a bound weight: put in the MFMA layout once
    pp = rt.prepare_projection(pd)
    emb = rt.empty((b, e), np.uint16)
    ids = rt.empty((b, k), np.int32)
    sc = rt.empty((b, k), np.float32)

    def step():
        rt.embed_pooled(td, md, tbd, pp, csd, out=emb)
        rt.score_topk(cands, "dot", emb, k, out=(ids, sc, None), quantized=True)

    fams = ["embed", "embed_transpose", "embed_finalize", "mq_scan", "mq_select", "q8_scan", "topk_merge", "query_encode"]
    step_s, fam, dev_ms, nt = _timed(rt, step, steps, warmup, fams, min_timed_s=MIN_TIMED_S)
    flops_a = 2.0 * b * t * d * e
    ops_b = 2.0 * b * n * d
    emb_t = flops_a / (fam["embed"][1] / 1000.0) / 1e12
    dom = "mq_scan" if fam["mq_scan"][0] else "q8_scan"
    sc_t = ops_b / (fam[dom][2] / 1000.0) / 1e12
    cands.close()
    return {
        "workload": "c4_embed_q8proj_then_q8dot_top50", "shape": {"q": b, "t": t, "d": d, "n": n, "k": k},
        "semantics": "BASELINE's q8 dot formula (query codes round(q*127), int32 accumulation)",
        "value": b * n / step_s, "unit": "candidates/s (end to end, embed included)",
        "ms_per_step": step_s * 1000.0, "timed_steps": nt, "device_ms_per_step": dev_ms, "kernels": _kernels(fam),
        "embed": {"tokens_per_s_kernel": b * t / (fam["embed"][1] / 1000.0),
                  "roofline": {"bound": "mfma", "achieved": emb_t, "peak": F16_PEAK, "unit": "TFLOP/s",
                               "frac": emb_t / F16_PEAK, "avg_launch_us": fam["embed"][1] * 1000.0}},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": sc_t, "peak": I8_PEAK, "unit": "TOP/s",
                     "frac": sc_t / I8_PEAK, "scan_us_per_step": fam[dom][2] * 1000.0, "ops_per_step": ops_b,
                     "bytes_per_step": n * (d + 4) + b * d * 2 + b * k * 8,
                     "traffic": profiled_traffic("mq8_scan_c4_dot_top50.md", "traffic_bytes_per_step"),
                     "traffic_source": "profiles/mq8_scan_c4_dot_top50.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; "
                                       "all scan passes of a step)",
                     "note": "all threshold passes of the scan together cover the N rows once"},
        **c4_cpu(tokens, mask, table, pcodes, cs, codes, scales, k, cpu_s),
    }


def c4_cpu(tokens, mask, table, pcodes, cs, codes, scales, k, cpu_s) -> dict:
    if cpu_s <= 0:
        return {"cpu_baseline": None, "fair_cpu": None}
    from oracle import oracle as orc

    b, t = tokens.shape
    n = codes.shape[0]
    nt = _fair_threads()

    def one(i):
        # one query end to end: its sequence's embedding, dotRows over the
        # dequantized rows, full-sort top-k
        j = i % b
        q16, _ = orc.embed(tokens[j:j + 1], mask[j:j + 1], table, proj_codes=pcodes, col_scale=cs)
        qf = orc.f16_to_f32(q16)[0]
        orc.topk(orc.ref_score_q8("dot", q16, codes, scales)[0], k)
        del qf

    cpu = _ref_cpu("candidates/s", n, cpu_s, one, "queries end to end (embed of one sequence, dotRows over the "
                   "dequantized q8 rows, full-sort topKTensor)", b)

    def fair_one(i):
        q = orc.fair_embed(tokens[(16 * i) % b:(16 * i) % b + 16], mask[(16 * i) % b:(16 * i) % b + 16], table,
                           proj_codes=pcodes, col_scale=cs, threads=nt)
        orc.fair_q8_topk("dot", orc.f32_to_f16(q), codes, scales, k, threads=nt)

    done, el = _budget_loop(cpu_s / 2, fair_one, b // 16)
    fair = {"value": done * 16 * n / el, "unit": "candidates/s", "cores": nt, "kind": "fair",
            "sample": "%d batches of 16 queries end to end (f32 embed, BASELINE's q8 dot on the int8 rows, heap "
                      "top-k), %d threads, %.1f s" % (done, nt, el)}
    return {"cpu_baseline": cpu, "fair_cpu": fair}


def run_enc(rt, steps, warmup, cpu_s) -> dict:
    """The encoder forward of examples/encoder_trainable_q8.manta
    (embed_pooled_batch) at C4's embed shape: 1024 sequences of 64 tokens,
    vocabulary 32000, d = 384, ffn width h = 1536; random q8 weights."""
    rng = np.random.default_rng(5)
    b, t, vocab, d, h = 1024, 64, 32000, 384, 1536
    tokens = rng.integers(0, vocab, size=(b, t), dtype=np.int32)
    mask = np.ones((b, t), np.int32)
    tcodes = rng.integers(-127, 128, size=(vocab, d), dtype=np.int8)
    tscales = np.full(vocab, 0.5 / 127.0, np.float32)
    dev = []
    for k, n in [(d, d), (d, d), (d, d), (d, d), (d, h), (h, d)]:
        dev.append((rt.to_device(rng.integers(-127, 128, size=(k, n), dtype=np.int8)),
                    rt.to_device(np.full(n, 1.0 / (127.0 * np.sqrt(k)), np.float32))))
    td, md, tcd, tsd = (rt.to_device(x) for x in (tokens, mask, tcodes, tscales))
    out = rt.empty((b, d), np.uint16)
    fams = ["encoder_gather", "encoder_gemm", "encoder_attention", "encoder_softmax", "encoder_layernorm",
            "normalize", "mean_pool", "encoder_out", "embed_transpose"]
    step_s, fam, dev_ms, nt = _timed(rt, lambda: rt.encoder_pooled(td, md, tcd, tsd, dev, out=out), steps, warmup,
                                     fams, min_timed_s=MIN_TIMED_S)
    r = b * t
    gemm_flops = 2.0 * r * d * d * 4 + 2.0 * r * d * h * 2
    attn_flops = 2.0 * 2.0 * b * t * t * d
    gemm_us = fam["encoder_gemm"][2] * 1000.0
    return {
        "workload": "enc_encoder_trainable_q8_pooled", "shape": {"b": b, "t": t, "vocab": vocab, "d": d, "h": h},
        "value": r / step_s, "unit": "tokens/s", "ms_per_step": step_s * 1000.0, "timed_steps": nt, "device_ms_per_step": dev_ms,
        "kernels": _kernels(fam),
        "roofline": {"bound": "mfma", "kernel": "embed_gemm2_kernel (f16 MFMA 32x32x16, 256x128 tiles; q/k/v/o, "
                                                "ffn_up with gelu and an f16 output, projection; q8 weights widened "
                                                "exactly, column scales after the f32 accumulation)",
                     "achieved": gemm_flops / (gemm_us * 1e-6) / 1e12, "peak": F16_PEAK, "unit": "TFLOP/s",
                     "frac": gemm_flops / (gemm_us * 1e-6) / 1e12 / F16_PEAK, "gemm_us_per_step": gemm_us,
                     "flops_per_step": gemm_flops, "attention_flops_per_step": attn_flops,
                     "weight_prep_us_per_step": fam["embed_transpose"][2] * 1000.0,
                     "note": "left operands rounded to f16 by the steps that produce them, f32 accumulation; "
                             "the attention products, softmax and layernorms stay f32"},
    }


def run_c0(rt, args) -> dict:
    from manta_amd import synth

    t_gen = time.perf_counter()
    queries, codes, scales = synth.config0(sets=args.sets)
    t_gen = time.perf_counter() - t_gen
    cands = rt.bind_q8(codes, scales)
    q_dev = rt.to_device(queries)
    ids = rt.empty((args.sets, K), np.int32)
    sc = rt.empty((args.sets, K), np.float32)
    # the headline: exactly W untimed warmup steps, then K timed ones
    step_s, fam, dev_ms, _ = _timed(rt, lambda: rt.score_topk(cands, "dot", q_dev, K, out=(ids, sc, None),
                                                              quantized=True),
                                    args.steps, args.warmup, ["q8_scan"], min_warm_s=0.0)
    # one fused launch per step: the uninstrumented run's device time per
    # step (two HIP events around the K timed steps) bounds the kernel's
    # duration; the per-launch event figure is the other bound
    scan_avg_s = fam["q8_scan"][1] / 1000.0
    if fam["q8_scan"][0] == 1.0:
        scan_avg_s = min(scan_avg_s, dev_ms / 1000.0)
    bytes_per_launch = args.sets * c0_bytes_per_problem()
    achieved = bytes_per_launch / scan_avg_s / 1e9

    # single-query latency (one problem per call, back to back)
    q1 = rt.to_device(queries[:1])
    one = rt.bind_q8(codes[0], scales[0])
    ids1 = rt.empty((1, K), np.int32)
    single_s, _, _, _ = _timed(rt, lambda: rt.score_topk(one, "dot", q1, K, out=(ids1, None, None), quantized=True),
                               200, 5, [])
    line = {
        "metric": "candidates scored/sec (q8 dot + top-k, BASELINE config 0 shape)",
        "value": args.sets * N / step_s,
        "unit": "candidates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1000.0,
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
            "semantics": "BASELINE config 0's q8 dot formula (query codes round(q*127), int32 accumulation)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "q8_scan (manta::q8_scan_kernel<0,16,1>, fused top-k incl. merge)",
            "achieved": achieved,
            "peak": HBM_PEAK,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK,
            "traffic": profiled_traffic("q8_scan_c0_batched.md") if args.sets == 32 else None,
            "traffic_source": "profiles/q8_scan_c0_batched.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
            "avg_launch_us": scan_avg_s * 1e6,
            "event_timed_launch_us": fam["q8_scan"][1] * 1000.0,
            "bytes_per_launch": bytes_per_launch,
        },
        "device_ms_per_step": dev_ms,
        "single_query_call_us": single_s * 1e6,
        "hbm_fraction_of_step": bytes_per_launch / step_s / 1e9 / HBM_PEAK,
        "gen_seconds": t_gen,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(codes, scales, queries, args.cpu_seconds)
        line["fair_cpu"] = fair_c0(codes, scales, queries, args.cpu_seconds / 2)
    else:
        line["cpu_baseline"] = None
        line["fair_cpu"] = None
    line["host"] = host_info()
    cands.close()
    one.close()
    return line


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sets", type=int, default=32, help="C0 problems per step")
    ap.add_argument("--workload", default="all", choices=["c0", "c1", "c2", "c3", "c4", "enc", "all", "full"],
                    help="c0 is the headline line; the others are added under 'configs' (all: c1-c4; "
                         "full: c1-c4 and the encoder)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB (PMC scaling run)")
    args = ap.parse_args()
    if args.copy_calibration_mb:
        return copy_calibration(args.copy_calibration_mb)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (candidate rows "
              "would shard across GPUs, each returning its own top-k for a KB-scale merge). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    from manta_amd import rocm

    rt = rocm.Runtime(0)
    extra = {"c1": run_c1, "c2": run_c2, "c3": run_c3, "c4": run_c4, "enc": run_enc}
    if args.workload == "all":
        todo = ["c1", "c2", "c3", "c4"]
    elif args.workload == "full":
        todo = list(extra)
    else:
        todo = [args.workload] if args.workload in extra else []
    heavy_steps = max(3, min(args.steps, 10))
    configs = {}
    for w in todo:
        print("bench: %s" % w, file=sys.stderr, flush=True)
        steps = args.steps if w == "c1" else heavy_steps
        cpu_s = 0.0 if args.no_cpu else args.cpu_seconds
        configs[w] = extra[w](rt, steps, min(args.warmup, 2) if w != "c1" else args.warmup, cpu_s)
    print("bench: c0", file=sys.stderr, flush=True)
    line = run_c0(rt, args)
    if configs:
        line["configs"] = configs
    rt.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
