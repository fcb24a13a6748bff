#!/usr/bin/env python3
"""Batched search throughput on one MI355X.

A step is one batched search (rotation, probe, candidate generation, one-bit
refinement, chunked full-bit selection, full-bit MaxSim, top-k) of Q queries
whose inputs are already in HBM, replayed as one captured HIP graph.

Prints one JSON line with queries/s, the roofline of the dominant kernel
(per-stage HIP events on the search stream), the oracle's CPU throughput on a
bounded sample, doc-tokens scored/s and recall@100 against exact MaxSim.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "queries/sec (Q=1024 batch) + doc-tokens scored/s, % of HBM roofline, recall@100"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3

WORKLOADS = {
    # 10,000 docs, doclens U[16,160], 2,048-centre mixture sigma 0.15,
    # n_clusters 4,096, ex_bits 4; nprobe 32, k_refine 1000, k_full_bit 100;
    # a batch of 1,024 queries (32 tokens, sigma 0.1 around random targets).
    "docs10k-q1024": dict(num_docs=10000, len_kind="uniform", len_lo=16, len_hi=160, centres=2048, sigma=0.15,
                          n_clusters=4096, ex_bits=4, nprobe=32, k_refine=1000, k_full_bit=100, num_chunks=5,
                          k=100, nq=1024, seed=1),
}
DEFAULT_WORKLOAD = "docs10k-q1024"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def percentile(sorted_ms, pct):
    """percentile_ms (apps/utils.cpp:186-197): linear interpolation."""
    if not sorted_ms:
        return 0.0
    pos = (min(max(pct, 0.0), 100.0) / 100.0) * (len(sorted_ms) - 1)
    lo, hi = int(np.floor(pos)), int(np.ceil(pos))
    w = pos - lo
    return sorted_ms[lo] * (1 - w) + sorted_ms[hi] * w


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-sample", type=int, default=32, help="queries timed on the CPU oracle (0 = skip)")
    ap.add_argument("--recall-sample", type=int, default=128, help="queries checked against exact MaxSim")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (queries shard without "
              "communication; see the multi-GPU note of the design document)", file=sys.stderr)
        return 2

    import chimera_amd
    from chimera_amd import capi, synthetic

    wl = WORKLOADS[args.workload]
    t0 = time.time()
    w = synthetic.generate(num_docs=wl["num_docs"], num_centres=wl["centres"], sigma=wl["sigma"], nq=wl["nq"],
                           seed=wl["seed"], len_kind=wl["len_kind"], len_lo=wl["len_lo"], len_hi=wl["len_hi"])
    log(f"generated {w.embeddings.shape[0]} tokens / {w.doc_lens.size} docs in {time.time() - t0:.1f}s")
    mod = chimera_amd.load_module()
    t0 = time.time()
    index = mod._build_index(w.embeddings, w.doc_lens.tolist(), wl["n_clusters"], wl["ex_bits"])
    log(f"built index in {time.time() - t0:.1f}s")

    nq, k = wl["nq"], wl["k"]
    ctx = capi.Context(index, wl["nprobe"], wl["k_refine"], wl["k_full_bit"], wl["num_chunks"], max_batch=nq)
    d_q = ctx.to_device(w.queries)
    d_ids = ctx.empty((nq, k), np.int64)
    d_sc = ctx.empty((nq, k), np.float32)
    d_cnt = ctx.empty((nq,), np.int32)

    # units of algorithmic work for this batch (from one traced run)
    tr = ctx.search_trace(w.queries, k, cand_capacity=1)
    cpos = index["cluster_pos"].astype(np.int64)
    sizes = cpos[1:] - cpos[:-1]
    visits = int(sizes[tr["labels"].astype(np.int64)].sum())
    lens = w.doc_lens.astype(np.int64)
    refined_tokens = int(sum(lens[tr["refined_ids"][q, :tr["refined_count"][q]]].sum() for q in range(nq)))
    fullbit_tokens = int(sum(lens[tr["fullbit_ids"][q, :tr["fullbit_count"][q]]].sum() for q in range(nq)))
    width = 1 + wl["ex_bits"]
    rows = nq * 32
    units = {
        "probe": ("mfma", 2.0 * rows * wl["n_clusters"] * 128, "TFLOP/s", FP32_PEAK_TFLOPS),
        "mark": ("hbm", 4.0 * visits, "GB/s", HBM_PEAK_GBS),
        "partial": ("hbm", 24.0 * visits, "GB/s", HBM_PEAK_GBS),
        "refine": ("hbm", 24.0 * refined_tokens, "GB/s", HBM_PEAK_GBS),
        "fullbit_topk": ("hbm", (16.0 * width + 4.0) * fullbit_tokens, "GB/s", HBM_PEAK_GBS),
    }

    # warm-up, capture, timed replays
    for _ in range(max(1, args.warmup)):
        ctx.search_device(d_q, nq, k, d_ids, d_sc, d_cnt)
    ctx.synchronize()
    ctx.graph_capture(d_q, nq, k, d_ids, d_sc, d_cnt)
    for _ in range(args.warmup):
        ctx.graph_launch()
    ctx.synchronize()
    t_start = time.perf_counter()
    event_ms = ctx.graph_time(args.steps)
    ctx.synchronize()
    wall_s = time.perf_counter() - t_start
    ms_per_step = wall_s * 1000.0 / args.steps
    qps = nq * args.steps / wall_s
    step_ms = sorted(ctx.graph_time(1) for _ in range(min(args.steps, 20)))
    ids_gpu = d_ids.numpy()
    log(f"{args.steps} steps: {ms_per_step:.3f} ms/step (events {event_ms / args.steps:.3f}), {qps:.0f} queries/s")

    # per-stage kernel times on the search stream
    ctx.set_profiling(True)
    prof_steps = max(1, min(args.steps, 5))
    for _ in range(prof_steps):
        ctx.search_device(d_q, nq, k, d_ids, d_sc, d_cnt)
    ctx.synchronize()
    stages = ctx.stage_times()
    ctx.set_profiling(False)
    dominant = max((n for n in stages if n in units), key=lambda n: stages[n][0])
    bound, amount, unit, peak = units[dominant]
    tot_ms, launches = stages[dominant]
    avg_s = tot_ms / launches / 1000.0
    per_launch = amount * prof_steps / launches
    achieved = per_launch / avg_s / (1e12 if unit == "TFLOP/s" else 1e9)
    roofline = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 5), "traffic": None, "kernel": dominant,
                "avg_launch_ms": round(tot_ms / launches, 4),
                "units_per_launch": per_launch}
    stage_ms = {n: round(v[0] / max(1, prof_steps), 4) for n, v in stages.items()}

    # recall@100 of the GPU results against exact MaxSim (query subset)
    rs = min(args.recall_sample, nq)
    gt, _ = synthetic.exact_maxsim_topk(w.embeddings, w.doc_lens, w.queries[:rs], 100)
    recall = synthetic.recall_at_k(gt, ids_gpu[:rs], 100)

    cpu = None
    if args.cpu_sample > 0:
        from oracle import oracle as orc

        oi = orc.Index(index)
        s = min(args.cpu_sample, nq)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        t0 = time.perf_counter()
        rid, _, _ = orc.search_batch(oi, w.queries[:s], wl["nprobe"], wl["k_refine"], wl["k_full_bit"],
                                     wl["num_chunks"], k)
        cpu_s = time.perf_counter() - t0
        agree = float(np.mean([np.array_equal(rid[q], ids_gpu[q]) for q in range(s)]))
        cpu = {"value": round(s / cpu_s, 3), "unit": "queries/s", "cores": threads, "kind": "port",
               "sample": f"{s} queries of this workload through the full scalar oracle (OpenMP over queries)",
               "seconds": round(cpu_s, 2), "ids_equal_to_gpu": agree}
        ref = orc.ref_lib()
        if ref is not None:
            import ctypes as C

            tok = 0
            t0 = time.perf_counter()
            for q in range(s):
                fc = int(tr["fullbit_count"][q])
                docs = np.ascontiguousarray(tr["fullbit_ids"][q, :fc])
                out = np.zeros(fc, np.float32)
                rot = np.ascontiguousarray(tr["rotated"][q])
                cbex = np.ascontiguousarray(tr["cbex"][q])
                ref.ref_full_bit_scores(rot.ctypes.data_as(C.c_void_p), cbex.ctypes.data_as(C.c_void_p),
                                        index["doc_ptrs"].ctypes.data_as(C.c_void_p),
                                        index["full_bit_codes"].ctypes.data_as(C.c_void_p),
                                        index["full_bit_factors"].ctypes.data_as(C.c_void_p), wl["ex_bits"],
                                        docs.ctypes.data_as(C.c_void_p), fc, out.ctypes.data_as(C.c_void_p))
                tok += int(lens[docs].sum())
            ref_s = time.perf_counter() - t0
            cpu["reference_fullbit_stage"] = {
                "doc_tokens_per_s": round(tok / ref_s, 1), "cores": threads, "kind": "reference",
                "sample": f"full-bit MaxSim of the same {s} queries' selected documents with the reference's "
                          "AVX-512 unpack + gemv_batch8 kernels (compute_full_bit_scores loop)"}

    scored = visits + refined_tokens + fullbit_tokens
    result = {
        "metric": METRIC, "value": round(qps, 2), "unit": "queries/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": args.workload, "num_docs": wl["num_docs"], "tokens": int(w.embeddings.shape[0]),
                   "n_clusters": wl["n_clusters"], "ex_bits": wl["ex_bits"], "nprobe": wl["nprobe"],
                   "k_refine": wl["k_refine"], "k_full_bit": wl["k_full_bit"], "num_chunks": wl["num_chunks"],
                   "k": k, "batch": nq, "seed": wl["seed"], "graph": True},
        "roofline": roofline, "cpu_baseline": cpu,
        "doc_tokens_scored_per_s": round(scored * args.steps / wall_s, 1),
        "work_per_batch": {"visits": visits, "refined_tokens": refined_tokens, "fullbit_tokens": fullbit_tokens},
        "stage_ms": stage_ms,
        "batch_latency_ms": {"p50": round(percentile(step_ms, 50), 4), "p99": round(percentile(step_ms, 99), 4)},
        "recall_at_100": round(recall, 4), "recall_sample": rs,
    }
    print(json.dumps(result), flush=True)
    for a in (d_q, d_ids, d_sc, d_cnt):
        a.free()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
