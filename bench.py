#!/usr/bin/env python3
"""Batched search throughput on one MI355X.

A step is one batched search (rotation, probe, candidate generation, one-bit
refinement, chunked full-bit selection, full-bit MaxSim, top-k) of Q queries
whose inputs are already in HBM, replayed as one captured HIP graph.

The corpus is generated on the device (Gaussian mixture on the unit sphere,
Philox-seeded), the index is built on the device, and recall@100 is measured
against exact MaxSim computed on the device. Prints one JSON line with
queries/s, the roofline of the dominant kernel (per-stage HIP events on the
search stream), the CPU oracle's throughput on a bounded sample, doc-tokens
scored/s and recall@100.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "queries/sec (Q=1024 batch) + doc-tokens scored/s, % of HBM roofline, recall@100"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

_E2E = dict(len_kind="lognormal", len_lo=8, len_hi=300, len_median=64.0, len_sigma=0.5, centres=16384,
            sigma=0.15, n_clusters=1 << 20, ex_bits=4, nprobe=128, k_refine=3000, k_full_bit=300, num_chunks=5,
            k=100, nq=1024)
_SWEEP = dict(num_docs=1_000_000, len_kind="uniform", len_lo=16, len_hi=160, centres=2048, sigma=0.15,
              n_clusters=524_288, nprobe=128, k_refine=3000, k_full_bit=300, num_chunks=5, k=100, nq=1024)
WORKLOADS = {
    # End-to-end batched search: 2,000,000 docs, clipped log-normal lengths
    # (median 64, sigma 0.5, [8, 300]) -> ~145M tokens of D=128 from a
    # 16,384-centre mixture (sigma 0.15); n_clusters 1,048,576, ex_bits 4;
    # 1,024 queries x 32 tokens; nprobe 128, k_refine 3000, k_full_bit 300.
    "docs2m-q1024": dict(num_docs=2_000_000, seed=5, **_E2E),
    # Residual-scoring sweep: 1,000,000 docs, lengths U[16,160] (~88M
    # tokens), 2,048-centre mixture, n_clusters 524,288, ex_bits 1/4/7.
    "docs1m-q1024-ex1": dict(ex_bits=1, seed=4, **_SWEEP),
    "docs1m-q1024-ex4": dict(ex_bits=4, seed=4, **_SWEEP),
    "docs1m-q1024-ex7": dict(ex_bits=7, seed=4, **_SWEEP),
    # Small index: 10,000 docs, lengths U[16,160], 2,048-centre mixture,
    # n_clusters 4,096, ex_bits 4; nprobe 32, k_refine 1000, k_full_bit 100.
    "docs10k-q1024": dict(num_docs=10_000, len_kind="uniform", len_lo=16, len_hi=160, centres=2048, sigma=0.15,
                          n_clusters=4096, ex_bits=4, nprobe=32, k_refine=1000, k_full_bit=100, num_chunks=5, k=100,
                          nq=1024, seed=1),
    # The same index and options with 64 queries per batch.
    "docs10k-q64": dict(num_docs=10_000, len_kind="uniform", len_lo=16, len_hi=160, centres=2048, sigma=0.15,
                        n_clusters=4096, ex_bits=4, nprobe=32, k_refine=1000, k_full_bit=100, num_chunks=5, k=100,
                        nq=64, seed=1),
}
DEFAULT_WORKLOAD = "docs2m-q1024"
# IVF centroid probe alone: 1,024 queries x 32 tokens = 32,768 unit-norm
# query vectors against a unit-norm Gaussian mixture of centroids (sigma
# 0.2), top-128 per vector; labels checked against the exact fp32 probe.
# MaxSim rescoring alone: 256 unit-norm Gaussian queries x 32 tokens, each
# with its own 300 candidate documents of U[16, 256] fp32 tokens from a
# 2,048-centre mixture (sigma 0.15); per-document MaxSim on the matrix cores,
# then the top 100 per query.
RESCORE_WORKLOADS = {
    "maxsim-q256-c300": dict(nq=256, cands=300, len_lo=16, len_hi=256, centres=2048, sigma=0.15, k=100, seed=2),
}
PROBE_WORKLOADS = {
    "probe-q1024-k65536": dict(n_clusters=65536, centres=2048, sigma=0.2, nprobe=128, nq=1024, seed=3),
    "probe-q1024-k1048576": dict(n_clusters=1 << 20, centres=16384, sigma=0.2, nprobe=128, nq=1024, seed=3),
}


# kernel behind each single-kernel stage (names as rocprofv3 reports them)
STAGE_KERNELS = {
    "probe_scan": "chimera::probe_mfma_kernel<1, 4>",
    "count": "chimera::cand_count_kernel",
    "emit": "chimera::cand_emit_staged_kernel",
    "reduce": "chimera::cand_reduce_kernel<8>",
    "refine": "chimera::refine_mfma_kernel",
    "fullbit": "chimera::fullbit_mfma_kernel",
}
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


def measured_traffic(workload: str, stage: str):
    """HBM bytes per launch of a stage's kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs (scaled by the copy-kernel calibration), or
    None when that kernel was not measured for this workload."""
    try:
        with open(TRAFFIC_FILE) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    entry = table.get(workload, {}).get(stage)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def percentile(sorted_ms, pct):
    """percentile_ms (apps/utils.cpp:186-197): linear interpolation."""
    if not sorted_ms:
        return 0.0
    pos = (min(max(pct, 0.0), 100.0) / 100.0) * (len(sorted_ms) - 1)
    lo, hi = int(np.floor(pos)), int(np.ceil(pos))
    w = pos - lo
    return sorted_ms[lo] * (1 - w) + sorted_ms[hi] * w


def topk_rows(scores: np.ndarray, k: int) -> np.ndarray:
    """Top-k column ids per row by score descending, ties to the lower id."""
    out = np.empty((scores.shape[0], k), np.int64)
    for r, row in enumerate(scores):
        kk = min(k, row.size)
        part = np.argpartition(-row, kk - 1)[:kk]
        thr = row[part].min()
        cand = np.nonzero(row >= thr)[0]
        order = np.lexsort((cand, -row[cand]))
        out[r] = cand[order[:kk]]
    return out


def cpu_info() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS) + sorted(PROBE_WORKLOADS) + sorted(RESCORE_WORKLOADS))
    ap.add_argument("--cpu-sample", type=int, default=16, help="queries timed on the CPU oracle (0 = skip)")
    ap.add_argument("--recall-sample", type=int, default=64, help="queries checked against exact MaxSim")
    ap.add_argument("--single-queries", type=int, default=256,
                    help="serial one-query searches timed after the batch, and the no-allocation entry point's "
                         "capacity and one-query time (0 = skip both)")
    ap.add_argument("--gemm-peak", action="store_true",
                    help="only time square 8192^3 matrix products in bf16, fp16 and fp32 through torch (the "
                         "vendor library's achievable matrix-core rate on this GPU, for comparison)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of MIB MiB (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (queries shard without "
              "communication, so N GPUs would each run this batch on a replica of the index)", file=sys.stderr)
        return 2

    if args.copy_calibration > 0:
        return copy_calibration(args.copy_calibration, args.steps)
    if args.gemm_peak:
        return gemm_peak(args.steps)

    import chimera_amd
    from chimera_amd import capi, synthetic

    if args.workload in PROBE_WORKLOADS:
        return probe_bench(args)
    if args.workload in RESCORE_WORKLOADS:
        return rescore_bench(args)
    wl = WORKLOADS[args.workload]
    nq, k, width = wl["nq"], wl["k"], 1 + wl["ex_bits"]
    ctx, corpus = build_workload(wl)
    queries, lens, ptrs, targets, d_emb, n_tok = (corpus[n] for n in ("queries", "lens", "ptrs", "targets",
                                                                        "d_emb", "n_tok"))

    d_q = ctx.to_device(queries)
    d_ids = ctx.empty((nq, k), np.int64)
    d_sc = ctx.empty((nq, k), np.float32)
    d_cnt = ctx.empty((nq,), np.int32)

    # units of algorithmic work for this batch (from one traced run)
    t0 = time.time()
    tr = ctx.search_trace(queries, k, cand_capacity=1)
    log(f"traced one batch in {time.time() - t0:.1f}s: mean |C| {tr['cand_count'].mean():.0f}, "
        f"max {tr['cand_count'].max()}")
    probe_cands = probe_candidate_stats(ctx, nq * 32)
    log(f"probe candidates per row: {probe_cands}")
    host_index = ctx.download() if args.cpu_sample > 0 else ctx.download(fields=("cluster_pos",))
    cpos = host_index["cluster_pos"].astype(np.int64)
    sizes = cpos[1:] - cpos[:-1]
    visits = int(sizes[tr["labels"].astype(np.int64)].sum())
    lens64 = lens.astype(np.int64)
    refined_tokens = int(sum(lens64[tr["refined_ids"][q, :tr["refined_count"][q]]].sum() for q in range(nq)))
    fullbit_tokens = int(sum(lens64[tr["fullbit_ids"][q, :tr["fullbit_count"][q]]].sum() for q in range(nq)))
    rows_q = nq * 32
    # stage -> (bound, algorithmic flops or bytes per batch, unit, peak); each
    # of these stages is one kernel launch per batch
    units = {
        "probe_scan": ("mfma", 2.0 * rows_q * wl["n_clusters"] * 128, "TFLOP/s", BF16_PEAK_TFLOPS),
        "count": ("hbm", 4.0 * visits, "GB/s", HBM_PEAK_GBS),
        "emit": ("hbm", 24.0 * visits, "GB/s", HBM_PEAK_GBS),
        "refine": ("hbm", 24.0 * refined_tokens, "GB/s", HBM_PEAK_GBS),
        "fullbit": ("hbm", (16.0 * width + 4.0) * fullbit_tokens, "GB/s", HBM_PEAK_GBS),
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
    step_ms = sorted(ctx.graph_time(1) for _ in range(50))
    ids_gpu = d_ids.numpy()
    log(f"{args.steps} steps: {ms_per_step:.3f} ms/step (events {event_ms / args.steps:.3f}), {qps:.0f} queries/s")

    # per-stage kernel times on the search stream
    ctx.set_profiling(True)
    prof_steps = max(1, min(args.steps, 3))
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
                "frac": round(achieved / peak, 5), "traffic": measured_traffic(args.workload, dominant),
                "kernel": STAGE_KERNELS.get(dominant, dominant), "stage": dominant,
                "avg_launch_ms": round(tot_ms / launches, 4), "units_per_launch": per_launch}
    stage_ms = {n: round(v[0] / prof_steps, 4) for n, v in stages.items()}
    stage_frac = {}
    for n, (b, amt, u, pk) in units.items():
        if stages[n][0] > 0:
            rate = amt * prof_steps / (stages[n][0] / 1000.0) / (1e12 if u == "TFLOP/s" else 1e9)
            stage_frac[n] = {"achieved": round(rate, 2), "unit": u, "frac": round(rate / pk, 4)}
    # the one-bit refine and the full-bit scoring also run on the matrix
    # cores: per doc token and query token, 128 products of each of the two
    # fp16 halves of the split query (16x16x32 fp16 instructions)
    for n, toks in (("refine", refined_tokens), ("fullbit", fullbit_tokens)):
        if n in stage_frac and stages[n][0] > 0:
            tf = 2.0 * 2.0 * 32 * 128 * toks * prof_steps / (stages[n][0] / 1000.0) / 1e12
            stage_frac[n]["matrix"] = {"fp16_tflops": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
    log(f"stage ms: {stage_ms}")

    single = None
    if args.single_queries > 0:
        single = single_query_latency(ctx, queries, k, args.single_queries, warmup=16)
        log(f"one query at a time: {single}")
    noalloc = None
    if args.single_queries > 0:
        noalloc = noalloc_capacity(ctx, d_q, nq, k, d_ids, d_sc, d_cnt)
        log(f"no-allocation entry point: {noalloc}")

    # what the matrix cores sustain with register operands (no memory
    # traffic) on this GPU now, per instruction type of the search: the
    # practical ceiling of the matrix-core stages under the power limit
    mc_loop = matrix_core_loop(ctx)
    log(f"matrix-core loops: {mc_loop}")
    if roofline["unit"] == "TFLOP/s" and mc_loop:
        lt = mc_loop["bf16_32x32x16"]["tflops"]
        roofline["matrix_core_loop_tflops"] = lt
        roofline["frac_of_matrix_core_loop"] = round(roofline["achieved"] / lt, 4)
    for n, kind in (("refine", "f16_16x16x32_bits"), ("fullbit", "f16_16x16x32")):
        if mc_loop and n in stage_frac and "matrix" in stage_frac[n]:
            m = stage_frac[n]["matrix"]
            m["matrix_core_loop_tflops"] = mc_loop[kind]["tflops"]
            m["frac_of_matrix_core_loop"] = round(m["fp16_tflops"] / mc_loop[kind]["tflops"], 4)

    # recall@100 of the GPU results against exact MaxSim (query subset)
    t0 = time.time()
    rs = min(args.recall_sample, nq)
    recall = None
    if rs > 0:
        d_ptrs = ctx.to_device(ptrs.astype(np.int32))
        gt_scores = ctx.exact_maxsim(d_emb, d_ptrs, queries[:rs])
        d_ptrs.free()
        gt = topk_rows(gt_scores, 100)
        recall = synthetic.recall_at_k(gt, ids_gpu[:rs], 100)
        log(f"recall@100 {recall:.4f} over {rs} queries (exact MaxSim in {time.time() - t0:.1f}s)")
    target_hit = float(np.mean([targets[q] in set(ids_gpu[q, :10].tolist()) for q in range(nq)]))
    d_emb.free()

    cpu = None
    if args.cpu_sample > 0:
        from oracle import oracle as orc

        oi = orc.Index(host_index)
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        # the reference's CPU stage: full-bit MaxSim of the batch's selected
        # documents (AVX-512 restatement), repeated to about 8 s of work
        fb_counts = tr["fullbit_count"].astype(np.int32)
        fb_docs = np.ascontiguousarray(tr["fullbit_ids"][:, :max(1, int(fb_counts.max()))])
        if orc.fullbit_baseline_available():
            reps, cpu_s, sc = 0, 0.0, None
            while reps == 0 or (cpu_s < 8.0 and reps < 20):
                t0 = time.perf_counter()
                sc = orc.fullbit_baseline(oi, tr["rotated"], tr["cbex"], fb_docs, fb_counts, threads)
                cpu_s += time.perf_counter() - t0
                reps += 1
            tok_s = fullbit_tokens * reps / cpu_s
            gpu_fb_ms = stage_ms.get("fullbit", 0.0)
            # scores: bit for bit the oracle's on a query sample, and the
            # GPU's matrix-core scores within their tolerance
            chk = min(4, nq)
            want = orc.full_bit_scores(oi, tr["rotated"][:chk], tr["cbex"][:chk], fb_docs[:chk])
            bit_equal = all(np.array_equal(sc[q, :fb_counts[q]].view(np.uint32), want[q, :fb_counts[q]].view(np.uint32))
                            for q in range(chk))
            rel = max(float(np.max(np.abs(sc[q, :fb_counts[q]] - tr["fullbit_scores"][q, :fb_counts[q]]) /
                                   np.maximum(np.abs(sc[q, :fb_counts[q]]), 1e-6))) for q in range(chk))
            cpu = {"value": round(tok_s, 1), "unit": "full-bit doc-tokens/s", "cores": threads, "kind": "port",
                   "sample": f"full-bit MaxSim of the {int(fb_counts.sum())} documents ({fullbit_tokens} doc tokens) "
                             f"the GPU selected for all {nq} queries of this batch, {reps}x, with the AVX-512 + "
                             f"OpenMP restatement of the reference's CPU stage on {cpu_info()}",
                   "seconds": round(cpu_s, 2), "gb_per_s": round((16.0 * width + 4.0) * tok_s / 1e9, 2),
                   "ms_per_query": round(cpu_s * 1000.0 / (reps * nq), 4),
                   "gpu_fullbit_doc_tokens_per_s": round(fullbit_tokens / (gpu_fb_ms / 1000.0), 1) if gpu_fb_ms else None,
                   "scores_bit_equal_to_oracle": bit_equal, "max_rel_diff_to_gpu": rel}
            log(f"CPU baseline: {tok_s:.3e} full-bit doc-tokens/s on {threads} threads ({reps} x {nq} queries)")
        else:
            cpu = {"value": None, "unit": "full-bit doc-tokens/s", "cores": threads, "kind": "port",
                   "sample": f"not run: {cpu_info()} has no AVX-512"}
        # the whole search in the scalar oracle on a bounded query sample
        s = min(args.cpu_sample, nq)
        t0 = time.perf_counter()
        rid, rsc, _ = orc.search_batch(oi, queries[:s], wl["nprobe"], wl["k_refine"], wl["k_full_bit"],
                                       wl["num_chunks"], k)
        pipe_s = time.perf_counter() - t0
        agree = float(np.mean([np.array_equal(rid[q], ids_gpu[q]) for q in range(s)]))
        # lists that differ only by documents whose scores agree within the
        # matrix-core scoring's tolerance (2e-5 against the oracle's for each
        # side, so 4e-5 between the two sorted score lists)
        ties = float(np.mean([np.array_equal(rid[q], ids_gpu[q]) or
                              bool(np.allclose(np.sort(rsc[q]), np.sort(tr["scores"][q]), rtol=4e-5, atol=1e-7))
                              for q in range(s)]))
        cpu["oracle_pipeline"] = {"queries_per_s": round(s / pipe_s, 3), "cores": threads,
                                  "sample": f"{s} queries through the whole search in the scalar oracle",
                                  "seconds": round(pipe_s, 2), "ids_equal_to_gpu": agree,
                                  "ids_equal_up_to_ties_in_tolerance": ties}
        log(f"CPU oracle: {s} queries in {pipe_s:.1f}s")

    scored = visits + refined_tokens + fullbit_tokens
    result = {
        "metric": METRIC, "value": round(qps, 2), "unit": "queries/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (generated on the device)",
        "config": {"workload": args.workload, "num_docs": wl["num_docs"], "tokens": n_tok,
                   "n_clusters": wl["n_clusters"], "ex_bits": wl["ex_bits"], "nprobe": wl["nprobe"],
                   "k_refine": wl["k_refine"], "k_full_bit": wl["k_full_bit"], "num_chunks": wl["num_chunks"],
                   "k": k, "batch": nq, "seed": wl["seed"], "graph": True},
        "roofline": roofline, "cpu_baseline": cpu,
        "doc_tokens_scored_per_s": round(scored * args.steps / wall_s, 1),
        "work_per_batch": {"visits": visits, "refined_tokens": refined_tokens, "fullbit_tokens": fullbit_tokens,
                           "mean_candidates_per_query": round(float(tr["cand_count"].mean()), 1)},
        "stage_ms": stage_ms, "stage_roofline": stage_frac,
        "batch_latency_ms": {"p50": round(percentile(step_ms, 50), 4), "p99": round(percentile(step_ms, 99), 4)},
        "per_query_latency_ms": single,
        "noalloc": noalloc,
        "recall_at_100": None if recall is None else round(recall, 4), "recall_sample": rs, "target_in_top10": round(target_hit, 4),
        "probe_candidates_per_row": probe_cands,
    }
    for a in (d_q, d_ids, d_sc, d_cnt):
        a.free()
    ctx.close()
    # the practical ceilings of this GPU, measured now in a child process
    vr = vendor_rates()
    if vr:
        if roofline["unit"] == "TFLOP/s":
            g = vr["gemm_8192"]["bf16"]["tflops"]
            roofline["vendor_gemm_bf16_tflops"] = g
            roofline["frac_of_vendor_gemm"] = round(roofline["achieved"] / g, 4)
        # HBM stages: counter traffic (committed rocprofv3 runs) over this
        # run's stage time, against the copy's read + write rate
        copy_gbs = vr["copy_2gib"]["read_plus_write_gbs"]
        for n, sf in stage_frac.items():
            tb = measured_traffic(args.workload, n)
            if sf["unit"] == "GB/s" and tb and stages[n][0] > 0:
                gbs = tb * stages[n][1] / (stages[n][0] / 1000.0) / 1e9
                sf["traffic_gbs"] = round(gbs, 1)
                sf["traffic_frac_of_copy"] = round(gbs / copy_gbs, 4)
        result["practical_ceilings"] = vr
    if mc_loop:
        result.setdefault("practical_ceilings", {})["matrix_core_loop"] = mc_loop
    print(json.dumps(result), flush=True)
    return 0


def matrix_core_loop(ctx) -> dict:
    """chimera_matrix_core_rate for the matrix-core instructions of the
    search (probe bf16 32x32x16, full-bit fp16 16x16x32, one-bit refine fp16
    16x16x32 with 0/1 code bits, fp32 probe 32x32x2) and the 0/1-bit loop
    with four independent VALU instructions per MFMA: TFLOP/s."""
    out = {}
    for kind in ("bf16_32x32x16", "f16_16x16x32", "f16_16x16x32_bits", "f32_32x32x2", "f16_16x16x32_bits_valu4"):
        ops = ctx.matrix_core_rate(kind, 20000 if kind != "f32_32x32x2" else 4000)
        out[kind] = {"tflops": round(ops / 1e12, 1)}
    return out


def build_workload(wl: dict):
    """A context holding the workload's index, built on the device from a
    corpus generated on the device (the host only draws lengths, centres and
    query picks), and the corpus: queries [nq, 32, 128] on the host, document
    lengths and offsets, query targets, the device embeddings and the token
    count."""
    import chimera_amd
    from chimera_amd import capi, synthetic

    nq = wl["nq"]
    chimera_amd.load_module()
    ctx = capi.Context(None, wl["nprobe"], wl["k_refine"], wl["k_full_bit"], wl["num_chunks"], max_batch=nq)
    t0 = time.time()
    rng = np.random.default_rng(wl["seed"])
    centres = synthetic.unit_centres(rng, wl["centres"], 128)
    lens = synthetic.doc_lengths(rng, wl["num_docs"], wl["len_kind"], wl["len_lo"], wl["len_hi"],
                                 wl.get("len_median", 64.0), wl.get("len_sigma", 0.5))
    ptrs = np.concatenate([[0], np.cumsum(lens, dtype=np.int64)])
    n_tok = int(ptrs[-1])
    d_centres = ctx.to_device(centres)
    d_emb = ctx.synth_tokens(d_centres, n_tok, wl["sigma"], seed=wl["seed"])
    d_centres.free()
    targets = rng.integers(0, lens.size, size=nq)
    picks = ptrs[targets][:, None] + (rng.random((nq, 32)) * lens[targets][:, None]).astype(np.int64)
    rows = ctx.gather_rows(d_emb, picks.reshape(-1)).reshape(nq, 32, 128)
    queries = rows + np.float32(0.1) * rng.standard_normal(rows.shape, dtype=np.float32)
    queries /= np.linalg.norm(queries, axis=2, keepdims=True)
    queries = np.ascontiguousarray(queries, np.float32)
    ctx.synchronize()
    log(f"generated {n_tok} tokens / {lens.size} docs and {nq} queries on the device in {time.time() - t0:.1f}s")

    t0 = time.time()
    ctx.build(d_emb, lens, wl["n_clusters"], wl["ex_bits"])
    log(f"built the index on the device in {time.time() - t0:.1f}s ({ctx.memory_usage() / 2**30:.1f} GiB)")
    return ctx, {"queries": queries, "lens": lens, "ptrs": ptrs, "targets": targets, "d_emb": d_emb,
                 "n_tok": n_tok}


def single_query_latency(ctx, queries: np.ndarray, k: int, n: int, warmup: int) -> dict:
    """Serial one-query searches through chimera_search (host query in, host
    ids out, one call after the other), the way the reference's search
    command times index.search (apps/search.cpp:96-106): per-call wall time,
    mean and percentiles with percentile_ms semantics (apps/utils.cpp:186-197),
    and the stage times of one eager query."""
    import ctypes as C

    from chimera_amd import capi

    L = capi.lib()
    nq = queries.shape[0]
    ids = np.full((1, k), -1, np.int64)
    sc = np.zeros((1, k), np.float32)
    cnt = np.zeros(1, np.int32)
    pi, ps, pc = (a.ctypes.data_as(C.c_void_p) for a in (ids, sc, cnt))
    qptr = [np.ascontiguousarray(queries[i:i + 1]) for i in range(min(nq, n + warmup))]

    def one(i):
        capi.check(L.chimera_search(ctx.handle, qptr[i % len(qptr)].ctypes.data_as(C.c_void_p), 1, k, pi, ps, pc))

    for i in range(warmup):
        one(i)
    lat = []
    for i in range(n):
        t0 = time.perf_counter()
        one(warmup + i)
        lat.append((time.perf_counter() - t0) * 1000.0)
    srt = sorted(lat)
    ctx.set_profiling(True)
    one(0)
    ctx.synchronize()
    stages = ctx.stage_times()
    ctx.set_profiling(False)
    return {"queries": n, "warmup": warmup, "mean_ms": round(float(np.mean(lat)), 4),
            "p50_ms": round(percentile(srt, 50), 4), "p90_ms": round(percentile(srt, 90), 4),
            "p99_ms": round(percentile(srt, 99), 4), "max_ms": round(srt[-1], 4),
            "stage_ms_one_query": {n_: round(v[0], 4) for n_, v in stages.items() if v[1] > 0}}


def noalloc_capacity(ctx, d_q, nq: int, k: int, d_ids, d_sc, d_cnt) -> dict:
    """The largest batch chimera_search_device_noalloc takes on this index
    (its capacity error names it when the whole batch does not fit the
    static workspace) and the time of one-query calls through it."""
    import re

    from chimera_amd import capi

    fit = nq
    try:
        ctx.search_device_noalloc(d_q, nq, k, d_ids, d_sc, d_cnt)
        ctx.synchronize()
    except capi.ChimeraError as e:
        m = re.search(r"at most (\d+) queries", str(e))
        if e.code != capi.ERR_CAPACITY or not m:
            raise
        fit = int(m.group(1))
    lat = []
    if fit >= 1:
        for i in range(40):
            t0 = time.perf_counter()
            ctx.search_device_noalloc(d_q, 1, k, d_ids, d_sc, d_cnt)
            ctx.synchronize()
            if i >= 8:
                lat.append((time.perf_counter() - t0) * 1000.0)
    return {"max_batch": fit, "static_workspace_mib": 64,
            "one_query_ms_p50": round(percentile(sorted(lat), 50), 4) if lat else None}


def probe_candidate_stats(ctx, nrows: int):
    """Centroids per query row that passed the matrix-core probe's filter in
    the last search (d' <= thr), the fraction of rows whose candidates
    overflowed and the fraction whose threshold estimate failed the rerank's
    check (both recomputed by the exact kernel); None when the matrix-core
    probe did not run."""
    try:
        c = ctx.probe_stats(nrows)
    except Exception:
        return None
    missed = c == 0xFFFFFFFE
    over = c == 0xFFFFFFFF
    ok = c[~(over | missed)].astype(np.float64)
    if ok.size == 0:
        return {"rows": nrows, "overflow_fraction": round(float(over.mean()), 6),
                "check_failed_fraction": round(float(missed.mean()), 6)}
    return {"rows": nrows, "mean": round(float(ok.mean()), 1), "p50": float(np.percentile(ok, 50)),
            "p99": float(np.percentile(ok, 99)), "max": int(ok.max()),
            "overflow_fraction": round(float(over.mean()), 6),
            "check_failed_fraction": round(float(missed.mean()), 6)}


def gemm_peak(steps: int) -> int:
    """Square 8192^3 products through torch (hipBLASLt) in bf16, fp16 and
    fp32: the rate the vendor's tuned GEMM sustains on this GPU, beside the
    nominal peaks the rooflines use. Runs in its own process (torch brings
    its own HIP runtime)."""
    import torch

    n, out = 8192, {}
    for name, dt, peak in (("bf16", torch.bfloat16, BF16_PEAK_TFLOPS), ("fp16", torch.float16, BF16_PEAK_TFLOPS),
                           ("fp32", torch.float32, FP32_PEAK_TFLOPS)):
        a = torch.randn(n, n, device="cuda:0", dtype=dt)
        b = torch.randn(n, n, device="cuda:0", dtype=dt)
        for _ in range(3):
            c = a @ b
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(max(1, steps)):
            c = a @ b
        torch.cuda.synchronize()
        s = (time.perf_counter() - t0) / max(1, steps)
        tf = 2.0 * n ** 3 / s / 1e12
        out[name] = {"ms": round(s * 1000.0, 4), "tflops": round(tf, 1), "nominal_peak": peak,
                     "frac_of_nominal": round(tf / peak, 4)}
        del a, b, c
    # a 2 GiB device-to-device copy: bytes read plus written per second
    src = torch.empty(2 << 30, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(max(1, steps)):
        dst.copy_(src)
    torch.cuda.synchronize()
    s = (time.perf_counter() - t0) / max(1, steps)
    copy = {"bytes": 2 << 30, "ms": round(s * 1000.0, 4), "read_plus_write_gbs": round(2.0 * (2 << 30) / s / 1e9, 1)}
    print(json.dumps({"gemm_8192": out, "copy_2gib": copy}))
    return 0


def vendor_rates():
    """bench.py --gemm-peak in a child process (torch loads its own HIP
    runtime, which cannot share this process with the library's): the rate
    of the vendor's tuned GEMM and of a device copy on this GPU, the
    practical ceilings beside the nominal peaks."""
    import subprocess

    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--gemm-peak", "--steps", "10"],
                           capture_output=True, text=True, timeout=300)
        for line in reversed(r.stdout.splitlines()):
            if line.startswith("{"):
                return json.loads(line)
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    return None


def copy_calibration(mib: int, steps: int) -> int:
    """Device-to-device copies of a known size: under rocprofv3 --pmc their
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) against mib * 1024 give the
    factor that turns those counters into bytes for the search kernels."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(max(1, steps)):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / max(1, steps)
    print(json.dumps({"copy_mib": mib, "steps": max(1, steps), "ms_per_copy": round(ms, 4),
                      "gb_s": round(2.0 * n / (ms / 1000.0) / 1e9, 1)}))
    return 0


def rescore_bench(args) -> int:
    """Times chimera_maxsim_rescore_device (MaxSim of each query's candidate
    documents on fp32 tokens, split into fp16 pairs on the matrix cores, then
    the top-k); scores of a query sample are compared with a float64 brute
    force."""
    from chimera_amd import capi, synthetic

    wl = RESCORE_WORKLOADS[args.workload]
    nq, cap, k = wl["nq"], wl["cands"], wl["k"]
    rng = np.random.default_rng(wl["seed"])
    centres = synthetic.unit_centres(rng, wl["centres"], 128)
    m = nq * cap
    lens = rng.integers(wl["len_lo"], wl["len_hi"] + 1, size=m).astype(np.int32)
    ptrs = np.concatenate([[0], np.cumsum(lens, dtype=np.int64)])
    n_tok = int(ptrs[-1])
    queries = rng.standard_normal((nq, 32, 128)).astype(np.float32)
    queries /= np.linalg.norm(queries, axis=2, keepdims=True)
    ids = np.arange(m, dtype=np.int32).reshape(nq, cap)  # query q's candidates are documents q*cap .. +cap-1
    ctx = capi.Context(None, 8, 100, 50, 5)
    d_c = ctx.to_device(centres)
    d_emb = ctx.synth_tokens(d_c, n_tok, wl["sigma"], seed=wl["seed"])
    d_c.free()
    d_ptrs = ctx.to_device(ptrs.astype(np.int32))
    d_q = ctx.to_device(queries)
    d_ids = ctx.to_device(ids)
    d_cnt = ctx.to_device(np.full(nq, cap, np.int32))
    d_sc = ctx.empty((nq, cap), np.float32)
    d_tid = ctx.empty((nq, k), np.int64)
    d_tsc = ctx.empty((nq, k), np.float32)
    d_tcnt = ctx.empty((nq,), np.int32)

    def step():
        ctx.maxsim_rescore_device(d_emb, d_ptrs, d_q, d_ids, d_cnt, k, d_sc, d_tid, d_tsc, d_tcnt)

    for _ in range(max(1, args.warmup)):
        step()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.synchronize()
    wall_s = time.perf_counter() - t0
    ctx.set_profiling(True)
    for _ in range(args.steps):
        step()
    ctx.synchronize()
    stages = ctx.stage_times()
    ctx.set_profiling(False)
    resc_ms = stages["rescore"][0] / max(1, stages["rescore"][1])
    topk_ms = stages["rescore_topk"][0] / max(1, stages["rescore_topk"][1])
    scores = d_sc.numpy()
    top_ids = d_tid.numpy()
    # float64 check on a query sample
    sample = min(nq, 8)
    rel, agree = 0.0, 0
    for q in range(sample):
        docs = ids[q]
        rows = ctx.gather_rows(d_emb, np.arange(ptrs[docs[0]], ptrs[docs[-1] + 1]))
        base = ptrs[docs[0]]
        qq = queries[q].astype(np.float64)
        want = np.array([(qq @ rows[ptrs[d] - base:ptrs[d + 1] - base].astype(np.float64).T).max(1).sum()
                         for d in docs])
        rel = max(rel, float(np.max(np.abs(scores[q] - want) / np.abs(want))))
        order = np.lexsort((-docs.astype(np.int64), -want))[:k]  # score desc, larger id first
        agree += int(np.array_equal(docs[order], top_ids[q]))
    for a in (d_emb, d_ptrs, d_q, d_ids, d_cnt, d_sc, d_tid, d_tsc, d_tcnt):
        a.free()
    ctx.close()
    ms = wall_s * 1000.0 / args.steps
    bytes_per_call = 512.0 * n_tok
    flops_per_call = 8192.0 * n_tok
    gbs = bytes_per_call / (resc_ms / 1000.0) / 1e9
    tfl = flops_per_call / (resc_ms / 1000.0) / 1e12
    result = {
        "metric": "MaxSim rescoring doc-tokens/s (fp32 tokens, top-100)", "value": round(n_tok / (ms / 1000.0), 1),
        "unit": "doc-tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": args.workload, "queries": nq, "candidates_per_query": cap, "doc_tokens": n_tok,
                   "k": k},
        "queries_per_s": round(nq / (ms / 1000.0), 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "chimera::maxsim_rescore_kernel", "avg_launch_ms": round(resc_ms, 4),
                     "units_per_launch": bytes_per_call},
        # the fp32 products run on the fp16 matrix cores as three split
        # products (hi*hi, hi*lo, lo*hi)
        "matrix": {"algorithmic_tflops": round(tfl, 2), "fp16_mfma_tflops": round(3.0 * tfl, 2),
                   "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(3.0 * tfl / BF16_PEAK_TFLOPS, 4)},
        "topk_ms": round(topk_ms, 4),
        "check": {"queries": sample, "max_rel_err_vs_f64": rel, "topk_equal_to_f64": agree / sample},
    }
    print(json.dumps(result), flush=True)
    return 0


def probe_bench(args) -> int:
    """Times chimera_probe_device (matrix-core probe) on one batch of query
    vectors; labels of a row sample are compared with the exact fp32 probe."""
    import ctypes as C

    from chimera_amd import capi, synthetic

    wl = PROBE_WORKLOADS[args.workload]
    k, nprobe, rows = wl["n_clusters"], wl["nprobe"], wl["nq"] * 32
    rng = np.random.default_rng(wl["seed"])
    centres = synthetic.unit_centres(rng, wl["centres"], 128)
    tmp = capi.Context(None, nprobe, nprobe, 1, 1, max_batch=1)
    d_c = tmp.to_device(centres)
    d_cent = tmp.synth_tokens(d_c, k, wl["sigma"], seed=wl["seed"])
    d_rows = tmp.synth_tokens(d_c, rows, wl["sigma"], seed=wl["seed"] + 1)
    cent = d_cent.numpy()
    qrows = d_rows.numpy()
    for a in (d_c, d_cent, d_rows):
        a.free()
    tmp.close()
    index = {
        "num_embeddings": k, "dimension": 128, "num_clusters": k, "ex_bits": 1,
        "flips": np.zeros(64, np.uint8), "doc_lens": np.array([k], np.int32),
        "doc_ptrs": np.array([0, k], np.int32), "cluster_pos": np.arange(k + 1, dtype=np.uint64),
        "clustered_codes": np.zeros(k * 16, np.uint8), "clustered_factors": np.ones(k, np.float32),
        "clustered_doc_ids": np.zeros(k, np.int32), "token_to_cluster_pos": np.arange(k, dtype=np.uint32),
        "full_bit_codes": np.zeros(k * 32, np.uint8), "full_bit_factors": np.ones(k, np.float32),
        "rotated_centroids": cent,
    }
    ctx = capi.Context(index, nprobe, nprobe, 1, 1, max_batch=wl["nq"])
    ctx.set_probe_mode(2)
    d_q = ctx.to_device(qrows)
    d_lab = ctx.empty((rows, nprobe), np.uint32)
    L = capi.lib()

    def probe():
        capi.check(L.chimera_probe_device(ctx.handle, capi.P(d_q.ptr), rows, nprobe, capi.P(d_lab.ptr)))

    for _ in range(max(1, args.warmup)):
        probe()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        probe()
    ctx.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    got = d_lab.numpy()
    cands = probe_candidate_stats(ctx, rows)
    ctx.set_profiling(True)
    for _ in range(args.steps):
        probe()
    ctx.synchronize()
    st = ctx.stage_times()
    ctx.set_profiling(False)
    parts = {n: round(st[n][0] / max(1, st[n][1]), 4) for n in ("probe_sample", "probe_scan", "probe_rerank")}
    # the same probe with the filter on fp32 operands (v_mfma_f32_32x32x2_f32)
    ctx.set_probe_mode(3)
    for _ in range(max(1, args.warmup)):
        probe()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        probe()
    ctx.synchronize()
    ms32 = (time.perf_counter() - t0) * 1000.0 / args.steps
    got32 = d_lab.numpy()
    cands32 = probe_candidate_stats(ctx, rows)
    ctx.set_profiling(True)
    for _ in range(args.steps):
        probe()
    ctx.synchronize()
    st32 = ctx.stage_times()
    ctx.set_profiling(False)
    parts32 = {n: round(st32[n][0] / max(1, st32[n][1]), 4) for n in ("probe_sample", "probe_scan", "probe_rerank")}
    # exact fp32 probe on a sample of rows
    sample = min(rows, 2048)
    ctx.set_probe_mode(1)
    d_s = ctx.to_device(qrows[:sample])
    d_sl = ctx.empty((sample, nprobe), np.uint32)
    capi.check(L.chimera_probe_device(ctx.handle, capi.P(d_s.ptr), sample, nprobe, capi.P(d_sl.ptr)))
    ctx.synchronize()
    exact = d_sl.numpy()
    same = float(np.mean(np.all(exact == got[:sample], axis=1)))
    same32 = float(np.mean(np.all(exact == got32[:sample], axis=1)))
    tflops = 2.0 * rows * k * 128 / (ms / 1000.0) / 1e12
    tflops32 = 2.0 * rows * k * 128 / (ms32 / 1000.0) / 1e12
    scan32 = 2.0 * rows * k * 128 / (parts32["probe_scan"] / 1000.0) / 1e12 if parts32["probe_scan"] > 0 else None
    result = {
        "metric": "IVF probe TFLOP/s (bf16 matrix-core filter + exact fp32 rerank)", "value": round(tflops, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": args.workload, "rows": rows, "n_clusters": k, "nprobe": nprobe},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None},
        "labels_equal_to_exact_fp32": same, "exact_sample_rows": sample, "probe_candidates_per_row": cands,
        "part_ms": parts, "filtered_pass_tflops": round(2.0 * rows * k * 128 / (parts["probe_scan"] / 1000.0) / 1e12, 1)
        if parts["probe_scan"] > 0 else None,
        # the fp32 matrix-core leg: the same labels from a filter on fp32
        # operands, against the 157.3 TFLOP/s fp32 matrix peak
        "fp32_matrix": {"ms_per_call": round(ms32, 4), "tflops": round(tflops32, 2), "peak": FP32_PEAK_TFLOPS,
                        "frac": round(tflops32 / FP32_PEAK_TFLOPS, 4), "part_ms": parts32,
                        "filtered_pass_tflops": round(scan32, 2) if scan32 else None,
                        "filtered_pass_frac": round(scan32 / FP32_PEAK_TFLOPS, 4) if scan32 else None,
                        "labels_equal_to_exact_fp32": same32, "probe_candidates_per_row": cands32},
    }
    print(json.dumps(result), flush=True)
    for a in (d_q, d_lab, d_s, d_sl):
        a.free()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
