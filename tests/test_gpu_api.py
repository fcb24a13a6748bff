"""GPU tests of the public surfaces: the pybind11 module (build / search /
save / load), device-pointer search, HIP graph replays, and recall at the
10k-document scale against brute-force exact MaxSim."""
import numpy as np
import pytest

from chimera_amd import capi, synthetic
from oracle import oracle as orc
from parity_checks import compare_query

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(small_index, small_workload):
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16)
    qs = small_workload.queries
    nq, k = qs.shape[0], 50
    ref_ids, ref_scores, ref_counts = ctx.search(qs, k)
    d_q = ctx.to_device(qs)
    d_ids = ctx.empty((nq, k), np.int64)
    d_sc = ctx.empty((nq, k), np.float32)
    d_cnt = ctx.empty((nq,), np.int32)
    ctx.graph_capture(d_q, nq, k, d_ids, d_sc, d_cnt)
    other = small_workload.queries[::-1].copy()
    for rep in range(4):
        ctx.graph_launch()
        ctx.synchronize()
        assert np.array_equal(d_ids.numpy(), ref_ids), f"replay {rep}"
        assert np.array_equal(d_sc.numpy(), ref_scores)
        assert np.array_equal(d_cnt.numpy(), ref_counts)
        # eager work on the same context between replays
        ids2, _, _ = ctx.search(other, 10)
        assert ids2.shape == (nq, 10)
    # device-pointer eager search equals the host entry point
    ctx.search_device(d_q, nq, k, d_ids, d_sc, d_cnt)
    ctx.synchronize()
    assert np.array_equal(d_ids.numpy(), ref_ids)
    for a in (d_q, d_ids, d_sc, d_cnt):
        a.free()
    ctx.close()


def test_pybind_build_search_save_load(tmp_path, chimera_mod, tiny_workload):
    w = tiny_workload
    idx = chimera_mod.ChimeraIndex.build(w.embeddings, w.doc_lens.tolist(), n_clusters=48, ex_bits=4, nprobe=8,
                                         k_refine=60, k_full_bit=20, num_chunks=3)
    single = idx.search(w.queries[0], k=10)
    batch = idx.search(w.queries, k=10)
    assert isinstance(single, list) and all(isinstance(x, int) for x in single)
    assert batch[0] == single
    idx.save(str(tmp_path / "ix"))
    idx2 = chimera_mod.ChimeraIndex.load(str(tmp_path / "ix"), nprobe=8, k_refine=60, k_full_bit=20, num_chunks=3)
    assert idx2.search(w.queries, k=10) == batch
    # same results as the oracle on the same index files
    oi = orc.Index(chimera_mod._read_index(str(tmp_path / "ix")))
    rid, rsc, rcnt = orc.search_batch(oi, w.queries, 8, 60, 20, 3, 10)
    for q in range(w.queries.shape[0]):
        assert batch[q] == rid[q, :rcnt[q]].tolist()
    with pytest.raises(ValueError):
        idx.search(w.queries[0][:, :64].copy(), k=10)
    with pytest.raises(ValueError):
        idx.search(w.queries[0], k=0)
    with pytest.raises(ValueError):
        chimera_mod.ChimeraIndex.load(str(tmp_path / "ix"), nprobe=49)


def test_config1_scale_recall():
    """10k documents, n_clusters 4096, ex_bits 4, nprobe 32, k_refine 1000,
    k_full_bit 100 (the small synthetic configuration), 32 queries: every
    query's trace against the oracle stage by stage (matrix-core scoring), the
    results equal to the trace's, and recall@100 against exact MaxSim within
    0.5 points of the oracle's."""
    import chimera_amd

    mod = chimera_amd.load_module()
    w = synthetic.generate(num_docs=10000, num_centres=2048, sigma=0.15, nq=32, seed=1)
    index = mod._build_index(w.embeddings, w.doc_lens.tolist(), 4096, 4)
    ctx = capi.Context(index, 32, 1000, 100, 5, max_batch=32)
    ids, scores, counts = ctx.search(w.queries, 100)
    t = ctx.search_trace(w.queries, 100)
    ctx.close()
    assert np.array_equal(t["ids"], ids)
    oi = orc.Index(index)
    for q in range(w.queries.shape[0]):
        compare_query(t, q, orc.search(oi, w.queries[q], 32, 1000, 100, 5, 100), False, oi, 100, 5)
    rid, rsc, rcnt = orc.search_batch(oi, w.queries, 32, 1000, 100, 5, 100)
    gt, _ = synthetic.exact_maxsim_topk(w.embeddings, w.doc_lens, w.queries, 100)
    r_gpu = synthetic.recall_at_k(gt, ids, 100)
    r_orc = synthetic.recall_at_k(gt, rid, 100)
    assert abs(r_gpu - r_orc) <= 0.005
    assert np.mean(ids[:, 0] == w.targets) >= 0.9


def test_search_command_end_to_end(tmp_path, chimera_mod, tiny_workload):
    """chimera_search on a saved index: the report lines of the reference's
    gpu_search, recall@10 = 1 against ground truth equal to the library's
    own results, and the batched line."""
    import re
    import struct
    import subprocess

    from chimera_amd import PKG_DIR

    w = tiny_workload
    idx = chimera_mod.ChimeraIndex.build(w.embeddings, w.doc_lens.tolist(), n_clusters=48, ex_bits=4, nprobe=8,
                                         k_refine=60, k_full_bit=20, num_chunks=3)
    idx.save(str(tmp_path / "ix"))
    res = idx.search(w.queries, k=10)
    nq = w.queries.shape[0]
    (tmp_path / "q.bin").write_bytes(struct.pack("<iii", nq, 32, 128) + w.queries.astype(np.float32).tobytes())
    (tmp_path / "gt.tsv").write_text("".join(f"{q}\t{d}\t{r + 1}\n" for q in range(nq) for r, d in enumerate(res[q])))
    print("chimera_search: tiny workload, 4 queries, k 10", flush=True)
    out = subprocess.run([str(PKG_DIR / "chimera_search"), "--query", str(tmp_path / "q.bin"), "--gt",
                          str(tmp_path / "gt.tsv"), "--index", str(tmp_path / "ix"), "--k", "10", "--warmup", "2",
                          "--nprobe", "8", "--k-refine", "60", "--k-full-bit", "20", "--num-chunks", "3"],
                         capture_output=True, text=True, timeout=110)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    lat = re.fullmatch(r"\[SEARCH\] latency_ms mean=(\S+) min=(\S+) p50=(\S+) p90=(\S+) p95=(\S+) p99=(\S+) "
                       r"max=(\S+) stddev=(\S+)", lines[0])
    assert lat, lines[0]
    v = [float(x) for x in lat.groups()]
    assert 0 < v[1] <= v[2] <= v[3] <= v[4] <= v[5] <= v[6]
    assert lines[1] == "[SEARCH] recall@10=1.000"
    assert re.fullmatch(r"\[SEARCH\] batch queries=4 ms=\S+ qps=\S+", lines[2]), lines[2]
