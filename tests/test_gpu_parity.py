"""HIP path against the oracle, stage by stage, through the C ABI.

Bars: integer results (rotated-query bits, probe labels, candidate lists,
code unpacking) bit-exact; S_cand bit-exact (the reference's shuffle-down
tree over the 32 clamped per-token maxima, whatever the order of the visit
records), hence the refined list identical; rotation, QueryState and, in
exact-scoring mode, S1, SF and the final ranking bit-exact. In the default
(matrix-core) scoring mode S1 and SF are within 2e-5 relative/absolute of
the reference arithmetic, the full-bit selection equals the reference's rule
applied to the GPU's S1, and the final ranking follows the GPU's SF exactly
and the reference arithmetic's SF up to swaps inside that tolerance. Every
query is checked in full: compare_query has no early exit."""
import numpy as np
import pytest

from chimera_amd import capi
from oracle import oracle as orc
from parity_checks import expected_shape, compare_query

pytestmark = pytest.mark.gpu

@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
@pytest.mark.parametrize("nprobe,k_refine,k_full_bit,num_chunks", [(32, 500, 100, 5), (8, 300, 300, 1),
                                                                   (64, 1000, 200, 3)])
def test_search_trace_matches_oracle(small_index, small_workload, nprobe, k_refine, k_full_bit, num_chunks, exact):
    ctx = capi.Context(small_index, nprobe, k_refine, k_full_bit, num_chunks, max_batch=16, exact=exact)
    qs = small_workload.queries[:6]
    t = ctx.search_trace(qs, k=100)
    oi = orc.Index(small_index)
    for q in range(qs.shape[0]):
        r = orc.search(oi, qs[q], nprobe, k_refine, k_full_bit, num_chunks, 100)
        compare_query(t, q, r, exact, oi, k_full_bit, num_chunks)
    ctx.close()


def test_search_matches_trace_and_oracle_batch(small_index, small_workload):
    """Exact-scoring mode: the batched search equals the oracle bit for bit
    on every query."""
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=True)
    ids, scores, counts = ctx.search(small_workload.queries, k=100)
    oi = orc.Index(small_index)
    rids, rscores, rcounts = orc.search_batch(oi, small_workload.queries, 32, 500, 100, 5, 100)
    assert np.array_equal(counts, rcounts)
    assert np.array_equal(ids, rids)
    assert np.array_equal(scores.view(np.uint32), rscores.view(np.uint32))
    ctx.close()


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_large_refined_lists(chimera_mod, exact):
    """k_refine 6,000 over 12,000 short documents: the selection sorts more
    than 4,096 keys and the full-bit selection 8,192 (the block sorts' widest
    register merge form) against the oracle."""
    from chimera_amd import synthetic

    w = synthetic.generate(num_docs=12000, num_centres=256, sigma=0.2, nq=4, seed=23, len_lo=4, len_hi=16)
    idx = chimera_mod._build_index(w.embeddings, w.doc_lens.tolist(), 1024, 4)
    nprobe, k_refine, k_full_bit, num_chunks = 64, 6000, 600, 5
    ctx = capi.Context(idx, nprobe, k_refine, k_full_bit, num_chunks, max_batch=4, exact=exact)
    t = ctx.search_trace(w.queries, k=100)
    ctx.close()
    oi = orc.Index(idx)
    for q in range(w.queries.shape[0]):
        assert int(t["refined_count"][q]) == k_refine
        r = orc.search(oi, w.queries[q], nprobe, k_refine, k_full_bit, num_chunks, 100)
        compare_query(t, q, r, exact, oi, k_full_bit, num_chunks)


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_search_is_deterministic(small_index, small_workload, exact):
    """Two runs of the same batch: every intermediate and result bit for bit
    equal (the candidate stage's visit records arrive in a different order
    each run)."""
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=exact)
    a = ctx.search_trace(small_workload.queries, k=50)
    b = ctx.search_trace(small_workload.queries, k=50)
    ctx.close()
    for key in a:
        assert np.array_equal(np.asarray(a[key]).view(np.uint8), np.asarray(b[key]).view(np.uint8)), key


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
@pytest.mark.parametrize("ex_bits", [1, 2, 3, 5, 6, 7])
def test_every_code_width(chimera_mod, tiny_workload, ex_bits, exact):
    w = tiny_workload
    idx = chimera_mod._build_index(w.embeddings, w.doc_lens.tolist(), 48, ex_bits)
    ctx = capi.Context(idx, 8, 60, 20, 3, max_batch=4, exact=exact)
    t = ctx.search_trace(w.queries, k=10)
    oi = orc.Index(idx)
    for q in range(w.queries.shape[0]):
        r = orc.search(oi, w.queries[q], 8, 60, 20, 3, 10)
        compare_query(t, q, r, exact, oi, 20, 3)
    ctx.close()


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_k_larger_than_results_and_edge_options(tiny_index, tiny_workload, exact):
    # k beyond the scored set, nprobe = n_clusters, one chunk per document
    ctx = capi.Context(tiny_index, 48, 120, 120, 120, max_batch=4, exact=exact)
    t = ctx.search_trace(tiny_workload.queries, k=500)
    oi = orc.Index(tiny_index)
    for q in range(tiny_workload.queries.shape[0]):
        r = orc.search(oi, tiny_workload.queries[q], 48, 120, 120, 120, 500)
        compare_query(t, q, r, exact, oi, 120, 120)
        assert (t["ids"][q, int(t["counts"][q]):] == -1).all()
    ctx.close()


def test_unpack_kernel_bit_exact(chimera_mod, small_index):
    ctx = capi.Context(small_index, 8, 100, 50, 5, max_batch=1)
    rng = np.random.default_rng(3)
    for w in range(1, 9):
        raw = rng.integers(0, 1 << w, size=(257, 128)).astype(np.uint8)
        raw[0] = (1 << w) - 1
        packed = chimera_mod._pack(raw, w)
        d_in = ctx.to_device(packed)
        d_out = ctx.empty((257, 128), np.uint8)
        capi.check(capi.lib().chimera_unpack_codes_device(ctx.handle, w, capi.P(d_in.ptr), capi.C.c_int64(257),
                                                          capi.P(d_out.ptr)))
        ctx.synchronize()
        assert np.array_equal(d_out.numpy(), raw)
        assert np.array_equal(orc.unpack(packed, w), raw)
        d_in.free()
        d_out.free()
    ctx.close()


def test_rotation_state_and_lut_bit_exact(small_index, small_workload):
    """chimera_rotate_lut_device against the oracle: rotated queries,
    QueryState sums and the one-bit LUT ([query][token][chunk][entry]),
    bit for bit (kernels.cu:402-428; rotator.hpp:281-334)."""
    ctx = capi.Context(small_index, 8, 100, 50, 5, max_batch=16)
    qs = np.ascontiguousarray(small_workload.queries, np.float32)
    nq = qs.shape[0]
    bufs = [ctx.to_device(qs), ctx.empty((nq, 32, 128), np.float32), ctx.empty((nq, 32), np.float32),
            ctx.empty((nq, 32), np.float32), ctx.empty((nq, 32, 32, 16), np.float32)]
    d_q, d_rot, d_cb1, d_cbex, d_lut = bufs
    capi.check(capi.lib().chimera_rotate_lut_device(ctx.handle, capi.P(d_q.ptr), nq, capi.P(d_rot.ptr),
                                                    capi.P(d_cb1.ptr), capi.P(d_cbex.ptr), capi.P(d_lut.ptr)))
    ctx.synchronize()
    rot, cb1, cbex, lut = (b.numpy() for b in bufs[1:])
    for b in bufs:
        b.free()
    ctx.close()
    oi = orc.Index(small_index)
    for q in range(nq):
        r = orc.search(oi, qs[q], 8, 100, 50, 5, 10)
        assert np.array_equal(rot[q].view(np.uint32), r["rotated"].view(np.uint32))
        assert np.array_equal(cb1[q].view(np.uint32), r["cb1"].view(np.uint32))
        assert np.array_equal(cbex[q].view(np.uint32), r["cbex"].view(np.uint32))
        assert np.array_equal(lut[q].view(np.uint32), r["lut"].view(np.uint32))
        assert np.array_equal(lut[q].view(np.uint32), orc.lut(rot[q]).view(np.uint32))


def test_probe_kernel_matches_brute_force(small_index, small_workload):
    ctx = capi.Context(small_index, 64, 100, 50, 5, max_batch=8)
    t = ctx.search_trace(small_workload.queries[:4], k=10)
    rot = t["rotated"].reshape(-1, 128)
    cent = small_index["rotated_centroids"].reshape(-1, 128)
    for nprobe in (1, 17, 64, 300, 1024):
        d_rot = ctx.to_device(rot)
        d_lab = ctx.empty((rot.shape[0], nprobe), np.uint32)
        capi.check(capi.lib().chimera_probe_device(ctx.handle, capi.P(d_rot.ptr), rot.shape[0], nprobe,
                                                   capi.P(d_lab.ptr)))
        ctx.synchronize()
        got = d_lab.numpy()
        d_rot.free()
        d_lab.free()
        assert np.array_equal(got, orc.probe(rot, cent, nprobe))
        # float64 brute force: same sets except exact-score ties at the boundary
        d64 = (cent.astype(np.float64) ** 2).sum(1)[None, :] - 2 * rot.astype(np.float64) @ cent.T.astype(np.float64)
        for i in range(rot.shape[0]):
            want = np.argsort(d64[i], kind="stable")[:nprobe]
            diff = set(want) ^ set(got[i].tolist())
            if diff:
                thr = d64[i][want[-1]]
                assert all(abs(d64[i][j] - thr) < 1e-5 for j in diff)
    ctx.close()


def _unit(v):
    return (v / np.linalg.norm(v, axis=-1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_repeated_tokens_take_the_exact_reduce(chimera_mod, exact):
    """Documents made of one token repeated 16-48 times: every visit of a
    probed document repeats its (doc, query token) key, thousands of
    duplicated keys per bucket, so the candidate reduce runs its exact
    per-token form. Candidate lists, S_cand and everything after them
    against the oracle."""
    from chimera_amd import synthetic

    rng = np.random.default_rng(21)
    centres = synthetic.unit_centres(rng, 24, 128)
    m = 400
    lens = rng.integers(16, 49, size=m).astype(np.int32)
    base = synthetic.mixture_tokens(rng, centres, m, 0.15)
    emb = np.repeat(base, lens, axis=0)
    q, _ = synthetic.make_queries(rng, emb, lens, 4)
    idx = chimera_mod._build_index(emb, lens.tolist(), 32, 4)
    ctx = capi.Context(idx, 8, 200, 50, 5, max_batch=4, exact=exact)
    t = ctx.search_trace(q, k=20)
    oi = orc.Index(idx)
    for i in range(q.shape[0]):
        r = orc.search(oi, q[i], 8, 200, 50, 5, 20)
        compare_query(t, i, r, exact, oi, 50, 5)
    ctx.close()


@pytest.mark.parametrize("n_clusters", [128, 2048])
@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_duplicate_documents_tie_in_doc_order(chimera_mod, exact, n_clusters):
    """5,000 copies of one two-token document among 1,000 others. The 32
    query tokens are one perturbed copy of the document's first token, so
    every copy's S_cand is a sum of 32 equal terms, an exact tie whatever the
    order of additions; more candidates than the selection's list reach its
    group threshold, and the exact selection must return the 100 lowest-id
    copies, as the reference's stable sort does. Every copy is visited by all
    32 query tokens, so a bucket of copies needs 32 slots per document and
    its reduce walks many slot chunks: 1,024-document buckets at 128
    clusters, 8,192 at 2,048 clusters, 8 records per thread in both."""
    from chimera_amd import synthetic

    rng = np.random.default_rng(22)
    centres = synthetic.unit_centres(rng, 64, 128)
    doc = synthetic.mixture_tokens(rng, centres[:2], 2, 0.05)
    others_lens = rng.integers(2, 9, size=1000).astype(np.int32)
    others = synthetic.mixture_tokens(rng, centres[8:], int(others_lens.sum()), 0.15)
    copies = 5000
    emb = np.concatenate([np.tile(doc, (copies, 1)), others]).astype(np.float32)
    lens = np.concatenate([np.full(copies, 2, np.int32), others_lens])
    nq = 3
    q = np.empty((nq, 32, 128), np.float32)
    for i in range(nq):
        q[i] = _unit(doc[0] + np.float32(0.05) * rng.standard_normal(128, dtype=np.float32))
    assert expected_shape(lens.size, int(lens.sum()), n_clusters, 4) == {128: (10, 8), 2048: (13, 8)}[n_clusters]
    idx = chimera_mod._build_index(emb, lens.tolist(), n_clusters, 4)
    ctx = capi.Context(idx, 4, 100, 20, 5, max_batch=4, exact=exact)
    t = ctx.search_trace(q, k=10)
    oi = orc.Index(idx)
    for i in range(nq):
        r = orc.search(oi, q[i], 4, 100, 20, 5, 10)
        assert int(t["cand_count"][i]) > 4096  # more than the selection's list holds
        s_top = float(r["cand_scores"][:copies].max())
        assert np.all(r["cand_scores"][:copies] == s_top)  # the copies tie exactly
        rc = int(t["refined_count"][i])
        assert np.array_equal(t["refined_ids"][i, :rc], r["refined_ids"])
        assert np.array_equal(r["refined_ids"], np.arange(100))  # lowest ids first
        compare_query(t, i, r, exact, oi, 20, 5)
    ctx.close()


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
@pytest.mark.parametrize("dim", [64, 96, 100])
def test_search_below_128_dimensions(chimera_mod, dim, exact):
    """Embeddings of d < 128 (zero-padded to 128 by the rotation): the whole
    search against the oracle, stage by stage."""
    from chimera_amd import synthetic

    w = synthetic.generate(num_docs=300, num_centres=48, sigma=0.15, nq=3, seed=30 + dim, dim=dim)
    idx = chimera_mod._build_index(w.embeddings, w.doc_lens.tolist(), 96, 4)
    ctx = capi.Context(idx, 16, 150, 40, 5, max_batch=4, exact=exact)
    t = ctx.search_trace(w.queries, k=20)
    oi = orc.Index(idx)
    for q in range(w.queries.shape[0]):
        r = orc.search(oi, w.queries[q], 16, 150, 40, 5, 20)
        compare_query(t, q, r, exact, oi, 40, 5)
    ctx.close()


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_candidate_sub_batches(small_index, small_workload, exact):
    """The candidate stage in sub-batches of 8 queries (as when a batch's
    visit records do not fit the workspace): the same results as one
    sub-batch, and each query against the oracle."""
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=exact)
    q = small_workload.queries
    ids1, sc1, cnt1 = ctx.search(q, k=50)
    ctx.set_candidate_batch(8)
    ids8, sc8, cnt8 = ctx.search(q, k=50)
    t = ctx.search_trace(q, k=50)
    ctx.set_candidate_batch(0)
    assert np.array_equal(ids1, ids8)
    assert np.array_equal(sc1.view(np.uint32), sc8.view(np.uint32))
    assert np.array_equal(cnt1, cnt8)
    oi = orc.Index(small_index)
    for i in range(q.shape[0]):
        r = orc.search(oi, q[i], 32, 500, 100, 5, 50)
        compare_query(t, i, r, exact, oi, 100, 5)
    ctx.close()


@pytest.mark.parametrize("exact", [True, False], ids=["exact", "mfma"])
def test_small_sub_batches_split_visits(small_index, small_workload, exact):
    """Batches of 1, 2, 3, 5 and 8 queries, whose count and emit kernels
    split each (query, token)'s visits over 16, 8, 4, 2 and 2 blocks, and 16
    queries in candidate sub-batches of 8 (2 blocks, the XCD-grouped grid):
    the same results as one 16-query sub-batch, bit for bit, as the reduce
    does not depend on the order of the records; a single-query trace against
    the oracle stage by stage."""
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=exact)
    q = small_workload.queries
    ids1, sc1, cnt1 = ctx.search(q, k=50)
    for n in (1, 2, 3, 5, 8):
        print(f"{n} queries", flush=True)
        ids, sc, cnt = ctx.search(q[:n], k=50)
        assert np.array_equal(ids, ids1[:n]), n
        assert np.array_equal(sc.view(np.uint32), sc1[:n].view(np.uint32)), n
        assert np.array_equal(cnt, cnt1[:n]), n
    ctx.set_candidate_batch(8)
    ids, sc, cnt = ctx.search(q, k=50)
    ctx.set_candidate_batch(0)
    assert np.array_equal(ids, ids1)
    assert np.array_equal(sc.view(np.uint32), sc1.view(np.uint32))
    assert np.array_equal(cnt, cnt1)
    t = ctx.search_trace(q[3:4], k=50)
    oi = orc.Index(small_index)
    r = orc.search(oi, q[3], 32, 500, 100, 5, 50)
    compare_query(t, 0, r, exact, oi, 100, 5)
    ctx.close()
