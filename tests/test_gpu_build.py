"""Index build on the device against the host build: every array of the
index files bit-exact (codes, factors, IVF lists, cluster order, rotated
centroids), for power-of-two and padded dimensions and every ex_bits."""
import numpy as np
import pytest

from chimera_amd import capi, synthetic

pytestmark = pytest.mark.gpu

KEYS = ["cluster_pos", "inv_list", "token_to_cluster_pos", "one_bit_codes", "one_bit_factors", "full_bit_codes",
        "full_bit_factors", "clustered_codes", "clustered_factors", "clustered_doc_ids", "rotated_centroids"]


def device_build(w, n_clusters, ex_bits, nprobe=8, k_refine=60, k_full_bit=20, num_chunks=3, max_batch=8):
    ctx = capi.Context(None, nprobe, k_refine, k_full_bit, num_chunks, max_batch=max_batch)
    ctx.build(w.embeddings, w.doc_lens, n_clusters, ex_bits)
    return ctx


def assert_same_index(cpu: dict, gpu: dict):
    for key in KEYS:
        a = np.asarray(cpu[key]).ravel()
        b = np.asarray(gpu[key]).ravel()
        assert a.dtype == b.dtype and a.shape == b.shape, key
        if a.dtype.kind == "f":
            bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
        else:
            bad = np.flatnonzero(a != b)
        assert bad.size == 0, f"{key}: {bad.size} of {a.size} differ, first at {bad[:5]}"


def workload(dim, seed, docs=300, lo=1, hi=40):
    rng = np.random.default_rng(seed)
    centres = synthetic.unit_centres(rng, 64, dim)
    lens = rng.integers(lo, hi + 1, size=docs).astype(np.int32)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    q, t = synthetic.make_queries(rng, emb, lens, 8)
    return synthetic.Workload(emb, lens, q, t)


@pytest.mark.parametrize("dim,ex_bits", [(128, 1), (128, 2), (128, 3), (128, 4), (128, 5), (128, 6), (128, 7),
                                         (100, 4), (64, 3)])
def test_device_build_equals_host_build(chimera_mod, dim, ex_bits):
    w = workload(dim, 100 + dim + ex_bits)
    cpu = chimera_mod._build_index(w.embeddings, w.doc_lens.tolist(), 96, ex_bits)
    ctx = device_build(w, 96, ex_bits)
    gpu = ctx.download()
    ctx.close()
    assert_same_index(cpu, gpu)


def test_device_build_small_index_and_search(chimera_mod, small_workload, small_index):
    """175k tokens, 1024 clusters: same bytes as the host build and the same
    search results as the uploaded host index."""
    w = small_workload
    ctx = capi.Context(None, 32, 500, 100, 5, max_batch=16)
    ctx.build(w.embeddings, w.doc_lens, 1024, 4)
    assert_same_index(small_index, ctx.download())
    ids, scores, counts = ctx.search(w.queries, 50)
    ref = capi.Context(small_index, 32, 500, 100, 5, max_batch=16)
    rids, rscores, rcounts = ref.search(w.queries, 50)
    ref.close()
    ctx.close()
    assert np.array_equal(ids, rids)
    assert np.array_equal(scores.view(np.uint32), rscores.view(np.uint32))
    assert np.array_equal(counts, rcounts)


def test_device_build_errors(small_workload):
    w = small_workload
    ctx = capi.Context(None, 8, 60, 20, 3, max_batch=8)
    emb = w.embeddings[:1000].copy()
    lens = np.array([500, 500], np.int32)
    with pytest.raises(capi.ChimeraError) as e:
        ctx.build(emb, np.array([500, 499], np.int32), 16, 4)
    assert e.value.code == capi.ERR_INVALID_ARGUMENT and "sum" in str(e.value)
    with pytest.raises(capi.ChimeraError) as e:
        ctx.build(emb, lens, 16, 8)
    assert e.value.code == capi.ERR_INVALID_ARGUMENT
    with pytest.raises(capi.ChimeraError) as e:
        ctx.build(emb, lens, 2000, 4)
    assert e.value.code == capi.ERR_INVALID_ARGUMENT
    bad = emb.copy()
    bad[17] = 0.0
    with pytest.raises(capi.ChimeraError) as e:
        ctx.build(bad, lens, 16, 4)
    assert e.value.code == capi.ERR_INVALID_ARGUMENT and "finite" in str(e.value)
    # the context is empty after a failed build and builds again afterwards
    with pytest.raises(capi.ChimeraError):
        ctx.search(w.queries[:1], 10)
    ctx.build(emb, lens, 16, 4)
    ids, _, counts = ctx.search(w.queries[:2], 10)
    assert ids.shape == (2, 10)
    ctx.close()
