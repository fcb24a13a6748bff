"""Candidate-stage shapes against the oracle.

The library sizes its document buckets per index: 2^b documents with b the
largest in [8, 13] whose expected visit records per bucket (rho per
document, rho = 32 nprobe N / (K M) for a uniform probe) fit 8 per reduce
thread, raised while there are more than 2,048 buckets (the emit's LDS
counters); a bucket raised past 8 records per thread takes the 12-record
reduce. Each bucket size gives the reduce a different document-to-thread
mapping (one document per thread up to 512-document buckets, then 2, 4, 8,
16). The small fixtures of the other tests land on 256-document buckets;
this index of 20,000 short documents (2-12 tokens) over 2,048 clusters,
probed at nprobe 4 to 64, takes every bucket size from 2^9 to 2^13, and an
index of 600,000 one-token documents over 64 clusters at nprobe 20 is
raised from 256- to 512-document buckets with 12 records per thread. Every
query is compared with the oracle stage by stage (candidate list and S_cand
bit-exact, refined list identical, S1 and SF within the matrix-core
tolerance)."""
import numpy as np
import pytest

from chimera_amd import capi, synthetic
from oracle import oracle as orc
from parity_checks import compare_query, expected_shape

pytestmark = pytest.mark.gpu

NPROBES = [4, 6, 8, 12, 16, 24, 32, 48, 64]
K_REFINE, K_FULL, CHUNKS, K = 400, 100, 4, 50


@pytest.fixture(scope="module")
def short_docs(chimera_mod):
    rng = np.random.default_rng(31)
    centres = synthetic.unit_centres(rng, 256, 128)
    lens = rng.integers(2, 13, size=20000).astype(np.int32)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    q, _ = synthetic.make_queries(rng, emb, lens, 4)
    idx = chimera_mod._build_index(emb, lens.tolist(), 2048, 4)
    return idx, q, lens


def test_nprobes_reach_every_shape(short_docs):
    _, _, lens = short_docs
    shapes = {expected_shape(lens.size, int(lens.sum()), 2048, n) for n in NPROBES}
    assert {b for b, _ in shapes} == {9, 10, 11, 12, 13}
    assert {h for _, h in shapes} == {8}


@pytest.mark.parametrize("nprobe", NPROBES)
def test_bucket_shape_matches_oracle(short_docs, nprobe):
    idx, q, lens = short_docs
    print("shape", expected_shape(lens.size, int(lens.sum()), 2048, nprobe), flush=True)
    ctx = capi.Context(idx, nprobe, K_REFINE, K_FULL, CHUNKS, max_batch=4)
    t = ctx.search_trace(q, k=K)
    ctx.close()
    oi = orc.Index(idx)
    for i in range(q.shape[0]):
        r = orc.search(oi, q[i], nprobe, K_REFINE, K_FULL, CHUNKS, K)
        compare_query(t, i, r, False, oi, K_FULL, CHUNKS)


def test_bucket_cap_raises_to_twelve_records_per_thread(chimera_mod):
    """600,000 one-token documents over 64 clusters at nprobe 20: rho = 10,
    so 256-document buckets fit 8 records per thread, but 2,344 of them
    exceed the emit's 2,048 bucket counters and the buckets grow to 512
    documents, about 5,100 records per item: the 12-record reduce. Every
    visited document of a bucket is visited by many query tokens, so items
    need several slot chunks."""
    num_docs, n_clusters, nprobe, nq = 600_000, 64, 20, 2
    assert expected_shape(num_docs, num_docs, n_clusters, nprobe) == (9, 12)
    rng = np.random.default_rng(41)
    ctx = capi.Context(None, nprobe, K_REFINE, K_FULL, CHUNKS, max_batch=nq)
    c = synthetic.unit_centres(rng, 64, 128)
    d_c = ctx.to_device(c)
    d_emb = ctx.synth_tokens(d_c, num_docs, 0.15, seed=41)
    d_c.free()
    picks = rng.integers(0, num_docs, size=nq * 32)
    rows = ctx.gather_rows(d_emb, picks).reshape(nq, 32, 128)
    q = rows + np.float32(0.1) * rng.standard_normal(rows.shape, dtype=np.float32)
    q = np.ascontiguousarray(q / np.linalg.norm(q, axis=2, keepdims=True), np.float32)
    print("building 600,000 one-token documents over 64 clusters", flush=True)
    ctx.build(d_emb, np.ones(num_docs, np.int32), n_clusters, 4)
    d_emb.free()
    t = ctx.search_trace(q, k=K)
    host = ctx.download()
    ctx.close()
    oi = orc.Index(host)
    for i in range(nq):
        r = orc.search(oi, q[i], nprobe, K_REFINE, K_FULL, CHUNKS, K)
        compare_query(t, i, r, False, oi, K_FULL, CHUNKS)
