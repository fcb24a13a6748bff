"""Candidate-stage shapes against the oracle.

The library sizes its document buckets per index: 2^b documents with b the
largest in [8, 13] whose expected visit records per bucket (rho per
document, rho = 32 nprobe N / (K M) for a uniform probe) fit 12 per reduce
thread, and the reduce holds 8 records per thread when they fit 8. Each
bucket size gives the reduce a different document-to-thread mapping (one
document per thread up to 512-document buckets, then 2, 4, 8, 16). The
small fixtures of the other tests land on 256-document buckets; this index
of 20,000 short documents (2-12 tokens) over 2,048 clusters, probed at
nprobe 4 to 64, takes every bucket size from 2^9 to 2^13 with both reduce
variants. Every query is compared with the oracle stage by stage (candidate
list and S_cand bit-exact, refined list identical, S1 and SF within the
matrix-core tolerance)."""
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
    assert {h for _, h in shapes} == {8, 12}


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
