"""The full-size synthetic configurations against the oracle, query by
query and stage by stage (matrix-core scoring):

  docs1m   1,000,000 documents, lengths U[16, 160] (~88M tokens), 2,048-centre
           mixture (sigma 0.15), n_clusters 524,288, ex_bits 1, 4 and 7
  docs2m   2,000,000 documents, clipped log-normal lengths (median 64,
           sigma 0.5, [8, 300]; ~145M tokens), 16,384-centre mixture,
           n_clusters 1,048,576, ex_bits 4

both with nprobe 128, k_refine 3000, k_full_bit 300, num_chunks 5, k 100 and
32 queries perturbed from random target documents. The corpus is generated
and the index built on the device; the oracle runs on the downloaded index."""
import concurrent.futures as cf

import numpy as np
import pytest

from chimera_amd import capi, synthetic
from oracle import oracle as orc
from parity_checks import compare_query

pytestmark = pytest.mark.gpu

NPROBE, K_REFINE, K_FULL, CHUNKS, K, NQ = 128, 3000, 300, 5, 100, 32


def device_corpus(ctx, num_docs, len_kind, lo, hi, centres, sigma, seed):
    """Tokens on the device, document lengths and NQ queries (host)."""
    rng = np.random.default_rng(seed)
    c = synthetic.unit_centres(rng, centres, 128)
    lens = synthetic.doc_lengths(rng, num_docs, len_kind, lo, hi, 64.0, 0.5)
    ptrs = np.concatenate([[0], np.cumsum(lens, dtype=np.int64)])
    d_c = ctx.to_device(c)
    d_emb = ctx.synth_tokens(d_c, int(ptrs[-1]), sigma, seed=seed)
    d_c.free()
    targets = rng.integers(0, lens.size, size=NQ)
    picks = ptrs[targets][:, None] + (rng.random((NQ, 32)) * lens[targets][:, None]).astype(np.int64)
    rows = ctx.gather_rows(d_emb, picks.reshape(-1)).reshape(NQ, 32, 128)
    q = rows + np.float32(0.1) * rng.standard_normal(rows.shape, dtype=np.float32)
    q /= np.linalg.norm(q, axis=2, keepdims=True)
    return d_emb, lens, np.ascontiguousarray(q, np.float32)


def check_against_oracle(num_docs, len_kind, lo, hi, centres, n_clusters, ex_bits, seed):
    ctx = capi.Context(None, NPROBE, K_REFINE, K_FULL, CHUNKS, max_batch=NQ)
    print(f"{num_docs} docs, {n_clusters} clusters, ex_bits {ex_bits}: generating and building", flush=True)
    d_emb, lens, queries = device_corpus(ctx, num_docs, len_kind, lo, hi, centres, 0.15, seed)
    ctx.build(d_emb, lens, n_clusters, ex_bits)
    d_emb.free()
    t = ctx.search_trace(queries, K)
    host = ctx.download()
    ctx.close()
    oi = orc.Index(host)
    with cf.ThreadPoolExecutor(max_workers=16) as ex:
        runs = list(ex.map(lambda q: orc.search(oi, queries[q], NPROBE, K_REFINE, K_FULL, CHUNKS, K), range(NQ)))
    for q in range(NQ):
        assert int(t["refined_count"][q]) == K_REFINE
        compare_query(t, q, runs[q], False, oi, K_FULL, CHUNKS)


@pytest.mark.parametrize("ex_bits", [1, 4, 7])
def test_docs1m_against_oracle(ex_bits):
    check_against_oracle(1_000_000, "uniform", 16, 160, 2048, 524_288, ex_bits, seed=4)


def test_docs2m_against_oracle():
    check_against_oracle(2_000_000, "lognormal", 8, 300, 16384, 1 << 20, 4, seed=5)
