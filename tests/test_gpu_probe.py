"""Matrix-core probe: labels equal to the exact fp32 probe of the oracle
(the same sequential-fma score, ties to the lower centroid ID)."""
import numpy as np
import pytest

from chimera_amd import capi, synthetic
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def centroid_index(centroids: np.ndarray) -> dict:
    """A minimal index whose only meaningful part is the centroid set: one
    token per cluster, one document."""
    k = centroids.shape[0]
    return {
        "num_embeddings": k, "dimension": 128, "num_clusters": k, "ex_bits": 1,
        "flips": np.zeros(64, np.uint8), "doc_lens": np.array([k], np.int32),
        "doc_ptrs": np.array([0, k], np.int32), "cluster_pos": np.arange(k + 1, dtype=np.uint64),
        "clustered_codes": np.zeros(k * 16, np.uint8), "clustered_factors": np.ones(k, np.float32),
        "clustered_doc_ids": np.zeros(k, np.int32), "token_to_cluster_pos": np.arange(k, dtype=np.uint32),
        "full_bit_codes": np.zeros(k * 32, np.uint8), "full_bit_factors": np.ones(k, np.float32),
        "rotated_centroids": np.ascontiguousarray(centroids, np.float32),
    }


def run_probe(ctx, rows: np.ndarray, nprobe: int) -> np.ndarray:
    d_rot = ctx.to_device(rows)
    d_lab = ctx.empty((rows.shape[0], nprobe), np.uint32)
    capi.check(capi.lib().chimera_probe_device(ctx.handle, capi.P(d_rot.ptr), rows.shape[0], nprobe,
                                               capi.P(d_lab.ptr)))
    ctx.synchronize()
    out = d_lab.numpy()
    d_rot.free()
    d_lab.free()
    return out


@pytest.mark.parametrize("k,nprobe,sigma", [(65536, 128, 0.2), (16384, 32, 0.2), (65536, 16, 0.05)])
def test_mfma_probe_equals_exact(k, nprobe, sigma):
    rng = np.random.default_rng(k + nprobe)
    centres = synthetic.unit_centres(rng, 2048, 128)
    cent = synthetic.mixture_tokens(rng, centres, k, sigma)
    rows = synthetic.mixture_tokens(rng, centres, 1024, sigma)
    ctx = capi.Context(centroid_index(cent), nprobe, nprobe, 1, 1, max_batch=32)
    ctx.set_probe_mode(2)
    got = run_probe(ctx, rows, nprobe)
    ctx.set_probe_mode(1)
    exact_gpu = run_probe(ctx, rows, nprobe)
    ctx.close()
    want = orc.probe(rows, cent, nprobe)
    assert np.array_equal(exact_gpu, want)
    assert np.array_equal(got, want)


def test_mfma_probe_in_search_matches_oracle(small_index, small_workload):
    # force the matrix-core probe inside a full search (nprobe 32 of 1024 clusters)
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=True)
    ctx.set_probe_mode(2)
    qs = small_workload.queries[:8]
    t = ctx.search_trace(qs, k=100)
    oi = orc.Index(small_index)
    for q in range(qs.shape[0]):
        r = orc.search(oi, qs[q], 32, 500, 100, 5, 100)
        assert np.array_equal(t["labels"][q], r["labels"])
        n = int(t["counts"][q])
        assert np.array_equal(t["ids"][q, :n], r["result_ids"])
    ctx.close()
