"""The CPU baseline (oracle/fullbit_avx512.cpp): the AVX-512 restatement of
the reference's full-bit MaxSim stage (search_impl.cu:510-574) returns the
oracle's full-bit scores bit for bit at every code width, with the unpack
layouts of every width exercised over random codes."""
import numpy as np
import pytest

from chimera_amd import synthetic
from oracle import oracle as orc

pytestmark = pytest.mark.skipif(not orc.fullbit_baseline_available(), reason="no AVX-512 on this CPU")


@pytest.mark.parametrize("ex_bits", range(1, 8))
def test_baseline_equals_oracle_full_bit_scores(chimera_mod, ex_bits):
    rng = np.random.default_rng(ex_bits)
    centres = synthetic.unit_centres(rng, 16, 128)
    lens = rng.integers(1, 30, size=80).astype(np.int32)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    idx = chimera_mod._build_index(emb, lens.tolist(), 16, ex_bits)
    oi = orc.Index(idx)
    nq, per = 3, 40
    q = synthetic.make_queries(rng, emb, lens, nq)[0]
    rot = orc.rotate(q.reshape(-1, 128), idx["flips"]).reshape(nq, 32, 128)
    cbex = np.stack([orc.query_state(rot[i], ex_bits)[1] for i in range(nq)])
    docs = rng.integers(0, lens.size, size=(nq, per)).astype(np.int32)
    counts = np.array([per, 17, 0], np.int32)
    got = orc.fullbit_baseline(oi, rot, cbex, docs, counts, threads=4)
    want = orc.full_bit_scores(oi, rot, cbex, docs)
    for i in range(nq):
        assert np.array_equal(got[i, :counts[i]].view(np.uint32), want[i, :counts[i]].view(np.uint32))
    assert (got[1, 17:] == 0).all() and (got[2] == 0).all()


@pytest.mark.parametrize("w", range(2, 9))
def test_baseline_unpack_on_random_codes(w):
    """Random packed bytes of width w as one document's codes: the score
    equals the oracle's, which unpacks with its own scalar loop."""
    rng = np.random.default_rng(w)
    n = 24
    ptrs = np.array([0, n], np.int32)
    codes = rng.integers(0, 256, size=n * 16 * w).astype(np.uint8)
    index = orc.Index({
        "num_embeddings": n, "dimension": 128, "num_clusters": 1, "ex_bits": w - 1,
        "doc_lens": np.array([n], np.int32), "doc_ptrs": ptrs, "cluster_pos": np.array([0, n], np.uint64),
        "clustered_codes": np.zeros(n * 16, np.uint8), "clustered_factors": np.zeros(n, np.float32),
        "clustered_doc_ids": np.zeros(n, np.int32), "token_to_cluster_pos": np.arange(n, dtype=np.uint32),
        "full_bit_codes": codes, "full_bit_factors": rng.uniform(0.5, 2.0, n).astype(np.float32),
        "rotated_centroids": np.zeros(128, np.float32), "flips": np.zeros(64, np.uint8),
    })
    rot = rng.standard_normal((1, 32, 128)).astype(np.float32)
    cbex = rng.standard_normal((1, 32)).astype(np.float32)
    docs = np.zeros((1, 1), np.int32)
    got = orc.fullbit_baseline(index, rot, cbex, docs, np.array([1], np.int32))
    want = orc.full_bit_scores(index, rot, cbex, docs)
    assert got.view(np.uint32)[0, 0] == want.view(np.uint32)[0, 0]
