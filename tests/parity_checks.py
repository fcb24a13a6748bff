"""Stage-by-stage comparison of a GPU search trace with the oracle's run of
the same query (shared by the GPU parity tests)."""
import numpy as np

from oracle import oracle as orc

# matrix-core one-bit and full-bit MaxSim against the reference's fp32 order
# (1e-4 relative)
S1_TOL = 2e-5
SF_TOL = 2e-5


def same_up_to_ties(got_ids, ref_ids, score_of, rtol):
    """Ranked lists equal, or differing only where the reference scores of
    the swapped documents agree within rtol."""
    got_ids, ref_ids = list(got_ids), list(ref_ids)
    if got_ids == ref_ids:
        return True
    if len(got_ids) != len(ref_ids):
        return False
    a = np.sort(np.array([score_of(d) for d in got_ids], np.float64))
    b = np.sort(np.array([score_of(d) for d in ref_ids], np.float64))
    return np.allclose(a, b, rtol=rtol, atol=1e-7)


def compare_query(t, q, r, exact, oi, k_full_bit, num_chunks):
    """Every stage of query q of trace t against the oracle's run r."""
    assert np.array_equal(t["rotated"][q], r["rotated"])
    assert np.array_equal(t["cb1"][q], r["cb1"])
    assert np.array_equal(t["cbex"][q], r["cbex"])
    assert np.array_equal(t["labels"][q], r["labels"])
    c = int(t["cand_count"][q])
    assert c == int(r["cand_count"][0])
    assert np.array_equal(t["candidates"][q, :c], r["candidates"])
    assert np.array_equal(t["cand_scores"][q, :c].view(np.uint32), r["cand_scores"].view(np.uint32))
    rc = int(t["refined_count"][q])
    assert rc == int(r["refined_count"][0])
    got_r = t["refined_ids"][q, :rc]
    assert np.array_equal(got_r, r["refined_ids"])
    fc = int(t["fullbit_count"][q])
    got_f = t["fullbit_ids"][q, :fc]
    order = np.argsort(got_f, kind="stable")
    n = int(t["counts"][q])
    if exact:
        assert np.array_equal(t["refined_scores"][q, :rc].view(np.uint32), r["refined_scores"].view(np.uint32))
        assert fc == int(r["fullbit_count"][0])
        assert np.array_equal(got_f[order], r["fullbit_ids"])
        assert np.array_equal(t["fullbit_scores"][q, :fc][order].view(np.uint32), r["fullbit_scores"].view(np.uint32))
        assert n == r["result_ids"].size
        assert np.array_equal(t["ids"][q, :n], r["result_ids"])
        assert np.array_equal(t["scores"][q, :n].view(np.uint32), r["result_scores"].view(np.uint32))
        return
    s1 = t["refined_scores"][q, :rc]
    np.testing.assert_allclose(s1, r["refined_scores"], rtol=S1_TOL, atol=S1_TOL)
    # the reference's chunk rule on the GPU's own one-bit scores
    sel = orc.chunk_select(s1, k_full_bit, num_chunks)
    want = np.sort(got_r[sel])
    assert np.array_equal(got_f[order], want)
    # against the oracle's own one-bit scores: a document may change sides
    # only where its oracle S1 has a near-tie (within twice the tolerance)
    # with another refined document
    got_set, ref_set = set(want.tolist()), set(r["fullbit_ids"].tolist())
    if got_set != ref_set:
        s1r = np.asarray(r["refined_scores"], np.float64)
        pos = {d: i for i, d in enumerate(r["refined_ids"].tolist())}
        tol = 2 * S1_TOL
        for d in got_set ^ ref_set:
            v = s1r[pos[d]]
            near = np.abs(s1r - v) <= tol * np.maximum(np.abs(s1r), abs(v)) + tol
            assert near.sum() >= 2, f"document {d} changes sides of the full-bit selection without a near-tie"
    sf = orc.full_bit_scores(oi, t["rotated"][q][None], t["cbex"][q][None], want[None, :].astype(np.int32))[0]
    got_sf = t["fullbit_scores"][q, :fc][order]
    np.testing.assert_allclose(got_sf, sf, rtol=SF_TOL, atol=SF_TOL)
    # the top-k follows the GPU's own scores exactly (ties: larger id first) ...
    keyed = sorted(zip(got_sf.tolist(), want.tolist()), key=lambda x: (-x[0], -x[1]))
    assert t["ids"][q, :n].tolist() == [d for _, d in keyed][:n]
    # ... and the reference arithmetic's ranking up to swaps inside the tolerance
    ref_keyed = sorted(zip(sf.tolist(), want.tolist()), key=lambda x: (-x[0], -x[1]))
    sf_of = dict(zip(want.tolist(), sf.tolist()))
    assert same_up_to_ties(t["ids"][q, :n], [d for _, d in ref_keyed][:n], sf_of.__getitem__, rtol=SF_TOL)


def expected_shape(num_docs, n_tokens, n_clusters, nprobe):
    """(log2 documents per bucket, records per reduce thread) as the library
    sizes the candidate stage: b the largest in [8, 13] whose expected
    visit records per bucket (rho per document, rho = 32 nprobe N / (K M)
    for a uniform probe) fit 8 per thread of a 512-thread reduce block,
    raised while there are more than 2,048 buckets; 12 records per thread
    when that raise leaves more than 8. Used to show which shapes a test's
    parameters reach."""
    rho = 32 * nprobe * n_tokens / (n_clusters * num_docs)
    b = 13
    while b > 8 and rho * 2**b > 8 * 512:
        b -= 1
    while b < 13 and -(-num_docs // 2**b) > 2048:
        b += 1
    return b, 8 if rho * 2**b <= 8 * 512 else 12
