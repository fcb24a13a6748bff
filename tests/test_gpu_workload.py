"""Device corpus generation and exact MaxSim ground truth
(include/chimera_workload.h) against numpy, and the matrix-core rate
utility's bounds."""
import numpy as np
import pytest

from conftest import gpu_available

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    if not gpu_available():
        pytest.fail("no HIP device visible")
    from chimera_amd import capi

    c = capi.Context(None, 8, 100, 50, 5)
    yield c
    c.close()


def _centres(k, seed):
    from chimera_amd import synthetic

    return synthetic.unit_centres(np.random.default_rng(seed), k, 128)


def test_synth_tokens_are_unit_mixture_and_deterministic(ctx):
    centres = _centres(64, 1)
    d_c = ctx.to_device(centres)
    sigma = 0.15
    a = ctx.synth_tokens(d_c, 5000, sigma, seed=7)
    b = ctx.synth_tokens(d_c, 5000, sigma, seed=7)
    c = ctx.synth_tokens(d_c, 5000, sigma, seed=8)
    x, y, z = a.numpy(), b.numpy(), c.numpy()
    for arr in (a, b, c, d_c):
        arr.free()
    assert np.array_equal(x, y)
    assert not np.array_equal(x, z)
    np.testing.assert_allclose(np.linalg.norm(x, axis=1), 1.0, atol=1e-5)
    # a token is (centre + sigma g) / |.|: its cosine with its centre
    # concentrates at 1 / sqrt(1 + 128 sigma^2); other centres are far
    best = (x @ centres.T).max(axis=1)
    expect = 1.0 / np.sqrt(1.0 + 128 * sigma * sigma)
    assert abs(float(np.median(best)) - expect) < 0.03
    # centre choice is uniform: every centre is used, none dominates
    counts = np.bincount((x @ centres.T).argmax(axis=1), minlength=64)
    assert counts.min() > 30 and counts.max() < 140
    # the noise is N(0, sigma^2) per dimension before normalisation
    lab = (x @ centres.T).argmax(axis=1)
    noise = x / best[:, None] - centres[lab]
    assert abs(float(noise.std()) - sigma) < 0.01


def test_gather_rows(ctx):
    rng = np.random.default_rng(3)
    src = rng.standard_normal((300, 128)).astype(np.float32)
    d = ctx.to_device(src)
    ids = rng.integers(0, 300, size=77)
    got = ctx.gather_rows(d, ids)
    d.free()
    assert np.array_equal(got, src[ids])


@pytest.mark.parametrize("nq", [1, 10])
def test_exact_maxsim_matches_numpy(ctx, nq):
    from chimera_amd import synthetic

    rng = np.random.default_rng(nq)
    # lengths around the 16-token tile: 1, 15, 16, 17, 32, 33 and random ones
    lens = np.concatenate([[1, 15, 16, 17, 32, 33], rng.integers(1, 70, size=250)]).astype(np.int32)
    centres = synthetic.unit_centres(rng, 32, 128)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    q, _ = synthetic.make_queries(rng, emb, lens, nq)
    ptrs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d_emb = ctx.to_device(emb)
    d_ptrs = ctx.to_device(ptrs)
    got = ctx.exact_maxsim(d_emb, d_ptrs, q)
    d_emb.free()
    d_ptrs.free()
    want = synthetic.exact_maxsim_scores(emb, lens, q)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    gt_ids, _ = synthetic.exact_maxsim_topk(emb, lens, q, 10)
    assert synthetic.recall_at_k(gt_ids, [np.argsort(-g, kind="stable")[:10] for g in got], 10) >= 0.99


def _maxsim_f64(emb, ptrs, q, doc):
    """sum_i max_t <q_i, x_t> in float64 for one document (-inf when empty)."""
    x = emb[ptrs[doc]:ptrs[doc + 1]].astype(np.float64)
    if x.shape[0] == 0:
        return -np.inf
    return float((q.astype(np.float64) @ x.T).max(axis=1).sum())


def test_maxsim_rescore_matches_float64(ctx):
    """MaxSim rescoring of candidate lists (the MaxSim rescoring microbench's
    shape: unit-norm Gaussian queries, candidate documents of U[16, 256]
    mixture tokens, top-100) against a float64 brute force: scores within
    1e-4 relative, top-k equal up to swaps inside that tolerance."""
    from chimera_amd import synthetic

    rng = np.random.default_rng(11)
    m = 1200
    lens = np.concatenate([[0, 1, 15, 16, 17, 31, 32, 33, 256], rng.integers(16, 257, size=m - 9)]).astype(np.int32)
    ptrs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    centres = synthetic.unit_centres(rng, 2048, 128)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    nq, cap, k = 7, 300, 100
    q = rng.standard_normal((nq, 32, 128)).astype(np.float32)
    q /= np.linalg.norm(q, axis=2, keepdims=True)
    ids = np.stack([rng.choice(m, size=cap, replace=False) for _ in range(nq)]).astype(np.int32)
    ids[0, :9] = np.arange(9)              # empty and tile-edge documents
    ids[1, 5] = -1                         # ids outside [0, m) score -inf
    ids[1, 6] = m
    counts = np.array([cap, cap, 0, 1, 137, cap, 60], np.int32)  # 60 < k: padded output
    d_emb = ctx.to_device(emb)
    d_ptrs = ctx.to_device(ptrs)
    try:
        sc, top_ids, top_sc, top_cnt = ctx.maxsim_rescore(d_emb, d_ptrs, q, ids, counts, k)
    finally:
        d_emb.free()
        d_ptrs.free()
    for qi in range(nq):
        n = counts[qi]
        want = np.array([_maxsim_f64(emb, ptrs, q[qi], d) if 0 <= d < m else -np.inf for d in ids[qi, :n]])
        got = sc[qi, :n].astype(np.float64)
        fin = np.isfinite(want)
        assert np.array_equal(np.isfinite(got), fin)
        assert np.all(got[~fin] == -np.inf)
        np.testing.assert_allclose(got[fin], want[fin], rtol=1e-4, atol=1e-5)
        kk = min(k, n)
        assert top_cnt[qi] == kk
        assert np.all(top_ids[qi, kk:] == -1)
        # returned scores are the rescored ones, in descending order
        np.testing.assert_array_equal(np.sort(top_sc[qi, :kk])[::-1], top_sc[qi, :kk])
        if kk == 0:
            continue
        # the top-k by the float64 scores, up to swaps inside the tolerance
        kth = np.sort(want)[::-1][kk - 1]
        tol = 1e-4 * max(1.0, abs(kth)) if np.isfinite(kth) else 0.0
        pos = {int(d): j for j, d in enumerate(ids[qi, :n])}
        for d in top_ids[qi, :kk]:
            w = want[pos[int(d)]]
            assert w >= kth - tol or (not np.isfinite(kth) and not np.isfinite(w))
    # ids with the -inf score rank after every finite candidate
    assert set(top_ids[1, :k].tolist()).isdisjoint({-1 & 0xFFFFFFFF, m})


def test_matrix_core_rate_is_below_the_nominal_peaks(ctx):
    """chimera_matrix_core_rate: every instruction type reports a rate
    above a tenth of its dense nominal peak (bf16/fp16 2.5 PFLOP/s, fp32
    157.3 TFLOP/s, int8 5 POP/s) and below it (with 5 % for the clock the
    peak is quoted at)."""
    peaks = {"bf16_32x32x16": 2500e12, "f16_16x16x32": 2500e12, "f16_16x16x32_bits": 2500e12,
             "f32_32x32x2": 157.3e12, "i8_32x32x32": 5000e12, "f16_16x16x32_bits_valu4": 2500e12}
    for kind, peak in peaks.items():
        ops = ctx.matrix_core_rate(kind, 2000)
        print(f"{kind}: {ops / 1e12:.1f} T/s", flush=True)
        assert 0.1 * peak < ops < 1.05 * peak, kind
