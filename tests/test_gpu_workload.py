"""Device corpus generation and exact MaxSim ground truth
(include/chimera_workload.h) against numpy."""
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
