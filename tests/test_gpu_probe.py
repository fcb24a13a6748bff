"""Matrix-core probe, on bf16 and on fp32 operands: labels equal to the
exact fp32 probe of the oracle (the same sequential-fma score, ties to the
lower centroid ID), from one query's 32 rows to 32,768."""
import numpy as np
import pytest

from chimera_amd import capi, synthetic
from oracle import oracle as orc
from test_probe_margin import margin  # the delta the kernels use

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


# probe modes: 2 the bf16 matrix-core filter, 3 the fp32 one (both with the
# exact fp32 rerank); 1 is the exact vector kernel
MODES = pytest.mark.parametrize("mode", [2, 3], ids=["bf16", "fp32"])


@MODES
@pytest.mark.parametrize("k,nprobe,sigma,nrows", [(65536, 128, 0.2, 1024), (16384, 32, 0.2, 1024),
                                                  (65536, 16, 0.05, 1024), (65536, 128, 0.2, 32)])
def test_mfma_probe_equals_exact(k, nprobe, sigma, nrows, mode):
    rng = np.random.default_rng(k + nprobe)
    centres = synthetic.unit_centres(rng, 2048, 128)
    cent = synthetic.mixture_tokens(rng, centres, k, sigma)
    rows = synthetic.mixture_tokens(rng, centres, nrows, sigma)
    ctx = capi.Context(centroid_index(cent), nprobe, nprobe, 1, 1, max_batch=32)
    print(f"probe mode {mode}: {nrows} rows x {k} centroids, nprobe {nprobe}", flush=True)
    ctx.set_probe_mode(mode)
    got = run_probe(ctx, rows, nprobe)
    ctx.set_probe_mode(1)
    exact_gpu = run_probe(ctx, rows, nprobe)
    ctx.close()
    want = orc.probe(rows, cent, nprobe)
    assert np.array_equal(exact_gpu, want)
    assert np.array_equal(got, want)


@MODES
def test_mfma_probe_at_the_microbench_size(mode):
    """The probe microbench's whole shape: 32,768 query vectors (1,024
    queries x 32 tokens) x 65,536 centroids, nprobe 128. Every row's labels
    equal the exact fp32 vector kernel's on the GPU, and 1,024 rows drawn
    over all row blocks equal the oracle's."""
    rng = np.random.default_rng(65536 + 128)
    centres = synthetic.unit_centres(rng, 2048, 128)
    cent = synthetic.mixture_tokens(rng, centres, 65536, 0.2)
    rows = synthetic.mixture_tokens(rng, centres, 32768, 0.2)
    ctx = capi.Context(centroid_index(cent), 128, 128, 1, 1, max_batch=1024)
    print(f"probe mode {mode}: 32768 rows x 65536 centroids, nprobe 128", flush=True)
    ctx.set_probe_mode(mode)
    got = run_probe(ctx, rows, 128)
    ctx.set_probe_mode(1)
    exact_gpu = run_probe(ctx, rows, 128)
    ctx.close()
    assert np.array_equal(got, exact_gpu)
    pick = np.sort(rng.choice(rows.shape[0], 1024, replace=False))
    assert np.array_equal(exact_gpu[pick], orc.probe(rows[pick], cent, 128))


def test_fp32_filter_keeps_fewer_candidates():
    """Without operand rounding the margin shrinks (probe_delta with eq =
    ecmax = 0), so fewer centroids pass the fp32 filter than the bf16 one;
    both label sets equal the exact probe's."""
    rng = np.random.default_rng(31)
    centres = synthetic.unit_centres(rng, 2048, 128)
    cent = synthetic.mixture_tokens(rng, centres, 65536, 0.2)
    rows = synthetic.mixture_tokens(rng, centres, 2048, 0.2)
    ctx = capi.Context(centroid_index(cent), 128, 128, 1, 1, max_batch=64)
    out = {}
    for mode in (2, 3, 1):
        ctx.set_probe_mode(mode)
        out[mode] = (run_probe(ctx, rows, 128), ctx.probe_stats(2048) if mode != 1 else None)
    ctx.close()
    bf, fp = out[2][1].astype(np.float64), out[3][1].astype(np.float64)
    assert (bf < 2048).all() and (fp < 2048).all()  # no overflow or failed check
    assert fp.mean() < 0.8 * bf.mean(), (fp.mean(), bf.mean())
    assert (fp >= 128).all()
    assert np.array_equal(out[2][0], out[1][0])
    assert np.array_equal(out[3][0], out[1][0])


@MODES
def test_mfma_probe_in_search_matches_oracle(small_index, small_workload, mode):
    # the matrix-core probe inside a full search (nprobe 32 of 1024 clusters)
    ctx = capi.Context(small_index, 32, 500, 100, 5, max_batch=16, exact=True)
    ctx.set_probe_mode(mode)
    qs = small_workload.queries[:8]
    t = ctx.search_trace(qs, k=100)
    oi = orc.Index(small_index)
    for q in range(qs.shape[0]):
        r = orc.search(oi, qs[q], 32, 500, 100, 5, 100)
        assert np.array_equal(t["labels"][q], r["labels"])
        n = int(t["counts"][q])
        assert np.array_equal(t["ids"][q, :n], r["result_ids"])
    ctx.close()


def _mixture(rng, k, sigma=0.2):
    centres = synthetic.unit_centres(rng, 2048, 128)
    return centres, synthetic.mixture_tokens(rng, centres, k, sigma)


@pytest.mark.parametrize("nrows,copies,first,tied,mode", [(1024, 4096, 8192, 256, 2), (32768, 6144, 8192, 256, 2),
                                                          (1024, 4096, 8192, 768, 2), (1024, 4096, 8192, 256, 3),
                                                          (32768, 6144, 8192, 256, 3)],
                         ids=["rerank-cap", "lane-cap", "many-flagged", "rerank-cap-fp32", "lane-cap-fp32"])
def test_overflowing_rows_fall_back_to_the_exact_kernel(nrows, copies, first, tied, mode):
    """Thousands of identical centroids tie exactly for the `tied` rows drawn
    next to them, so every copy passes the filter. With 1,024 rows the
    copies spread over 16 centroid splits and a row collects 4,096
    candidates, more than the rerank's key area (1,024 at nprobe 64: its
    flag); with 32,768 rows the split holds all 192 tiles of copies and a
    lane's 128-entry sub-list overflows during the filtered pass (the
    kernel's flag). Up to 512 flagged rows are recomputed by the exact
    kernels split over the centroids, more (768) by the row-block exact
    kernel: either way their labels are the first nprobe copies (ties to
    the lower id), the other rows equal the oracle's."""
    rng = np.random.default_rng(nrows + copies + tied)
    centres, cent = _mixture(rng, 65536)
    v = synthetic.unit_centres(rng, 1, 128)[0]
    cent[first:first + copies] = v
    rows = synthetic.mixture_tokens(rng, centres, nrows, 0.2)
    near = v[None, :] + np.float32(0.05) * rng.standard_normal((tied, 128), dtype=np.float32)
    rows[:tied] = near / np.linalg.norm(near, axis=1, keepdims=True)
    nprobe = 64
    ctx = capi.Context(centroid_index(cent), nprobe, nprobe, 1, 1, max_batch=nrows // 32)
    ctx.set_probe_mode(mode)
    got = run_probe(ctx, rows, nprobe)
    stats = ctx.probe_stats(nrows)
    ctx.set_probe_mode(1)
    exact_gpu = run_probe(ctx, rows, nprobe)
    ctx.close()
    flagged = (stats == 0xFFFFFFFF) | (stats > 2048)
    assert flagged[:tied].all(), "the tied rows must take the overflow path"
    assert flagged[tied:].sum() < 0.05 * (nrows - tied)
    want_tied = first + np.arange(nprobe, dtype=np.uint32)
    assert (got[:tied] == want_tied[None, :]).all()
    assert np.array_equal(got, exact_gpu)
    sample = np.concatenate([np.arange(8), tied + rng.choice(nrows - tied, 248, replace=False)])
    assert np.array_equal(got[sample], orc.probe(rows[sample], cent, nprobe))


def test_mfma_probe_with_aligned_bf16_rounding():
    """Every row q = s * (1 + 2^-8 - 2^-20) (random signs s) rounds to s in
    bf16. Each row has a family of 32 centroids next to it: 12 of kind A,
    s * (values just below 1 + 2^-8, rounding down to 1), and 20 of kind B,
    s * (values just above 1 + 2^-8, rounding up to 1 + 2^-7). In fp32 the
    family's scores are equal up to rounding noise, but the bf16 score of an
    A exceeds its exact score by about 2.0 while a B's barely moves, so the
    exact top-nprobe holds A centroids whose bf16 scores lie about 2 above
    the bf16 threshold: the filter keeps them only if the margin covers the
    operands' rounding (the row's |q - q_b| and the centroids' max
    |c - c_b|). Labels must equal the oracle's."""
    rng = np.random.default_rng(99)
    down = 1.0 + 2 ** -8 - 2 ** -20
    nrows, fam, n_a, nprobe = 1024, 32, 12, 16
    sign = rng.choice([-1.0, 1.0], (nrows, 128))
    rows = (sign * down).astype(np.float32)
    mag = np.empty((nrows, fam, 128))
    mag[:, :n_a] = 1.0 + 2 ** -8 - rng.uniform(2 ** -20, 2 ** -13, (nrows, n_a, 128))
    mag[:, n_a:] = 1.0 + 2 ** -8 + rng.uniform(2 ** -20, 2 ** -13, (nrows, fam - n_a, 128))
    cent = (sign[:, None, :] * mag).reshape(-1, 128).astype(np.float32)
    kind_a = np.tile(np.arange(fam) < n_a, nrows)
    perm = rng.permutation(cent.shape[0])
    cent, kind_a = cent[perm], kind_a[perm]
    ctx = capi.Context(centroid_index(cent), nprobe, nprobe, 1, 1, max_batch=nrows // 32)
    cmax, ecmax = ctx.probe_bounds()
    assert ecmax > 0.95 * 2 ** -8 * np.sqrt(128)  # the centroids' rounding is near its maximum
    ctx.set_probe_mode(2)
    got = run_probe(ctx, rows, nprobe)
    stats = ctx.probe_stats(nrows)
    ctx.close()
    # no row overflows; the families of 32 near-ties make the threshold
    # estimate miss on a few rows, which the exact kernel recomputes
    assert (stats != 0xFFFFFFFF).all()
    assert ((stats == 0xFFFFFFFE) | (stats <= 2048)).all()
    assert (stats == 0xFFFFFFFE).mean() < 0.1
    want = orc.probe(rows, cent, nprobe)
    assert kind_a[want].sum() > nrows  # exact labels do include A centroids
    assert np.array_equal(got, want)


def _bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even bf16 of float32 values, as float32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def _plan_stride_and_rank(k: int, nprobe: int) -> tuple[int, int]:
    """The matrix-core probe's sample stride and threshold rank for k
    centroids (the plan's rule), used only to build inputs that defeat the
    threshold estimate."""
    ntiles = k // 32
    s = 8 if ntiles >= 64 * nprobe else 4 if ntiles >= 16 * nprobe else 1
    f, z = 1.0 / s, 4.5
    b = z * np.sqrt(1.0 - f)
    x = 0.5 * (b + np.sqrt(b * b + 4.0 * f * nprobe))
    return s, int(min(nprobe, max(1, np.ceil(x * x - 1e-9))))


@pytest.mark.parametrize("ring", [True, False], ids=["check-fails", "too-few-candidates"])
def test_rows_whose_threshold_estimate_misses_fall_back(ring):
    """The filter threshold comes from the r-th smallest sampled tile minimum
    (65,536 centroids, nprobe 64: every 4th tile sampled, r = 41), an
    estimate of the centroid of rank about 164. For 6 rows it is made to
    miss: r + 8 centroids close to the row, one in each of as many sampled
    tiles, set the threshold at the r-th of them (U), and 100 more lie in
    unsampled tiles at d = U + delta (ring) or are absent. With the ring a
    row has more than 64 candidates, but only r < 64 of them have d' <= U,
    so the rerank's check fails; without it the row has fewer than 64.
    Either way the row must be recomputed exactly (stats 0xFFFFFFFE) and
    every row's labels equal the oracle's."""
    rng = np.random.default_rng(7 if ring else 8)
    k, nprobe, nrows, bad = 65536, 64, 1024, 6
    stride, r = _plan_stride_and_rank(k, nprobe)
    assert r < nprobe and bad * (r + 8) * stride <= k // 32
    n_a = r + 8
    centres, cent = _mixture(rng, k)
    rows = synthetic.mixture_tokens(rng, centres, nrows, 0.2)
    cos_a = 0.95 - 0.0005 * np.arange(n_a)
    for j in range(bad):
        v = rows[j].astype(np.float64)
        u = rng.standard_normal((n_a, 128))
        u -= (u @ v)[:, None] * v[None, :]
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        a_idx = 32 * stride * (n_a * j + np.arange(n_a)) + (j % 32)
        cent[a_idx] = (cos_a[:, None] * v + np.sqrt(1 - cos_a ** 2)[:, None] * u).astype(np.float32)
    ecmax = float(np.max(np.linalg.norm(cent - _bf16(cent), axis=1)))
    cmax = float(np.max(np.linalg.norm(cent, axis=1)))
    for j in range(bad):
        v = rows[j].astype(np.float64)
        u = rng.standard_normal((100, 128))
        u -= (u @ v)[:, None] * v[None, :]
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        eq = float(np.linalg.norm(rows[j] - _bf16(rows[j])))
        delta = margin(float(np.linalg.norm(rows[j])), eq, cmax * 1.001, ecmax * 1.001)
        u_d = 1.0 - 2.0 * cos_a[r - 1]
        cos_b = (1.0 - (u_d + delta)) / 2.0 - 1e-6 * np.arange(100)
        t = 25 * j + np.arange(100) // 4
        b_idx = 32 * (4 * t + 1) + (np.arange(100) % 4) * 8 + (j % 8)  # tiles 4t + 1: never sampled
        if ring:
            cent[b_idx] = (cos_b[:, None] * v + np.sqrt(1 - cos_b ** 2)[:, None] * u).astype(np.float32)
    ctx = capi.Context(centroid_index(cent), nprobe, nprobe, 1, 1, max_batch=nrows // 32)
    ctx.set_probe_mode(2)
    got = run_probe(ctx, rows, nprobe)
    stats = ctx.probe_stats(nrows)
    ctx.close()
    assert (stats[:bad] == 0xFFFFFFFE).all(), stats[:bad]
    assert ((stats[bad:] == 0xFFFFFFFE) | (stats[bad:] == 0xFFFFFFFF)).mean() < 0.05
    sample = np.concatenate([np.arange(bad), bad + rng.choice(nrows - bad, 120, replace=False)])
    assert np.array_equal(got[sample], orc.probe(rows[sample], cent, nprobe))
