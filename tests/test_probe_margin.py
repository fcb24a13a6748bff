"""The matrix-core probe's error margin, on the CPU.

The probe keeps every centroid whose bf16 score d' (bf16 operands, fp32
accumulation from -|c|^2/2) is within U + 2 delta and rescores those in fp32,
so its labels equal the exact probe's only if delta bounds |d' - d| for every
centroid (d = |c|^2 - 2<q,c>, the oracle's sequential-fmaf score). This file
checks chimera_probe_margin (the delta the kernels use) against d' emulated
on the CPU, with bf16 round-to-nearest-even reproduced bit by bit and the fp32
accumulation taken in several orders, on adversarial vectors whose every
component sits just off a bf16 midpoint (all rounding errors aligned), on
mixed magnitudes and scales, and on random data. The aligned case also shows
the bound is tight there (within 5 %), so a bound missing a factor of two
fails."""
import ctypes as C

import numpy as np
import pytest

from chimera_amd import capi
from oracle import oracle as orc


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def bf16_by_definition(x: np.ndarray) -> np.ndarray:
    """The same rounding chosen from the two bfloat16 neighbours of x."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32)
    lo = (u & np.uint32(0xFFFF0000)).view(np.float32)
    hi = ((u & np.uint32(0xFFFF0000)) + np.uint32(0x10000)).view(np.float32)
    dl = np.abs(x.astype(np.float64) - lo.astype(np.float64))
    dh = np.abs(hi.astype(np.float64) - x.astype(np.float64))
    lo_even = ((lo.view(np.uint32) >> 16) & 1) == 0
    return np.where((dl < dh) | ((dl == dh) & lo_even), lo, hi)


def margin(qn: float, eq: float, cmax: float, ecmax: float) -> float:
    f = capi.lib().chimera_probe_margin
    f.restype = C.c_float
    f.argtypes = [C.c_float, C.c_float, C.c_float, C.c_float]
    return float(f(qn, eq, cmax, ecmax))


def exact_scores(q: np.ndarray, cents: np.ndarray) -> np.ndarray:
    """The oracle's fp32 score (sequential fmaf dot and norm)."""
    L = orc.lib()
    L.oracle_probe_score.argtypes = [C.c_void_p, C.c_void_p]
    q = np.ascontiguousarray(q, np.float32)
    return np.array([L.oracle_probe_score(q.ctypes.data, np.ascontiguousarray(c, np.float32).ctypes.data)
                     for c in cents], np.float64)


def bf16_scores(q: np.ndarray, cents: np.ndarray, norms: np.ndarray) -> np.ndarray:
    """d' = -2 acc under four fp32 accumulation orders of -N/2 and the
    128 exact bf16 products; returns [orders, centroids]."""
    qb = bf16_rne(q).astype(np.float64)
    out = []
    for c, n in zip(cents, norms):
        cb = bf16_rne(c).astype(np.float64)
        p = qb * cb  # exact: 8-bit by 8-bit significands
        start = np.float32(-0.5 * np.float32(n))
        exact = np.float32(np.float64(start) + p.sum())
        seq = start
        for v in p.astype(np.float32):
            seq = np.float32(seq + v)
        blk = start  # one rounding per 16-product step
        for k in range(8):
            blk = np.float32(np.float64(blk) + p[16 * k:16 * k + 16].sum())
        tree = np.concatenate([[start], p.astype(np.float32), np.zeros(127, np.float32)]).astype(np.float32)
        while tree.size > 1:
            tree = (tree[0::2] + tree[1::2]).astype(np.float32)
        out.append([-2.0 * float(a) for a in (exact, seq, blk, tree[0])])
    return np.array(out).T


def check_bound(q: np.ndarray, cents: np.ndarray):
    """max |d' - d| over the centroids and orders, and the probe's delta."""
    q = q.astype(np.float32)
    cents = cents.astype(np.float32)
    d = exact_scores(q, cents)
    norms = np.array([np.float32(sum(np.float64(v) * v for v in c)) for c in cents], np.float32)
    dp = bf16_scores(q, cents, norms)
    worst = float(np.max(np.abs(dp - d[None, :])))
    qn = float(np.linalg.norm(q.astype(np.float64)))
    eq = float(np.linalg.norm(q.astype(np.float64) - bf16_rne(q)))
    cmax = float(np.max(np.linalg.norm(cents.astype(np.float64), axis=1))) * (1 + 1e-4)
    ecmax = float(np.max(np.linalg.norm(cents.astype(np.float64) - bf16_rne(cents), axis=1))) * (1 + 1e-4)
    return worst, margin(qn, eq, cmax, ecmax)


def test_bf16_rounding_matches_its_definition():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32),
                        (rng.standard_normal(2000) * 1e-30).astype(np.float32),
                        (rng.standard_normal(2000) * 1e30).astype(np.float32)])
    # exact midpoints between neighbouring bfloat16 values, both parities
    mids = ((rng.integers(0x0080, 0x7F00, 4000, dtype=np.uint32) << 16) | 0x8000).view(np.float32)
    x = np.concatenate([x, mids, -mids, np.float32([0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8])])
    assert np.array_equal(bf16_rne(x).view(np.uint32), bf16_by_definition(x).view(np.uint32))
    assert bf16_rne(np.float32([1.0 + 2 ** -8]))[0] == 1.0  # tie to even
    assert bf16_rne(np.float32([1.0 + 3 * 2 ** -8]))[0] == np.float32(1.0 + 2 ** -6)


@pytest.mark.parametrize("v", [1.0 + 2 ** -8 - 2 ** -20, 1.0 + 2 ** -8 + 2 ** -20], ids=["down", "up"])
def test_aligned_rounding_errors_are_covered_and_the_bound_is_tight(v):
    """Every component of q and c one step below (or above) a bf16 midpoint:
    all 256 roundings move the same way, and |d' - d| reaches about
    2 * 2^-7 |q||c| = 2.0."""
    q = np.full(128, v, np.float32)
    cents = np.stack([np.full(128, v, np.float32), np.full(128, -v, np.float32)])
    worst, delta = check_bound(q, cents)
    assert worst > 1.9
    assert worst <= delta <= 1.05 * worst


def test_aligned_errors_with_mixed_magnitudes_and_signs():
    rng = np.random.default_rng(7)
    for trial in range(20):
        mag = 2.0 ** rng.integers(-6, 3, 128)
        sign = rng.choice([-1.0, 1.0], 128)
        off = 2 ** -8 - 2 ** -20 if trial % 2 == 0 else 2 ** -8 + 2 ** -20
        q = (sign * mag * (1.0 + off)).astype(np.float32)
        cents = np.stack([q, -q, (sign * (1.0 + off)).astype(np.float32), q * np.float32(3.0)])
        worst, delta = check_bound(q, cents)
        assert worst <= delta, (trial, worst, delta)


@pytest.mark.parametrize("scale", [2.0 ** -20, 1.0, 2.0 ** 20])
def test_random_rows_and_centroids_at_any_scale(scale):
    rng = np.random.default_rng(11)
    q = (rng.standard_normal(128) * scale).astype(np.float32)
    cents = (rng.standard_normal((64, 128)) * scale).astype(np.float32)
    worst, delta = check_bound(q, cents)
    assert worst <= delta


def test_margin_arithmetic():
    # no rounding error in the operands leaves the accumulation terms only
    assert margin(1.0, 0.0, 1.0, 0.0) < 1e-3
    # the operand terms enter through |q - q_b| |c| + |q| |c - c_b|, doubled
    base = margin(1.0, 0.0, 1.0, 0.0)
    assert margin(1.0, 2 ** -9, 1.0, 0.0) - base == pytest.approx(2 * 2 ** -9 * (1 + 2 ** -8), rel=2e-3)
    assert margin(1.0, 0.0, 1.0, 2 ** -9) - base == pytest.approx(2 * 2 ** -9, rel=2e-3)
    # monotone in every argument
    for args in [(2.0, 0.01, 1.0, 0.01), (1.0, 0.02, 1.0, 0.01), (1.0, 0.01, 2.0, 0.01), (1.0, 0.01, 1.0, 0.02)]:
        assert margin(*args) > margin(1.0, 0.01, 1.0, 0.01)
