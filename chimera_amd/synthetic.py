"""Seeded synthetic workloads (Gaussian mixtures on the unit sphere).

Token = centre[uniform] + sigma * N(0, I), L2-normalised. A query picks a
random target document, samples 32 of its tokens with replacement, adds
N(0, query_sigma^2) noise and re-normalises. Document lengths are uniform
integers or a clipped log-normal.

The generator is numpy-only and draws in chunks so that large corpora do not
need a float64 copy.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Workload:
    embeddings: np.ndarray   # float32 [N, D]
    doc_lens: np.ndarray     # int32 [M]
    queries: np.ndarray      # float32 [Q, 32, D]
    targets: np.ndarray      # int64 [Q] target document of each query


def unit_centres(rng: np.random.Generator, k: int, dim: int) -> np.ndarray:
    c = rng.standard_normal((k, dim), dtype=np.float32)
    c /= np.linalg.norm(c, axis=1, keepdims=True)
    return c


def doc_lengths(rng: np.random.Generator, m: int, kind: str = "uniform", lo: int = 16, hi: int = 160,
                median: float = 64.0, sigma: float = 0.5) -> np.ndarray:
    if kind == "uniform":
        return rng.integers(lo, hi + 1, size=m).astype(np.int32)
    if kind == "lognormal":
        v = np.exp(np.log(median) + sigma * rng.standard_normal(m))
        return np.clip(np.rint(v), lo, hi).astype(np.int32)
    raise ValueError(kind)


def mixture_tokens(rng: np.random.Generator, centres: np.ndarray, n: int, sigma: float,
                   chunk: int = 1 << 20) -> np.ndarray:
    dim = centres.shape[1]
    out = np.empty((n, dim), dtype=np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        lab = rng.integers(0, centres.shape[0], size=e - s)
        x = centres[lab] + np.float32(sigma) * rng.standard_normal((e - s, dim), dtype=np.float32)
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        out[s:e] = x
    return out


def make_queries(rng: np.random.Generator, embeddings: np.ndarray, doc_lens: np.ndarray, nq: int,
                 sigma: float = 0.1, qlen: int = 32) -> tuple[np.ndarray, np.ndarray]:
    ptrs = np.concatenate([[0], np.cumsum(doc_lens, dtype=np.int64)])
    targets = rng.integers(0, doc_lens.size, size=nq)
    dim = embeddings.shape[1]
    q = np.empty((nq, qlen, dim), dtype=np.float32)
    for i, t in enumerate(targets):
        pick = rng.integers(ptrs[t], ptrs[t + 1], size=qlen)
        v = embeddings[pick] + np.float32(sigma) * rng.standard_normal((qlen, dim), dtype=np.float32)
        v /= np.linalg.norm(v, axis=1, keepdims=True)
        q[i] = v
    return q, targets.astype(np.int64)


def generate(num_docs: int, num_centres: int, sigma: float, nq: int, seed: int, dim: int = 128,
             len_kind: str = "uniform", len_lo: int = 16, len_hi: int = 160, query_sigma: float = 0.1) -> Workload:
    rng = np.random.default_rng(seed)
    centres = unit_centres(rng, num_centres, dim)
    lens = doc_lengths(rng, num_docs, len_kind, len_lo, len_hi)
    emb = mixture_tokens(rng, centres, int(lens.sum()), sigma)
    q, t = make_queries(rng, emb, lens, nq, query_sigma)
    return Workload(emb, lens, q, t)


def exact_maxsim_scores(embeddings: np.ndarray, doc_lens: np.ndarray, queries: np.ndarray,
                        chunk_tokens: int = 1 << 17) -> np.ndarray:
    """Brute-force MaxSim: score[q, d] = sum_i max_{t in d} <q_i, o_t>.

    fp32 dot products (BLAS), per-document max over token ranges, sum over the
    query tokens in float64. Returns float64 [Q, M]."""
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq, ql, dim = q.shape
    qf = q.reshape(nq * ql, dim)
    ptrs = np.concatenate([[0], np.cumsum(doc_lens, dtype=np.int64)])
    m = doc_lens.size
    best = np.empty((nq * ql, m), dtype=np.float32)
    d0 = 0
    while d0 < m:
        # whole documents per chunk
        d1 = int(np.searchsorted(ptrs, ptrs[d0] + chunk_tokens, side="right")) - 1
        d1 = max(d1, d0 + 1)
        d1 = min(d1, m)
        t0, t1 = ptrs[d0], ptrs[d1]
        sims = qf @ embeddings[t0:t1].T
        best[:, d0:d1] = np.maximum.reduceat(sims, (ptrs[d0:d1] - t0).astype(np.int64), axis=1)
        d0 = d1
    return best.reshape(nq, ql, m).astype(np.float64).sum(1)


def exact_maxsim_topk(embeddings: np.ndarray, doc_lens: np.ndarray, queries: np.ndarray, k: int):
    """Top-k documents by exact MaxSim (ties to the lower doc ID):
    (ids [Q, k] int64, scores [Q, M] float64)."""
    scores = exact_maxsim_scores(embeddings, doc_lens, queries)
    ids = np.argsort(-scores, axis=1, kind="stable")[:, :k]
    return ids, scores


def recall_at_k(gt: np.ndarray, got: list, k: int) -> float:
    """compute_recall (apps/utils.cpp:265-290): |top-k ∩ gt[:k]| / (nq * k)."""
    hits = 0
    for g, r in zip(gt, got):
        s = set(list(r)[:k])
        hits += sum(1 for x in list(g)[:k] if x in s)
    return hits / (len(got) * k)
