"""Seeded synthetic workloads (Gaussian mixtures on the unit sphere).

Token = centre[uniform] + sigma * N(0, I), L2-normalised. A query picks a
random target document, samples 32 of its tokens with replacement, adds
N(0, query_sigma^2) noise and re-normalises. Document lengths are uniform
integers or a clipped log-normal.

The generator is numpy-only and draws in chunks so that large corpora do not
need a float64 copy; `generate_torch` produces the same distribution directly
on a GPU for the large configurations.
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


def exact_maxsim_topk(embeddings: np.ndarray, doc_lens: np.ndarray, queries: np.ndarray, k: int,
                      device: str = "cpu", block: int = 1 << 18):
    """Brute-force MaxSim ground truth: score(d) = sum_i max_t <q_i, o_t>.

    fp32 products accumulated by torch (fp32 on CPU or GPU); returns
    (ids [Q, k] int64 ordered by descending score, scores [Q, M] float64).
    """
    import torch

    dev = torch.device(device)
    emb = torch.from_numpy(embeddings)
    lens = torch.from_numpy(doc_lens.astype(np.int64))
    doc_of = torch.repeat_interleave(torch.arange(lens.numel()), lens).to(dev)
    qs = torch.from_numpy(queries).to(dev)
    nq, ql, dim = qs.shape
    m = lens.numel()
    best = torch.full((nq * ql, m), float("-inf"), dtype=torch.float32, device=dev)
    qf = qs.reshape(nq * ql, dim)
    for s in range(0, emb.shape[0], block):
        e = min(emb.shape[0], s + block)
        sims = qf @ emb[s:e].to(dev).T                    # [Q*32, b]
        idx = doc_of[s:e].unsqueeze(0).expand(nq * ql, -1)
        best.scatter_reduce_(1, idx, sims, reduce="amax", include_self=True)
    scores = best.reshape(nq, ql, m).to(torch.float64).sum(1)
    top = torch.topk(scores, k, dim=1).indices
    return top.cpu().numpy(), scores.cpu().numpy()


def recall_at_k(gt: np.ndarray, got: list, k: int) -> float:
    """compute_recall (apps/utils.cpp:265-290): |top-k ∩ gt[:k]| / (nq * k)."""
    hits = 0
    for g, r in zip(gt, got):
        s = set(list(r)[:k])
        hits += sum(1 for x in list(g)[:k] if x in s)
    return hits / (len(got) * k)
