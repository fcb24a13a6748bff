"""ctypes access to the oracle (oracle/liboracle.so) and to the compiled
reference host sources (oracle/_ref/libchimera_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py, never by the product.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libchimera_ref.so"

_c = ctypes
P = _c.c_void_p


class OracleIndex(_c.Structure):
    _fields_ = [("n", _c.c_int64), ("dim", _c.c_int64), ("n_clusters", _c.c_int64), ("ex_bits", _c.c_int64),
                ("num_docs", _c.c_int64), ("doc_ptrs", P), ("cluster_pos", P), ("clustered_codes", P),
                ("clustered_factors", P), ("clustered_doc_ids", P), ("token_to_cluster_pos", P),
                ("full_codes", P), ("full_factors", P), ("rotated_centroids", P), ("flips", P)]


class OracleOptions(_c.Structure):
    _fields_ = [("nprobe", _c.c_int32), ("k_refine", _c.c_int32), ("k_full_bit", _c.c_int32),
                ("num_chunks", _c.c_int32)]


class OracleResult(_c.Structure):
    _fields_ = [("rotated", P), ("cb1", P), ("cbex", P), ("lut", P), ("labels", P), ("cand_count", P),
                ("candidates", P), ("cand_scores", P), ("cand_cap", _c.c_int64), ("refined_count", P),
                ("refined_ids", P), ("refined_scores", P), ("fullbit_count", P), ("fullbit_ids", P),
                ("fullbit_scores", P), ("fullbit_cap", _c.c_int64), ("result_count", P), ("result_ids", P),
                ("result_scores", P)]


def _ptr(a):
    return a.ctypes.data_as(P) if a is not None else None


def ensure_built() -> None:
    """make on the oracle library: a no-op when it is up to date, a rebuild
    when a source is newer (a library built before a change lacks its
    symbols). Without make, an existing library is used as it is."""
    try:
        subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)
    except (OSError, subprocess.CalledProcessError):
        if not LIB.exists():
            raise


_lib = None


def lib():
    global _lib
    if _lib is None:
        ensure_built()
        _lib = _c.CDLL(str(LIB))
        _lib.oracle_search.restype = _c.c_int32
        _lib.oracle_probe_score.restype = _c.c_float
        _lib.oracle_full_bit_score.restype = _c.c_float
        _lib.oracle_one_bit_est.restype = _c.c_float
        _lib.oracle_one_bit_est.argtypes = [P, P, _c.c_float, _c.c_float]
    return _lib


def ref_lib():
    """The compiled reference host sources, or None where they are absent."""
    if not REF_LIB.exists():
        return None
    return _c.CDLL(str(REF_LIB))


class Index:
    """Keeps the numpy arrays of an index (dict from chimera._build_index /
    chimera._read_index) alive behind an OracleIndex struct."""

    def __init__(self, d: dict):
        self.arrays = {k: (np.ascontiguousarray(v) if isinstance(v, np.ndarray) else v) for k, v in d.items()}
        a = self.arrays
        self.num_docs = int(a["doc_lens"].size)
        self.struct = OracleIndex(
            int(a["num_embeddings"]), int(a["dimension"]), int(a["num_clusters"]), int(a["ex_bits"]), self.num_docs,
            _ptr(a["doc_ptrs"]), _ptr(a["cluster_pos"]), _ptr(a["clustered_codes"]), _ptr(a["clustered_factors"]),
            _ptr(a["clustered_doc_ids"]), _ptr(a["token_to_cluster_pos"]), _ptr(a["full_bit_codes"]),
            _ptr(a["full_bit_factors"]), _ptr(a["rotated_centroids"]), _ptr(a["flips"]))


def search(index: Index, query: np.ndarray, nprobe: int, k_refine: int, k_full_bit: int, num_chunks: int,
           k: int, detail: bool = True) -> dict:
    """One query through every stage; returns the intermediate arrays."""
    L = lib()
    q = np.ascontiguousarray(query, dtype=np.float32)
    M = index.num_docs
    out = {
        "rotated": np.zeros((32, 128), np.float32), "cb1": np.zeros(32, np.float32),
        "cbex": np.zeros(32, np.float32), "lut": np.zeros((32, 32, 16), np.float32),
        "labels": np.zeros((32, nprobe), np.uint32), "cand_count": np.zeros(1, np.int32),
        "candidates": np.zeros(M, np.int32), "cand_scores": np.zeros(M, np.float32),
        "refined_count": np.zeros(1, np.int32), "refined_ids": np.zeros(k_refine, np.int32),
        "refined_scores": np.zeros(k_refine, np.float32), "fullbit_count": np.zeros(1, np.int32),
        "fullbit_ids": np.zeros(k_refine, np.int32), "fullbit_scores": np.zeros(k_refine, np.float32),
        "result_count": np.zeros(1, np.int32), "result_ids": np.full(k, -1, np.int64),
        "result_scores": np.zeros(k, np.float32),
    }
    if not detail:
        for key in ("lut", "candidates", "cand_scores"):
            out[key] = None
    r = OracleResult(_ptr(out["rotated"]), _ptr(out["cb1"]), _ptr(out["cbex"]), _ptr(out["lut"]),
                     _ptr(out["labels"]), _ptr(out["cand_count"]), _ptr(out["candidates"]),
                     _ptr(out["cand_scores"]), M, _ptr(out["refined_count"]), _ptr(out["refined_ids"]),
                     _ptr(out["refined_scores"]), _ptr(out["fullbit_count"]), _ptr(out["fullbit_ids"]),
                     _ptr(out["fullbit_scores"]), k_refine, _ptr(out["result_count"]), _ptr(out["result_ids"]),
                     _ptr(out["result_scores"]))
    opt = OracleOptions(nprobe, k_refine, k_full_bit, num_chunks)
    L.oracle_search(_c.byref(index.struct), _ptr(q), _c.byref(opt), k, _c.byref(r))
    c = int(out["cand_count"][0])
    rc = int(out["refined_count"][0])
    fc = int(out["fullbit_count"][0])
    n = int(out["result_count"][0])
    res = dict(out)
    if detail:
        res["candidates"] = out["candidates"][:c]
        res["cand_scores"] = out["cand_scores"][:c]
    res["refined_ids"] = out["refined_ids"][:rc]
    res["refined_scores"] = out["refined_scores"][:rc]
    res["fullbit_ids"] = out["fullbit_ids"][:fc]
    res["fullbit_scores"] = out["fullbit_scores"][:fc]
    res["result_ids"] = out["result_ids"][:n]
    res["result_scores"] = out["result_scores"][:n]
    return res


def search_batch(index: Index, queries: np.ndarray, nprobe: int, k_refine: int, k_full_bit: int,
                 num_chunks: int, k: int):
    """Final results of many queries (OpenMP over queries): ids [Q, k] padded
    with -1, scores, counts."""
    L = lib()
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq = q.shape[0]
    ids = np.full((nq, k), -1, np.int64)
    scores = np.zeros((nq, k), np.float32)
    counts = np.zeros(nq, np.int32)
    opt = OracleOptions(nprobe, k_refine, k_full_bit, num_chunks)
    L.oracle_search_batch(_c.byref(index.struct), _ptr(q), nq, _c.byref(opt), k, _ptr(ids), _ptr(scores),
                          _ptr(counts))
    return ids, scores, counts


def probe(rotated: np.ndarray, centroids: np.ndarray, nprobe: int) -> np.ndarray:
    L = lib()
    r = np.ascontiguousarray(rotated, dtype=np.float32)
    c = np.ascontiguousarray(centroids, dtype=np.float32)
    out = np.zeros((r.shape[0], nprobe), np.uint32)
    L.oracle_probe(_ptr(r), r.shape[0], _ptr(c), _c.c_int64(c.shape[0]), nprobe, _ptr(out))
    return out


def unpack(packed: np.ndarray, width: int) -> np.ndarray:
    L = lib()
    p = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros((p.shape[0], 128), np.uint8)
    for i in range(p.shape[0]):
        L.oracle_unpack(_ptr(p[i]), width, _ptr(out[i]))
    return out


def rotate(x: np.ndarray, flips: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = np.ascontiguousarray(flips, dtype=np.uint8)
    out = np.zeros((x.shape[0], 128), np.float32)
    for i in range(x.shape[0]):
        L.oracle_rotate(_ptr(x[i]), x.shape[1], _ptr(f), _ptr(out[i]))
    return out


def query_state(rotated: np.ndarray, ex_bits: int):
    L = lib()
    r = np.ascontiguousarray(rotated, dtype=np.float32)
    cb1 = np.zeros(r.shape[0], np.float32)
    cbex = np.zeros(r.shape[0], np.float32)
    a, b = _c.c_float(), _c.c_float()
    for i in range(r.shape[0]):
        L.oracle_query_state(_ptr(r[i]), ex_bits, _c.byref(a), _c.byref(b))
        cb1[i], cbex[i] = a.value, b.value
    return cb1, cbex


def lut(rotated: np.ndarray) -> np.ndarray:
    L = lib()
    r = np.ascontiguousarray(rotated, dtype=np.float32)
    out = np.zeros((r.shape[0], 32, 16), np.float32)
    for i in range(r.shape[0]):
        L.oracle_lut(_ptr(r[i]), _ptr(out[i]))
    return out


def full_bit_scores(index: Index, rotated: np.ndarray, cbex: np.ndarray, docs: np.ndarray) -> np.ndarray:
    """SF of docs[q, j] for query q (rotated [Q, 32, 128], cbex [Q, 32])."""
    L = lib()
    r = np.ascontiguousarray(rotated, dtype=np.float32)
    cb = np.ascontiguousarray(cbex, dtype=np.float32)
    d = np.ascontiguousarray(docs, dtype=np.int32)
    out = np.zeros(d.shape, np.float32)
    L.oracle_full_bit_batch(_c.byref(index.struct), _ptr(r), _ptr(cb), d.shape[0], _ptr(d), d.shape[1], _ptr(out))
    return out


def chunk_select(s1: np.ndarray, k_full_bit: int, num_chunks: int) -> np.ndarray:
    """Boolean mask of the refined documents the chunk rule sends to full-bit
    scoring, given their one-bit scores in refined order."""
    L = lib()
    v = np.ascontiguousarray(s1, dtype=np.float32)
    out = np.zeros(v.size, np.uint8)
    L.oracle_chunk_select(_ptr(v), v.size, k_full_bit, num_chunks, _ptr(out))
    return out.astype(bool)


def fullbit_baseline_available() -> bool:
    return bool(lib().cpu_fullbit_avx512_available())


def fullbit_baseline(index: Index, rotated: np.ndarray, cbex: np.ndarray, docs: np.ndarray, counts: np.ndarray,
                     threads: int = 0) -> np.ndarray:
    """The AVX-512 full-bit MaxSim of docs[q, :counts[q]] for query q
    (rotated [Q, 32, 128], cbex [Q, 32]) on `threads` OpenMP threads (0: all):
    the CPU baseline of the scoring stage. Raises where AVX-512 is absent."""
    L = lib()
    r = np.ascontiguousarray(rotated, dtype=np.float32)
    cb = np.ascontiguousarray(cbex, dtype=np.float32)
    d = np.ascontiguousarray(docs, dtype=np.int32)
    c = np.ascontiguousarray(counts, dtype=np.int32)
    out = np.zeros(d.shape, np.float32)
    rc = L.cpu_fullbit_batch(_c.byref(index.struct), _ptr(r), _ptr(cb), d.shape[0], _ptr(d), d.shape[1], _ptr(c),
                             _ptr(out), threads)
    if rc != 0:
        raise RuntimeError("the CPU baseline needs AVX-512 (avx512f/bw/vl/dq)")
    return out
