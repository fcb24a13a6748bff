"""ctypes binding of the C ABI in include/chimera_hip.h (libchimera_hip.so).

Used by the tests and bench.py to drive the HIP path directly. Loading fails
loudly when the library is missing; there is no fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import HIP_LIB

P = C.c_void_p

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_RUNTIME = 2
ERR_HIP = 3
ERR_CAPACITY = 4

EXPORTED = [
    "chimera_create", "chimera_destroy", "chimera_last_error", "chimera_device_count", "chimera_upload_index",
    "chimera_memory_usage", "chimera_search", "chimera_search_device", "chimera_graph_capture",
    "chimera_graph_launch", "chimera_synchronize", "chimera_stream", "chimera_search_trace",
    "chimera_rotate_lut_device", "chimera_probe_device", "chimera_unpack_codes_device",
]


class SearchOptions(C.Structure):
    _fields_ = [("nprobe", C.c_int32), ("k_refine", C.c_int32), ("k_full_bit", C.c_int32),
                ("cagra_itopk_size", C.c_int32), ("num_chunks", C.c_int32)]


class IndexDesc(C.Structure):
    _fields_ = [("num_embeddings", C.c_uint64), ("dimension", C.c_uint64), ("num_clusters", C.c_uint64),
                ("ex_bits", C.c_uint64), ("num_docs", C.c_uint64), ("doc_ptrs", P), ("cluster_pos", P),
                ("clustered_codes", P), ("clustered_factors", P), ("clustered_doc_ids", P),
                ("token_to_cluster_pos", P), ("full_codes", P), ("full_factors", P), ("rotated_centroids", P),
                ("rotator_flips", P)]


class Trace(C.Structure):
    _fields_ = [("rotated", P), ("cb1_sumq", P), ("cbex_sumq", P), ("labels", P), ("candidate_count", P),
                ("candidates", P), ("candidate_scores", P), ("cand_capacity", C.c_int64), ("refined_count", P),
                ("refined_ids", P), ("refined_scores", P), ("fullbit_count", P), ("fullbit_ids", P),
                ("fullbit_scores", P), ("fullbit_capacity", C.c_int64)]


class ChimeraError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not HIP_LIB.exists():
            raise ImportError(f"{HIP_LIB} is missing: run __graft_entry__.build()")
        _lib = C.CDLL(str(HIP_LIB))
        _lib.chimera_last_error.restype = C.c_char_p
        _lib.chimera_destroy.restype = None
    return _lib


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return C.c_void_p(a)
    return a.ctypes.data_as(P)


def check(code: int) -> None:
    if code != OK:
        raise ChimeraError(code, lib().chimera_last_error().decode())


class Context:
    """One chimera_ctx with an uploaded index. `index` is the dict returned by
    chimera._build_index / chimera._read_index."""

    def __init__(self, index: dict, nprobe: int, k_refine: int, k_full_bit: int, num_chunks: int,
                 max_batch: int = 64, device: int = 0, cagra_itopk_size: int = 150):
        L = lib()
        self._ctx = P()
        check(L.chimera_create(C.byref(self._ctx), device))
        self.arrays = {k: (np.ascontiguousarray(v) if isinstance(v, np.ndarray) else v) for k, v in index.items()}
        a = self.arrays
        self.dim = int(a["dimension"])
        self.num_docs = int(a["doc_lens"].size)
        self.desc = IndexDesc(int(a["num_embeddings"]), self.dim, int(a["num_clusters"]), int(a["ex_bits"]),
                              self.num_docs, _ptr(a["doc_ptrs"]), _ptr(a["cluster_pos"]),
                              _ptr(a["clustered_codes"]), _ptr(a["clustered_factors"]),
                              _ptr(a["clustered_doc_ids"]), _ptr(a["token_to_cluster_pos"]),
                              _ptr(a["full_bit_codes"]), _ptr(a["full_bit_factors"]), _ptr(a["rotated_centroids"]),
                              _ptr(a["flips"]))
        self.options = SearchOptions(nprobe, k_refine, k_full_bit, cagra_itopk_size, num_chunks)
        self.max_batch = max_batch
        check(L.chimera_upload_index(self._ctx, C.byref(self.desc), C.byref(self.options), max_batch))

    def close(self) -> None:
        if self._ctx:
            lib().chimera_destroy(self._ctx)
            self._ctx = P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._ctx

    def memory_usage(self) -> int:
        v = C.c_uint64()
        check(lib().chimera_memory_usage(self._ctx, C.byref(v)))
        return v.value

    def search(self, queries: np.ndarray, k: int):
        q = np.ascontiguousarray(queries, dtype=np.float32)
        nq = q.shape[0]
        ids = np.full((nq, k), -1, np.int64)
        scores = np.zeros((nq, k), np.float32)
        counts = np.zeros(nq, np.int32)
        check(lib().chimera_search(self._ctx, _ptr(q), nq, k, _ptr(ids), _ptr(scores), _ptr(counts)))
        return ids, scores, counts

    def search_trace(self, queries: np.ndarray, k: int, cand_capacity: int | None = None) -> dict:
        q = np.ascontiguousarray(queries, dtype=np.float32)
        nq = q.shape[0]
        o = self.options
        ccap = cand_capacity or self.num_docs
        fcap = o.k_refine
        t = {
            "rotated": np.zeros((nq, 32, 128), np.float32), "cb1": np.zeros((nq, 32), np.float32),
            "cbex": np.zeros((nq, 32), np.float32), "labels": np.zeros((nq, 32, o.nprobe), np.uint32),
            "cand_count": np.zeros(nq, np.int32), "candidates": np.zeros((nq, ccap), np.int32),
            "cand_scores": np.zeros((nq, ccap), np.float32), "refined_count": np.zeros(nq, np.int32),
            "refined_ids": np.zeros((nq, o.k_refine), np.int32),
            "refined_scores": np.zeros((nq, o.k_refine), np.float32), "fullbit_count": np.zeros(nq, np.int32),
            "fullbit_ids": np.zeros((nq, fcap), np.int32), "fullbit_scores": np.zeros((nq, fcap), np.float32),
        }
        tr = Trace(_ptr(t["rotated"]), _ptr(t["cb1"]), _ptr(t["cbex"]), _ptr(t["labels"]), _ptr(t["cand_count"]),
                   _ptr(t["candidates"]), _ptr(t["cand_scores"]), ccap, _ptr(t["refined_count"]),
                   _ptr(t["refined_ids"]), _ptr(t["refined_scores"]), _ptr(t["fullbit_count"]),
                   _ptr(t["fullbit_ids"]), _ptr(t["fullbit_scores"]), fcap)
        ids = np.full((nq, k), -1, np.int64)
        scores = np.zeros((nq, k), np.float32)
        counts = np.zeros(nq, np.int32)
        check(lib().chimera_search_trace(self._ctx, _ptr(q), nq, k, _ptr(ids), _ptr(scores), _ptr(counts),
                                         C.byref(tr)))
        t.update(ids=ids, scores=scores, counts=counts)
        return t
