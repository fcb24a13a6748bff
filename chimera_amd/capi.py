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
    "chimera_device_alloc", "chimera_device_free", "chimera_copy_to_device", "chimera_copy_to_host",
    "chimera_set_profiling", "chimera_stage_times", "chimera_graph_time", "chimera_set_exact_scoring",
    "chimera_set_probe_mode", "chimera_set_candidate_batch", "chimera_build_index_device", "chimera_download_index",
    "chimera_probe_margin", "chimera_probe_bounds", "chimera_probe_stats", "chimera_visit_bound",
    "chimera_search_device_noalloc", "chimera_device_memory_info",
    # include/chimera_workload.h
    "chimera_synth_tokens_device", "chimera_gather_rows_device", "chimera_exact_maxsim_device",
    "chimera_maxsim_rescore_device", "chimera_matrix_core_rate",
]

# chimera_matrix_core_rate kinds: instruction and operands
MATRIX_CORE_KINDS = {"bf16_32x32x16": 0, "f16_16x16x32": 1, "f16_16x16x32_bits": 2, "f32_32x32x2": 3,
                     "i8_32x32x32": 4, "f16_16x16x32_bits_valu4": 5}

STAGES = ["rotate_lut", "probe_sample", "probe_scan", "probe_rerank", "count", "offsets", "emit", "reduce",
          "select_refine", "refine", "chunk_select", "fullbit", "topk", "rescore", "rescore_topk"]


class SearchOptions(C.Structure):
    _fields_ = [("nprobe", C.c_int32), ("k_refine", C.c_int32), ("k_full_bit", C.c_int32),
                ("cagra_itopk_size", C.c_int32), ("num_chunks", C.c_int32)]


class IndexDesc(C.Structure):
    _fields_ = [("num_embeddings", C.c_uint64), ("dimension", C.c_uint64), ("num_clusters", C.c_uint64),
                ("ex_bits", C.c_uint64), ("num_docs", C.c_uint64), ("doc_ptrs", P), ("cluster_pos", P),
                ("clustered_codes", P), ("clustered_factors", P), ("clustered_doc_ids", P),
                ("token_to_cluster_pos", P), ("full_codes", P), ("full_factors", P), ("rotated_centroids", P),
                ("rotator_flips", P)]


class IndexHost(C.Structure):
    _fields_ = [("cluster_pos", P), ("inv_list", P), ("token_to_cluster_pos", P), ("one_bit_codes", P),
                ("one_bit_factors", P), ("full_codes", P), ("full_factors", P), ("clustered_codes", P),
                ("clustered_factors", P), ("clustered_doc_ids", P), ("rotated_centroids", P)]


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


def visit_bound(cluster_pos: np.ndarray, nprobe: int) -> int:
    """Per-query candidate visit bound of an index's IVF offsets
    (chimera_visit_bound; raises ChimeraError past the 32-bit offsets)."""
    cp = np.ascontiguousarray(cluster_pos, np.uint64)
    if cp.ndim != 1 or cp.size == 0:
        raise ValueError("cluster_pos must hold n_clusters + 1 offsets")
    v = C.c_int64()
    check(lib().chimera_visit_bound(_ptr(cp), C.c_uint64(cp.size - 1), nprobe, C.byref(v)))
    return v.value


class Context:
    """One chimera_ctx. `index` is the dict returned by chimera._build_index /
    chimera._read_index and is uploaded at once; with index=None the context
    stays empty until build() builds an index on the device."""

    def __init__(self, index: dict | None, nprobe: int, k_refine: int, k_full_bit: int, num_chunks: int,
                 max_batch: int = 64, device: int = 0, cagra_itopk_size: int = 150, exact: bool = False):
        L = lib()
        self._ctx = P()
        check(L.chimera_create(C.byref(self._ctx), device))
        self.options = SearchOptions(nprobe, k_refine, k_full_bit, cagra_itopk_size, num_chunks)
        self.max_batch = max_batch
        self.arrays = None
        if index is not None:
            self.arrays = {k: (np.ascontiguousarray(v) if isinstance(v, np.ndarray) else v)
                           for k, v in index.items()}
            a = self.arrays
            self._set_shape(int(a["num_embeddings"]), int(a["dimension"]), int(a["num_clusters"]),
                            int(a["ex_bits"]), a["doc_lens"])
            self.desc = IndexDesc(self.n, self.dim, self.n_clusters, self.ex_bits, self.num_docs,
                                  _ptr(a["doc_ptrs"]), _ptr(a["cluster_pos"]), _ptr(a["clustered_codes"]),
                                  _ptr(a["clustered_factors"]), _ptr(a["clustered_doc_ids"]),
                                  _ptr(a["token_to_cluster_pos"]), _ptr(a["full_bit_codes"]),
                                  _ptr(a["full_bit_factors"]), _ptr(a["rotated_centroids"]), _ptr(a["flips"]))
            check(L.chimera_upload_index(self._ctx, C.byref(self.desc), C.byref(self.options), max_batch))
        if exact:
            self.set_exact_scoring(True)

    def _set_shape(self, n, dim, n_clusters, ex_bits, doc_lens) -> None:
        self.n, self.dim, self.n_clusters, self.ex_bits = n, dim, n_clusters, ex_bits
        self.doc_lens = np.ascontiguousarray(doc_lens, np.int32)
        self.num_docs = int(self.doc_lens.size)

    def build(self, embeddings, doc_lens, n_clusters: int, ex_bits: int, centroid_ids=None, flips=None) -> None:
        """Builds the index on the device (chimera_build_index_device) from
        embeddings [N, d]: a numpy array or a DeviceArray already resident.
        Centroid ids and flip bytes default to the reference's seeded
        reservoir sample and rotator (seed 42)."""
        lens = np.ascontiguousarray(doc_lens, np.int32)
        own = None
        if isinstance(embeddings, DeviceArray):
            d_emb = embeddings
        else:
            own = d_emb = self.to_device(np.ascontiguousarray(embeddings, np.float32))
        n, dim = d_emb.shape
        if centroid_ids is None or flips is None:
            from . import load_module
            mod = load_module()
            if centroid_ids is None:
                centroid_ids = np.asarray(mod._sample_centroid_ids(n, n_clusters), np.int64)
            if flips is None:
                flips = mod._rotator_flips(42, dim)
        ids = np.ascontiguousarray(centroid_ids, np.int64)
        fl = np.ascontiguousarray(flips, np.uint8)
        try:
            check(lib().chimera_build_index_device(self._ctx, P(d_emb.ptr), C.c_uint64(n), C.c_uint64(dim),
                                                   _ptr(lens), C.c_uint64(lens.size), C.c_uint64(n_clusters),
                                                   C.c_uint64(ex_bits), _ptr(ids), _ptr(fl), C.byref(self.options),
                                                   self.max_batch))
        finally:
            if own is not None:
                own.free()
        self._set_shape(n, dim, n_clusters, ex_bits, lens)
        self.flips = fl.copy()

    def download(self, fields=None) -> dict:
        """The index arrays, in the form of chimera._build_index's dict
        (only `fields` of the device arrays when given)."""
        n, K, W = self.n, self.n_clusters, 1 + self.ex_bits
        out = {
            "cluster_pos": np.zeros(K + 1, np.uint64), "inv_list": np.zeros(n, np.uint32),
            "token_to_cluster_pos": np.zeros(n, np.uint32), "one_bit_codes": np.zeros(2 * n, np.uint64),
            "one_bit_factors": np.zeros(n, np.float32), "full_bit_codes": np.zeros(n * 16 * W, np.uint8),
            "full_bit_factors": np.zeros(n, np.float32), "clustered_codes": np.zeros(n * 16, np.uint8),
            "clustered_factors": np.zeros(n, np.float32), "clustered_doc_ids": np.zeros(n, np.int32),
            "rotated_centroids": np.zeros(K * 128, np.float32),
        } if fields is None else {}
        if fields is not None:
            shapes = {"cluster_pos": (K + 1, np.uint64), "inv_list": (n, np.uint32),
                      "token_to_cluster_pos": (n, np.uint32), "one_bit_codes": (2 * n, np.uint64),
                      "one_bit_factors": (n, np.float32), "full_bit_codes": (n * 16 * W, np.uint8),
                      "full_bit_factors": (n, np.float32), "clustered_codes": (n * 16, np.uint8),
                      "clustered_factors": (n, np.float32), "clustered_doc_ids": (n, np.int32),
                      "rotated_centroids": (K * 128, np.float32)}
            out = {f: np.zeros(shapes[f][0], shapes[f][1]) for f in fields}
        h = IndexHost(*(_ptr(out.get(f)) for f in ("cluster_pos", "inv_list", "token_to_cluster_pos", "one_bit_codes",
                                               "one_bit_factors", "full_bit_codes", "full_bit_factors",
                                               "clustered_codes", "clustered_factors", "clustered_doc_ids",
                                               "rotated_centroids")))
        check(lib().chimera_download_index(self._ctx, C.byref(h)))
        out.update(num_embeddings=n, dimension=self.dim, num_clusters=K, ex_bits=self.ex_bits,
                   flips=getattr(self, "flips", None) if self.arrays is None else self.arrays["flips"],
                   doc_lens=self.doc_lens,
                   doc_ptrs=np.concatenate([[0], np.cumsum(self.doc_lens, dtype=np.int64)]).astype(np.int32))
        return out

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

    def device_memory_info(self) -> tuple[int, int]:
        """(free, total) bytes of device memory on the context's device."""
        f, t = C.c_uint64(), C.c_uint64()
        check(lib().chimera_device_memory_info(self._ctx, C.byref(f), C.byref(t)))
        return f.value, t.value

    # ---- device memory owned by this context's device ----
    def alloc(self, nbytes: int) -> int:
        p = P()
        check(lib().chimera_device_alloc(self._ctx, C.byref(p), C.c_size_t(nbytes)))
        return p.value

    def free(self, ptr: int) -> None:
        check(lib().chimera_device_free(self._ctx, P(ptr)))

    def to_device(self, arr: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(arr)
        d = DeviceArray(self, a.shape, a.dtype)
        check(lib().chimera_copy_to_device(self._ctx, P(d.ptr), _ptr(a), C.c_size_t(a.nbytes)))
        return d

    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)

    def probe_bounds(self) -> tuple[float, float]:
        """(cmax, ecmax) of the matrix-core probe's error margin."""
        cm, ec = C.c_float(), C.c_float()
        check(lib().chimera_probe_bounds(self._ctx, C.byref(cm), C.byref(ec)))
        return cm.value, ec.value

    def probe_stats(self, nrows: int) -> np.ndarray:
        """Filtered candidates per row of the last matrix-core probe
        (0xFFFFFFFF: the row overflowed, 0xFFFFFFFE: its threshold estimate
        failed the rerank's check; both were recomputed exactly)."""
        out = np.zeros(nrows, np.uint32)
        check(lib().chimera_probe_stats(self._ctx, nrows, _ptr(out)))
        return out

    def set_probe_mode(self, mode: int) -> None:
        check(lib().chimera_set_probe_mode(self._ctx, mode))

    def set_candidate_batch(self, queries: int) -> None:
        check(lib().chimera_set_candidate_batch(self._ctx, queries))

    def set_exact_scoring(self, exact: bool) -> None:
        check(lib().chimera_set_exact_scoring(self._ctx, 1 if exact else 0))

    def synchronize(self) -> None:
        check(lib().chimera_synchronize(self._ctx))

    def set_profiling(self, enable: bool) -> None:
        check(lib().chimera_set_profiling(self._ctx, 1 if enable else 0))

    def stage_times(self) -> dict:
        ms = np.zeros(len(STAGES), np.float64)
        n = np.zeros(len(STAGES), np.int64)
        check(lib().chimera_stage_times(self._ctx, _ptr(ms), _ptr(n)))
        return {name: (float(ms[i]), int(n[i])) for i, name in enumerate(STAGES)}

    def search_device(self, d_queries: "DeviceArray", nq: int, k: int, d_ids: "DeviceArray",
                      d_scores: "DeviceArray", d_counts: "DeviceArray") -> None:
        check(lib().chimera_search_device(self._ctx, P(d_queries.ptr), nq, k, P(d_ids.ptr), P(d_scores.ptr),
                                          P(d_counts.ptr)))

    def search_device_noalloc(self, d_queries: "DeviceArray", nq: int, k: int, d_ids: "DeviceArray",
                              d_scores: "DeviceArray", d_counts: "DeviceArray") -> None:
        """chimera_search_device_noalloc: the same search on the library's
        static device workspace (no allocation)."""
        check(lib().chimera_search_device_noalloc(self._ctx, P(d_queries.ptr), nq, k, P(d_ids.ptr),
                                                  P(d_scores.ptr), P(d_counts.ptr)))

    def graph_capture(self, d_queries, nq, k, d_ids, d_scores, d_counts) -> None:
        check(lib().chimera_graph_capture(self._ctx, P(d_queries.ptr), nq, k, P(d_ids.ptr), P(d_scores.ptr),
                                          P(d_counts.ptr)))

    def graph_launch(self) -> None:
        check(lib().chimera_graph_launch(self._ctx))

    def graph_time(self, iters: int) -> float:
        ms = C.c_float()
        check(lib().chimera_graph_time(self._ctx, iters, C.byref(ms)))
        return ms.value

    # ---- workload generation and ground truth (include/chimera_workload.h) ----
    def synth_tokens(self, d_centres: "DeviceArray", n: int, sigma: float, seed: int) -> "DeviceArray":
        """n mixture tokens [n, 128] on the device (Philox-seeded)."""
        out = DeviceArray(self, (n, 128), np.float32)
        try:
            check(lib().chimera_synth_tokens_device(self._ctx, P(d_centres.ptr), C.c_int64(d_centres.shape[0]), 128,
                                                    C.c_uint64(n), C.c_float(sigma), C.c_uint64(seed), P(out.ptr)))
        except Exception:
            out.free()
            raise
        return out

    def gather_rows(self, d_src: "DeviceArray", ids: np.ndarray) -> np.ndarray:
        """Host copy of rows ids of a device matrix [*, dim], padded to 128."""
        ids = np.ascontiguousarray(ids, np.int64).reshape(-1)
        d_ids = self.to_device(ids)
        out = DeviceArray(self, (ids.size, 128), np.float32)
        try:
            check(lib().chimera_gather_rows_device(self._ctx, P(d_src.ptr), d_src.shape[1], P(d_ids.ptr),
                                                   C.c_int64(ids.size), P(out.ptr)))
            return out.numpy()
        finally:
            out.free()
            d_ids.free()

    def exact_maxsim(self, d_emb: "DeviceArray", d_doc_ptrs: "DeviceArray", queries: np.ndarray) -> np.ndarray:
        """Exact MaxSim scores [nq, num_docs] of host queries [nq, 32, 128]
        against a device corpus."""
        q = np.ascontiguousarray(queries, np.float32)
        nq = q.shape[0]
        m = d_doc_ptrs.shape[0] - 1
        d_q = self.to_device(q)
        d_s = DeviceArray(self, (nq, m), np.float32)
        try:
            check(lib().chimera_exact_maxsim_device(self._ctx, P(d_emb.ptr), P(d_doc_ptrs.ptr), C.c_int64(m),
                                                    P(d_q.ptr), nq, P(d_s.ptr)))
            return d_s.numpy()
        finally:
            d_s.free()
            d_q.free()

    def matrix_core_rate(self, kind: str, iters: int = 20000) -> float:
        """ops/s of one matrix-core instruction type with register operands
        on the context's device (synchronous); kind is a key of
        MATRIX_CORE_KINDS."""
        ops = C.c_double()
        check(lib().chimera_matrix_core_rate(self._ctx, MATRIX_CORE_KINDS[kind], iters, C.byref(ops)))
        return ops.value

    def maxsim_rescore_device(self, d_emb: "DeviceArray", d_doc_ptrs: "DeviceArray", d_queries: "DeviceArray",
                              d_cand_ids: "DeviceArray", d_cand_counts: "DeviceArray", k: int,
                              d_cand_scores: "DeviceArray", d_top_ids: "DeviceArray | None" = None,
                              d_top_scores: "DeviceArray | None" = None,
                              d_top_counts: "DeviceArray | None" = None) -> None:
        """chimera_maxsim_rescore_device on device buffers (asynchronous):
        candidate ids [nq, cap] int32, counts [nq] int32, scores [nq, cap]."""
        nq, cap = d_cand_ids.shape
        m = d_doc_ptrs.shape[0] - 1
        ptr = lambda a: None if a is None else P(a.ptr)
        check(lib().chimera_maxsim_rescore_device(
            self._ctx, P(d_emb.ptr), P(d_doc_ptrs.ptr), C.c_int64(m), P(d_queries.ptr), nq, P(d_cand_ids.ptr),
            P(d_cand_counts.ptr), cap, k, P(d_cand_scores.ptr), ptr(d_top_ids), ptr(d_top_scores),
            ptr(d_top_counts)))

    def maxsim_rescore(self, d_emb: "DeviceArray", d_doc_ptrs: "DeviceArray", queries: np.ndarray,
                       cand_ids: np.ndarray, cand_counts: np.ndarray, k: int):
        """Host wrapper: (candidate scores [nq, cap], top ids [nq, k],
        top scores [nq, k], top counts [nq])."""
        q = np.ascontiguousarray(queries, np.float32)
        ids = np.ascontiguousarray(cand_ids, np.int32)
        nq, cap = ids.shape
        bufs = [self.to_device(q), self.to_device(ids), self.to_device(np.ascontiguousarray(cand_counts, np.int32)),
                DeviceArray(self, (nq, cap), np.float32), DeviceArray(self, (nq, max(k, 1)), np.int64),
                DeviceArray(self, (nq, max(k, 1)), np.float32), DeviceArray(self, (nq,), np.int32)]
        try:
            d_q, d_ids, d_cnt, d_sc, d_tid, d_tsc, d_tcnt = bufs
            self.maxsim_rescore_device(d_emb, d_doc_ptrs, d_q, d_ids, d_cnt, k, d_sc, d_tid, d_tsc, d_tcnt)
            return d_sc.numpy(), d_tid.numpy()[:, :k], d_tsc.numpy()[:, :k], d_tcnt.numpy()
        finally:
            for b in bufs:
                b.free()

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


class DeviceArray:
    """A device allocation made through the C ABI (no other HIP runtime is
    loaded into the process)."""

    def __init__(self, ctx: Context, shape, dtype):
        self.ctx = ctx
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = ctx.alloc(self.nbytes)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().chimera_copy_to_host(self.ctx.handle, _ptr(out), P(self.ptr), C.c_size_t(self.nbytes)))
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx.free(self.ptr)
            self.ptr = 0
