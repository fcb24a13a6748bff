/*
 * chimera_hip.h - C ABI of the MI355X (gfx950) scoring path.
 *
 * Plain pointers and sizes only. Every function returns CHIMERA_OK (0) or an
 * error code; chimera_last_error() returns the message of the last failure on
 * the calling thread. The C++ class Chimera::chimera_index maps the codes to
 * the reference's exception types (cpp/include/chimera/chimera_index.cuh:34-41
 * check_cuda -> std::runtime_error; option and shape errors ->
 * std::invalid_argument, chimera_index.cu:27-36, search_impl.cu:50-60).
 *
 * One context owns one HIP stream and the device copy of one index. A context
 * is not thread-safe, like one reference chimera_index (its Workspace and
 * streams are shared, chimera_index_internal.cuh:13-49).
 *
 * Functions named *_device take device pointers and run asynchronously on the
 * context's stream; the others take host pointers and return when done.
 */
#ifndef CHIMERA_HIP_H_
#define CHIMERA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHIMERA_OK 0
#define CHIMERA_ERR_INVALID_ARGUMENT 1 /* maps to std::invalid_argument */
#define CHIMERA_ERR_RUNTIME 2          /* maps to std::runtime_error */
#define CHIMERA_ERR_HIP 3              /* a HIP runtime call failed; runtime_error */
#define CHIMERA_ERR_CAPACITY 4         /* a fixed workspace bound was exceeded; runtime_error */

#define CHIMERA_QUERY_LEN 32   /* Q_DOCLEN, config.cuh:8 */
#define CHIMERA_PADDED_DIM 128 /* PADDED_DIM, config.cuh:7 */

typedef struct chimera_ctx chimera_ctx;

/* Mirrors Chimera::SearchOptions (chimera_index.cuh:26-32). */
typedef struct {
    int32_t nprobe;
    int32_t k_refine;
    int32_t k_full_bit;
    int32_t cagra_itopk_size; /* validated, unused: the probe is exact */
    int32_t num_chunks;
} chimera_search_options;

/*
 * Host view of one loaded index: the arrays of the reference's index files
 * (doc_1bit.bin, doc_full.bin, cluster_1bit.bin, ivf.bin, doclens.bin and the
 * rotated centroids), as read by chimera_index::load (chimera_index.cu:54-173).
 */
typedef struct {
    uint64_t num_embeddings; /* N */
    uint64_t dimension;      /* d, 64..128 */
    uint64_t num_clusters;
    uint64_t ex_bits;        /* 1..7, full codes are W = 1 + ex_bits bits */
    uint64_t num_docs;       /* M */
    const int32_t* doc_ptrs;              /* [M + 1] prefix of doc_lens */
    const uint64_t* cluster_pos;          /* [num_clusters + 1] (ivf.bin) */
    const uint8_t* clustered_codes;       /* [N * 16] one-bit codes, cluster order */
    const float* clustered_factors;       /* [N] one-bit factors, cluster order */
    const int32_t* clustered_doc_ids;     /* [N] cluster order */
    const uint32_t* token_to_cluster_pos; /* [N] token order */
    const uint8_t* full_codes;            /* [N * 16 * (1 + ex_bits)] token order */
    const float* full_factors;            /* [N] token order */
    const float* rotated_centroids;       /* [num_clusters * 128] */
    const uint8_t* rotator_flips;         /* [64] FhtKac flip bytes */
} chimera_index_desc;

/* Intermediate results of one batch, copied to host buffers the caller owns.
 * Any pointer may be NULL to skip that stage. Counts are per query. */
typedef struct {
    float* rotated;           /* [nq * 32 * 128] */
    float* cb1_sumq;          /* [nq * 32] */
    float* cbex_sumq;         /* [nq * 32] */
    uint32_t* labels;         /* [nq * 32 * nprobe] probed clusters, nearest first */
    int32_t* candidate_count; /* [nq] |C| */
    int32_t* candidates;      /* [nq * cand_capacity] ascending doc IDs */
    float* candidate_scores;  /* [nq * cand_capacity] S_cand per candidate */
    int64_t cand_capacity;
    int32_t* refined_count;   /* [nq] R = min(k_refine, |C|) */
    int32_t* refined_ids;     /* [nq * k_refine] in S_cand order */
    float* refined_scores;    /* [nq * k_refine] one-bit MaxSim S1 */
    int32_t* fullbit_count;   /* [nq] */
    int32_t* fullbit_ids;     /* [nq * fullbit_capacity] docs scored at full precision */
    float* fullbit_scores;    /* [nq * fullbit_capacity] full-bit MaxSim SF */
    int64_t fullbit_capacity;
} chimera_trace;

/* Replaces chimera_index::begin_initialization and the Workspace streams
 * (chimera_index.cu:42-48, utils.cu:444-449). device is the HIP ordinal. */
int chimera_create(chimera_ctx** out, int device);

/* Replaces chimera_index::release_resources (utils.cu:477-550). NULL-safe. */
void chimera_destroy(chimera_ctx* ctx);

/* Message of the last failure on the calling thread ("" if none). */
const char* chimera_last_error(void);

/* Number of visible HIP devices, or -1 with an error message. */
int chimera_device_count(void);

/* Replaces chimera_index::initialize_search_state, compute_candidate_bounds
 * and allocate_workspace (chimera_index.cu:175-248, utils.cu:217-456): copies
 * the index to HBM, validates options (chimera_index.cu:27-36,94-96) and sizes
 * every workspace for batches of up to max_batch queries. */
int chimera_upload_index(chimera_ctx* ctx, const chimera_index_desc* desc,
                         const chimera_search_options* options, int32_t max_batch);

/* The candidate stage's per-query visit bound that chimera_upload_index
 * sizes its workspace with (the reference sizes the same arrays from the
 * largest clusters, utils.cu:217-264,299-456): 32 x the token count of the
 * nprobe largest clusters of cluster_pos [n_clusters + 1] into *visits.
 * Fails with CHIMERA_ERR_CAPACITY when that exceeds the 32-bit visit
 * offsets (2^31 - 1), and CHIMERA_ERR_RUNTIME for decreasing offsets.
 * Host arithmetic only: no context, no device. */
int chimera_visit_bound(const uint64_t* cluster_pos, uint64_t n_clusters, int32_t nprobe, int64_t* visits);

/* Device bytes held by the context (index + workspace). */
int chimera_memory_usage(chimera_ctx* ctx, uint64_t* bytes);

/* Free and total bytes of device memory on the context's device
 * (hipMemGetInfo). No counterpart in the reference. */
int chimera_device_memory_info(chimera_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes);

/* Batched replacement of chimera_index::search / search_one
 * (search_impl.cu:40-116 and everything it calls, 118-574). queries is
 * [nq, 32, d] fp32 on the host. For query q, out_ids[q*k .. q*k+k) holds the
 * top documents in descending full-bit score (ties: larger ID first,
 * search_impl.cu:409,496-500), padded with -1; out_counts[q] is how many are
 * valid; out_scores may be NULL. */
int chimera_search(chimera_ctx* ctx, const float* queries, int32_t nq, int32_t k,
                   int64_t* out_ids, float* out_scores, int32_t* out_counts);

/* Same, with all pointers in device memory; asynchronous on the context's
 * stream (no host synchronisation inside). */
int chimera_search_device(chimera_ctx* ctx, const float* d_queries, int32_t nq, int32_t k,
                          int64_t* d_out_ids, float* d_out_scores, int32_t* d_out_counts);

/* chimera_search_device without allocating: no counterpart in the reference.
 * It is for callers that cannot allocate device memory around a search
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The per-batch workspace (rotated queries, LUTs, probe labels,
 * visit records, candidate and refined lists, the status word) comes from a
 * static 64 MiB device array that the library holds on each GPU until the
 * process ends, instead of the context's workspace; the matrix-core probe
 * uses the context's probe buffers, allocated at upload like those of
 * chimera_search_device, and the status is copied into a word of the
 * context at the end of the call. Results equal chimera_search_device's. A
 * batch whose workspace exceeds 64 MiB is rejected with CHIMERA_ERR_CAPACITY
 * (the message names the largest batch that fits this index). Every call on
 * one GPU shares that array: calls that overlap on one GPU (any contexts,
 * any streams) race. Asynchronous on the context's stream;
 * chimera_synchronize reports capacity errors. Stage timing
 * (chimera_set_profiling) does not cover these calls. */
int chimera_search_device_noalloc(chimera_ctx* ctx, const float* d_queries, int32_t nq, int32_t k,
                                  int64_t* d_out_ids, float* d_out_scores, int32_t* d_out_counts);

/* Captures chimera_search_device for a fixed (nq, k) and these pointers into a
 * HIP graph owned by the context; chimera_graph_launch replays it. */
int chimera_graph_capture(chimera_ctx* ctx, const float* d_queries, int32_t nq, int32_t k,
                          int64_t* d_out_ids, float* d_out_scores, int32_t* d_out_counts);
int chimera_graph_launch(chimera_ctx* ctx);

/* Waits for all work queued on the context's stream. */
int chimera_synchronize(chimera_ctx* ctx);

/* The context's stream as an opaque handle (a hipStream_t). */
int chimera_stream(chimera_ctx* ctx, void** stream);

/* chimera_search plus intermediate results (for parity checks). */
int chimera_search_trace(chimera_ctx* ctx, const float* queries, int32_t nq, int32_t k,
                         int64_t* out_ids, float* out_scores, int32_t* out_counts,
                         chimera_trace* trace);

/* Scoring arithmetic. mode 0 (default): one-bit and full-bit MaxSim on the
 * matrix cores (split-fp16 query, error ~2^-22 of the largest query
 * component; scores within 2e-5 of the reference's). mode 1: the reference's
 * LUT and fp32 AVX-512 arithmetic, bit for bit (slower, for verification). */
int chimera_set_exact_scoring(chimera_ctx* ctx, int mode);

/* Centroid probe implementation: 0 automatic (the matrix-core probe at every
 * batch size whenever the index allows it: at least nprobe sampled groups
 * of 32-centroid tiles and nprobe <= 1024, else the fp32 vector kernel),
 * 1 the fp32 vector kernel, 2 the same as 0, 3 the matrix-core probe on
 * fp32 operands (v_mfma_f32_32x32x2_f32 filter, a margin without operand
 * rounding, the same exact rerank) where 0 would use bf16 operands. All
 * give the same labels. */
int chimera_set_probe_mode(chimera_ctx* ctx, int mode);

/* Queries per candidate-stage sub-batch (rounded down to a multiple of 8, at
 * least 8, at most what the workspace allocated at upload holds; <= 0
 * restores that). The candidate stage runs in sub-batches when the visit
 * records of a whole batch do not fit the workspace; results do not depend
 * on the size. Applies to searches and graph captures after the call. No
 * counterpart in the reference (its workspace is per query,
 * search_impl.cu:72-116). */
int chimera_set_candidate_batch(chimera_ctx* ctx, int32_t queries);

/* ---- device memory and timing for callers without a HIP runtime of their own ---- */

/* hipMalloc / hipFree on the context's device. */
int chimera_device_alloc(chimera_ctx* ctx, void** ptr, size_t bytes);
int chimera_device_free(chimera_ctx* ctx, void* ptr);
/* Copies on the context's stream; they return when the copy is complete. */
int chimera_copy_to_device(chimera_ctx* ctx, void* d_dst, const void* src, size_t bytes);
int chimera_copy_to_host(chimera_ctx* ctx, void* dst, const void* d_src, size_t bytes);

/* Per-stage HIP-event timing on the context's stream. While enabled, every
 * eager chimera_search* call records events around each kernel launch and
 * accumulates its duration; chimera_stage_times returns, for each of the
 * CHIMERA_STAGES stages, total milliseconds and launch counts since the last
 * reset (enable=1 resets). Graph replays are not timed per stage. */
#define CHIMERA_STAGES 15
/* stage ids: 0 rotate+LUT, 1 probe sampled pass + threshold, 2 probe
 * filtered pass (the whole exact probe when the matrix-core probe is not
 * used), 3 probe rerank, 4 visit count, 5 visit offsets, 6 visit records
 * (one-bit estimates), 7 candidate reduce (S_cand), 8 refine select,
 * 9 one-bit refine, 10 chunk select, 11 full-bit, 12 final top-k;
 * 13 MaxSim rescoring and 14 its top-k (chimera_maxsim_rescore_device) */
int chimera_set_profiling(chimera_ctx* ctx, int enable);
int chimera_stage_times(chimera_ctx* ctx, double* ms, int64_t* launches);

/* Wall time of `iters` replays of the captured graph, bracketed by HIP
 * events on the context's stream; *ms is the total. */
int chimera_graph_time(chimera_ctx* ctx, int32_t iters, float* ms);

/* ---- index build on the device ---- */

/* Writable host buffers for chimera_download_index, in the layout of the
 * index files (build_index.cu:503-557). Any pointer may be NULL to skip that
 * array. */
typedef struct {
    uint64_t* cluster_pos;          /* [num_clusters + 1] (ivf.bin) */
    uint32_t* inv_list;             /* [N] cluster position -> token (ivf.bin) */
    uint32_t* token_to_cluster_pos; /* [N] token order */
    uint8_t* one_bit_codes;         /* [N * 16] token order (doc_1bit.bin) */
    float* one_bit_factors;         /* [N] token order */
    uint8_t* full_codes;            /* [N * 16 * (1 + ex_bits)] token order (doc_full.bin) */
    float* full_factors;            /* [N] token order */
    uint8_t* clustered_codes;       /* [N * 16] cluster order (cluster_1bit.bin) */
    float* clustered_factors;       /* [N] */
    int32_t* clustered_doc_ids;     /* [N] */
    float* rotated_centroids;       /* [num_clusters * 128] (centroids.carga) */
} chimera_index_host;

/* Builds an index from device-resident embeddings [N, dimension] (fp32,
 * row-major) straight into the context, ready to search: replaces
 * chimera_index::build (build_index.cu:394-501) after centroid sampling.
 * centroid_ids [num_clusters] are the sampled token ids
 * (sample_centroids, build_index.cu:159-184) and rotator_flips the 64
 * FhtKac flip bytes (rotator.hpp:183-189), both computed on the host. The
 * assignment is the exact nearest centroid (|c|^2 - 2<x,c>, fp32, ties to
 * the lower id) in place of the CAGRA search of assign_embeddings
 * (build_index.cu:186-219); encoding follows quantization.cpp:32-193 and the
 * layout ivf_pg.cpp:110-126 and build_index.cu:328-363. Errors and messages
 * of validate_build_inputs (build_index.cu:75-126); a zero or non-finite
 * embedding is rejected with CHIMERA_ERR_INVALID_ARGUMENT. Returns when the
 * build is complete. */
int chimera_build_index_device(chimera_ctx* ctx, const float* d_embeddings, uint64_t num_embeddings,
                               uint64_t dimension, const int32_t* doc_lens, uint64_t num_docs,
                               uint64_t num_clusters, uint64_t ex_bits, const int64_t* centroid_ids,
                               const uint8_t* rotator_flips, const chimera_search_options* opt,
                               int32_t max_batch);

/* Copies the index arrays of the context to host memory (the data that
 * chimera_index::save writes, build_index.cu:503-557). inv_list and
 * token_to_cluster_pos are available for indexes built on the device. */
int chimera_download_index(chimera_ctx* ctx, chimera_index_host* out);

/* ---- single-stage entry points on device pointers (parity tests) ---- */

/* Rotation, QueryState and one-bit LUT for nq queries: replaces the host
 * FhtKacRotator::rotate loop and QueryState (search_impl.cu:73-82,
 * rotator.hpp:281-334, chimera_index_internal.cuh:51-65) and
 * precompute_one_bit_lut_kernel (kernels.cu:402-428). d_lut is laid out
 * [nq][32 query tokens][32 chunks][16 entries], the reference's order; any
 * output may be NULL. */
int chimera_rotate_lut_device(chimera_ctx* ctx, const float* d_queries, int32_t nq,
                              float* d_rotated, float* d_cb1_sumq, float* d_cbex_sumq,
                              float* d_lut);

/* Exact centroid probe replacing IVF_PG::search_centroids / cuVS CAGRA
 * (ivf_pg.cpp:37-65): for each of nrows rotated query vectors, the nprobe
 * centroids of the uploaded index with the smallest |c|^2 - 2<q,c> (fp32,
 * ties to the lower ID), nearest first. */
int chimera_probe_device(chimera_ctx* ctx, const float* d_rotated, int32_t nrows, int32_t nprobe,
                         uint32_t* d_labels);

/* Error bound of the matrix-core probe, which replaces the approximate
 * CAGRA search of ivf_pg.cpp:37-65 with an exact one: for a rotated query row
 * q with qn = |q|, eq = |q - bf16(q)| and centroids with cmax >= max |c|,
 * ecmax >= max |c - bf16(c)| (bf16 by round-to-nearest-even), the returned
 * delta bounds |d' - d| for every centroid, where d = |c|^2 - 2<q,c> is the
 * exact fp32 score and d' the score of the bf16 operands accumulated in fp32.
 * The probe keeps the centroids with d' <= thr (thr = U + 2 delta, U an
 * estimate of the d' of rank 2 nprobe from a sample of the centroids),
 * checks that nprobe of them have d' <= thr - 2 delta (which puts every
 * exact top-nprobe centroid among them) and rescores those near the
 * nprobe-th in fp32, so its labels equal the exact probe's; a row that fails
 * the check is recomputed by the exact kernel. Pure arithmetic: no context,
 * no device. */
float chimera_probe_margin(float qn, float eq, float cmax, float ecmax);

/* The cmax and ecmax the context's matrix-core probe uses (ecmax is 0 when
 * the matrix-core probe is not set up for the index). */
int chimera_probe_bounds(chimera_ctx* ctx, float* cmax, float* ecmax);

/* Per-row candidate counts of the last matrix-core probe on the context
 * (after a search or chimera_probe_device that used it): candidates[r] is
 * the number of centroids of row r that passed d' <= thr, 0xFFFFFFFF when
 * the row's candidate sub-lists overflowed or it had more candidates than
 * the rerank holds (8 nprobe rounded up to a power of two in [1024, 2048]),
 * or 0xFFFFFFFE when fewer than nprobe candidates had d' <= thr - 2 delta
 * (the threshold estimate was too low). Those rows are recomputed by the
 * exact kernel. No counterpart in the reference (its CAGRA probe keeps no
 * such count). */
int chimera_probe_stats(chimera_ctx* ctx, int32_t nrows, uint32_t* candidates);

/* Unpacks n packed W-bit codes of 128 dimensions into bytes, the integers
 * the reference's unpack_fxu{W} functions convert (space.hpp:604-801). */
int chimera_unpack_codes_device(chimera_ctx* ctx, int32_t width, const uint8_t* d_packed,
                                int64_t n, uint8_t* d_raw);

#ifdef __cplusplus
}
#endif

#endif /* CHIMERA_HIP_H_ */
