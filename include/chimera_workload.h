/*
 * chimera_workload.h - synthetic corpora and exact MaxSim ground truth on the
 * device, for benchmarks and recall measurement at corpus sizes the host
 * cannot generate or brute-force in reasonable time.
 *
 * These entry points have no counterpart in the reference's scoring path:
 * the reference's apps generate nothing (they read embeddings from files,
 * cpp/apps/utils.cpp) and compute recall against supplied ground truth
 * (cpp/apps/utils.cpp:265-290). Same conventions as chimera_hip.h: a status
 * code per call, chimera_last_error() for the message, device pointers,
 * asynchronous on the context's stream.
 */
#ifndef CHIMERA_WORKLOAD_H_
#define CHIMERA_WORKLOAD_H_

#include <stddef.h>
#include <stdint.h>

#include "chimera_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Gaussian-mixture tokens on the unit sphere: token t takes centre
 * u(t) * n_centres (u uniform in [0, 1)), adds sigma * N(0, I) per dimension
 * and is L2-normalised. Randomness is Philox4x32-10 keyed by seed with the
 * token index as counter, so any slice of the corpus can be regenerated.
 * d_centres [n_centres, 128], d_out [n, 128]; dim must be 128. */
int chimera_synth_tokens_device(chimera_ctx* ctx, const float* d_centres, int64_t n_centres, int32_t dim,
                                uint64_t n, float sigma, uint64_t seed, float* d_out);

/* d_out[r] = d_src[d_ids[r]] for r < n: rows of dim floats gathered into
 * rows of 128 floats (zero-padded when dim < 128). */
int chimera_gather_rows_device(chimera_ctx* ctx, const float* d_src, int32_t dim, const int64_t* d_ids, int64_t n,
                               float* d_out);

/* Exact MaxSim of nq queries [nq, 32, 128] against every document of an
 * un-quantised corpus: d_scores[q * num_docs + d] = sum over the 32 query
 * tokens i of max over tokens t of document d of <q_i, x_t>, fp32 products
 * on the matrix cores. d_doc_ptrs [num_docs + 1] are token offsets into
 * d_embeddings [*, 128]. */
int chimera_exact_maxsim_device(chimera_ctx* ctx, const float* d_embeddings, const int32_t* d_doc_ptrs,
                                int64_t num_docs, const float* d_queries, int32_t nq, float* d_scores);

/* MaxSim rescoring of per-query candidate lists on un-quantised tokens: the
 * full-bit rescoring stage of the search (compute_full_bit_scores,
 * cpp/src/search_impl.cu:510-574) with fp32 tokens in place of W-bit codes,
 * followed by its final top-k (search_impl.cu:409,489-500).
 * For query q (d_queries [nq, 32, 128]) and j < min(d_cand_counts[q],
 * cand_cap): d_cand_scores[q * cand_cap + j] = sum over the 32 query tokens i
 * of max over the tokens t of document d_cand_ids[q * cand_cap + j] of
 * <q_i, x_t> (fp32 operands split into fp16 hi + lo pairs on the matrix
 * cores, within about 2^-21 of |q_i||x_t| per product); an id outside
 * [0, num_docs) or an empty document scores -inf. With k > 0,
 * d_top_ids / d_top_scores [nq, k] receive the k best candidates by score
 * descending, ties to the larger document id (the reference's max-heap of
 * (score, id)), padded with -1 / 0, and d_top_counts [nq] their number
 * (d_top_scores may be NULL). cand_cap must be in [1, 8192], nq at most
 * 65535. */
int chimera_maxsim_rescore_device(chimera_ctx* ctx, const float* d_embeddings, const int32_t* d_doc_ptrs,
                                  int64_t num_docs, const float* d_queries, int32_t nq, const int32_t* d_cand_ids,
                                  const int32_t* d_cand_counts, int32_t cand_cap, int32_t k, float* d_cand_scores,
                                  int64_t* d_top_ids, float* d_top_scores, int32_t* d_top_counts);

/* Matrix-core throughput on the context's device with register operands
 * (no memory traffic), every SIMD running eight waves of independent
 * accumulation chains: kind 0 v_mfma_f32_32x32x16_bf16 (the probe's), 1
 * v_mfma_f32_16x16x32_f16, 2 the same with 0/1 code bits as the A operand
 * (the one-bit refine's), 3 v_mfma_f32_32x32x2_f32 (the fp32 probe's), 4
 * v_mfma_i32_32x32x32_i8, 5 kind 2 with four independent one-cycle integer
 * VALU instructions after each MFMA (whether vector-ALU issue overlaps the
 * matrix cores on one SIMD). iters rounds per wave, three launches to settle
 * the clock, then one timed launch: *ops_per_second (2 per multiply-add).
 * Synchronous; it allocates and frees its own small buffers. A measurement
 * utility with no reference counterpart: the rate the matrix cores sustain
 * under their power limit, against which the matrix-core stages are
 * judged. */
int chimera_matrix_core_rate(chimera_ctx* ctx, int32_t kind, int32_t iters, double* ops_per_second);

#ifdef __cplusplus
}
#endif

#endif /* CHIMERA_WORKLOAD_H_ */
