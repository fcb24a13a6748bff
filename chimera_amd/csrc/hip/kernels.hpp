// Host-side launchers of the gfx950 kernels (all asynchronous on `s`).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace chimera {

int pow2_at_least(int v);
int probe_buffer_cap(int nprobe);

// Raises the dynamic LDS limit of the kernels that use more than 64 KB.
hipError_t configure_kernels(int nbk, int nprobe, int k_refine, int fb_cap);
hipError_t configure_candidate_kernels(int nbk, int k_refine);
hipError_t configure_score_kernels(int k_refine, int fb_cap);
hipError_t configure_query_kernels(int nprobe);

hipError_t launch_rotate_lut(hipStream_t s, const float* queries, int nq, int dim, const uint8_t* flips,
                             int ex_bits, float* rot, float* cb1, float* cbex, float* lut);
hipError_t launch_centroid_norms(hipStream_t s, const float* c, int64_t k, float* norms);
hipError_t launch_probe_exact(hipStream_t s, const float* rot, int nrows, const float* centroids,
                              const float* norms, int64_t k, int nprobe, uint32_t* labels);
// Buffers of the exact recomputation of flagged probe rows: up to list_cap
// flagged rows are listed and scored against centroid splits in parallel
// (partial holds list_cap * kExactPartialKeys keys: splits * nprobe per
// row); beyond list_cap flagged rows (or with list null) the row-block exact
// kernel recomputes them.
constexpr int kExactPartialKeys = 8192;
constexpr int kExactFallbackRows = 512;
struct ExactFallback {
    uint32_t* list = nullptr;     // [list_cap]
    uint32_t* nflag = nullptr;    // [1]
    uint64_t* partial = nullptr;  // [list_cap * kExactPartialKeys]
    int list_cap = 0;
};
// Centroid splits of the flagged-row recomputation for nprobe.
int exact_fallback_splits(int nprobe);
// Work split of the matrix-core probe (kernels_probe_mfma.hip).
struct ProbePlan {
    int row_blocks;
    int splits;
    int tiles_per_split;
    int sample_stride;
    int n_sampled;
    int group_tiles;  // sampled tiles per group minimum of the sampled pass
    int u_rank;       // rank (1-based) of the group minimum that sets the filter threshold
    int lane_cap;  // candidate sub-list entries per (row, split, lane half)
    bool usable;
};
// Rows of sub-list storage (buffers hold rows * 2 * lane_cap candidates and
// rows * 2 counts) that cover every plan for up to max_rows rows.
size_t probe_sublist_rows(int max_rows, int num_cus);
ProbePlan plan_probe_mfma(int nrows, int64_t k, int nprobe, int num_cus);
// bf16 centroids [k, 128], -|c|^2/2 [k] for the matrix-core probe, and the
// bits of max |c - c_b| over the centroids into *err_max (a non-negative
// float; the launcher clears it first).
hipError_t launch_probe_centroids(hipStream_t s, const float* c, const float* norms, int64_t k, uint16_t* cbf,
                                  float* nhalf, uint32_t* err_max);
// Bound on |d' - d| between the matrix-core score d' (bf16 operands, fp32
// accumulation) and the exact fp32 score d of one row against any centroid:
// qn = |q|, eq = |q - bf16(q)|, cmax >= max |c|, ecmax >= max |c - bf16(c)|.
__host__ __device__ float probe_delta(float qn, float eq, float cmax, float ecmax);
// part -1 runs the whole probe; 0 the sampled pass and threshold, 1 the
// full filtered pass, 2 the exact rerank (and the exact kernel for rows
// whose candidates overflowed), in that order. With f32 the two passes run
// on fp32 operands (centroids as given, v_mfma_f32_32x32x2_f32) and the
// margin drops the bf16 rounding terms; the labels are the same.
// rval holds probe_sublist_rows * 2 * lane_cap records of 16 fp16 values
// (8 words), rtile and cnt probe_sublist_rows * 2 * lane_cap and * 2
// entries. row_cand [nrows] receives each row's number of filtered
// candidates (0xFFFFFFFF for a row whose sub-list overflowed or whose
// candidates exceed the rerank's key area (8 nprobe, at least 1024), 0xFFFFFFFE for a row
// whose threshold failed the rerank's check); both kinds of row are
// recomputed by the exact kernel.
hipError_t launch_probe_mfma(hipStream_t s, const ProbePlan& p, const float* rot, int nrows, const uint16_t* cbf,
                             const float* nhalf, const float* centroids, const float* norms, int64_t k, float cmax,
                             float ecmax, int nprobe, float* gm, float* thr, uint32_t* rval, uint32_t* rtile,
                             uint32_t* cnt, uint32_t* row_flag, uint32_t* row_cand, uint32_t* labels,
                             const ExactFallback& fb, int part = -1, bool f32 = false);
// Nearest centroid (top-1, exact fp32 labels) of rows [nrows, 128] on the
// matrix cores; buf holds nrows * 2 * splits * lane_cap candidates, cnt
// nrows * 2 * splits counts, ukey and row_flag nrows entries.
ProbePlan plan_assign_top1(int nrows, int64_t k, int num_cus);
hipError_t launch_assign_top1(hipStream_t s, const ProbePlan& p, const float* rows, int nrows, const uint16_t* cbf,
                              const float* nhalf, const float* centroids, const float* norms, int64_t k, float cmax,
                              float ecmax, uint32_t* ukey, uint2* buf, uint32_t* cnt, uint32_t* row_flag,
                              uint32_t* labels, const ExactFallback& fb);
// Exact probe of the flagged rows: listed and split over the centroids (fb),
// or by the row-block kernel when more than fb.list_cap rows are flagged.
hipError_t launch_probe_exact_flagged(hipStream_t s, const float* rot, int nrows, const float* centroids,
                                      const float* norms, int64_t k, int nprobe, const uint32_t* row_flag,
                                      uint32_t* labels, const ExactFallback& fb);
hipError_t launch_unpack_codes(hipStream_t s, int width, const uint8_t* packed, int64_t n, uint8_t* raw);

// Candidate stage (kernels_candidates.hip). Per sub-batch of qs queries:
// vcnt [qs][nbk][32][parts] visit counts then offsets (parts > 1 only for
// small sub-batches: the query stride is then parts times larger), vtot
// [qs], rec [qs][vcap] records then candidates, tcount [qs][nbk], gstat
// and gsec [qs][nbk][groups per bucket].
struct CandidateArgs {
    const uint32_t* labels;
    int nprobe;
    const uint64_t* cluster_pos;
    const uint8_t* codes_clu;
    const float* f1_clu;
    const int32_t* doc_clu;
    int64_t n_clusters;
    int64_t num_docs;
    const float* lut;
    const float* cb1;
    int blog;  // documents per bucket = 2^blog
    int held;  // visit records per reduce thread kept in registers (8 or 12)
    int nbk;
    uint32_t* vcnt;
    uint32_t* vtot;
    uint2* rec;
    int64_t vcap;
    uint32_t* tcount;
    float2* gstat;
    uint2* gsec;  // per group {second-largest S bits (-1 when fewer than two), doc of the largest}
    uint16_t* gkey;  // per group the top 16 bits of its max S as an ordered key (the selection's radix keys)
    int k_refine;
    int32_t* ccount;
    int32_t* rcount;
    int32_t* rids;
    float* rscore;
    uint32_t* err;
    int num_cus;
    int wqs;  // queries the candidate state (vcnt, vtot, rec, ...) holds
};
int cand_buckets(int64_t num_docs, int blog);
// Bucket size (log2) of the candidate stage for an index: the largest in
// [kMinBucketLog2, kMaxBucketLog2] at which a (query, bucket) item expects at
// most 8,192 visit records, given 32 query tokens x nprobe clusters of the
// mean size spread over the documents (and at most the staged emit's bucket
// count).
// Candidate-stage shape of an index: documents per bucket 2^blog and the
// visit records each reduce thread keeps in registers (8 or 12).
struct CandShape {
    int blog;
    int held;
};
CandShape cand_shape(int64_t num_docs, int64_t n_tokens, int64_t n_clusters, int nprobe);
int select_list_cap(int k_refine);
// phase 0 count, 1 offsets, 2 emit, 3 reduce, 4 select
hipError_t launch_candidates(hipStream_t s, const CandidateArgs& a, int q_base, int qs, int phase);
hipError_t launch_cand_compact(hipStream_t s, const CandidateArgs& a, int qs, int64_t cap, int32_t* cand,
                               float* score);

hipError_t launch_refine_lut(hipStream_t s, int nq, int k_refine, const float* lut, const float* cb1,
                             const int32_t* rcount, const int32_t* rids, const int32_t* doc_ptrs,
                             const uint8_t* codes_tok, const float* f1_tok, float* s1);
// codes_tok and f1_tok hold kRefinePadTokens tokens past the index's last one
// (any values): a 64-token group that crosses the end is loaded whole.
constexpr int kRefinePadTokens = 64;
hipError_t launch_refine_mfma(hipStream_t s, int nq, int k_refine, const float* rot, const float* cb1,
                              const int32_t* rcount, const int32_t* rids, const int32_t* doc_ptrs,
                              const uint8_t* codes_tok, const float* f1_tok, float* s1, int num_cus);
hipError_t launch_chunk_select(hipStream_t s, int nq, const float* s1, const int32_t* rcount, const int32_t* rids,
                               int k_refine, int k_full_bit, int num_chunks, int fb_cap, int32_t* fcount,
                               int32_t* fids, uint32_t* err);
hipError_t launch_fullbit(hipStream_t s, int nq, const float* rot, const float* cbex, const int32_t* fcount,
                          const int32_t* fids, int fb_cap, const int32_t* doc_ptrs, const uint8_t* full_codes,
                          const float* full_factors, int width, float* fscores);
// Full-bit MaxSim on the matrix cores (width 2..8), scores within ~1e-6
// relative of the reference's fp32 arithmetic. full_codes and full_factors
// hold kFullbitPadTokens tokens past the index's last one (any values): a
// 16-token tile that crosses the end is loaded whole.
constexpr int kFullbitPadTokens = 16;
hipError_t launch_fullbit_mfma(hipStream_t s, int nq, const float* rot, const float* cbex, const int32_t* fcount,
                               const int32_t* fids, int fb_cap, const int32_t* doc_ptrs, const uint8_t* full_codes,
                               const float* full_factors, int width, float* fscores, int num_cus);
hipError_t launch_final_topk(hipStream_t s, int nq, const int32_t* fcount, const int32_t* fids,
                             const float* fscores, int fb_cap, int k, int64_t* out_ids, float* out_scores,
                             int32_t* out_counts);

// Index build (kernels_build.hip).
hipError_t launch_encode_tokens(hipStream_t s, const float* emb, int64_t n, int dim, const uint8_t* flips,
                                int ex_bits, int num_cus, uint8_t* codes1, float* f1, uint8_t* full, float* fF,
                                uint32_t* status);
// out[r] = src[ids ? ids[r] : r] zero-padded to 128 floats, rotated when asked.
hipError_t launch_gather_rows(hipStream_t s, const float* src, int dim, const int64_t* ids, int64_t nrows,
                              const uint8_t* flips, bool rotate, float* out);
// Stable sort of (label, token) pairs by label; temp == nullptr queries the
// scratch size into *temp_bytes.
hipError_t launch_sort_assignments(hipStream_t s, const uint32_t* labels, int64_t n, int64_t k, uint32_t* keys_out,
                                   uint32_t* vals_in, uint32_t* vals_out, void* temp, size_t* temp_bytes);
hipError_t launch_layout(hipStream_t s, const uint32_t* sorted_keys, const uint32_t* inv, int64_t n, int64_t k,
                         const int32_t* doc_ptrs, int64_t m, const uint8_t* codes_tok, const float* f1_tok,
                         int32_t* token_doc, uint64_t* cluster_pos, uint8_t* codes_clu, float* f1_clu,
                         int32_t* doc_clu, uint32_t* runs);

// Token-order copies of the clustered one-bit data: out[t] = in[pos[t]].
hipError_t launch_gather_token_order(hipStream_t s, const uint8_t* codes_clu, const float* f1_clu,
                                     const uint32_t* tok2pos, int64_t n, uint8_t* codes_tok, float* f1_tok);
// Fill n 32-bit words with v (graph-safe replacement for memset).
hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, int64_t n, uint32_t v);
hipError_t launch_copy_u32(hipStream_t s, uint32_t* dst, const uint32_t* src, int64_t n);

}  // namespace chimera
