// Chimera oracle: a scalar CPU restatement of the reference's search path.
//
// TEST INFRASTRUCTURE ONLY. It is the checker for the HIP implementation and
// the CPU baseline of bench.py; nothing in the product links or calls it.
//
// Every function follows the reference file:line named in its comment, with
// the reference's floating-point operation order, so that integer results
// (codes, candidate lists, probe labels) match bit for bit and float results
// match bit for bit wherever the reference's order is reproducible on a CPU:
//   rotation            rotator.hpp:129-334, fht_avx.cpp:219-591 (stages 1,2,4,..)
//   QueryState          chimera_index_internal.cuh:51-65
//   one-bit LUT         kernels.cu:402-428
//   one-bit estimator   kernels.cu:361-375 and 491-504
//   candidate set       kernels.cu:117-173, 206-278; search_impl.cu:118-262
//   S_cand              kernels.cu:280-400 (max over a token's visits of a doc,
//                       clamped at 0) and 175-204 (shfl-down tree over 32)
//   refined set R       CUB stable descending radix sort, search_impl.cu:245-261
//   S1                  kernels.cu:430-575 (max from -FLT_MAX, tree sum)
//   full-bit selection  search_impl.cu:405-494 (nth_element ties: lower
//                       refined index first here; the reference leaves them
//                       unspecified)
//   full-bit score SF   search_impl.cu:510-574 with gemv_batch8_avx512
//                       (space.hpp:806-850: 16 fma lanes, reduce 8,4,2,1)
//   final top-k         search_impl.cu:409,489-500 (ties: larger doc ID)
// The centroid probe is exact (|c|^2 - 2<q,c>, sequential fmaf, ties to the
// lower ID) where the reference calls cuVS CAGRA, an approximate graph search
// whose output no file here can reproduce: the probe labels are "parity
// unpinned" against the reference and pinned instead against brute force.
//
// How each function is pinned independently of this file:
//   rotation, flips, encoders, pack/unpack, full-bit score SF
//       known answers of the reference's own host code compiled here
//       (tests/golden/reference_host.npz, tests/test_codec_golden.py), plus
//       the Hadamard closed form of the rotation
//   QueryState, LUT        closed forms (tests/test_codec_golden.py)
//   probe, candidate set, S_cand, refined set, S1, full-bit selection, SF,
//   final top-k            tests/test_oracle_pins.py: float64 brute force
//       and closed forms, the union of the probed clusters, a stable sort,
//       a literal simulation of the reference's chunk loop with nth_element
//       partitions in random order, and heap pops; on an index with exact
//       duplicate documents so that every ranked stage has ties
//
// Build: oracle/Makefile (g++ -O2 -fopenmp -ffp-contract=off).

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <utility>
#include <vector>

#include "oracle_index.h"

namespace {

constexpr int kDim = 128;
constexpr int kQ = 32;
constexpr int kChunks = 32;   // NUM_CHUNKS, config.cuh:17-18
constexpr int kLut = 16;      // LUT_SIZE

int floor_log2(int x) {
    int r = 0;
    while (x > 1) {
        ++r;
        x >>= 1;
    }
    return r;
}

void fwht(float* x, int n) {
    for (int h = 1; h < n; h <<= 1)
        for (int i = 0; i < n; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
}

void flip_sign(const uint8_t* flip, float* x, int n) {
    for (int j = 0; j < n; ++j)
        if ((flip[j >> 3] >> (j & 7)) & 1) x[j] = -x[j];
}

// rotator.hpp:281-334 with padded_dim = 128.
void rotate(const float* src, int dim, const uint8_t* flips, float* dst) {
    for (int j = 0; j < kDim; ++j) dst[j] = j < dim ? src[j] : 0.0f;
    const int trunc = 1 << floor_log2(dim);
    const float fac = 1.0F / std::sqrt(static_cast<float>(trunc));
    const int stride = kDim / 8;
    if (trunc == kDim) {
        for (int r = 0; r < 4; ++r) {
            flip_sign(flips + r * stride, dst, kDim);
            fwht(dst, trunc);
            for (int j = 0; j < trunc; ++j) dst[j] = dst[j] * fac;
        }
        return;
    }
    const int start = kDim - trunc;
    for (int r = 0; r < 4; ++r) {
        flip_sign(flips + r * stride, dst, kDim);
        float* seg = (r & 1) ? dst + start : dst;
        fwht(seg, trunc);
        for (int j = 0; j < trunc; ++j) seg[j] = seg[j] * fac;
        for (int i = 0; i < kDim / 2; ++i) {
            const float x = dst[i], y = dst[i + kDim / 2];
            dst[i] = x + y;
            dst[i + kDim / 2] = x - y;
        }
    }
    for (int j = 0; j < kDim; ++j) dst[j] = dst[j] * 0.25F;
}

// Shuffle-down tree over 32 values: offsets 16, 8, 4, 2, 1 (kernels.cu:195-198;
// the 128-thread shared-memory tree of kernels.cu:557-570 reduces to the same
// order because lanes 32..127 contribute +0).
float tree32(const float* v) {
    float a[32];
    for (int i = 0; i < 32; ++i) a[i] = v[i];
    for (int off = 16; off >= 1; off >>= 1)
        for (int i = 0; i < off; ++i) a[i] = a[i] + a[i + off];
    return a[0];
}

// _mm512_reduce_add_ps as GCC defines it: halves 8, 4, 2, 1.
float reduce16(const float* v) {
    float a[16];
    for (int i = 0; i < 16; ++i) a[i] = v[i];
    for (int off = 8; off >= 1; off >>= 1)
        for (int i = 0; i < off; ++i) a[i] = a[i] + a[i + off];
    return a[0];
}

inline int nibble(const uint8_t* code, int c) { return (code[c >> 1] >> ((c & 1) * 4)) & 0xF; }

// kernels.cu:361-375 / 497-504: ip accumulates the 32 chunk entries in order.
inline float one_bit_est(const float* lut_i, const uint8_t* code, float cb1, float factor) {
    float ip = 0.0f;
    for (int c = 0; c < kChunks; ++c) ip += lut_i[c * kLut + nibble(code, c)];
    return (ip - cb1) * factor;
}

void unpack(const uint8_t* in, int width, uint8_t* raw) {
    // Inverse of pack_excode.hpp:13-297 for 128 dimensions.
    switch (width) {
        case 1:
            for (int b = 0; b < kDim; b += 16) {
                const int v = in[b / 8] | (in[b / 8 + 1] << 8);
                for (int i = 0; i < 16; ++i) raw[b + i] = (v >> i) & 1;
            }
            return;
        case 2:
            for (int b = 0; b < kDim / 16; ++b)
                for (int k = 0; k < 4; ++k)
                    for (int m = 0; m < 4; ++m) raw[16 * b + 4 * k + m] = (in[4 * b + m] >> (2 * k)) & 3;
            return;
        case 4:
            for (int b = 0; b < kDim / 16; ++b)
                for (int m = 0; m < 8; ++m) {
                    raw[16 * b + m] = in[8 * b + m] & 15;
                    raw[16 * b + 8 + m] = in[8 * b + m] >> 4;
                }
            return;
        case 6:
            for (int b = 0; b < kDim / 16; ++b) {
                const uint8_t* p = in + 12 * b;
                for (int m = 0; m < 8; ++m) {
                    raw[16 * b + m] = p[m] & 15;
                    raw[16 * b + 8 + m] = p[m] >> 4;
                }
                for (int k = 0; k < 4; ++k)
                    for (int m = 0; m < 4; ++m) raw[16 * b + 4 * k + m] |= ((p[8 + m] >> (2 * k)) & 3) << 4;
            }
            return;
        case 8:
            std::memcpy(raw, in, kDim);
            return;
        default: {  // 3, 5, 7: 64-dimension blocks with a u64 of top bits
            const int bytes = 64 * width / 8;
            for (int blk = 0; blk < 2; ++blk) {
                const uint8_t* p = in + blk * bytes;
                uint8_t* r = raw + 64 * blk;
                if (width == 3) {
                    for (int k = 0; k < 4; ++k)
                        for (int m = 0; m < 16; ++m) r[16 * k + m] = (p[m] >> (2 * k)) & 3;
                } else if (width == 5) {
                    for (int m = 0; m < 16; ++m) {
                        r[m] = p[m] & 15;
                        r[16 + m] = p[m] >> 4;
                        r[32 + m] = p[16 + m] & 15;
                        r[48 + m] = p[16 + m] >> 4;
                    }
                } else {
                    for (int m = 0; m < 16; ++m) {
                        r[m] = p[m] & 63;
                        r[16 + m] = p[16 + m] & 63;
                        r[32 + m] = p[32 + m] & 63;
                        r[48 + m] = (p[m] >> 6) | ((p[16 + m] >> 6) << 2) | ((p[32 + m] >> 6) << 4);
                    }
                }
                uint64_t top;
                std::memcpy(&top, p + bytes - 8, 8);
                for (int i = 0; i < 64; i += 8)
                    for (int k = 0; k < 8; ++k) r[i + k] |= ((top >> (8 * k + i / 8)) & 1) << (width - 1);
            }
            return;
        }
    }
}

}  // namespace

extern "C" {

struct oracle_options {
    int32_t nprobe, k_refine, k_full_bit, num_chunks;
};

// Per-query outputs; any pointer may be NULL. Capacities are element counts.
struct oracle_result {
    float* rotated;            // [32*128]
    float* cb1;                // [32]
    float* cbex;               // [32]
    float* lut;                // [32*32*16]
    uint32_t* labels;          // [32*nprobe]
    int32_t* cand_count;       // [1]
    int32_t* candidates;       // [cand_cap]
    float* cand_scores;        // [cand_cap]
    int64_t cand_cap;
    int32_t* refined_count;    // [1]
    int32_t* refined_ids;      // [k_refine]
    float* refined_scores;     // [k_refine]
    int32_t* fullbit_count;    // [1]
    int32_t* fullbit_ids;      // [fullbit_cap], ascending doc ID
    float* fullbit_scores;     // [fullbit_cap]
    int64_t fullbit_cap;
    int32_t* result_count;     // [1]
    int64_t* result_ids;       // [k]
    float* result_scores;      // [k]
};

void oracle_rotate(const float* src, int32_t dim, const uint8_t* flips, float* dst) {
    rotate(src, dim, flips, dst);
}

// chimera_index_internal.cuh:58-64
void oracle_query_state(const float* rotated, int32_t ex_bits, float* cb1, float* cbex) {
    float sumq = 0.0f;
    for (int j = 0; j < kDim; ++j) sumq = sumq + rotated[j];
    *cb1 = sumq * ((1 << 1) - 1) / 2.0f;
    *cbex = sumq * ((1 << (ex_bits + 1)) - 1) / 2.0f;
}

// kernels.cu:402-428 for one query token: lut[c*16 + e].
void oracle_lut(const float* rotated, float* lut) {
    for (int c = 0; c < kChunks; ++c)
        for (int e = 0; e < kLut; ++e) {
            float s = 0.0f;
            for (int b = 0; b < 4; ++b)
                if ((e >> b) & 1) s += rotated[c * 4 + b];
            lut[c * kLut + e] = s;
        }
}

void oracle_unpack(const uint8_t* packed, int32_t width, uint8_t* raw) { unpack(packed, width, raw); }

float oracle_one_bit_est(const float* lut_i, const uint8_t* code, float cb1, float factor) {
    return one_bit_est(lut_i, code, cb1, factor);
}

// Exact probe score |c|^2 - 2<q,c>, both by sequential fmaf over 128 dims.
float oracle_probe_score(const float* q, const float* c) {
    float dot = 0.0f, nrm = 0.0f;
    for (int j = 0; j < kDim; ++j) {
        dot = std::fmaf(q[j], c[j], dot);
        nrm = std::fmaf(c[j], c[j], nrm);
    }
    return nrm - 2.0f * dot;
}

void oracle_probe(const float* rotated, int32_t nrows, const float* centroids, int64_t n_clusters,
                  int32_t nprobe, uint32_t* labels) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int r = 0; r < nrows; ++r) {
        std::vector<std::pair<float, uint32_t>> s(static_cast<size_t>(n_clusters));
        for (int64_t c = 0; c < n_clusters; ++c)
            s[c] = {oracle_probe_score(rotated + static_cast<size_t>(r) * kDim, centroids + c * kDim),
                    static_cast<uint32_t>(c)};
        std::partial_sort(s.begin(), s.begin() + nprobe, s.end());
        for (int p = 0; p < nprobe; ++p) labels[static_cast<size_t>(r) * nprobe + p] = s[p].second;
    }
}

// Full-bit MaxSim of one document (search_impl.cu:526-573).
float oracle_full_bit_score(const oracle_index* idx, int32_t doc, const float* rotated /*[32*128]*/,
                            const float* cbex /*[32]*/) {
    const int width = static_cast<int>(1 + idx->ex_bits);
    const size_t stride = static_cast<size_t>(16 * width);
    float max_ts[kQ];
    for (int i = 0; i < kQ; ++i) max_ts[i] = -std::numeric_limits<float>::infinity();
    uint8_t raw[kDim];
    float decoded[kDim];
    for (int32_t t = idx->doc_ptrs[doc]; t < idx->doc_ptrs[doc + 1]; ++t) {
        unpack(idx->full_codes + static_cast<size_t>(t) * stride, width, raw);
        for (int j = 0; j < kDim; ++j) decoded[j] = static_cast<float>(raw[j]);
        const float f = idx->full_factors[t];
        for (int i = 0; i < kQ; ++i) {
            const float* q = rotated + i * kDim;
            float lane[16];
            for (int m = 0; m < 16; ++m) {
                float acc = 0.0f;
                for (int s = 0; s < kDim / 16; ++s) acc = std::fmaf(decoded[16 * s + m], q[16 * s + m], acc);
                lane[m] = acc;
            }
            const float ip = reduce16(lane);
            const float combined = (ip - cbex[i]) * f;
            max_ts[i] = std::max(max_ts[i], combined);
        }
    }
    float s16[16];
    for (int m = 0; m < 16; ++m) s16[m] = max_ts[m] + max_ts[16 + m];
    return reduce16(s16);
}

// Chunked full-bit selection (search_impl.cu:341-494) over the one-bit scores
// s1[0..R) of the refined list: chunks are contiguous slices of ceil(R/n_ch);
// after chunk c the carry is the top min(F, end_c) of the first end_c
// documents and the top min(F (c+1) / n_ch, carry) of those are selected.
// Ties (unspecified in the reference's nth_element) go to the lower index.
void oracle_chunk_select(const float* s1, int32_t R, int32_t k_full_bit, int32_t num_chunks, uint8_t* selected) {
    for (int r = 0; r < R; ++r) selected[r] = 0;
    if (R <= 0) return;
    const int F = std::min(k_full_bit, R);
    const int n_ch = std::min(num_chunks, R);
    const int chunk = (R + n_ch - 1) / n_ch;
    std::vector<int> by_s1(R);
    for (int r = 0; r < R; ++r) by_s1[r] = r;
    std::stable_sort(by_s1.begin(), by_s1.end(), [&](int a, int b) { return s1[a] > s1[b]; });
    for (int c = 0; c < n_ch; ++c) {
        const int end = std::min((c + 1) * chunk, R);
        const int carry = std::min(F, end);
        const int target = std::min(F * (c + 1) / n_ch, carry);
        int taken = 0;
        for (int s = 0; s < R && taken < target; ++s)
            if (by_s1[s] < end) {
                selected[by_s1[s]] = 1;
                ++taken;
            }
    }
}

// Appendix-B search of one query. Returns 0.
int32_t oracle_search(const oracle_index* idx, const float* query, const oracle_options* opt,
                      int32_t k, oracle_result* out) {
    const int dim = static_cast<int>(idx->dim);
    const int nprobe = opt->nprobe;
    const size_t M = static_cast<size_t>(idx->num_docs);

    // 1. rotation, QueryState, LUT
    std::vector<float> rot(kQ * kDim), cb1(kQ), cbex(kQ), lut(kQ * kChunks * kLut);
    for (int i = 0; i < kQ; ++i) {
        rotate(query + i * dim, dim, idx->flips, &rot[i * kDim]);
        oracle_query_state(&rot[i * kDim], static_cast<int>(idx->ex_bits), &cb1[i], &cbex[i]);
        oracle_lut(&rot[i * kDim], &lut[i * kChunks * kLut]);
    }
    if (out->rotated) std::memcpy(out->rotated, rot.data(), rot.size() * 4);
    if (out->cb1) std::memcpy(out->cb1, cb1.data(), kQ * 4);
    if (out->cbex) std::memcpy(out->cbex, cbex.data(), kQ * 4);
    if (out->lut) std::memcpy(out->lut, lut.data(), lut.size() * 4);

    // 2. probe
    std::vector<uint32_t> labels(static_cast<size_t>(kQ) * nprobe);
    for (int i = 0; i < kQ; ++i) {
        std::vector<std::pair<float, uint32_t>> s(static_cast<size_t>(idx->n_clusters));
        for (int64_t c = 0; c < idx->n_clusters; ++c)
            s[c] = {oracle_probe_score(&rot[i * kDim], idx->rotated_centroids + c * kDim), static_cast<uint32_t>(c)};
        std::partial_sort(s.begin(), s.begin() + nprobe, s.end());
        for (int p = 0; p < nprobe; ++p) labels[static_cast<size_t>(i) * nprobe + p] = s[p].second;
    }
    if (out->labels) std::memcpy(out->labels, labels.data(), labels.size() * 4);

    // 3-4. candidate set and S_cand
    std::vector<uint8_t> touched(M, 0);
    std::vector<float> partial;  // [M*32] only where touched; keep dense for clarity
    partial.assign(M * kQ, 0.0f);
    for (int i = 0; i < kQ; ++i) {
        const float* lut_i = &lut[i * kChunks * kLut];
        for (int p = 0; p < nprobe; ++p) {
            const uint32_t label = labels[static_cast<size_t>(i) * nprobe + p];
            if (label >= static_cast<uint64_t>(idx->n_clusters)) continue;
            for (uint64_t pos = idx->cluster_pos[label]; pos < idx->cluster_pos[label + 1]; ++pos) {
                const int32_t doc = idx->clustered_doc_ids[pos];
                if (doc < 0 || static_cast<size_t>(doc) >= M) continue;
                touched[doc] = 1;
                const float e = one_bit_est(lut_i, idx->clustered_codes + pos * 16, cb1[i], idx->clustered_factors[pos]);
                if (e > 0.0f) {
                    float& slot = partial[static_cast<size_t>(doc) * kQ + i];
                    slot = std::fmax(e, slot);
                }
            }
        }
    }
    std::vector<int32_t> cand;
    std::vector<float> cand_score;
    for (size_t d = 0; d < M; ++d)
        if (touched[d]) {
            cand.push_back(static_cast<int32_t>(d));
            cand_score.push_back(tree32(&partial[d * kQ]));
        }
    const int C = static_cast<int>(cand.size());
    if (out->cand_count) *out->cand_count = C;
    if (out->candidates)
        for (int c = 0; c < C && c < out->cand_cap; ++c) out->candidates[c] = cand[c];
    if (out->cand_scores)
        for (int c = 0; c < C && c < out->cand_cap; ++c) out->cand_scores[c] = cand_score[c];

    auto set_empty = [&]() {
        if (out->refined_count) *out->refined_count = 0;
        if (out->fullbit_count) *out->fullbit_count = 0;
        if (out->result_count) *out->result_count = 0;
        return 0;
    };
    if (C == 0) return set_empty();

    // 5. stable descending sort, keep R
    std::vector<int> order(C);
    for (int c = 0; c < C; ++c) order[c] = c;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cand_score[a] > cand_score[b]; });
    const int R = std::min(opt->k_refine, C);
    std::vector<int32_t> refined(R);
    for (int r = 0; r < R; ++r) refined[r] = cand[order[r]];

    // 6. one-bit MaxSim
    std::vector<float> s1(R);
    for (int r = 0; r < R; ++r) {
        const int32_t doc = refined[r];
        float mx[kQ];
        for (int i = 0; i < kQ; ++i) mx[i] = -FLT_MAX;
        for (int32_t t = idx->doc_ptrs[doc]; t < idx->doc_ptrs[doc + 1]; ++t) {
            const uint32_t pos = idx->token_to_cluster_pos[t];
            const uint8_t* code = idx->clustered_codes + static_cast<size_t>(pos) * 16;
            const float f = idx->clustered_factors[pos];
            for (int i = 0; i < kQ; ++i)
                mx[i] = std::fmax(mx[i], one_bit_est(&lut[i * kChunks * kLut], code, cb1[i], f));
        }
        s1[r] = tree32(mx);
    }
    if (out->refined_count) *out->refined_count = R;
    if (out->refined_ids) std::memcpy(out->refined_ids, refined.data(), R * 4);
    if (out->refined_scores) std::memcpy(out->refined_scores, s1.data(), R * 4);

    // 7. chunked full-bit selection (search_impl.cu:341-494)
    std::vector<uint8_t> selected(R, 0);
    oracle_chunk_select(s1.data(), R, opt->k_full_bit, opt->num_chunks, selected.data());

    // 8. full-bit scores and 9. final top-k
    std::vector<std::pair<float, int32_t>> scored;
    for (int r = 0; r < R; ++r)
        if (selected[r]) scored.push_back({oracle_full_bit_score(idx, refined[r], rot.data(), cbex.data()), refined[r]});
    std::vector<std::pair<float, int32_t>> asc = scored;
    std::sort(asc.begin(), asc.end(), [](const auto& a, const auto& b) { return a.second < b.second; });
    if (out->fullbit_count) *out->fullbit_count = static_cast<int32_t>(asc.size());
    for (size_t j = 0; j < asc.size() && static_cast<int64_t>(j) < out->fullbit_cap; ++j) {
        if (out->fullbit_ids) out->fullbit_ids[j] = asc[j].second;
        if (out->fullbit_scores) out->fullbit_scores[j] = asc[j].first;
    }
    std::sort(scored.begin(), scored.end(), [](const auto& a, const auto& b) {
        return a.first != b.first ? a.first > b.first : a.second > b.second;
    });
    const int kk = std::min<int>(k, static_cast<int>(scored.size()));
    if (out->result_count) *out->result_count = kk;
    for (int j = 0; j < kk; ++j) {
        if (out->result_ids) out->result_ids[j] = scored[j].second;
        if (out->result_scores) out->result_scores[j] = scored[j].first;
    }
    return 0;
}

// Many queries in parallel; results only (ids [nq*k] padded with -1).
void oracle_search_batch(const oracle_index* idx, const float* queries, int32_t nq,
                         const oracle_options* opt, int32_t k, int64_t* ids, float* scores,
                         int32_t* counts) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int q = 0; q < nq; ++q) {
        oracle_result r{};
        int32_t cnt = 0;
        r.result_count = &cnt;
        r.result_ids = ids + static_cast<size_t>(q) * k;
        r.result_scores = scores ? scores + static_cast<size_t>(q) * k : nullptr;
        for (int j = 0; j < k; ++j) ids[static_cast<size_t>(q) * k + j] = -1;
        oracle_search(idx, queries + static_cast<size_t>(q) * kQ * idx->dim, opt, k, &r);
        counts[q] = cnt;
    }
}

// Full-bit MaxSim over explicit (query, doc) lists: the CPU baseline of the
// full-bit stage. docs[q*per_query + j]; out[q*per_query + j].
void oracle_full_bit_batch(const oracle_index* idx, const float* rotated /*[nq*32*128]*/,
                           const float* cbex /*[nq*32]*/, int32_t nq, const int32_t* docs,
                           int32_t per_query, float* out) {
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
    for (int q = 0; q < nq; ++q)
        for (int j = 0; j < per_query; ++j) {
            const int32_t d = docs[static_cast<size_t>(q) * per_query + j];
            out[static_cast<size_t>(q) * per_query + j] =
                d < 0 ? 0.0f : oracle_full_bit_score(idx, d, rotated + static_cast<size_t>(q) * kQ * kDim, cbex + q * kQ);
        }
}

}  // extern "C"
