// CPU baseline of the scoring path: full-bit MaxSim of per-query document
// lists with AVX-512 and OpenMP over documents, a restatement of the
// reference's CPU stage compute_full_bit_scores (search_impl.cu:510-574):
//   per document token: the W-bit code unpacked to 128 floats (the layouts
//   of pack_excode.hpp:13-297), a GEMV against the 32 rotated query tokens
//   with 16 fma lanes over 8 steps of 16 dimensions and eight query rows at a
//   time (gemv_batch8_avx512, space.hpp:806-850), the 16 lanes summed by
//   halves (8, 4, 2, 1, as _mm512_reduce_add_ps), then (ip - cbex) * factor
//   and the running max over the document's tokens; the 32 maxima summed as
//   two 16-lane vectors and reduced by halves.
// The operation order is the reference's, so the scores equal the oracle's
// oracle_full_bit_score bit for bit (tests/test_cpu_baseline.py).
//
// TEST INFRASTRUCTURE ONLY: bench.py times it as the CPU baseline; nothing in
// the product links or calls it. The AVX-512 code is compiled for that
// target only (function attributes) and entered after a run-time CPU check.

#include <immintrin.h>
#include <omp.h>

#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "oracle_index.h"

namespace {

constexpr int kDim = 128;
constexpr int kQ = 32;

inline uint64_t ld64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}
inline uint32_t ld32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
inline void st64(uint8_t* p, uint64_t v) { std::memcpy(p, &v, 8); }
inline void st32(uint8_t* p, uint32_t v) { std::memcpy(p, &v, 4); }

constexpr uint64_t kLo2 = 0x0303030303030303ull, kLo4 = 0x0F0F0F0F0F0F0F0Full, kLo6 = 0x3F3F3F3F3F3F3F3Full,
                   kBit0 = 0x0101010101010101ull;

// top bits of a 64-dimension block: bit (8b + g) of top is bit (W - 1) of
// raw[8g + b] (pack_excode.hpp:56-102)
inline void or_top_bits(uint8_t* r, uint64_t top, int shift) {
    for (int g = 0; g < 8; ++g) st64(r + 8 * g, ld64(r + 8 * g) | (((top >> g) & kBit0) << shift));
}

// W-bit codes of 128 dimensions to bytes, eight lanes of 8 bits at a time
void unpack_swar(const uint8_t* in, int width, uint8_t* raw) {
    switch (width) {
        case 2:  // per 16 dims, 4 bytes: byte m bits 2k..2k+1 = raw[4k + m]
            for (int b = 0; b < kDim / 16; ++b) {
                const uint32_t x = ld32(in + 4 * b);
                for (int k = 0; k < 4; ++k) st32(raw + 16 * b + 4 * k, (x >> (2 * k)) & 0x03030303u);
            }
            return;
        case 4:  // per 16 dims, 8 bytes: byte m = raw[m] | raw[8 + m] << 4
            for (int b = 0; b < kDim / 16; ++b) {
                const uint64_t x = ld64(in + 8 * b);
                st64(raw + 16 * b, x & kLo4);
                st64(raw + 16 * b + 8, (x >> 4) & kLo4);
            }
            return;
        case 6:  // the W = 4 layout plus a u32 of bits 4-5 per 16 dims
            for (int b = 0; b < kDim / 16; ++b) {
                const uint8_t* p = in + 12 * b;
                const uint64_t x = ld64(p);
                const uint32_t y = ld32(p + 8);
                uint8_t* r = raw + 16 * b;
                st64(r, x & kLo4);
                st64(r + 8, (x >> 4) & kLo4);
                for (int k = 0; k < 4; ++k) st32(r + 4 * k, ld32(r + 4 * k) | (((y >> (2 * k)) & 0x03030303u) << 4));
            }
            return;
        case 8:
            std::memcpy(raw, in, kDim);
            return;
        case 3:  // per 64 dims, 24 bytes: byte m bits 2k..2k+1 = raw[16k + m] & 3, top bit 2
            for (int blk = 0; blk < 2; ++blk) {
                const uint8_t* p = in + 24 * blk;
                uint8_t* r = raw + 64 * blk;
                const uint64_t w0 = ld64(p), w1 = ld64(p + 8);
                for (int k = 0; k < 4; ++k) {
                    st64(r + 16 * k, (w0 >> (2 * k)) & kLo2);
                    st64(r + 16 * k + 8, (w1 >> (2 * k)) & kLo2);
                }
                or_top_bits(r, ld64(p + 16), 2);
            }
            return;
        case 5:  // per 64 dims, 40 bytes: two nibble-split 16-byte groups, top bit 4
            for (int blk = 0; blk < 2; ++blk) {
                const uint8_t* p = in + 40 * blk;
                uint8_t* r = raw + 64 * blk;
                for (int g = 0; g < 2; ++g)
                    for (int h = 0; h < 2; ++h) {
                        const uint64_t w = ld64(p + 16 * g + 8 * h);
                        st64(r + 32 * g + 8 * h, w & kLo4);
                        st64(r + 32 * g + 16 + 8 * h, (w >> 4) & kLo4);
                    }
                or_top_bits(r, ld64(p + 32), 4);
            }
            return;
        case 7:  // per 64 dims, 56 bytes: three 6-bit groups carrying the fourth's bits, top bit 6
            for (int blk = 0; blk < 2; ++blk) {
                const uint8_t* p = in + 56 * blk;
                uint8_t* r = raw + 64 * blk;
                for (int h = 0; h < 2; ++h) {
                    const uint64_t x0 = ld64(p + 8 * h), x1 = ld64(p + 16 + 8 * h), x2 = ld64(p + 32 + 8 * h);
                    st64(r + 8 * h, x0 & kLo6);
                    st64(r + 16 + 8 * h, x1 & kLo6);
                    st64(r + 32 + 8 * h, x2 & kLo6);
                    st64(r + 48 + 8 * h,
                         ((x0 >> 6) & kLo2) | (((x1 >> 6) & kLo2) << 2) | (((x2 >> 6) & kLo2) << 4));
                }
                or_top_bits(r, ld64(p + 48), 6);
            }
            return;
        default:
            std::memset(raw, 0, kDim);
            return;
    }
}

__attribute__((target("avx512f,avx512bw,avx512vl,avx512dq"))) inline float reduce_halves(__m512 v) {
    const __m256 lo = _mm512_castps512_ps256(v);
    const __m256 hi = _mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(v), 1));
    const __m256 s8 = _mm256_add_ps(lo, hi);
    const __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(s8), _mm256_extractf128_ps(s8, 1));
    const __m128 s2 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
    const __m128 s1 = _mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 1));
    return _mm_cvtss_f32(s1);
}

__attribute__((target("avx512f,avx512bw,avx512vl,avx512dq"))) float score_doc(const oracle_index* idx, int32_t doc,
                                                                             const float* q /*[32*128]*/,
                                                                             const float* cbex /*[32]*/) {
    const int width = static_cast<int>(1 + idx->ex_bits);
    const size_t stride = static_cast<size_t>(16 * width);
    alignas(64) uint8_t raw[kDim];
    alignas(64) float ip[kQ];
    __m512 mx0 = _mm512_set1_ps(-std::numeric_limits<float>::infinity());
    __m512 mx1 = mx0;
    const __m512 cb0 = _mm512_loadu_ps(cbex), cb1 = _mm512_loadu_ps(cbex + 16);
    for (int32_t t = idx->doc_ptrs[doc]; t < idx->doc_ptrs[doc + 1]; ++t) {
        unpack_swar(idx->full_codes + static_cast<size_t>(t) * stride, width, raw);
        if (t + 1 < idx->doc_ptrs[doc + 1]) __builtin_prefetch(idx->full_codes + static_cast<size_t>(t + 1) * stride);
        __m512 d[8];
        for (int s = 0; s < 8; ++s)
            d[s] = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm_load_si128(reinterpret_cast<const __m128i*>(raw + 16 * s))));
        for (int j = 0; j < kQ; j += 8) {
            __m512 acc[8];
            for (int r = 0; r < 8; ++r) acc[r] = _mm512_setzero_ps();
            for (int s = 0; s < 8; ++s)
                for (int r = 0; r < 8; ++r)
                    acc[r] = _mm512_fmadd_ps(d[s], _mm512_loadu_ps(q + (j + r) * kDim + 16 * s), acc[r]);
            for (int r = 0; r < 8; ++r) ip[j + r] = reduce_halves(acc[r]);
        }
        const __m512 f = _mm512_set1_ps(idx->full_factors[t]);
        mx0 = _mm512_max_ps(mx0, _mm512_mul_ps(_mm512_sub_ps(_mm512_load_ps(ip), cb0), f));
        mx1 = _mm512_max_ps(mx1, _mm512_mul_ps(_mm512_sub_ps(_mm512_load_ps(ip + 16), cb1), f));
    }
    return reduce_halves(_mm512_add_ps(mx0, mx1));
}

}  // namespace

extern "C" {

int cpu_fullbit_avx512_available(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512dq");
}

// Full-bit MaxSim of docs[q * per_query + j], j < counts[q], for query q
// (rotated [nq, 32, 128], cbex [nq, 32]) into out (same layout), with
// `threads` OpenMP threads over (query, document) pairs, dynamic schedule
// of one document (search_impl.cu:525). Returns -1 without AVX-512.
int cpu_fullbit_batch(const oracle_index* idx, const float* rotated, const float* cbex, int32_t nq, const int32_t* docs,
                      int32_t per_query, const int32_t* counts, float* out, int32_t threads) {
    if (!cpu_fullbit_avx512_available()) return -1;
    std::vector<int64_t> pairs;
    for (int32_t q = 0; q < nq; ++q)
        for (int32_t j = 0; j < counts[q] && j < per_query; ++j) pairs.push_back(static_cast<int64_t>(q) * per_query + j);
    const int64_t np = static_cast<int64_t>(pairs.size());
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : omp_get_max_threads())
    for (int64_t p = 0; p < np; ++p) {
        const int64_t e = pairs[static_cast<size_t>(p)];
        const int64_t q = e / per_query;
        out[e] = score_doc(idx, docs[e], rotated + q * kQ * kDim, cbex + q * kQ);
    }
    return 0;
}

}  // extern "C"
