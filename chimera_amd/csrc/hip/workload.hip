// Synthetic corpora and exact MaxSim ground truth on the device
// (include/chimera_workload.h).
#include "capi_internal.hpp"
#include "chimera_workload.h"
#include "common.hpp"
#include "kernels.hpp"

#include <cmath>
#include <string>

namespace chimera {

namespace {

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as
// easy as 1, 2, 3", SC 2011): ten rounds of two 32x32->64 multiplies with
// the published multipliers and Weyl key increments.
struct U4 {
    uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 philox4x32_10(U4 ctr, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = 0xD2511F53u * ctr.x;
        const uint32_t hi0 = __umulhi(0xD2511F53u, ctr.x);
        const uint32_t lo1 = 0xCD9E8D57u * ctr.z;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, ctr.z);
        ctr = U4{hi1 ^ ctr.y ^ k0, lo1, hi0 ^ ctr.w ^ k1, lo0};
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return ctr;
}

}  // namespace

// One wave per token: lane l draws dimensions 2l and 2l+1 with one
// Box-Muller pair; lane 0's remaining 64 bits pick the centre.
__global__ __launch_bounds__(256) void synth_tokens_kernel(const float* __restrict__ centres, int64_t n_centres,
                                                           uint64_t n, float sigma, uint64_t seed,
                                                           float* __restrict__ out) {
    const int l = lane_id();
    const uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
    const uint64_t waves = static_cast<uint64_t>(gridDim.x) * (blockDim.x / kWave);
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * (blockDim.x / kWave) + wave_id(); t < n; t += waves) {
        const U4 r = philox4x32_10(U4{static_cast<uint32_t>(t), static_cast<uint32_t>(t >> 32),
                                      static_cast<uint32_t>(l), 0x5EEDu},
                                   k0, k1);
        const uint64_t pick64 = (static_cast<uint64_t>(r.w) << 32) | r.z;
        const uint64_t pick_l0 = static_cast<uint64_t>(__shfl(static_cast<long long>(pick64), 0, kWave));
        const uint64_t ci = static_cast<uint64_t>((static_cast<unsigned __int128>(pick_l0) * n_centres) >> 64);
        const float u1 = (static_cast<float>(r.x >> 8) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = static_cast<float>(r.y >> 8) * (1.0f / 16777216.0f);           // [0, 1)
        const float rad = sqrtf(-2.0f * logf(u1));
        float sn, cs;
        sincosf(6.2831853071795864f * u2, &sn, &cs);
        const float2 c = reinterpret_cast<const float2*>(centres + ci * kDim)[l];
        const float a = c.x + sigma * (rad * cs);
        const float b = c.y + sigma * (rad * sn);
        float ss = a * a + b * b;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, kWave);
        const float inv = 1.0f / sqrtf(ss);
        reinterpret_cast<float2*>(out + t * kDim)[l] = make_float2(a * inv, b * inv);
    }
}

typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kGtQueriesPerBlock = 8;  // one query per wave
constexpr int kGtDocsPerBlock = 32;

// Query operand of v_mfma_f32_16x16x4_f32 for MaxSim: lane l holds query
// tokens l%16 (half 0) and 16 + l%16 (half 1), dimensions 32*(l/16) + s in
// step s.
__device__ __forceinline__ void load_query_operand(const float* __restrict__ query, int c, int g, float (&bq)[2][32]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float4* src = reinterpret_cast<const float4*>(query + (16 * h + c) * kDim + 32 * g);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 x = src[v];
            bq[h][4 * v + 0] = x.x;
            bq[h][4 * v + 1] = x.y;
            bq[h][4 * v + 2] = x.z;
            bq[h][4 * v + 3] = x.w;
        }
    }
}

// MaxSim of one document (tokens [start, end) of emb) against the query in
// bq, on the matrix cores (v_mfma_f32_16x16x4_f32). A tile of 16 document
// tokens is A (lane l: token l%16), a half of the query's 32 tokens is B, and
// lane group g = l/16 supplies dimensions g*32 + s in step s, so 32 steps
// cover all 128 dimensions. D lane l holds tokens 4g..4g+3 against query
// token l%16. The next tile's loads are issued before the current tile's
// matrix-core work; rows past the end read the last token and are masked.
// Returns sum over the 32 query tokens of the max over the document's tokens
// of <q_i, x_t> (fp32 products, fp32 accumulation), -inf for an empty
// document; every lane gets the value.
__device__ __forceinline__ float doc_maxsim(const float* __restrict__ emb, int start, int end,
                                            const float (&bq)[2][32], int c, int g) {
    float mx0 = -INFINITY, mx1 = -INFINITY;
    auto load = [&](int t0, float (&a)[32]) {
        const int tok = t0 + c < end ? t0 + c : end - 1;
        const float4* src = reinterpret_cast<const float4*>(emb + static_cast<size_t>(tok) * kDim + 32 * g);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 x = src[v];
            a[4 * v + 0] = x.x;
            a[4 * v + 1] = x.y;
            a[4 * v + 2] = x.z;
            a[4 * v + 3] = x.w;
        }
    };
    auto tile = [&](const float (&a)[32], int t0) {
        float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 32; ++s) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bq[0][s], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bq[1][s], acc1, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (t0 + 4 * g + r < end) {
                mx0 = fmaxf(mx0, acc0[r]);
                mx1 = fmaxf(mx1, acc1[r]);
            }
        }
    };
    if (start < end) {
        float a0[32], a1[32];
        load(start, a0);
        for (int t0 = start;;) {
            if (t0 + 16 < end) load(t0 + 16, a1);
            tile(a0, t0);
            t0 += 16;
            if (t0 >= end) break;
            if (t0 + 16 < end) load(t0 + 16, a0);
            tile(a1, t0);
            t0 += 16;
            if (t0 >= end) break;
        }
    }
    mx0 = fmaxf(mx0, __shfl_xor(mx0, 16, kWave));
    mx0 = fmaxf(mx0, __shfl_xor(mx0, 32, kWave));
    mx1 = fmaxf(mx1, __shfl_xor(mx1, 16, kWave));
    mx1 = fmaxf(mx1, __shfl_xor(mx1, 32, kWave));
    float v = mx0 + mx1;  // query tokens c and 16 + c
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Exact MaxSim of nq queries against every document: one query per wave, and
// all waves of a block walk the same documents, so a token tile is fetched
// from HBM once per block.
__global__ __launch_bounds__(kGtQueriesPerBlock * kWave) void exact_maxsim_kernel(
    const float* __restrict__ emb, const int32_t* __restrict__ doc_ptrs, int64_t m, const float* __restrict__ queries,
    int nq, float* __restrict__ scores) {
    const int q = blockIdx.y * kGtQueriesPerBlock + wave_id();
    if (q >= nq) return;
    const int l = lane_id();
    const int c = l & 15;
    const int g = l >> 4;
    float bq[2][32];
    load_query_operand(queries + static_cast<size_t>(q) * kQ * kDim, c, g, bq);
    const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kGtDocsPerBlock;
    const int64_t d1 = d0 + kGtDocsPerBlock < m ? d0 + kGtDocsPerBlock : m;
    for (int64_t d = d0; d < d1; ++d) {
        const float v = doc_maxsim(emb, doc_ptrs[d], doc_ptrs[d + 1], bq, c, g);
        if (l == 0) scores[static_cast<size_t>(q) * m + d] = v;
    }
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// Query operand of v_mfma_f32_16x16x32_f16 for the rescoring kernel: query
// token t (lane l holds t = l%16 in half 0, 16 + l%16 in half 1) is scaled
// by the power of two 2^sq(t) that puts its largest component in
// [512, 1024) and split into fp16 hi + lo; lane group g = l/16 supplies
// dimensions 32g + 8kk .. +7 in k step kk. inv[h] = 2^-sq of the lane's
// token in half h.
__device__ __forceinline__ void load_query_split(const float* __restrict__ query, int c, int g, half8_t (&bq)[4][2][2],
                                                 float (&inv)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float4* src = reinterpret_cast<const float4*>(query + (16 * h + c) * kDim + 32 * g);
        float v[32];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const float4 x = src[u];
            v[4 * u + 0] = x.x;
            v[4 * u + 1] = x.y;
            v[4 * u + 2] = x.z;
            v[4 * u + 3] = x.w;
        }
        float mx = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) mx = fmaxf(mx, fabsf(v[j]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        int e = 0;
        frexpf(mx > 0.0f ? mx : 1.0f, &e);
        const float sc = ldexpf(1.0f, 10 - e);
        inv[h] = ldexpf(1.0f, e - 10);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = v[8 * kk + j] * sc;
                const _Float16 hi = static_cast<_Float16>(x);
                bq[kk][h][0][j] = hi;
                bq[kk][h][1][j] = static_cast<_Float16>(x - static_cast<float>(hi));
            }
    }
}

// MaxSim of one document against a split query (load_query_split) on the
// fp16 matrix cores (v_mfma_f32_16x16x32_f16: A lane l holds row l%16,
// k (l/16)*8 .. +7; B lane l holds column l%16; D lane l holds rows
// (l/16)*4 .. +3 of column l%16). A tile of 16 document tokens is scaled by
// the power of two 2^st that puts its largest component in [512, 1024) and
// split into fp16 hi + lo; <x, q> 2^(st+sq) = xh qh + xh ql + xl qh (+ the
// dropped xl ql, below 2^-21 of |x||q|), accumulated in fp32. The max over a
// tile's rows is scaled back by 2^-st, the document's max by 2^-sq.
// One tile's loads at a time: three waves per SIMD hide their latency
// (a second tile in registers would leave two).
// Rows past the end read the last token and are masked; -inf for an empty
// document; every lane gets the value.
__device__ __forceinline__ float doc_maxsim_split(const float* __restrict__ emb, int start, int end,
                                                  const half8_t (&bq)[4][2][2], const float (&inv)[2], int c,
                                                  int g) {
    float mx0 = -INFINITY, mx1 = -INFINITY;
    auto load = [&](int t0, float (&a)[32]) {
        const int tok = t0 + c < end ? t0 + c : end - 1;
        const float4* src = reinterpret_cast<const float4*>(emb + static_cast<size_t>(tok) * kDim + 32 * g);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 x = src[v];
            a[4 * v + 0] = x.x;
            a[4 * v + 1] = x.y;
            a[4 * v + 2] = x.z;
            a[4 * v + 3] = x.w;
        }
    };
    auto tile = [&](const float (&a)[32], int t0) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) m = fmaxf(m, fabsf(a[j]));
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
        int e = 0;
        frexpf(m > 0.0f ? m : 1.0f, &e);
        const float sc = ldexpf(1.0f, 10 - e);
        float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            half8_t xh, xl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = a[8 * kk + j] * sc;
                const _Float16 hi = static_cast<_Float16>(x);
                xh[j] = hi;
                xl[j] = static_cast<_Float16>(x - static_cast<float>(hi));
            }
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq[kk][0][0], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq[kk][1][0], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq[kk][0][1], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq[kk][1][1], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bq[kk][0][0], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bq[kk][1][0], acc1, 0, 0, 0);
        }
        float t0m = -INFINITY, t1m = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (t0 + 4 * g + r < end) {
                t0m = fmaxf(t0m, acc0[r]);
                t1m = fmaxf(t1m, acc1[r]);
            }
        }
        const float is = ldexpf(1.0f, e - 10);
        mx0 = fmaxf(mx0, t0m * is);
        mx1 = fmaxf(mx1, t1m * is);
    };
    for (int t0 = start; t0 < end; t0 += 16) {
        float a0[32];
        load(t0, a0);
        tile(a0, t0);
    }
    mx0 = fmaxf(mx0, __shfl_xor(mx0, 16, kWave));
    mx0 = fmaxf(mx0, __shfl_xor(mx0, 32, kWave));
    mx1 = fmaxf(mx1, __shfl_xor(mx1, 16, kWave));
    mx1 = fmaxf(mx1, __shfl_xor(mx1, 32, kWave));
    float v = mx0 * inv[0] + mx1 * inv[1];  // query tokens c and 16 + c
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

constexpr int kRescoreWaves = 4;
constexpr int kRescoreDocsPerBlock = 16;
// the top-k sorts a query's candidates in LDS as 8-byte keys: 64 KB
constexpr int kRescoreMaxCandidates = 8192;
constexpr int kStageRescore = 13;
constexpr int kStageRescoreTopk = 14;

// MaxSim of each query's candidate documents (doc_maxsim_split: fp16
// matrix cores, split operands): block (x, q) takes candidates
// x * kRescoreDocsPerBlock .. +kRescoreDocsPerBlock - 1 of query q, one per
// wave at a time. Candidates with an id outside [0, m) score -inf.
__global__ __launch_bounds__(kRescoreWaves * kWave) void maxsim_rescore_kernel(
    const float* __restrict__ emb, const int32_t* __restrict__ doc_ptrs, int64_t m, const float* __restrict__ queries,
    const int32_t* __restrict__ cand_ids, const int32_t* __restrict__ cand_counts, int cap,
    float* __restrict__ scores) {
    const int q = blockIdx.y;
    const int cnt = cand_counts[q];
    const int n = cnt < 0 ? 0 : (cnt < cap ? cnt : cap);
    const int j0 = static_cast<int>(blockIdx.x) * kRescoreDocsPerBlock;
    const int j1 = j0 + kRescoreDocsPerBlock < n ? j0 + kRescoreDocsPerBlock : n;
    if (j0 >= j1) return;
    const int l = lane_id();
    const int c = l & 15;
    const int g = l >> 4;
    half8_t bq[4][2][2];
    float inv[2];
    load_query_split(queries + static_cast<size_t>(q) * kQ * kDim, c, g, bq, inv);
    for (int j = j0 + wave_id(); j < j1; j += kRescoreWaves) {
        const int32_t d = cand_ids[static_cast<size_t>(q) * cap + j];
        float v = -INFINITY;
        if (d >= 0 && d < m) v = doc_maxsim_split(emb, doc_ptrs[d], doc_ptrs[d + 1], bq, inv, c, g);
        if (l == 0) scores[static_cast<size_t>(q) * cap + j] = v;
    }
}


// Matrix-core throughput with register operands: every wave runs `iters`
// rounds of independent accumulation chains of one instruction type on
// operands derived from seed words (random bits; kind 2 keeps only 0/1 in
// the A operand, as the one-bit refine's code bits), so no memory traffic
// limits the rate and the GPU's clock under that load decides it; acc
// keeps the results alive.
typedef __bf16 mc_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mc_f16x8 __attribute__((ext_vector_type(8)));
typedef float mc_f4 __attribute__((ext_vector_type(4)));
typedef float mc_f16 __attribute__((ext_vector_type(16)));
typedef int mc_i4 __attribute__((ext_vector_type(4)));
typedef int mc_i16 __attribute__((ext_vector_type(16)));

template <int kKind>
__global__ __launch_bounds__(256) void matrix_core_loop_kernel(int iters, uint32_t seed, float* __restrict__ acc) {
    uint32_t w[8];
    uint32_t x = seed ^ (blockIdx.x * 256u + threadIdx.x) * 0x9E3779B9u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x ^= x << 13;
        x ^= x >> 17;
        x ^= x << 5;
        w[i] = x;
    }
    float out = 0.0f;
    if constexpr (kKind == 0 || kKind == 1 || kKind == 2 || kKind == 5) {
        // 16-bit operands with exponents below 2^1 (finite products)
        uint32_t a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = kKind == 2 || kKind == 5 ? w[i] & 0x3C003C00u : w[i] & 0x3BFF3BFFu;
            b[i] = w[4 + i] & 0x3BFF3BFFu;
        }
        if constexpr (kKind == 0) {
            mc_bf16x8 av, bv;
            __builtin_memcpy(&av, a, 16);
            __builtin_memcpy(&bv, b, 16);
            mc_f16 c0 = {}, c1 = {};
            for (int it = 0; it < iters; ++it) {
                c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, c1, 0, 0, 0);
            }
            out = c0[0] + c1[1];
        } else {
            mc_f16x8 av, bv;
            __builtin_memcpy(&av, a, 16);
            __builtin_memcpy(&bv, b, 16);
            mc_f4 c0 = {}, c1 = {}, c2 = {}, c3 = {};
            // kind 5: four independent one-cycle integer VALU instructions
            // after each MFMA (emitted as written, on registers no MFMA reads)
            uint32_t x0 = w[0], x1 = w[1], x2 = w[2], x3 = w[3];
            const uint32_t y = w[5];
            auto valu4 = [&]() {
                if constexpr (kKind == 5) {
                    asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x0) : "v"(y));
                    asm volatile("v_add_u32 %0, %0, %1" : "+v"(x1) : "v"(y));
                    asm volatile("v_xor_b32 %0, %0, %1" : "+v"(x2) : "v"(y));
                    asm volatile("v_add_u32 %0, %0, %1" : "+v"(x3) : "v"(y));
                }
            };
            for (int it = 0; it < iters; ++it) {
                c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c0, 0, 0, 0);
                valu4();
                c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c1, 0, 0, 0);
                valu4();
                c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c2, 0, 0, 0);
                valu4();
                c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c3, 0, 0, 0);
                valu4();
            }
            out = c0[0] + c1[1] + c2[2] + c3[3] + static_cast<float>((x0 ^ x1 ^ x2 ^ x3) & 1u);
        }
    } else if constexpr (kKind == 3) {
        const float av = __uint_as_float((w[0] & 0x3FFFFFFFu) | 0x30000000u);
        const float bv = __uint_as_float((w[1] & 0x3FFFFFFFu) | 0x30000000u);
        mc_f16 c0 = {}, c1 = {};
        for (int it = 0; it < iters; ++it) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, c1, 0, 0, 0);
        }
        out = c0[0] + c1[1];
    } else {
        mc_i4 av, bv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            av[i] = static_cast<int>(w[i]);
            bv[i] = static_cast<int>(w[4 + i]);
        }
        mc_i16 c0 = {}, c1 = {};
        for (int it = 0; it < iters; ++it) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, c1, 0, 0, 0);
        }
        out = static_cast<float>(c0[0] + c1[1]);
    }
    acc[blockIdx.x * 256 + threadIdx.x] = out;
}

}  // namespace chimera

using namespace chimera;

extern "C" {

int chimera_synth_tokens_device(chimera_ctx* ctx, const float* d_centres, int64_t n_centres, int32_t dim, uint64_t n,
                                float sigma, uint64_t seed, float* d_out) {
    hipStream_t s;
    const int rc = api_enter(ctx, &s);
    if (rc != CHIMERA_OK) return rc;
    if (dim != kDim) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "synthetic tokens are generated with dim 128 only");
    if (n_centres <= 0 || !d_centres || (n > 0 && !d_out))
        return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "synthetic tokens need centres and an output buffer");
    if (n == 0) return CHIMERA_OK;
    const uint64_t waves = n < (uint64_t{1} << 20) ? n : (uint64_t{1} << 20);
    const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
    hipLaunchKernelGGL(synth_tokens_kernel, dim3(blocks), dim3(256), 0, s, d_centres, n_centres, n, sigma, seed, d_out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return api_fail(CHIMERA_ERR_HIP, std::string("synthetic token kernel failed: ") + hipGetErrorString(e));
    return CHIMERA_OK;
}

int chimera_gather_rows_device(chimera_ctx* ctx, const float* d_src, int32_t dim, const int64_t* d_ids, int64_t n,
                               float* d_out) {
    hipStream_t s;
    const int rc = api_enter(ctx, &s);
    if (rc != CHIMERA_OK) return rc;
    if (dim < 1 || dim > kDim) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "row dimension must be in [1, 128]");
    if (n < 0) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "negative row count");
    if (n == 0) return CHIMERA_OK;
    if (!d_src || !d_ids || !d_out) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    const hipError_t e = launch_gather_rows(s, d_src, dim, d_ids, n, nullptr, false, d_out);
    if (e != hipSuccess) return api_fail(CHIMERA_ERR_HIP, std::string("row gather failed: ") + hipGetErrorString(e));
    return CHIMERA_OK;
}

int chimera_exact_maxsim_device(chimera_ctx* ctx, const float* d_embeddings, const int32_t* d_doc_ptrs,
                                int64_t num_docs, const float* d_queries, int32_t nq, float* d_scores) {
    hipStream_t s;
    const int rc = api_enter(ctx, &s);
    if (rc != CHIMERA_OK) return rc;
    if (num_docs < 0 || nq < 0) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "negative size");
    if (num_docs == 0 || nq == 0) return CHIMERA_OK;
    if (!d_embeddings || !d_doc_ptrs || !d_queries || !d_scores) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    const int64_t bx = (num_docs + kGtDocsPerBlock - 1) / kGtDocsPerBlock;
    if (bx > 0x7FFFFFFF) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "too many documents");
    const dim3 grid(static_cast<unsigned>(bx), static_cast<unsigned>((nq + kGtQueriesPerBlock - 1) / kGtQueriesPerBlock));
    hipLaunchKernelGGL(exact_maxsim_kernel, grid, dim3(kGtQueriesPerBlock * kWave), 0, s, d_embeddings, d_doc_ptrs,
                       num_docs, d_queries, nq, d_scores);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return api_fail(CHIMERA_ERR_HIP, std::string("exact MaxSim kernel failed: ") + hipGetErrorString(e));
    return CHIMERA_OK;
}

int chimera_maxsim_rescore_device(chimera_ctx* ctx, const float* d_embeddings, const int32_t* d_doc_ptrs,
                                  int64_t num_docs, const float* d_queries, int32_t nq, const int32_t* d_cand_ids,
                                  const int32_t* d_cand_counts, int32_t cand_cap, int32_t k, float* d_cand_scores,
                                  int64_t* d_top_ids, float* d_top_scores, int32_t* d_top_counts) {
    hipStream_t s;
    const int rc = api_enter(ctx, &s);
    if (rc != CHIMERA_OK) return rc;
    if (num_docs < 0 || nq < 0 || k < 0) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "negative size");
    if (cand_cap < 1 || cand_cap > kRescoreMaxCandidates)
        return api_fail(CHIMERA_ERR_INVALID_ARGUMENT,
                        "candidate capacity must be in [1, " + std::to_string(kRescoreMaxCandidates) + "]");
    if (nq > 65535) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "at most 65535 queries per call");
    if (nq == 0) return CHIMERA_OK;
    if (!d_embeddings || !d_doc_ptrs || !d_queries || !d_cand_ids || !d_cand_counts || !d_cand_scores)
        return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    if (k > 0 && (!d_top_ids || !d_top_counts)) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "null top-k output");
    const dim3 grid(static_cast<unsigned>((cand_cap + kRescoreDocsPerBlock - 1) / kRescoreDocsPerBlock),
                    static_cast<unsigned>(nq));
    stage_begin(ctx, kStageRescore);
    hipLaunchKernelGGL(maxsim_rescore_kernel, grid, dim3(kRescoreWaves * kWave), 0, s, d_embeddings, d_doc_ptrs,
                       num_docs, d_queries, d_cand_ids, d_cand_counts, cand_cap, d_cand_scores);
    hipError_t e = hipGetLastError();
    stage_end(ctx);
    if (e != hipSuccess) return api_fail(CHIMERA_ERR_HIP, std::string("MaxSim rescoring kernel failed: ") + hipGetErrorString(e));
    if (k == 0) return CHIMERA_OK;
    stage_begin(ctx, kStageRescoreTopk);
    e = launch_final_topk(s, nq, d_cand_counts, d_cand_ids, d_cand_scores, cand_cap, k, d_top_ids, d_top_scores,
                          d_top_counts);
    stage_end(ctx);
    if (e != hipSuccess) return api_fail(CHIMERA_ERR_HIP, std::string("rescoring top-k kernel failed: ") + hipGetErrorString(e));
    return CHIMERA_OK;
}

int chimera_matrix_core_rate(chimera_ctx* ctx, int32_t kind, int32_t iters, double* ops_per_second) {
    hipStream_t s;
    const int rc = api_enter(ctx, &s);
    if (rc != CHIMERA_OK) return rc;
    if (kind < 0 || kind > 5) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "matrix-core kind must be in [0, 5]");
    if (iters < 1 || iters > 1000000) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "iters must be in [1, 1000000]");
    if (!ops_per_second) return api_fail(CHIMERA_ERR_INVALID_ARGUMENT, "null argument");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess || cus < 1)
        return api_fail(CHIMERA_ERR_HIP, "device attributes");
    // two 256-thread blocks per SIMD: 8 waves per SIMD keep every chain fed
    const int blocks = cus * 8;
    // {ops per instruction} x {instructions per round}
    static const double kOps[6] = {2.0 * 32 * 32 * 16 * 2, 2.0 * 16 * 16 * 32 * 4, 2.0 * 16 * 16 * 32 * 4,
                                   2.0 * 32 * 32 * 2 * 2,  2.0 * 32 * 32 * 32 * 2, 2.0 * 16 * 16 * 32 * 4};
    float* acc = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&acc, static_cast<size_t>(blocks) * 256 * sizeof(float));
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    float ms = 0.0f;
    // three launches to bring the clock to its level under this load, then
    // the timed one
    for (int rep = 0; rep < 4 && e == hipSuccess; ++rep) {
        if (rep == 3) e = hipEventRecord(e0, s);
        if (e != hipSuccess) break;
        switch (kind) {
            case 0: hipLaunchKernelGGL(matrix_core_loop_kernel<0>, dim3(blocks), dim3(256), 0, s, iters, 12345u, acc); break;
            case 1: hipLaunchKernelGGL(matrix_core_loop_kernel<1>, dim3(blocks), dim3(256), 0, s, iters, 12345u, acc); break;
            case 2: hipLaunchKernelGGL(matrix_core_loop_kernel<2>, dim3(blocks), dim3(256), 0, s, iters, 12345u, acc); break;
            case 3: hipLaunchKernelGGL(matrix_core_loop_kernel<3>, dim3(blocks), dim3(256), 0, s, iters, 12345u, acc); break;
            case 5: hipLaunchKernelGGL(matrix_core_loop_kernel<5>, dim3(blocks), dim3(256), 0, s, iters, 12345u, acc); break;
            default: hipLaunchKernelGGL(matrix_core_loop_kernel<4>, dim3(blocks), dim3(256), 0, s, iters, 12345u, acc); break;
        }
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(e1, s);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (acc) (void)hipFree(acc);
    if (e != hipSuccess) return api_fail(CHIMERA_ERR_HIP, std::string("matrix-core loop failed: ") + hipGetErrorString(e));
    const double total = static_cast<double>(blocks) * 4.0 * iters * kOps[kind];
    *ops_per_second = ms > 0.0f ? total / (static_cast<double>(ms) * 1e-3) : 0.0;
    return CHIMERA_OK;
}

}  // extern "C"
