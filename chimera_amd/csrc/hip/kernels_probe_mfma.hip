// Centroid probe on the matrix cores with labels equal to the exact fp32
// probe (|c|^2 - 2<q,c> by sequential fmaf, ties to the lower ID).
//
//   pass A  bf16 MFMA scores d' of every query row against a sample of
//           32-centroid tiles; per (row, group of sampled tiles) the
//           minimum d'.
//   thresh  thr = U + 2*delta, U the u_rank-th smallest group minimum, where
//           delta bounds |d' - d| for every centroid of the row (probe_delta:
//           the bf16 rounding of both operands through |q - q_b| and
//           max |c - c_b|, plus the fp32 accumulation of either order).
//           With one tile in s sampled, U sits near the centroid of rank
//           s * u_rank = 2 nprobe: an estimate, which the rerank checks.
//   pass B  bf16 MFMA scores of every centroid; a lane whose 16 values hold
//           a d' <= thr stores them (as v = acc + thr/2, fp16 rounded
//           toward zero) with their tile into the row's records.
//   rerank  the candidates (v >= 0) of the records; v* = their nprobe-th
//           largest v. If v* >= delta (less the fp16 error), nprobe
//           centroids have d' <= thr - 2 delta, hence d <= thr - delta, so
//           the exact nprobe-th best T <= thr - delta and every exact
//           top-nprobe centroid c has d'(c) <= T + delta <= thr: all of them
//           are candidates. Candidates with v >= v* - delta - (fp16 error)
//           are rescored in fp32 and sorted by (score, id).
// Rows whose records overflow or whose v* fails the check are flagged and
// recomputed by the exact kernel, so labels never depend on the estimate.
//
// MFMA: v_mfma_f32_32x32x16_bf16 with centroids as A (rows i, 32 per tile)
// and query rows as B (columns j): lane l holds column l%32 and tile rows
// (r/4)*8 + (l/32)*4 + r%4 of the accumulator, so one lane compares 16
// centroids against one row's threshold. The accumulators start at
// -|c|^2/2, so acc = <q_b,c_b> - |c|^2/2 = -d'/2 and d' <= t is acc >= -t/2
// (exact: scaling by powers of two): the per-tile test is a max over the
// lane's 16 values and one compare, with no per-value arithmetic.
#include <cmath>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace chimera {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

namespace {

constexpr int kProbeWaves = 8;                 // waves per block
constexpr int kRowsPerWave = 64;               // 2 column blocks of 32
constexpr int kColBlocks = kRowsPerWave / 32;
constexpr int kRowsPerBlock = kProbeWaves * kRowsPerWave;
constexpr int kStageTiles = 8;                 // 32-centroid tiles staged per iteration
constexpr int kGroupTiles = 4;                 // sampled tiles per group minimum of the sampled pass (large k)
constexpr int kTileBytes = 32 * kDim * 2;      // 32 centroid rows of 256 B, chunks swizzled
constexpr int kWaitVmcnt0 = 0x0F70;            // s_waitcnt vmcnt(0), expcnt and lgkmcnt not waited on
constexpr int kProbeLaneCap = 128;             // sub-list entries per (row, split, lane half) of the probe
constexpr int kProbeMaxCandidates = 2048;      // candidates per row the rerank sorts in LDS
constexpr int kTop1LaneCap = 256;              // sub-list entries of the top-1 search
constexpr int kMaxSublists = 1024;             // 2 * splits
constexpr int64_t kMaxGroups = 16384;          // sampled group minima per row of the probe

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float bf16_round(float f) { return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_rne(f)) << 16); }

// |q| and |q - q_b| of one 128-float row, q_b its bf16 (RNE) copy: sums of
// squares over the wave (lane l reads elements l and l + 64). q - q_b is
// exact in fp32 (the two are within a factor of two of each other).
__device__ __forceinline__ float2 row_norms_wave(const float* __restrict__ row) {
    const int l = lane_id();
    const float a = row[l], b = row[l + 64];
    const float ea = a - bf16_round(a), eb = b - bf16_round(b);
    float ss = a * a + b * b, es = ea * ea + eb * eb;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        ss += __shfl_xor(ss, o, kWave);
        es += __shfl_xor(es, o, kWave);
    }
    return make_float2(sqrtf(ss), sqrtf(es));
}

}  // namespace

// Bound on |d' - d| for every centroid c of one row q. d = N - 2<q,c> is the
// exact probe's score (sequential fmaf dot, N = |c|^2 from norms[]), d' =
// -2 acc with acc the matrix cores' fp32 sum of -N/2 and the 128 products
// of the bf16 operands q_b, c_b. Arguments: qn = |q|, eq = |q - q_b|, cmax
// >= max |c| and ecmax >= max |c - c_b| over the centroids.
//   <q_b,c_b> - <q,c> = <q_b - q, c_b> + <q, c_b - c>, so by Cauchy-Schwarz
//     |<q_b,c_b> - <q,c>| <= eq |c_b| + qn |c - c_b|
//                         <= eq cmax (1 + 2^-8) + qn ecmax
//     (RNE to bf16 moves each component by at most 2^-8 of itself);
//   the matrix-core sum of 129 terms of magnitude sum at most
//     |q_b||c_b| + N/2 <= 1.02 qn cmax + cmax^2 / 2 is allowed 2^-13 of that
//     (16x the 129 * 2^-24 of round-to-nearest accumulation);
//   the sequential fmaf dot carries at most 128 * 2^-24 < 2^-16 of qn cmax;
//   the final roundings of N - 2 dot and of the threshold sums U + 2 delta
//     are below 2^-22 (cmax^2 + 2 qn cmax).
// d' and d differ by twice the dot-product errors; the total is inflated by
// 2^-10 for the fp32 evaluation of this bound and of its norm arguments.
// With every component of q and c at 1 + 2^-8 - 2^-20 (each rounds down by
// almost 2^-8) the first term is reached: eq cmax + qn ecmax ~ 2^-7 qn cmax.
__host__ __device__ float probe_delta(float qn, float eq, float cmax, float ecmax) {
    const float cb = cmax * (1.0f + 0.00390625f);
    const float dot_err = eq * cb + qn * ecmax + 0.0001220703125f * (1.02f * qn * cmax + 0.5f * cmax * cmax) +
                          0.0000152587890625f * qn * cmax;
    const float round_err = 0.0000002384185791f * (cmax * cmax + 2.0f * qn * cmax);
    return (2.0f * dot_err + round_err) * (1.0f + 0.0009765625f);
}

namespace {

// Two floats converted to fp16 toward zero (v_cvt_pkrtz_f16_f32), a in the
// low half of the word: |h| <= |x|, the sign kept (a negative x gives a
// negative value or -0), and values beyond the fp16 range become +-65504.
__device__ __forceinline__ uint32_t rtz_half2_bits(float a, float b) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(a, b);
    uint32_t w;
    __builtin_memcpy(&w, &h, 4);
    return w;
}

// fp16 bits (sign clear) as a float: exact
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    _Float16 v;
    const uint16_t b = static_cast<uint16_t>(h);
    __builtin_memcpy(&v, &b, 2);
    return static_cast<float>(v);
}

// a + b rounded up and a - b rounded down (OCML's directed-rounding adds)
__device__ __forceinline__ float add_up(float a, float b) { return __ocml_add_rtp_f32(a, b); }
__device__ __forceinline__ float sub_down(float a, float b) { return __ocml_sub_rtn_f32(a, b); }

// LDS address space view of a pointer into a __shared__ array, as the
// direct-to-LDS loads take their destination
__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(void* p) {
    return (__attribute__((address_space(3))) void*)(p);
}

}  // namespace

// bf16 copies of the centroids, the probe's accumulator start -|c|^2/2 and
// max over centroids of |c - c_b| (atomicMax on the bits of a non-negative
// float into *err_max, which the caller clears). One wave per centroid.
__global__ __launch_bounds__(256) void probe_centroids_kernel(const float* __restrict__ c,
                                                              const float* __restrict__ norms, int64_t k,
                                                              uint16_t* __restrict__ out, float* __restrict__ nhalf,
                                                              uint32_t* __restrict__ err_max) {
    const int64_t cen = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave_id();
    if (cen >= k) return;
    const int l = lane_id();
    const float2 v = reinterpret_cast<const float2*>(c + cen * kDim)[l];
    const uint16_t hx = f32_to_bf16_rne(v.x), hy = f32_to_bf16_rne(v.y);
    reinterpret_cast<uint32_t*>(out + cen * kDim)[l] = static_cast<uint32_t>(hx) | (static_cast<uint32_t>(hy) << 16);
    const float ex = v.x - __uint_as_float(static_cast<uint32_t>(hx) << 16);
    const float ey = v.y - __uint_as_float(static_cast<uint32_t>(hy) << 16);
    float es = ex * ex + ey * ey;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) es += __shfl_xor(es, o, kWave);
    if (l == 0) {
        nhalf[cen] = -0.5f * norms[cen];
        atomicMax(err_max, __float_as_uint(sqrtf(es)));
    }
}

// MODE 0: minima of groups of G sampled tiles into gm[row][group]
//         (each the d' of a distinct centroid).
// MODE 1: every (tile, lane) whose 16 values hold a d' <= thr[row] appends a
//         record to the lane's own sub-list L = (row * splits + split) * 2 + hk:
//         the tile into rtile[L * lane_cap + n], the 16 values v = acc - th
//         (th = -thr/2; the fp32 difference converted to fp16 toward zero,
//         two per word) into rval[(L * lane_cap + n) * 2 ...] as two 16-byte
//         halves; the record count goes to cnt[L] (no atomics). A hit is
//         acc >= th, which is v >= 0: the sign of the fp32 difference, which
//         the conversion keeps (-0 for tiny misses). The rerank picks the
//         hits out of the records.
// MODE 2: minimum d' over the sampled tiles into ukey[row] (ordered key).
// MODE 3: candidates {id, d' bits} with d' <= ukey[row] + 2 * probe_delta of
//         the row into buf[L * lane_cap ...], their number into cnt[L].
//
// Staging: the tiles of a stage go from global memory straight into LDS
// (global_load_lds_dwordx4, no registers on the way), into one of two
// separately declared buffers, so the compiler sees that the reads of one
// buffer do not depend on the loads still landing in the other. A tile is
// 32 unpadded 256-byte centroid rows; chunk h (16 bytes) of centroid c sits
// at c * 256 + 16 * (h ^ (c & 15)), so 16 lanes reading the same chunk of
// 16 consecutive centroids cover all 16 bank groups of 256 bytes.
// Slots of tiles past the split or past k load centroid 0 and get the
// initial value -inf, which makes every accumulator of theirs -inf: never
// a hit and never a minimum.
template <int MODE, int G = kGroupTiles>
__global__ __launch_bounds__(kProbeWaves * kWave) void probe_mfma_kernel(
    const float* __restrict__ rot, int nrows, const uint16_t* __restrict__ cbf, const float* __restrict__ nhalf,
    int64_t k, int tiles_per_split, int sample_stride, float* __restrict__ gm, const float* __restrict__ thr,
    uint2* __restrict__ buf, uint4* __restrict__ rval, uint32_t* __restrict__ rtile, uint32_t* __restrict__ cnt,
    int lane_cap, uint32_t* __restrict__ row_flag, uint32_t* __restrict__ ukey, float cmax, float ecmax,
    int row_blocks, int splits) {
    __shared__ __align__(16) unsigned char stage0[kStageTiles * kTileBytes];
    __shared__ __align__(16) unsigned char stage1[kStageTiles * kTileBytes];
    __shared__ __align__(16) float snorm0[kStageTiles * 32];
    __shared__ __align__(16) float snorm1[kStageTiles * 32];
    __shared__ float gbuf[MODE == 0 ? kRowsPerBlock * 8 : 1];  // MODE 0: [row of the block][column mod 8]
    const int l = lane_id();
    const int w = wave_id();
    const int j = l & 31;
    const int hk = l >> 5;  // k half within a 16-wide k step
    // 1-D grid of row_blocks * splits blocks. The XCDs take block ids
    // round-robin; with splits a multiple of 8, XCD x runs only splits x,
    // x + 8, ..., row blocks fastest, so the blocks resident on one XCD stream
    // the same centroid tiles at the same time and share its L2.
    int rb, sp;
    if (splits % 8 == 0) {
        const int kx = static_cast<int>(blockIdx.x) >> 3;
        sp = (static_cast<int>(blockIdx.x) & 7) + 8 * (kx / row_blocks);
        rb = kx % row_blocks;
    } else {
        rb = static_cast<int>(blockIdx.x) % row_blocks;
        sp = static_cast<int>(blockIdx.x) / row_blocks;
    }
    const int row0 = rb * kRowsPerBlock + w * kRowsPerWave;
    const int64_t ntiles = (k + 31) / 32;
    const int64_t n_sampled = (ntiles + sample_stride - 1) / sample_stride;
    static_assert(kStageTiles % G == 0, "whole groups per stage");
    constexpr int kGroupsPerStage = kStageTiles / G;
    const int64_t n_groups = (n_sampled + G - 1) / G;
    const int64_t t_begin = static_cast<int64_t>(sp) * tiles_per_split;
    const int64_t t_end = min<int64_t>(ntiles, t_begin + tiles_per_split);

    // query operands (bf16, RNE) for this wave's column blocks
    bf16x8_t bq[kColBlocks][8];
    float th[kColBlocks];    // acc-space threshold -t/2: hit iff acc >= th
    float rmax[kColBlocks];  // MODE 2: max acc = -(min d')/2
    int lcnt[kColBlocks];
    float gmax[kColBlocks][kGroupsPerStage];
    size_t sub[kColBlocks];  // first entry of the lane's sub-list
#pragma unroll
    for (int cb = 0; cb < kColBlocks; ++cb) {
        const int row = row0 + 32 * cb + j;
        const bool ok = row < nrows;
        const float* src = rot + static_cast<size_t>(ok ? row : 0) * kDim;
        float ss = 0.0f, es = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = ok ? src[16 * s + 8 * hk + e] : 0.0f;
                const uint16_t h = f32_to_bf16_rne(v);
                if (MODE == 3) {
                    const float ev = v - __uint_as_float(static_cast<uint32_t>(h) << 16);
                    ss = __fmaf_rn(v, v, ss);
                    es = __fmaf_rn(ev, ev, es);
                }
                __bf16 b;
                __builtin_memcpy(&b, &h, 2);
                bq[cb][s][e] = b;
            }
        rmax[cb] = -INFINITY;
        lcnt[cb] = 0;
        sub[cb] = ((static_cast<size_t>(ok ? row : 0) * splits + sp) * 2 + hk) * lane_cap;
        if (MODE == 1) {
            th[cb] = ok ? -0.5f * thr[row] : INFINITY;
        } else if (MODE == 3) {
            // the two lane halves hold the two halves of the row
            const float qn = sqrtf(ss + __shfl_xor(ss, 32, kWave));
            const float eq = sqrtf(es + __shfl_xor(es, 32, kWave));
            th[cb] = ok ? -0.5f * (ordered_to_float(ukey[row]) + 2.0f * probe_delta(qn, eq, cmax, ecmax)) : INFINITY;
        } else {
            th[cb] = INFINITY;
        }
    }

    // iterate over tiles of this split (every sample_stride-th in MODE 0 and 2),
    // kStageTiles at a time through the two LDS buffers
    auto tile_of = [&](int64_t it) -> int64_t { return t_begin + it * sample_stride; };
    const int64_t n_it_tiles = (t_end - t_begin + sample_stride - 1) / sample_stride;
    const int64_t n_iter = (n_it_tiles + kStageTiles - 1) / kStageTiles;

    // thread t fills slot t (centroid t/16, swizzled chunk) of every tile of
    // the stage; waves 0..3 fill the stage's 256 initial values
    static_assert(kProbeWaves * kWave == 32 * 16, "one 16-byte slot per thread per tile");
    static_assert(kStageTiles * 32 <= kProbeWaves * kWave, "one initial value per thread at most");
    static_assert(kColBlocks == 2, "the skewed tile schedule pairs two column blocks");
    const int fc = static_cast<int>(threadIdx.x) >> 4;
    const int fh = (static_cast<int>(threadIdx.x) & 15) ^ (fc & 15);
    auto fetch = [&](int64_t iter, unsigned char* sb, float* nb) {
#pragma unroll
        for (int tt = 0; tt < kStageTiles; ++tt) {
            const int64_t it = iter * kStageTiles + tt;
            const int64_t cen = tile_of(it) * 32 + fc;
            const int64_t src = it < n_it_tiles && cen < k ? cen : 0;
            __builtin_amdgcn_global_load_lds(cbf + src * kDim + fh * 8, lds_ptr(sb + tt * kTileBytes + w * 1024), 16, 0,
                                             0);
        }
        if (w * kWave < kStageTiles * 32) {
            const int n = w * kWave + l;
            const int64_t it = iter * kStageTiles + (n >> 5);
            const int64_t cen = tile_of(it) * 32 + (n & 31);
            if (it < n_it_tiles && cen < k) {
                __builtin_amdgcn_global_load_lds(nhalf + cen, lds_ptr(nb + w * kWave), 4, 0, 0);
            } else {
                nb[n] = -INFINITY;
            }
        }
    };

    // MODE 0: tiles_per_split is a multiple of kStageTiles * sample_stride,
    // so stage iter of this split holds groups gcol0 + kGroupsPerStage * iter + h
    const int64_t gcol0 = (t_begin / sample_stride) / G;
    auto compute = [&](int64_t iter, const unsigned char* sb, const float* nb) {
        if (row0 >= nrows) return;
#pragma unroll
        for (int cb = 0; cb < kColBlocks; ++cb)
#pragma unroll
            for (int h = 0; h < kGroupsPerStage; ++h) gmax[cb][h] = -INFINITY;
        // A fragment s of a tile (eight 16-byte reads per lane per tile)
        auto load_a = [&](int tt, int s) {
            const unsigned char* tb = sb + tt * kTileBytes + j * (kDim * 2);
            bf16x8_t f;
            const uint4 v = *reinterpret_cast<const uint4*>(tb + (((2 * s + hk) ^ (j & 15)) << 4));
            __builtin_memcpy(&f, &v, 16);
            return f;
        };
        // per-tile test of one column block (16 values per lane)
        auto check = [&](int cb, const float16_t& acc, int64_t tile, int tt) {
            float m = acc[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) m = fmaxf(m, acc[r]);
            if (MODE == 0 || MODE == 2) {
                m = wave_max_xor32(m);
                if (MODE == 2) {
                    rmax[cb] = fmaxf(rmax[cb], m);
                } else {
                    gmax[cb][tt / G] = fmaxf(gmax[cb][tt / G], m);
                }
            } else if (MODE == 1) {
                // a lane with a hit stores its whole tile column (no
                // per-value tests here: the rerank does them)
                const bool hit = m >= th[cb];  // th is +inf past the last row
                if (hit && lcnt[cb] < lane_cap) {
                    const size_t e = sub[cb] + static_cast<size_t>(lcnt[cb]);
                    const float t = th[cb];
                    auto pk = [&](int r) { return rtz_half2_bits(acc[r] - t, acc[r + 1] - t); };
                    uint4* dv = rval + e * 2;
                    dv[0] = make_uint4(pk(0), pk(2), pk(4), pk(6));
                    dv[1] = make_uint4(pk(8), pk(10), pk(12), pk(14));
                    rtile[e] = static_cast<uint32_t>(tile);
                }
                lcnt[cb] += hit ? 1 : 0;
            } else if (m >= th[cb]) {  // MODE 3; th is +inf past the last row
                // four values at a time, then one at a time: the wave
                // skips what no lane hits, so a rare hit costs a
                // compare per group of four and per value of one group
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const float mg = fmaxf(fmaxf(acc[4 * g4], acc[4 * g4 + 1]), fmaxf(acc[4 * g4 + 2], acc[4 * g4 + 3]));
                    if (mg >= th[cb]) {
#pragma unroll
                        for (int rr = 0; rr < 4; ++rr) {
                            const int r = 4 * g4 + rr;
                            if (acc[r] >= th[cb]) {
                                const int64_t cen = tile * 32 + g4 * 8 + hk * 4 + rr;
                                if (lcnt[cb] < lane_cap)
                                    buf[sub[cb] + lcnt[cb]] = make_uint2(static_cast<uint32_t>(cen),
                                                                         __float_as_uint(-2.0f * acc[r]));
                                ++lcnt[cb];
                            }
                        }
                    }
                }
            }
        };
        // accumulators start at -|c|^2/2 of the lane's 16 centroids: the
        // first MFMA of each chain takes them as its C operand from
        // registers loaded one tile ahead, so no chain waits on LDS for them
        auto ninit = [&](int tt) {
            float16_t v16;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 v = *reinterpret_cast<const float4*>(&nb[tt * 32 + g * 8 + hk * 4]);
                v16[4 * g + 0] = v.x;
                v16[4 * g + 1] = v.y;
                v16[4 * g + 2] = v.z;
                v16[4 * g + 3] = v.w;
            }
            return v16;
        };
        // One register set holds the A fragments: fragment s of the next
        // tile replaces fragment s of this one once the second chain has
        // issued its MFMA s, eight MFMAs before the next tile needs it.
        float16_t acc1;
        float16_t nx = ninit(0);
        bf16x8_t a[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) a[s] = load_a(0, s);
#pragma unroll
        for (int tt = 0; tt < kStageTiles; ++tt) {
            const int64_t tile = tile_of(iter * kStageTiles + tt);
            const bool more = tt + 1 < kStageTiles;
            // Skewed schedule: the check of one column block's tile runs
            // after the other column block's MFMA chain has been issued, so
            // its results are ready and the matrix cores are not left idle
            // while the check waits on them (chains of dependent MFMAs issue
            // back to back). Column block 1 of the last tile is checked
            // after the loop.
            float16_t acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], bq[0][0], nx, 0, 0, 0);
#pragma unroll
            for (int s = 1; s < 8; ++s) acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq[0][s], acc0, 0, 0, 0);
            if (tt > 0) check(1, acc1, tile - sample_stride, tt - 1);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], bq[1][0], nx, 0, 0, 0);
            if (more) {
                nx = ninit(tt + 1);
                a[0] = load_a(tt + 1, 0);
            }
#pragma unroll
            for (int s = 1; s < 8; ++s) {
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], bq[1][s], acc1, 0, 0, 0);
                if (more) a[s] = load_a(tt + 1, s);
            }
            check(0, acc0, tile, tt);
        }
        check(1, acc1, tile_of(iter * kStageTiles + kStageTiles - 1), kStageTiles - 1);
        if (MODE == 0) {
            // The wave's group minima gather in LDS and leave as runs of up
            // to 8 consecutive groups per row (32-byte writes instead of
            // scattered 4-byte ones); runs end at multiples of 8 columns.
            const int64_t col = gcol0 + kGroupsPerStage * iter;
            float* gb = gbuf + w * kRowsPerWave * 8;
            if (hk == 0) {
#pragma unroll
                for (int cb = 0; cb < kColBlocks; ++cb)
#pragma unroll
                    for (int h = 0; h < kGroupsPerStage; ++h)
                        gb[(32 * cb + j) * 8 + static_cast<int>((col + h) & 7)] = -2.0f * gmax[cb][h];
            }
            const int64_t last = col + kGroupsPerStage - 1;
            const int slotc = static_cast<int>(last & 7);
            if (slotc == 7 || iter + 1 == n_iter) {
                wave_lds_sync();
                const int64_t cbase = last - slotc;
                const int s0 = cbase < gcol0 ? static_cast<int>(gcol0 - cbase) : 0;
                for (int v = l; v < kRowsPerWave * 8; v += kWave) {
                    const int rl = v >> 3, sl = v & 7;
                    const int row = row0 + rl;
                    if (sl >= s0 && sl <= slotc && row < nrows && cbase + sl < n_groups)
                        gm[static_cast<size_t>(row) * n_groups + cbase + sl] = gb[rl * 8 + sl];
                }
                wave_lds_sync();  // the next run overwrites the slots
            }
        }
    };

    // Stage iter is read from buffer iter % 2. At the top of each stage the
    // wave's own loads have landed (vmcnt 0) and the barrier makes every
    // wave's visible; it also ends the reads of the other buffer, which the
    // loads of the next stage then overwrite.
    if (n_iter > 0) fetch(0, stage0, snorm0);
    for (int64_t iter = 0; iter < n_iter; iter += 2) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        if (iter + 1 < n_iter) fetch(iter + 1, stage1, snorm1);
        compute(iter, stage0, snorm0);
        if (iter + 1 >= n_iter) break;
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        if (iter + 2 < n_iter) fetch(iter + 2, stage0, snorm0);
        compute(iter + 1, stage1, snorm1);
    }
    if (MODE == 2) {
#pragma unroll
        for (int cb = 0; cb < kColBlocks; ++cb) {
            const int row = row0 + 32 * cb + j;
            if (hk == 0 && row < nrows) atomicMin(&ukey[row], float_to_ordered(-2.0f * rmax[cb]));
        }
    }
    if (MODE == 1 || MODE == 3) {
#pragma unroll
        for (int cb = 0; cb < kColBlocks; ++cb) {
            const int row = row0 + 32 * cb + j;
            if (row < nrows) {
                cnt[(static_cast<size_t>(row) * splits + sp) * 2 + hk] =
                    static_cast<uint32_t>(lcnt[cb] < lane_cap ? lcnt[cb] : lane_cap);
                if (lcnt[cb] > lane_cap) row_flag[row] = 1u;
            }
        }
    }
}

// The sampled and filtered passes on fp32 operands (v_mfma_f32_32x32x2_f32):
// the same tiles, accumulator layout, group minima and records as
// probe_mfma_kernel, so the threshold, rerank and exact fallback are shared.
// With exact operands d' differs from d only by the accumulation orders, so
// the margin is probe_delta with no rounding of q or c (eq = ecmax = 0) and
// far fewer centroids lie between the nprobe-th and thr.
//
// A block is 16 waves of one 32-row column block each (512 rows, as
// probe_mfma_kernel): a wave's 64 query values per lane fit with four
// waves per SIMD. K ordering: the sum over the 128 dimensions is order-free
// for the filter, so MFMA step s (0..63) takes dimension 64 * hk + s in lane
// half hk (A and B alike): a lane's query values and each 16-byte A read are
// contiguous. Staging: fp32 tiles of 32 rows of 512 bytes, four tiles per
// stage (two 64 KB buffers); chunk c (dimensions 4c .. 4c + 3) of centroid
// i sits at i * 512 + 16 * (c ^ (i & 31)), so the 32 lanes of a lane half,
// reading the same chunk of 32 centroids, cover 32 distinct chunk columns.
constexpr int kF32StageTiles = 4;
constexpr int kF32TileBytes = 32 * kDim * 4;
constexpr int kF32Waves = kRowsPerBlock / 32;

template <int MODE, int G = kGroupTiles>
__global__ __launch_bounds__(kF32Waves * kWave) void probe_mfma_f32_kernel(
    const float* __restrict__ rot, int nrows, const float* __restrict__ cen32, const float* __restrict__ nhalf,
    int64_t k, int tiles_per_split, int sample_stride, float* __restrict__ gm, const float* __restrict__ thr,
    uint4* __restrict__ rval, uint32_t* __restrict__ rtile, uint32_t* __restrict__ cnt, int lane_cap,
    uint32_t* __restrict__ row_flag, int row_blocks, int splits) {
    static_assert(MODE == 0 || MODE == 1, "the sampled and filtered passes");
    __shared__ __align__(16) unsigned char stage0[kF32StageTiles * kF32TileBytes];
    __shared__ __align__(16) unsigned char stage1[kF32StageTiles * kF32TileBytes];
    __shared__ __align__(16) float snorm0[kF32StageTiles * 32];
    __shared__ __align__(16) float snorm1[kF32StageTiles * 32];
    __shared__ float gbuf[MODE == 0 ? kRowsPerBlock * 8 : 1];  // MODE 0: [row of the block][column mod 8]
    const int l = lane_id();
    const int w = wave_id();
    const int j = l & 31;
    const int hk = l >> 5;
    int rb, sp;  // XCD-aware split order, as probe_mfma_kernel
    if (splits % 8 == 0) {
        const int kx = static_cast<int>(blockIdx.x) >> 3;
        sp = (static_cast<int>(blockIdx.x) & 7) + 8 * (kx / row_blocks);
        rb = kx % row_blocks;
    } else {
        rb = static_cast<int>(blockIdx.x) % row_blocks;
        sp = static_cast<int>(blockIdx.x) / row_blocks;
    }
    const int row0 = rb * kRowsPerBlock + w * 32;
    const int64_t ntiles = (k + 31) / 32;
    const int64_t n_sampled = (ntiles + sample_stride - 1) / sample_stride;
    static_assert(kF32StageTiles % G == 0, "whole groups per stage");
    constexpr int kGroupsPerStage = kF32StageTiles / G;
    const int64_t n_groups = (n_sampled + G - 1) / G;
    const int64_t t_begin = static_cast<int64_t>(sp) * tiles_per_split;
    const int64_t t_end = min<int64_t>(ntiles, t_begin + tiles_per_split);

    const int row = row0 + j;
    const bool row_ok = row < nrows;
    float bq[64];  // q[row][64 hk + s]
    {
        const float4* src = reinterpret_cast<const float4*>(rot + static_cast<size_t>(row_ok ? row : 0) * kDim + 64 * hk);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float4 v = row_ok ? src[u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            bq[4 * u] = v.x;
            bq[4 * u + 1] = v.y;
            bq[4 * u + 2] = v.z;
            bq[4 * u + 3] = v.w;
        }
    }
    const float th = MODE == 1 && row_ok ? -0.5f * thr[row] : INFINITY;  // hit iff acc >= th
    int lcnt = 0;
    float gmax[kGroupsPerStage];
    const size_t sub = ((static_cast<size_t>(row_ok ? row : 0) * splits + sp) * 2 + hk) * lane_cap;

    auto tile_of = [&](int64_t it) -> int64_t { return t_begin + it * sample_stride; };
    const int64_t n_it_tiles = (t_end - t_begin + sample_stride - 1) / sample_stride;
    const int64_t n_iter = (n_it_tiles + kF32StageTiles - 1) / kF32StageTiles;

    // thread t fills chunk position t of every tile of the stage
    static_assert(kF32Waves * kWave * 16 == kF32TileBytes, "one 16-byte chunk per thread per tile");
    static_assert(kF32StageTiles * 32 <= kF32Waves * kWave, "one initial value per thread at most");
    const int fi = static_cast<int>(threadIdx.x) >> 5;                 // centroid of the chunk position
    const int fc = (static_cast<int>(threadIdx.x) & 31) ^ (fi & 31);   // its logical chunk
    auto fetch = [&](int64_t iter, unsigned char* sb, float* nb) {
#pragma unroll
        for (int tt = 0; tt < kF32StageTiles; ++tt) {
            const int64_t it = iter * kF32StageTiles + tt;
            const int64_t cen = tile_of(it) * 32 + fi;
            const int64_t src = it < n_it_tiles && cen < k ? cen : 0;
            __builtin_amdgcn_global_load_lds(cen32 + src * kDim + 4 * fc,
                                             lds_ptr(sb + tt * kF32TileBytes + w * 1024), 16, 0, 0);
        }
        if (w * kWave < kF32StageTiles * 32) {
            const int n = w * kWave + l;
            const int64_t it = iter * kF32StageTiles + (n >> 5);
            const int64_t cen = tile_of(it) * 32 + (n & 31);
            if (it < n_it_tiles && cen < k) {
                __builtin_amdgcn_global_load_lds(nhalf + cen, lds_ptr(nb + w * kWave), 4, 0, 0);
            } else {
                nb[n] = -INFINITY;
            }
        }
    };

    const int64_t gcol0 = (t_begin / sample_stride) / G;
    auto compute = [&](int64_t iter, const unsigned char* sb, const float* nb) {
        if (row0 >= nrows) return;
#pragma unroll
        for (int h = 0; h < kGroupsPerStage; ++h) gmax[h] = -INFINITY;
        // chunk 16 hk + g of centroid j sits at ((16 hk) ^ j ^ g) << 4 in its
        // row; the lane's part is recomputed per tile from a value the
        // compiler treats as new (an XOR and an add per 16-byte read) rather
        // than held in 16 registers
        auto load_a = [&](int tt, int g, uint32_t xo) {
            const unsigned char* tb = sb + tt * kF32TileBytes + j * (kDim * 4);
            return *reinterpret_cast<const float4*>(tb + (xo ^ (static_cast<uint32_t>(g) << 4)));
        };
        auto check = [&](const float16_t& acc, int64_t tile, int tt) {
            float m = acc[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) m = fmaxf(m, acc[r]);
            if (MODE == 0) {
                m = wave_max_xor32(m);
                gmax[tt / G] = fmaxf(gmax[tt / G], m);
            } else {
                const bool hit = m >= th;  // th is +inf past the last row
                if (hit && lcnt < lane_cap) {
                    const size_t e = sub + static_cast<size_t>(lcnt);
                    auto pk = [&](int r) { return rtz_half2_bits(acc[r] - th, acc[r + 1] - th); };
                    uint4* dv = rval + e * 2;
                    dv[0] = make_uint4(pk(0), pk(2), pk(4), pk(6));
                    dv[1] = make_uint4(pk(8), pk(10), pk(12), pk(14));
                    rtile[e] = static_cast<uint32_t>(tile);
                }
                lcnt += hit ? 1 : 0;
            }
        };
        auto ninit = [&](int tt) {
            float16_t v16;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 v = *reinterpret_cast<const float4*>(&nb[tt * 32 + g * 8 + hk * 4]);
                v16[4 * g + 0] = v.x;
                v16[4 * g + 1] = v.y;
                v16[4 * g + 2] = v.z;
                v16[4 * g + 3] = v.w;
            }
            return v16;
        };
#pragma unroll
        for (int tt = 0; tt < kF32StageTiles; ++tt) {
            const int64_t tile = tile_of(iter * kF32StageTiles + tt);
            float16_t acc = ninit(tt);
            uint32_t xo = static_cast<uint32_t>((16 * hk) ^ j) << 4;
            asm volatile("" : "+v"(xo));
            float4 a = load_a(tt, 0, xo);
#pragma unroll
            for (int g = 0; g < 16; ++g) {
                const float4 an = load_a(tt, g < 15 ? g + 1 : g, xo);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, bq[4 * g], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, bq[4 * g + 1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, bq[4 * g + 2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, bq[4 * g + 3], acc, 0, 0, 0);
                a = an;
            }
            check(acc, tile, tt);
        }
        if (MODE == 0) {
            const int64_t col = gcol0 + kGroupsPerStage * iter;
            float* gb = gbuf + w * 32 * 8;
            if (hk == 0) {
#pragma unroll
                for (int h = 0; h < kGroupsPerStage; ++h) gb[j * 8 + static_cast<int>((col + h) & 7)] = -2.0f * gmax[h];
            }
            const int64_t last = col + kGroupsPerStage - 1;
            const int slotc = static_cast<int>(last & 7);
            if (slotc == 7 || iter + 1 == n_iter) {
                wave_lds_sync();
                const int64_t cbase = last - slotc;
                const int s0 = cbase < gcol0 ? static_cast<int>(gcol0 - cbase) : 0;
                for (int v = l; v < 32 * 8; v += kWave) {
                    const int rl = v >> 3, sl = v & 7;
                    const int r = row0 + rl;
                    if (sl >= s0 && sl <= slotc && r < nrows && cbase + sl < n_groups)
                        gm[static_cast<size_t>(r) * n_groups + cbase + sl] = gb[rl * 8 + sl];
                }
                wave_lds_sync();
            }
        }
    };

    if (n_iter > 0) fetch(0, stage0, snorm0);
    for (int64_t iter = 0; iter < n_iter; iter += 2) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        if (iter + 1 < n_iter) fetch(iter + 1, stage1, snorm1);
        compute(iter, stage0, snorm0);
        if (iter + 1 >= n_iter) break;
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
        if (iter + 2 < n_iter) fetch(iter + 2, stage0, snorm0);
        compute(iter + 1, stage1, snorm1);
    }
    if (MODE == 1 && row_ok) {
        cnt[(static_cast<size_t>(row) * splits + sp) * 2 + hk] = static_cast<uint32_t>(lcnt < lane_cap ? lcnt : lane_cap);
        if (lcnt > lane_cap) row_flag[row] = 1u;
    }
}

// U = rank-th smallest sampled group minimum per row, by an 8-bit radix
// select over ordered keys staged in LDS; thr = U + 2*delta. One 256-thread
// block per row; the row's minima are contiguous (gm[row][group]). delta
// takes |q - bf16(q)| times eq_weight: 1 for bf16 query operands, 0 for
// fp32 ones (with ecmax 0 too).
__global__ __launch_bounds__(256) void probe_threshold_kernel(const float* __restrict__ gm, int n_sampled,
                                                              int nrows, int rank, const float* __restrict__ rot,
                                                              float cmax, float ecmax, float eq_weight,
                                                              float* __restrict__ thr) {
    extern __shared__ uint32_t skey[];  // [n_sampled]
    __shared__ __align__(16) int hist[256];
    __shared__ uint32_t s_prefix;
    __shared__ int s_rem;
    const int row = blockIdx.x;
    if (row >= nrows) return;
    const float* src = gm + static_cast<size_t>(row) * n_sampled;
    for (int g = threadIdx.x; g < n_sampled; g += blockDim.x) skey[g] = float_to_ordered(src[g]);
    __syncthreads();
    const uint32_t prefix = block_radix_select_u32([&](int g) { return skey[g]; }, n_sampled, rank - 1, hist,
                                                   &s_prefix, &s_rem);
    if (threadIdx.x < kWave) {
        const float2 nq = row_norms_wave(rot + static_cast<size_t>(row) * kDim);
        if (threadIdx.x == 0)
            thr[row] = ordered_to_float(prefix) + 2.0f * probe_delta(nq.x, eq_weight * nq.y, cmax, ecmax);
    }
}

// The same U and thr with one wave per row and the row's minima in registers
// (kPerLane per lane, for rows of at most 64 kPerLane minima): four 8-bit
// radix passes over the ordered keys, each a wave-local histogram (lanes that
// share the first active lane's digit add through it) and a scan of its bins
// (lane L holds bins 4L .. 4L + 3), with no block barriers.
template <int kPerLane>
__global__ __launch_bounds__(256) void probe_threshold_wave_kernel(const float* __restrict__ gm, int n_groups,
                                                                   int nrows, int rank, const float* __restrict__ rot,
                                                                   float cmax, float ecmax, float eq_weight,
                                                                   float* __restrict__ thr) {
    __shared__ __align__(16) int hist_all[4][256];
    const int l = lane_id();
    const int row = static_cast<int>(blockIdx.x) * 4 + wave_id();
    if (row >= nrows) return;
    int* hist = hist_all[wave_id()];
    const float* src = gm + static_cast<size_t>(row) * n_groups;
    uint32_t key[kPerLane];
#pragma unroll
    for (int u = 0; u < kPerLane; ++u) {
        const int g = u * kWave + l;
        key[u] = g < n_groups ? float_to_ordered(src[g]) : 0u;
    }
    uint32_t prefix = 0u, pmask = 0u;
    int rem = rank;  // position (1-based, ascending) within the keys that share the prefix
    for (int shift = 24; shift >= 0; shift -= 8) {
        *reinterpret_cast<int4*>(&hist[4 * l]) = make_int4(0, 0, 0, 0);
        wave_lds_sync();
#pragma unroll
        for (int u = 0; u < kPerLane; ++u)
            wave_hist_add(hist, u * kWave + l < n_groups && (key[u] & pmask) == prefix, (key[u] >> shift) & 255u);
        wave_lds_sync();
        const int4 h = *reinterpret_cast<const int4*>(&hist[4 * l]);
        const int hv[4] = {h.x, h.y, h.z, h.w};
        const int own = h.x + h.y + h.z + h.w;
        const int incl = wave_inclusive_scan(own);
        const int excl = incl - own;
        // at least rem keys share the prefix, so exactly one lane holds the digit
        const bool mine = excl < rem && incl >= rem;
        int bin = 0, cum = 0;
        if (mine) {
            cum = excl;
            int qd = 0;
            while (qd < 3 && cum + hv[qd] < rem) {
                cum += hv[qd];
                ++qd;
            }
            bin = 4 * l + qd;
        }
        const uint64_t who = __ballot(mine);
        const int src_lane = who != 0ull ? __ffsll(static_cast<long long>(who)) - 1 : kWave - 1;
        bin = __builtin_amdgcn_readlane(bin, src_lane);
        cum = __builtin_amdgcn_readlane(cum, src_lane);
        prefix |= static_cast<uint32_t>(bin) << shift;
        rem -= cum;
        pmask |= 255u << shift;
        wave_lds_sync();  // the next pass clears hist
    }
    const float2 nq = row_norms_wave(rot + static_cast<size_t>(row) * kDim);
    if (l == 0) thr[row] = ordered_to_float(prefix) + 2.0f * probe_delta(nq.x, eq_weight * nq.y, cmax, ecmax);
}

// Exact labels from the records. The candidates are the record values with
// v >= 0 (d' <= thr); v* = their nprobe-th largest v (a radix select over
// 16-bit keys). With eta >= |v~ - v| for every stored v~ (the fp32
// difference and the fp16 truncation: 2^-9 v~max + 2^-13, which also covers
// fp16 denormals flushed to zero):
//   check   v* >= delta + eta: nprobe candidates have v >= delta, i.e. d' <=
//           thr - 2 delta, so T <= thr - delta (T the exact nprobe-th best)
//           and every exact top-nprobe centroid c has d'(c) <= T + delta <=
//           thr: it is a candidate (v(c) >= 0). A row that fails is flagged.
//           When U is the nprobe-th group minimum (`rigorous`), nprobe
//           distinct centroids have d' <= U = thr - 2 delta by construction
//           and the check is skipped.
//   cutoff  T <= thr - 2 (v* - eta) + delta, so d'(c) <= T + delta gives
//           v(c) >= v* - eta - delta and v~(c) >= v* - delta - 2 eta: only
//           those are rescored in fp32 (sequential fmaf dot, |c|^2 - 2<q,c>)
//           and sorted by (score, id); the first nprobe are the labels.
// Both bounds are evaluated with directed rounding. One wave per row
// (kRerankWaves rows per block, each with its own LDS key area), so every
// step synchronises one wave only; the row's records are the concatenation
// of its nsub sub-lists. Rows with more than max_n candidates (row_cand
// 0xFFFFFFFF), a saturated value or a failed check (0xFFFFFFFE) are left to
// the exact kernel.
constexpr int kRerankWaves = 2;
__global__ __launch_bounds__(kRerankWaves * kWave) void probe_rerank_kernel(
    const float* __restrict__ rot, int nrows, const float* __restrict__ centroids, const float* __restrict__ norms,
    const uint4* __restrict__ rval, const uint32_t* __restrict__ rtile, const uint32_t* __restrict__ cnt,
    int lane_cap, int nsub, int max_n, int nprobe, bool rigorous, float cmax, float ecmax, float eq_weight,
    uint32_t* __restrict__ row_flag, uint32_t* __restrict__ row_cand, uint32_t* __restrict__ labels) {
    extern __shared__ uint64_t smem_keys[];  // [kRerankWaves][max_n]
    __shared__ float qs[kRerankWaves][kDim];
    __shared__ __align__(16) int hist_all[kRerankWaves][256];
    const int w = wave_id();
    const int l = lane_id();
    const int row = static_cast<int>(blockIdx.x) * kRerankWaves + w;
    if (row >= nrows) return;
    if (row_flag[row]) {
        if (l == 0) row_cand[row] = 0xFFFFFFFFu;  // a sub-list overflowed in the filtered pass
        return;
    }
    uint64_t* keys = smem_keys + static_cast<size_t>(w) * max_n;
    float* q = qs[w];
    int* hist = hist_all[w];
#pragma unroll
    for (int t = l; t < kDim; t += kWave) q[t] = rot[static_cast<size_t>(row) * kDim + t];
    const float2 nq = row_norms_wave(rot + static_cast<size_t>(row) * kDim);
    // candidates {key, id}, key = 0x7FFF - (fp16 bits of v): the bits of
    // non-negative fp16 values order as the values, so keys ascend as v
    // descends. The records of 64 sub-lists at a time form one index space
    // (the sub-lists' exclusive prefix sums in LDS; a lane finds its record's
    // sub-list by binary search), which the wave walks 64 records at a time,
    // loading the next 64 while it files the hits of the current ones.
    int n = 0;
    uint32_t hmax = 0u;  // largest v's bits (>= 0x7BFF: saturated, inf or NaN)
    const uint32_t* c_row = cnt + static_cast<size_t>(row) * nsub;
    int* pre = hist;  // [64] exclusive prefix of the sub-list counts
    for (int s0 = 0; s0 < nsub; s0 += kWave) {
        const int ns = nsub - s0 < kWave ? nsub - s0 : kWave;
        const int mycnt = l < ns ? static_cast<int>(c_row[s0 + l]) : 0;
        const int cincl = wave_inclusive_scan(mycnt);
        const int total = __builtin_amdgcn_readlane(cincl, kWave - 1);
        pre[l] = cincl - mycnt;
        wave_lds_sync();
        // record g of this group: tile, 8 value words, lane half of its sub-list
        struct Rec {
            uint4 a, b;
            uint32_t tile;
            int hk;
        };
        // (index 0 stands in past the end: every load is in bounds and
        // unconditional, so a batch's loads are in flight together)
        auto fetch = [&](int g) {
            Rec r;
            const int gc = g < total ? g : 0;
            int sl = 0;
#pragma unroll
            for (int step = 32; step >= 1; step >>= 1)
                if (sl + step < ns && pre[sl + step] <= gc) sl += step;
            const size_t e = (static_cast<size_t>(row) * nsub + s0 + sl) * lane_cap + (gc - pre[sl]);
            r.tile = rtile[e];
            r.a = rval[e * 2];
            r.b = rval[e * 2 + 1];
            r.hk = (s0 + sl) & 1;
            return r;
        };
        constexpr int kDepth = 4;  // record batches of the wave in flight
        for (int gb = 0; gb < total; gb += kDepth * kWave) {
            Rec batch[kDepth];
#pragma unroll
            for (int u = 0; u < kDepth; ++u) batch[u] = fetch(gb + u * kWave + l);
#pragma unroll
            for (int u = 0; u < kDepth; ++u) {
                const int g0 = gb + u * kWave;
                if (g0 >= total) break;
                const Rec& cur = batch[u];
                const bool live = g0 + l < total;
                const uint32_t wv[8] = {cur.a.x, cur.a.y, cur.a.z, cur.a.w, cur.b.x, cur.b.y, cur.b.z, cur.b.w};
                uint32_t hits = 0u;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t h = (wv[r >> 1] >> (16 * (r & 1))) & 0xFFFFu;
                    const bool hit = live && h < 0x8000u;
                    hits |= (hit ? 1u : 0u) << r;
                    hmax = hit && h > hmax ? h : hmax;
                }
                const int c = __popc(hits);
                const int incl = wave_inclusive_scan(c);
                int pos = n + incl - c;
                for (uint32_t h = hits; h != 0u; h &= h - 1u) {
                    const int r = __ffs(h) - 1;
                    const uint32_t id =
                        cur.tile * 32u + static_cast<uint32_t>((r >> 2) * 8 + cur.hk * 4 + (r & 3));
                    uint32_t word = wv[0];
#pragma unroll
                    for (int x = 1; x < 8; ++x) word = (r >> 1) == x ? wv[x] : word;
                    const uint32_t hb = (word >> (16 * (r & 1))) & 0xFFFFu;
                    if (pos < max_n) keys[pos] = (static_cast<uint64_t>(0x7FFFu - hb) << 32) | id;
                    ++pos;
                }
                n += __builtin_amdgcn_readlane(incl, kWave - 1);
            }
        }
        wave_lds_sync();  // the next group overwrites pre[]
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t x = static_cast<uint32_t>(__shfl_xor(static_cast<int>(hmax), o, kWave));
        hmax = x > hmax ? x : hmax;
    }
    if (n > max_n || n < nprobe || hmax >= 0x7BFFu) {
        if (l == 0) {
            row_cand[row] = n > max_n ? 0xFFFFFFFFu : 0xFFFFFFFEu;
            row_flag[row] = 1u;
        }
        return;
    }
    wave_lds_sync();
    // key of rank nprobe (ascending), i.e. v*: two 8-bit radix passes over
    // the wave's 16-bit keys with a wave-local histogram; lanes that share
    // the first active lane's digit add through it
    uint32_t prefix = 0, pmask = 0;
    int rem = nprobe;
    for (int shift = 8; shift >= 0; shift -= 8) {
        *reinterpret_cast<int4*>(&hist[4 * l]) = make_int4(0, 0, 0, 0);
        wave_lds_sync();
        for (int base = 0; base < n; base += kWave) {
            const int t = base + l;
            uint32_t digit = 0u;
            bool act = false;
            if (t < n) {
                const uint32_t key = static_cast<uint32_t>(keys[t] >> 32);
                act = (key & pmask) == prefix;
                digit = (key >> shift) & 255u;
            }
            const uint64_t live = __ballot(act);
            if (live == 0ull) continue;
            const int leader = __ffsll(static_cast<long long>(live)) - 1;
            const uint32_t d0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(digit), leader));
            const uint64_t same = __ballot(act && digit == d0);
            if (l == leader) atomicAdd(&hist[d0], __popcll(same));
            if (act && digit != d0) atomicAdd(&hist[digit], 1);
        }
        wave_lds_sync();
        const int4 h = *reinterpret_cast<const int4*>(&hist[4 * l]);
        const int hv[4] = {h.x, h.y, h.z, h.w};
        const int own = h.x + h.y + h.z + h.w;
        const int incl = wave_inclusive_scan(own);
        const int excl = incl - own;
        // exactly one lane holds the digit (at least rem keys share prefix)
        int bin = 0, cum = 0;
        const bool mine = excl < rem && incl >= rem;
        if (mine) {
            cum = excl;
            int qd = 0;
            while (qd < 3 && cum + hv[qd] < rem) {
                cum += hv[qd];
                ++qd;
            }
            bin = 4 * l + qd;
        }
        const uint64_t who = __ballot(mine);
        const int src_lane = who ? __ffsll(static_cast<long long>(who)) - 1 : kWave - 1;
        bin = __shfl(bin, src_lane, kWave);
        cum = __shfl(cum, src_lane, kWave);
        prefix |= static_cast<uint32_t>(bin) << shift;
        rem -= cum;
        pmask |= 255u << shift;
    }
    const float vstar = half_bits_to_float(0x7FFFu - prefix);
    const float delta = probe_delta(nq.x, eq_weight * nq.y, cmax, ecmax);
    const float eta = add_up(half_bits_to_float(hmax) * 0.001953125f, 0.0001220703125f);
    // (not needed when the threshold is the nprobe-th group minimum itself:
    // those nprobe distinct centroids have d' <= thr - 2 delta by
    // construction, while the check, through v's fp16 rounding, could not
    // certify the one lying exactly at U)
    if (!rigorous && !(vstar >= add_up(delta, eta))) {
        if (l == 0) {
            row_cand[row] = 0xFFFFFFFEu;
            row_flag[row] = 1u;
        }
        return;
    }
    if (l == 0) row_cand[row] = static_cast<uint32_t>(n);
    const float vcut = sub_down(vstar, add_up(delta, 2.0f * eta));
    // candidates with v~ >= vcut compacted to the front (in place: a lane
    // writes at or below the position it read), then rescored exactly
    int m = 0;
    for (int base = 0; base < n; base += kWave) {
        const int t = base + l;
        const uint64_t kv = t < n ? keys[t] : ~0ull;
        const bool keep = t < n && half_bits_to_float(0x7FFFu - static_cast<uint32_t>(kv >> 32)) >= vcut;
        const uint64_t bal = __ballot(keep);
        const int before = __popcll(bal & ((1ull << l) - 1ull));
        wave_lds_sync();
        if (keep) keys[m + before] = kv;
        m += __popcll(bal);
        wave_lds_sync();
    }
    // at least one key per lane (the key area holds at least max_n >= 64)
    const int sort_m = pow2_at_least_dev(m < kWave ? kWave : m);
    for (int t = l; t < sort_m; t += kWave) {
        uint64_t key = ~0ull;
        if (t < m) {
            const uint32_t c = static_cast<uint32_t>(keys[t] & 0xFFFFFFFFu);
            const float4* cv = reinterpret_cast<const float4*>(centroids + static_cast<size_t>(c) * kDim);
            // the whole 512-byte row is requested at once (one round trip per
            // 64 candidates), then the chain runs in sequence
            float4 v[kDim / 4];
#pragma unroll
            for (int u = 0; u < kDim / 4; ++u) v[u] = cv[u];
            float dot = 0.0f;
#pragma unroll
            for (int u = 0; u < kDim / 4; ++u) {
                const float4 qv = *reinterpret_cast<const float4*>(&q[4 * u]);
                dot = __fmaf_rn(qv.x, v[u].x, dot);
                dot = __fmaf_rn(qv.y, v[u].y, dot);
                dot = __fmaf_rn(qv.z, v[u].z, dot);
                dot = __fmaf_rn(qv.w, v[u].w, dot);
            }
            const float score = norms[c] - 2.0f * dot;
            key = (static_cast<uint64_t>(float_to_ordered(score)) << 32) | c;
        }
        keys[t] = key;  // t < m reads only its own entry
    }
    wave_lds_sync();
    // sort of keys[0, sort_m) by the wave in registers (lane l holds keys
    // [K l, K l + K)), then the first nprobe are the labels
    auto sort_store = [&](auto kk) {
        constexpr int K = decltype(kk)::value;
        uint64_t r[K];
#pragma unroll
        for (int j = 0; j < K; ++j) r[j] = keys[K * l + j];
        sort_keys_regs<K, false>(r, keys, sort_m, l);
#pragma unroll
        for (int j = 0; j < K; ++j)
            if (K * l + j < nprobe)
                labels[static_cast<size_t>(row) * nprobe + K * l + j] = static_cast<uint32_t>(r[j] & 0xFFFFFFFFu);
    };
    switch (sort_m / kWave) {
        case 1: sort_store(std::integral_constant<int, 1>{}); return;
        case 2: sort_store(std::integral_constant<int, 2>{}); return;
        case 4: sort_store(std::integral_constant<int, 4>{}); return;
        case 8: sort_store(std::integral_constant<int, 8>{}); return;
        case 16: sort_store(std::integral_constant<int, 16>{}); return;
        default: break;
    }
    // more than 1,024 keys: the bitonic network in LDS
    for (int size = 2; size <= sort_m; size <<= 1) {
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int t = l; t < sort_m / 2; t += kWave) {
                const int a = 2 * t - (t & (stride - 1));
                const int b = a + stride;
                const bool up = (a & size) == 0;
                const uint64_t x = keys[a], y = keys[b];
                if ((x > y) == up) {
                    keys[a] = y;
                    keys[b] = x;
                }
            }
            wave_lds_sync();
        }
    }
    for (int t = l; t < nprobe; t += kWave)
        labels[static_cast<size_t>(row) * nprobe + t] = static_cast<uint32_t>(keys[t] & 0xFFFFFFFFu);
}

// Nearest centroid of each row among its buffered candidates by the exact
// fp32 score (sequential fmaf dot, ties to the lower id). One wave per row;
// rows with no candidate or a flag are left to the exact kernel.
__global__ __launch_bounds__(256) void probe_top1_rerank_kernel(const float* __restrict__ rows, int nrows,
                                                                const float* __restrict__ centroids,
                                                                const float* __restrict__ norms,
                                                                const uint2* __restrict__ buf,
                                                                const uint32_t* __restrict__ cnt, int lane_cap,
                                                                int nsub, uint32_t* __restrict__ row_flag,
                                                                uint32_t* __restrict__ labels) {
    const int row = blockIdx.x * 4 + wave_id();
    const int l = lane_id();
    if (row >= nrows) return;
    if (row_flag[row]) return;
    const float4* q = reinterpret_cast<const float4*>(rows + static_cast<size_t>(row) * kDim);
    uint64_t best = ~0ull;
    uint32_t total = 0;
    for (int sb = 0; sb < nsub; ++sb) {
        const uint32_t n = cnt[static_cast<size_t>(row) * nsub + sb];
        total += n;
        const uint2* src = buf + (static_cast<size_t>(row) * nsub + sb) * lane_cap;
        for (uint32_t t = l; t < n; t += kWave) {
            const uint32_t c = src[t].x;
            const float4* cv = reinterpret_cast<const float4*>(centroids + static_cast<size_t>(c) * kDim);
            float dot = 0.0f;
            for (int j4 = 0; j4 < kDim / 4; ++j4) {
                const float4 a = q[j4];
                const float4 v = cv[j4];
                dot = __fmaf_rn(a.x, v.x, dot);
                dot = __fmaf_rn(a.y, v.y, dot);
                dot = __fmaf_rn(a.z, v.z, dot);
                dot = __fmaf_rn(a.w, v.w, dot);
            }
            const float score = norms[c] - 2.0f * dot;
            const uint64_t key = (static_cast<uint64_t>(float_to_ordered(score)) << 32) | c;
            best = key < best ? key : best;
        }
    }
    if (total == 0) {
        if (l == 0) row_flag[row] = 1u;
        return;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(best), m, kWave);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(best >> 32), m, kWave);
        const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
        best = o < best ? o : best;
    }
    if (l == 0) labels[row] = static_cast<uint32_t>(best & 0xFFFFFFFFu);
}

// ---- launchers ----

hipError_t launch_probe_centroids(hipStream_t s, const float* c, const float* norms, int64_t k, uint16_t* cbf,
                                  float* nhalf, uint32_t* err_max) {
    hipError_t e = launch_fill_u32(s, err_max, 1, 0u);
    if (e != hipSuccess || k == 0) return e;
    hipLaunchKernelGGL(probe_centroids_kernel, dim3(static_cast<unsigned>((k + 3) / 4)), dim3(256), 0, s, c, norms, k,
                       cbf, nhalf, err_max);
    return hipGetLastError();
}

ProbePlan plan_probe_mfma(int nrows, int64_t k, int nprobe, int num_cus) {
    ProbePlan p{};
    const int64_t ntiles = (k + 31) / 32;
    p.row_blocks = (nrows + kRowsPerBlock - 1) / kRowsPerBlock;
    // Every 8th tile is sampled when that leaves at least 8 nprobe sampled
    // tiles (large k, where the sampled pass costs most), else every 4th when
    // that leaves at least 4 nprobe, else every tile. The sampled pass keeps
    // one minimum per group of 4 sampled tiles when that still gives at least
    // 4 nprobe group minima, else one per sampled tile.
    p.sample_stride = ntiles >= static_cast<int64_t>(64) * nprobe   ? 8
                      : ntiles >= static_cast<int64_t>(16) * nprobe ? 4
                                                                     : 1;
    // the threshold kernel stages a row's group minima in 64 KB of LDS
    const int64_t max_sampled = kMaxGroups * kGroupTiles;
    p.sample_stride = static_cast<int>(std::max<int64_t>(p.sample_stride, (ntiles + max_sampled - 1) / max_sampled));
    p.n_sampled = static_cast<int>((ntiles + p.sample_stride - 1) / p.sample_stride);
    p.group_tiles = p.n_sampled / kGroupTiles >= 4 * nprobe || p.n_sampled > kMaxGroups ? kGroupTiles : 1;
    // The threshold rank r. With a fraction f = 1/s of the tiles sampled and
    // the centroids near the top spread over many groups, the r-th smallest
    // group minimum U has about r/f centroids at or below it, with standard
    // deviation sqrt(r (1 - f))/f. The rerank's check fails when fewer than
    // nprobe are, so r is the least with r/f - z sqrt(r (1 - f))/f >= nprobe
    // for z = 4.5: with x = sqrt(r), x = (z sqrt(1 - f) + sqrt(z^2 (1 - f) +
    // 4 f nprobe)) / 2. At most nprobe, which it is when every tile is
    // sampled (where the check cannot fail); 63 (s = 4) and 44 (s = 8) at
    // nprobe 128.
    {
        const double f = 1.0 / p.sample_stride, z = 4.5;
        const double b = z * std::sqrt(1.0 - f);
        const double x = 0.5 * (b + std::sqrt(b * b + 4.0 * f * nprobe));
        p.u_rank = static_cast<int>(std::min<double>(nprobe, std::max(1.0, std::ceil(x * x - 1e-9))));
    }
    // One block fits a CU at a time (its LDS). A single row block takes one
    // split per CU (one query at docs2m: sampled pass 42 -> 35 us, filtered
    // pass 73 -> 67 us, and half the sub-lists for the rerank to walk, 75 ->
    // 58 us); more row blocks take two blocks per CU in turn, as fewer splits
    // there overflow sub-lists.
    const int want_blocks = p.row_blocks == 1 ? num_cus : 2 * num_cus;
    int64_t splits = std::max<int64_t>(1, want_blocks / std::max(1, p.row_blocks));
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, ntiles / kStageTiles));
    if (splits >= 8) splits = splits / 8 * 8;  // one split per XCD group
    p.tiles_per_split = static_cast<int>((ntiles + splits - 1) / splits);
    p.splits = static_cast<int>((ntiles + p.tiles_per_split - 1) / p.tiles_per_split);
    // splits cover whole stages of kStageTiles sampled tiles
    const int unit = kStageTiles * p.sample_stride;
    p.tiles_per_split = (p.tiles_per_split + unit - 1) / unit * unit;
    p.splits = static_cast<int>((ntiles + p.tiles_per_split - 1) / p.tiles_per_split);
    p.lane_cap = kProbeLaneCap;
    const int n_groups = (p.n_sampled + p.group_tiles - 1) / p.group_tiles;
    p.usable = n_groups >= nprobe && n_groups <= kMaxGroups && nprobe <= 1024 && 2 * p.splits <= kMaxSublists;
    return p;
}

hipError_t launch_probe_mfma(hipStream_t s, const ProbePlan& p, const float* rot, int nrows, const uint16_t* cbf,
                             const float* nhalf, const float* centroids, const float* norms, int64_t k, float cmax,
                             float ecmax, int nprobe, float* gm, float* thr, uint32_t* rval, uint32_t* rtile,
                             uint32_t* cnt, uint32_t* row_flag, uint32_t* row_cand, uint32_t* labels,
                             const ExactFallback& fb, int part, bool f32) {
    uint4* rv = reinterpret_cast<uint4*>(rval);
    hipError_t e = hipSuccess;
    const dim3 grid(p.row_blocks * p.splits);
    const int n_groups = (p.n_sampled + p.group_tiles - 1) / p.group_tiles;
    // fp32 operands: no rounding of q or c enters the margin
    const float ec = f32 ? 0.0f : ecmax;
    const float eqw = f32 ? 0.0f : 1.0f;
    if (part < 0 || part == 0) {
        if ((e = launch_fill_u32(s, row_flag, nrows, 0u)) != hipSuccess) return e;
        // pass A over sampled tiles: gm index = sampled tile number, so the
        // split grid walks sampled tiles in order
        if (f32) {
            if (p.group_tiles == kGroupTiles)
                hipLaunchKernelGGL((probe_mfma_f32_kernel<0, kGroupTiles>), grid, dim3(kF32Waves * kWave), 0, s, rot,
                                   nrows, centroids, nhalf, k, p.tiles_per_split, p.sample_stride, gm, thr, nullptr,
                                   nullptr, cnt, p.lane_cap, row_flag, p.row_blocks, p.splits);
            else
                hipLaunchKernelGGL((probe_mfma_f32_kernel<0, 1>), grid, dim3(kF32Waves * kWave), 0, s, rot, nrows,
                                   centroids, nhalf, k, p.tiles_per_split, p.sample_stride, gm, thr, nullptr, nullptr,
                                   cnt, p.lane_cap, row_flag, p.row_blocks, p.splits);
        } else if (p.group_tiles == kGroupTiles) {
            hipLaunchKernelGGL((probe_mfma_kernel<0, kGroupTiles>), grid, dim3(kProbeWaves * kWave), 0, s, rot, nrows,
                               cbf, nhalf, k, p.tiles_per_split, p.sample_stride, gm, thr, nullptr, nullptr, nullptr,
                               cnt, p.lane_cap, row_flag, nullptr, cmax, ecmax, p.row_blocks, p.splits);
        } else {
            hipLaunchKernelGGL((probe_mfma_kernel<0, 1>), grid, dim3(kProbeWaves * kWave), 0, s, rot, nrows, cbf,
                               nhalf, k, p.tiles_per_split, p.sample_stride, gm, thr, nullptr, nullptr, nullptr, cnt,
                               p.lane_cap, row_flag, nullptr, cmax, ecmax, p.row_blocks, p.splits);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        const dim3 wgrid((nrows + 3) / 4);
        if (n_groups <= 8 * kWave)
            hipLaunchKernelGGL(probe_threshold_wave_kernel<8>, wgrid, dim3(256), 0, s, gm, n_groups, nrows, p.u_rank,
                               rot, cmax, ec, eqw, thr);
        else if (n_groups <= 16 * kWave)
            hipLaunchKernelGGL(probe_threshold_wave_kernel<16>, wgrid, dim3(256), 0, s, gm, n_groups, nrows,
                               p.u_rank, rot, cmax, ec, eqw, thr);
        else if (n_groups <= 32 * kWave)
            hipLaunchKernelGGL(probe_threshold_wave_kernel<32>, wgrid, dim3(256), 0, s, gm, n_groups, nrows,
                               p.u_rank, rot, cmax, ec, eqw, thr);
        else
            hipLaunchKernelGGL(probe_threshold_kernel, dim3(nrows), dim3(256), static_cast<size_t>(n_groups) * 4, s,
                               gm, n_groups, nrows, p.u_rank, rot, cmax, ec, eqw, thr);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (part < 0 || part == 1) {
        if (f32)
            hipLaunchKernelGGL(probe_mfma_f32_kernel<1>, grid, dim3(kF32Waves * kWave), 0, s, rot, nrows, centroids,
                               nhalf, k, p.tiles_per_split, 1, gm, thr, rv, rtile, cnt, p.lane_cap, row_flag,
                               p.row_blocks, p.splits);
        else
            hipLaunchKernelGGL(probe_mfma_kernel<1>, grid, dim3(kProbeWaves * kWave), 0, s, rot, nrows, cbf, nhalf, k,
                               p.tiles_per_split, 1, gm, thr, nullptr, rv, rtile, cnt, p.lane_cap, row_flag, nullptr,
                               cmax, ecmax, p.row_blocks, p.splits);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (part < 0 || part == 2) {
        // key area per row: 8 nprobe (a power of two in [1024, 2048]), about
        // four times the usual candidate count at nprobe 128; the LDS it
        // takes sets the rerank's occupancy (16 waves per CU at 1024)
        int max_n = 1024;
        while (max_n < 8 * nprobe && max_n < kProbeMaxCandidates) max_n *= 2;
        hipLaunchKernelGGL(probe_rerank_kernel, dim3((nrows + kRerankWaves - 1) / kRerankWaves),
                           dim3(kRerankWaves * kWave), static_cast<size_t>(kRerankWaves) * max_n * 8, s, rot, nrows,
                           centroids, norms, rv, rtile, cnt, p.lane_cap, 2 * p.splits, max_n, nprobe,
                           p.u_rank >= nprobe, cmax, ec, eqw, row_flag, row_cand, labels);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // rows that overflowed or failed the check: exact recomputation
        e = launch_probe_exact_flagged(s, rot, nrows, centroids, norms, k, nprobe, row_flag, labels, fb);
    }
    return e;
}

size_t probe_sublist_rows(int max_rows, int num_cus) {
    // rows * splits <= max(rows, 2 * num_cus * kRowsPerBlock) for every plan
    return static_cast<size_t>(std::max<int64_t>(max_rows, int64_t{2} * num_cus * kRowsPerBlock));
}

ProbePlan plan_assign_top1(int nrows, int64_t k, int num_cus) {
    ProbePlan p{};
    const int64_t ntiles = (k + 31) / 32;
    p.row_blocks = (nrows + kRowsPerBlock - 1) / kRowsPerBlock;
    // a 1/16 sample of the tiles bounds the nearest d' from above
    p.sample_stride = ntiles >= 64 ? 16 : 1;
    p.n_sampled = static_cast<int>((ntiles + p.sample_stride - 1) / p.sample_stride);
    int64_t splits = std::max<int64_t>(1, (2 * static_cast<int64_t>(num_cus)) / std::max(1, p.row_blocks));
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, ntiles / (kStageTiles * p.sample_stride)));
    p.tiles_per_split = static_cast<int>((ntiles + splits - 1) / splits);
    p.tiles_per_split = (p.tiles_per_split + p.sample_stride - 1) / p.sample_stride * p.sample_stride;
    p.splits = static_cast<int>((ntiles + p.tiles_per_split - 1) / p.tiles_per_split);
    p.lane_cap = kTop1LaneCap;
    p.group_tiles = 1;
    p.u_rank = 1;
    p.usable = true;
    return p;
}

hipError_t launch_assign_top1(hipStream_t s, const ProbePlan& p, const float* rows, int nrows, const uint16_t* cbf,
                              const float* nhalf, const float* centroids, const float* norms, int64_t k, float cmax,
                              float ecmax, uint32_t* ukey, uint2* buf, uint32_t* cnt, uint32_t* row_flag,
                              uint32_t* labels, const ExactFallback& fb) {
    if (nrows == 0) return hipSuccess;
    hipError_t e = launch_fill_u32(s, ukey, nrows, 0xFFFFFFFFu);
    if (e != hipSuccess) return e;
    if ((e = launch_fill_u32(s, row_flag, nrows, 0u)) != hipSuccess) return e;
    const dim3 grid(p.row_blocks * p.splits);
    hipLaunchKernelGGL(probe_mfma_kernel<2>, grid, dim3(kProbeWaves * kWave), 0, s, rows, nrows, cbf, nhalf, k,
                       p.tiles_per_split, p.sample_stride, nullptr, nullptr, buf, nullptr, nullptr, cnt, p.lane_cap,
                       row_flag, ukey, cmax, ecmax, p.row_blocks, p.splits);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(probe_mfma_kernel<3>, grid, dim3(kProbeWaves * kWave), 0, s, rows, nrows, cbf, nhalf, k,
                       p.tiles_per_split, 1, nullptr, nullptr, buf, nullptr, nullptr, cnt, p.lane_cap, row_flag, ukey,
                       cmax, ecmax, p.row_blocks, p.splits);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(probe_top1_rerank_kernel, dim3((nrows + 3) / 4), dim3(256), 0, s, rows, nrows, centroids, norms,
                       buf, cnt, p.lane_cap, 2 * p.splits, row_flag, labels);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return launch_probe_exact_flagged(s, rows, nrows, centroids, norms, k, 1, row_flag, labels, fb);
}

}  // namespace chimera
