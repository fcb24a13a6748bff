// Candidate generation for a sub-batch of queries:
//   mark     the candidate bitmap (kernels.cu:206-278)
//   scan     popcount prefix and the ascending candidate list (kernels.cu:117-173)
//   partial  S_cand = sum over query tokens of the max positive one-bit
//            estimate of each candidate (kernels.cu:280-400 + 175-204)
//   select   the first min(k_refine, C) candidates by S_cand descending,
//            ties by ascending doc ID (CUB stable sort, search_impl.cu:245-261)
#include "common.hpp"
#include "kernels.hpp"

namespace chimera {

namespace {

// Block b of a (qs rounded up to 8) x 32 grid -> (query, token). The eight
// XCDs take blocks round-robin, so all 32 token blocks of one query land on
// the same XCD and share its L2 (query state lives there).
__device__ __forceinline__ void xcd_map(int b, int& qq, int& i) {
    const int xcd = b & 7;
    const int slot = b >> 3;
    i = slot & 31;
    qq = (slot >> 5) * 8 + xcd;
}

__device__ __forceinline__ uint32_t hash32(uint32_t x) { return x * 2654435761u; }

}  // namespace

__global__ __launch_bounds__(256) void mark_kernel(const uint32_t* __restrict__ labels, int q_base, int qs,
                                                   int nprobe, const uint64_t* __restrict__ cluster_pos,
                                                   const int32_t* __restrict__ doc_clu, int64_t n_clusters,
                                                   int64_t num_docs, int nb, uint32_t* __restrict__ bitmap) {
    int qq, i;
    xcd_map(blockIdx.x, qq, i);
    if (qq >= qs) return;
    const uint32_t* lab = labels + (static_cast<size_t>(q_base + qq) * kQ + i) * nprobe;
    uint32_t* bm = bitmap + static_cast<size_t>(qq) * nb;
    const int nw = blockDim.x / kWave;
    for (int p = wave_id(); p < nprobe; p += nw) {
        const uint32_t label = lab[p];
        if (label >= static_cast<uint64_t>(n_clusters)) continue;
        const uint64_t start = cluster_pos[label];
        const uint64_t end = cluster_pos[label + 1];
        for (uint64_t pos = start + lane_id(); pos < end; pos += kWave) {
            const int32_t doc = doc_clu[pos];
            if (doc >= 0 && doc < num_docs) atomicOr(&bm[doc >> 5], 1u << (doc & 31));
        }
    }
}

// One block of 1024 threads per query: exclusive popcount prefix per bitmap
// word and the candidate IDs in ascending order.
__global__ __launch_bounds__(1024) void scan_kernel(const uint32_t* __restrict__ bitmap, int nb, int qs,
                                                    uint32_t* __restrict__ offs, int32_t* __restrict__ cand,
                                                    int64_t cap, int32_t* __restrict__ ccount,
                                                    uint32_t* __restrict__ err) {
    __shared__ int scratch[17];
    const int qq = blockIdx.x;
    if (qq >= qs) return;
    const uint32_t* bm = bitmap + static_cast<size_t>(qq) * nb;
    uint32_t* of = offs + static_cast<size_t>(qq) * nb;
    int32_t* cd = cand + static_cast<size_t>(qq) * cap;
    int carry = 0;
    for (int base = 0; base < nb; base += blockDim.x) {
        const int b = base + threadIdx.x;
        const uint32_t v = b < nb ? bm[b] : 0u;
        const int c = __popc(v);
        int total;
        const int incl = block_inclusive_scan_shared(c, scratch, &total);
        const int excl = carry + incl - c;
        if (b < nb) {
            of[b] = static_cast<uint32_t>(excl);
            if (excl + c <= cap) {
                uint32_t bits = v;
                int k = excl;
                while (bits) {
                    const int bit = __ffs(bits) - 1;
                    cd[k++] = b * 32 + bit;
                    bits &= bits - 1;
                }
            } else {
                atomicOr(err, kErrCandOverflow);
            }
        }
        carry += total;
    }
    if (threadIdx.x == 0) ccount[qq] = carry;
}

namespace {
constexpr int kDupCap = 2048;    // LDS dedupe slots
constexpr int kDupLimit = 1536;  // distinct duplicated docs handled per pass

__device__ __forceinline__ int dup_slot0(int doc) { return static_cast<int>(hash32(static_cast<uint32_t>(doc)) >> 21); }

__device__ __forceinline__ void dup_insert(int* keys, int* count, int doc) {
    int h = dup_slot0(doc);
    for (int probe = 0; probe < kDupCap; ++probe) {
        const int k = atomicCAS(&keys[h], -1, doc);
        if (k == -1) {
            atomicAdd(count, 1);
            return;
        }
        if (k == doc) return;
        h = (h + 1) & (kDupCap - 1);
    }
}

__device__ __forceinline__ int dup_find(const int* keys, int doc) {
    int h = dup_slot0(doc);
    for (int probe = 0; probe < kDupCap; ++probe) {
        const int k = keys[h];
        if (k == doc) return h;
        if (k == -1) return -1;
        h = (h + 1) & (kDupCap - 1);
    }
    return -1;
}

__device__ __forceinline__ bool in_part(int doc, int part, int nparts) {
    return nparts == 1 || static_cast<int>((hash32(static_cast<uint32_t>(doc)) >> 8) % static_cast<uint32_t>(nparts)) == part;
}
}  // namespace

// One block per (query, token): visits every token of the token's probed
// clusters. A doc visited more than once by this query token must contribute
// only its maximum estimate (kernels.cu:381-396). Pass 1 finds such docs with
// an LDS bitmap (exact when num_docs <= bitmap bits, otherwise a superset) and
// records them in an LDS set; pass 2 computes the estimates, adds unique
// positive ones straight into S_cand and max-reduces duplicated ones in LDS
// before adding them once. When too many duplicated docs appear, the doc
// space is split into hash parts processed one after another.
__global__ __launch_bounds__(512) void partial_kernel(
    const uint32_t* __restrict__ labels, int q_base, int qs, int nprobe, const uint64_t* __restrict__ cluster_pos,
    const uint8_t* __restrict__ codes_clu, const float* __restrict__ f1_clu, const int32_t* __restrict__ doc_clu,
    int64_t n_clusters, int64_t num_docs, const float* __restrict__ lut, const float* __restrict__ cb1,
    const uint32_t* __restrict__ bitmap, const uint32_t* __restrict__ offs, int nb, int bm_log2,
    float* __restrict__ S, int64_t cap, uint32_t* __restrict__ err) {
    extern __shared__ uint32_t lbm[];
    __shared__ float llut[kChunks * kLut];
    __shared__ int dkey[kDupCap];
    __shared__ uint32_t dval[kDupCap];
    __shared__ int dcount;
    __shared__ int dtotal;
    int qq, i;
    xcd_map(blockIdx.x, qq, i);
    if (qq >= qs) return;
    const int q = q_base + qq;
    for (int t = threadIdx.x; t < kChunks * kLut; t += blockDim.x)
        llut[t] = lut[static_cast<size_t>(q) * kLutPerQuery + t * kQ + i];
    const float cb = cb1[q * kQ + i];
    const uint32_t* lab = labels + (static_cast<size_t>(q) * kQ + i) * nprobe;
    const uint32_t* bmq = bitmap + static_cast<size_t>(qq) * nb;
    const uint32_t* ofq = offs + static_cast<size_t>(qq) * nb;
    float* sq = S + static_cast<size_t>(qq) * cap;
    const uint32_t bmask = (1u << bm_log2) - 1u;
    const int bm_words = static_cast<int>((1u << bm_log2) / 32u) > 0 ? static_cast<int>((1u << bm_log2) / 32u) : 1;
    const int nw = blockDim.x / kWave;
    const int l = lane_id();

    auto rank_of = [&](int doc) -> int {
        const int wd = doc >> 5;
        return static_cast<int>(ofq[wd]) + __popc(bmq[wd] & ((1u << (doc & 31)) - 1u));
    };

    int nparts = 1;
    bool first = true;
    for (int part = 0; part < nparts; ++part) {
        for (int t = threadIdx.x; t < bm_words; t += blockDim.x) lbm[t] = 0u;
        for (int t = threadIdx.x; t < kDupCap; t += blockDim.x) {
            dkey[t] = -1;
            dval[t] = 0u;
        }
        if (threadIdx.x == 0) {
            dcount = 0;
            dtotal = 0;
        }
        __syncthreads();
        // pass 1: docs visited more than once
        for (int p = wave_id(); p < nprobe; p += nw) {
            const uint32_t label = lab[p];
            if (label >= static_cast<uint64_t>(n_clusters)) continue;
            const uint64_t end = cluster_pos[label + 1];
            for (uint64_t pos = cluster_pos[label] + l; pos < end; pos += kWave) {
                const int32_t doc = doc_clu[pos];
                if (doc < 0 || doc >= num_docs || !in_part(doc, part, nparts)) continue;
                const uint32_t b = static_cast<uint32_t>(doc) & bmask;
                const uint32_t bit = 1u << (b & 31);
                const uint32_t old = atomicOr(&lbm[b >> 5], bit);
                if (old & bit) {
                    atomicAdd(&dtotal, 1);
                    if (dcount < kDupCap - 64) dup_insert(dkey, &dcount, doc);
                }
            }
        }
        __syncthreads();
        if (dcount > kDupLimit) {
            if (first) {
                const int want = (2 * dtotal + kDupLimit - 1) / kDupLimit + 1;
                nparts = want < 2 ? 2 : want;
                first = false;
                part = -1;
                __syncthreads();
                continue;
            }
            if (threadIdx.x == 0) atomicOr(err, kErrDupOverflow);
        }
        first = false;
        // pass 2: estimates
        for (int p = wave_id(); p < nprobe; p += nw) {
            const uint32_t label = lab[p];
            if (label >= static_cast<uint64_t>(n_clusters)) continue;
            const uint64_t end = cluster_pos[label + 1];
            for (uint64_t pos = cluster_pos[label] + l; pos < end; pos += kWave) {
                const int32_t doc = doc_clu[pos];
                if (doc < 0 || doc >= num_docs || !in_part(doc, part, nparts)) continue;
                const uint4 code = *reinterpret_cast<const uint4*>(codes_clu + pos * kCodeBytes);
                float ip = 0.0f;
#pragma unroll
                for (int c = 0; c < kChunks; ++c) ip += llut[c * kLut + code_nibble(code, c)];
                const float e = (ip - cb) * f1_clu[pos];
                if (e > 0.0f) {
                    const int slot = dup_find(dkey, doc);
                    if (slot >= 0) {
                        atomicMax(&dval[slot], __float_as_uint(e));
                    } else {
                        const int rk = rank_of(doc);
                        if (rk < cap) atomicAdd(&sq[rk], e);
                    }
                }
            }
        }
        __syncthreads();
        for (int t = threadIdx.x; t < kDupCap; t += blockDim.x) {
            const int doc = dkey[t];
            const uint32_t v = dval[t];
            if (doc >= 0 && v != 0u) {
                const int rk = rank_of(doc);
                if (rk < cap) atomicAdd(&sq[rk], __uint_as_float(v));
            }
        }
        __syncthreads();
    }
}

// Top-R by S_cand per query (one 1024-thread block): 8-bit radix select of
// the R-th largest key, stable compaction (ties in ascending candidate order,
// i.e. ascending doc ID), LDS bitonic sort by (score desc, doc asc).
__global__ __launch_bounds__(1024) void select_refine_kernel(const float* __restrict__ S,
                                                             const int32_t* __restrict__ cand,
                                                             const int32_t* __restrict__ ccount, int64_t cap,
                                                             int q_base, int qs, int k_refine, int sort_cap,
                                                             int32_t* __restrict__ rcount, int32_t* __restrict__ rids,
                                                             float* __restrict__ rscore) {
    extern __shared__ uint64_t keys[];  // [sort_cap]
    __shared__ int hist[256];
    __shared__ int scratch[17];
    __shared__ uint32_t s_prefix;
    __shared__ int s_remaining;
    const int qq = blockIdx.x;
    if (qq >= qs) return;
    const int q = q_base + qq;
    const int C = ccount[qq] < cap ? ccount[qq] : static_cast<int>(cap);
    const int R = C < k_refine ? C : k_refine;
    if (threadIdx.x == 0) rcount[q] = R;
    if (R == 0) return;
    const float* sq = S + static_cast<size_t>(qq) * cap;
    const int32_t* cq = cand + static_cast<size_t>(qq) * cap;
    uint32_t prefix = 0, pmask = 0;
    int remaining = R;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int t = threadIdx.x; t < 256; t += blockDim.x) hist[t] = 0;
        __syncthreads();
        for (int idx = threadIdx.x; idx < C; idx += blockDim.x) {
            const uint32_t key = float_to_ordered(sq[idx]);
            if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            int cum = 0;
            int sel = 0;
            for (int b = 255; b >= 0; --b) {
                if (cum + hist[b] >= remaining) {
                    sel = b;
                    break;
                }
                cum += hist[b];
            }
            s_prefix = prefix | (static_cast<uint32_t>(sel) << shift);
            s_remaining = remaining - cum;
        }
        __syncthreads();
        prefix = s_prefix;
        remaining = s_remaining;
        pmask |= 255u << shift;
    }
    const uint32_t T = prefix;
    const int need_ties = remaining;
    int tie_carry = 0, out_carry = 0;
    for (int base = 0; base < C; base += blockDim.x) {
        const int idx = base + threadIdx.x;
        uint32_t key = 0;
        if (idx < C) key = float_to_ordered(sq[idx]);
        const int is_eq = (idx < C && key == T) ? 1 : 0;
        int tot;
        const int tie_incl = block_inclusive_scan_shared(is_eq, scratch, &tot);
        const int tie_rank = tie_carry + tie_incl - is_eq;
        tie_carry += tot;
        const int sel = (idx < C && (key > T || (is_eq && tie_rank < need_ties))) ? 1 : 0;
        const int pos_incl = block_inclusive_scan_shared(sel, scratch, &tot);
        const int pos = out_carry + pos_incl - sel;
        out_carry += tot;
        if (sel && pos < sort_cap) keys[pos] = (static_cast<uint64_t>(~key) << 32) | static_cast<uint32_t>(idx);
    }
    for (int t = R + threadIdx.x; t < sort_cap; t += blockDim.x) keys[t] = ~0ull;
    __syncthreads();
    for (int size = 2; size <= sort_cap; size <<= 1) {
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < sort_cap / 2; t += blockDim.x) {
                const int a = 2 * t - (t & (stride - 1));
                const int b = a + stride;
                const bool up = (a & size) == 0;
                const uint64_t x = keys[a], y = keys[b];
                if ((x > y) == up) {
                    keys[a] = y;
                    keys[b] = x;
                }
            }
            __syncthreads();
        }
    }
    for (int t = threadIdx.x; t < R; t += blockDim.x) {
        const int idx = static_cast<int>(keys[t] & 0xFFFFFFFFu);
        rids[static_cast<size_t>(q) * k_refine + t] = cq[idx];
        if (rscore) rscore[static_cast<size_t>(q) * k_refine + t] = sq[idx];
    }
}

// ---- launchers ----

hipError_t configure_candidate_kernels(int64_t num_docs, int k_refine) {
    const int lg = partial_bitmap_log2(num_docs);
    const int partial_shm = static_cast<int>((size_t{1} << lg) / 8 < 4 ? 4 : (size_t{1} << lg) / 8);
    hipError_t e = hipSuccess;
    if (partial_shm > 64 * 1024)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(partial_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                partial_shm);
    if (e != hipSuccess) return e;
    const int sel_shm = pow2_at_least(k_refine < 2 ? 2 : k_refine) * 8;
    if (sel_shm > 64 * 1024)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(select_refine_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, sel_shm);
    return e;
}

static int grid_for(int qs) { return ((qs + 7) / 8) * 8 * kQ; }

hipError_t launch_mark(hipStream_t s, const uint32_t* labels, int q_base, int qs, int nprobe,
                       const uint64_t* cluster_pos, const int32_t* doc_clu, int64_t n_clusters, int64_t num_docs,
                       int nb, uint32_t* bitmap) {
    hipLaunchKernelGGL(mark_kernel, dim3(grid_for(qs)), dim3(256), 0, s, labels, q_base, qs, nprobe, cluster_pos,
                       doc_clu, n_clusters, num_docs, nb, bitmap);
    return hipGetLastError();
}

hipError_t launch_scan(hipStream_t s, const uint32_t* bitmap, int nb, int qs, uint32_t* offs, int32_t* cand,
                       int64_t cap, int32_t* ccount, uint32_t* err) {
    hipLaunchKernelGGL(scan_kernel, dim3(qs), dim3(1024), 0, s, bitmap, nb, qs, offs, cand, cap, ccount, err);
    return hipGetLastError();
}

int partial_bitmap_log2(int64_t num_docs) {
    int lg = 5;
    while (lg < 20 && (int64_t{1} << lg) < num_docs) ++lg;
    return lg;
}

hipError_t launch_partial(hipStream_t s, const uint32_t* labels, int q_base, int qs, int nprobe,
                          const uint64_t* cluster_pos, const uint8_t* codes_clu, const float* f1_clu,
                          const int32_t* doc_clu, int64_t n_clusters, int64_t num_docs, const float* lut,
                          const float* cb1, const uint32_t* bitmap, const uint32_t* offs, int nb, float* S,
                          int64_t cap, uint32_t* err) {
    const int lg = partial_bitmap_log2(num_docs);
    const size_t shm = (size_t{1} << lg) / 8 < 4 ? 4 : (size_t{1} << lg) / 8;
    hipLaunchKernelGGL(partial_kernel, dim3(grid_for(qs)), dim3(512), shm, s, labels, q_base, qs, nprobe,
                       cluster_pos, codes_clu, f1_clu, doc_clu, n_clusters, num_docs, lut, cb1, bitmap, offs, nb, lg,
                       S, cap, err);
    return hipGetLastError();
}

int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

hipError_t launch_select_refine(hipStream_t s, const float* S, const int32_t* cand, const int32_t* ccount,
                                int64_t cap, int q_base, int qs, int k_refine, int32_t* rcount, int32_t* rids,
                                float* rscore) {
    const int sort_cap = pow2_at_least(k_refine < 2 ? 2 : k_refine);
    hipLaunchKernelGGL(select_refine_kernel, dim3(qs), dim3(1024), static_cast<size_t>(sort_cap) * 8, s, S, cand,
                       ccount, cap, q_base, qs, k_refine, sort_cap, rcount, rids, rscore);
    return hipGetLastError();
}

}  // namespace chimera
