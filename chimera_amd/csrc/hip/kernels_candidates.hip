// Candidate generation for a sub-batch of queries, bucketed by document
// range. Restates mark_candidate_documents / count / materialize /
// partial_score / sum_partial_scores (kernels.cu:117-400) and the top-k_refine
// sort (search_impl.cu:160-261) without per-visit global atomics:
//
//   count    visits per (query, document bucket, query token)
//   offsets  exclusive scan of those counts: every (bucket, token) owns an
//            exact slice of the query's record area
//   emit     one record (doc, token, one-bit estimate) per visit, placed with
//            LDS counters
//   reduce   one block per (query, bucket): the touched documents, the
//            maximum estimate per (doc, token), S_cand = sum over tokens of
//            the positive maxima; candidates written in ascending doc order
//            with per-64-document group statistics
//   select   the first min(k_refine, C) candidates by S_cand descending,
//            ties by ascending doc ID (the reference's stable sort)
//
// A visit is (query token i, token position p) with p in one of the clusters
// probed by i; a document is a candidate when any of its tokens is visited
// (kernels.cu:206-278), and S_cand(d) = sum_i max(0, max over i's visits of d
// of est1(i, p)) (kernels.cu:381-396, 175-204).
#include "common.hpp"
#include "kernels.hpp"

namespace chimera {

namespace {

// Block b of the count and emit grids -> (query, token, part): the visits
// of a (query, token) are split into `parts` consecutive ranges, one block
// each (parts > 1 only for small sub-batches, which would otherwise leave
// most CUs idle). From 8 queries on, the grid is (qs rounded up to 8) x 32 x
// parts and the eight XCDs take blocks round-robin, so all blocks of one
// query land on the same XCD and share its L2; below 8 queries the grid is
// qs x 32 x parts, spread over every XCD. Returns false for a block past
// the sub-batch.
__device__ __forceinline__ bool cand_block(int b, int qs, int parts, int& qq, int& i, int& part) {
    if (qs >= 8) {
        const int slot = b >> 3;
        part = slot % parts;
        i = (slot / parts) & (kQ - 1);
        qq = (slot / (parts * kQ)) * 8 + (b & 7);
    } else {
        part = b % parts;
        i = (b / parts) % kQ;
        qq = b / (parts * kQ);
    }
    return qq < qs;
}

// The largest r in [0, n) with offs[r] <= v, for ascending offs with
// offs[0] <= v < offs[n]: the run holding visit v (never an empty run).
__device__ __forceinline__ int run_of(const uint32_t* offs, int n, uint32_t v) {
    int lo = 0, hi = n;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (offs[mid] <= v)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

// Visits [first, end) of part `part` of `parts` out of `total`.
__device__ __forceinline__ void part_range(int total, int part, int parts, int& first, int& end) {
    first = static_cast<int>(static_cast<int64_t>(total) * part / parts);
    end = static_cast<int>(static_cast<int64_t>(total) * (part + 1) / parts);
}

constexpr int kReduceThreads = 512;
constexpr int kReduceHeldMax = 12;  // records per reduce thread kept in registers, at most
constexpr int kWords = kMaxBucketDocs / 32;  // bitmap words of the largest bucket: thread t < words owns word t
constexpr int kSlotCap = 2048;               // (document, token) maxima held in LDS per chunk
constexpr int kChunkSlots = kSlotCap - kQ;   // slot bases per chunk: a document's slots never straddle
constexpr int kWideCap = kSlotCap / 3 + 1;   // documents of three or more tokens per chunk (3 slots each)
constexpr int kMaxChunks = (kMaxBucketDocs * kQ + kChunkSlots - 1) / kChunkSlots + 1;
static_assert(kWords <= kReduceThreads && (1 << (kMinBucketLog2 - 5)) % 2 == 0,
              "one bitmap word per thread, whole 64-document groups");

constexpr int rev5(int r) {
    return ((r & 1) << 4) | ((r & 2) << 2) | (r & 4) | ((r & 8) >> 2) | ((r & 16) >> 4);
}

// The shuffle-down tree of kernels.cu:195-198 (for o = 16, 8, 4, 2, 1: lane
// l += lane l + o) as one thread evaluates it, lane 0's result: leaf l is
// token l's maximum, slots[sb + rank of l in tm] when bit l of tm is set, +0
// otherwise. Step o pairs leaves that differ in bit log2(o), so the tree is
// the balanced pairwise sum of the leaves in bit-reversed order (leaf
// rev5(r) at position r): the leaves are taken in that order with one
// partial sum per level, the left operand of each pair being the lower
// positions (a + b = b + a bit for bit, so only the pairing matters). Every
// leaf is loaded, a token that did not visit from [sb, sb + popcount(tm)]:
// at most kSlotCap, so slots holds kSlotCap + 1 words.
__device__ __forceinline__ float tree_sum32(const uint32_t* slots, uint32_t sb, uint32_t tm) {
    float part[5];
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < kQ; ++r) {
        const int l = rev5(r);
        const float x = __uint_as_float(slots[sb + static_cast<uint32_t>(__popc(tm & ((1u << l) - 1u)))]);
        s = (tm >> l) & 1u ? x : 0.0f;
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            if (((r >> k) & 1) == 0) {
                part[k] = s;
                break;
            }
            s = part[k] + s;
        }
    }
    return s;
}
static_assert(kQ == 32, "the tree is over 32 tokens");

// Appends the slice documents d0 + j of the set bits j of `bits` to the wide
// list, one LDS atomic per wave. A chunk's wide documents hold at least 3 of
// its slots each, so the list cannot overflow.
static_assert(3 * kWideCap > kSlotCap, "every wide document of a chunk fits the list");
__device__ __forceinline__ void append_wide(uint32_t bits, int d0, uint16_t* wide, int* nwide) {
    const int n = __popc(bits);
    const int incl = wave_inclusive_scan(n);
    int base = 0;
    if (lane_id() == kWave - 1 && incl > 0) base = atomicAdd(nwide, incl);
    int k = __builtin_amdgcn_readlane(base, kWave - 1) + incl - n;
    for (uint32_t m = bits; m != 0u; m &= m - 1u) wide[k++] = static_cast<uint16_t>(d0 + __ffs(m) - 1);
}

// Walks part `part` of `parts` of the visits of (query, token): f(pos, doc)
// for every token position of the probed clusters in that range of visits.
// The probed runs' bounds are loaded once and their lengths scanned in LDS,
// then the block's threads take consecutive visit indices across run
// boundaries, so every load is independent and a wave's loads are
// contiguous. runs/offs are LDS arrays of kMaxProbe (+1) entries; every
// thread of the block must call this.
constexpr int kMaxProbe = 2048;
constexpr int kStagedMaxBuckets = 2048;  // the staged emit keeps per-bucket counters in LDS
constexpr int kStageVisits = 4096;       // visits per staging chunk

template <typename F>
__device__ __forceinline__ void for_each_visit(const uint32_t* lab, int nprobe, const uint64_t* __restrict__ cluster_pos,
                                               const int32_t* __restrict__ doc_clu, int64_t n_clusters,
                                               int64_t num_docs, uint32_t* runs, uint32_t* offs, int* scratch,
                                               int part, int parts, F&& f) {
    // per-thread share of the probes, then a block scan of the run lengths
    const int per = (nprobe + static_cast<int>(blockDim.x) - 1) / static_cast<int>(blockDim.x);
    const int p0 = static_cast<int>(threadIdx.x) * per;
    int mine = 0;
    for (int p = p0; p < p0 + per && p < nprobe; ++p) {
        const uint32_t label = lab[p];
        uint32_t len = 0, st = 0;
        if (label < static_cast<uint64_t>(n_clusters)) {
            st = static_cast<uint32_t>(cluster_pos[label]);
            len = static_cast<uint32_t>(cluster_pos[label + 1] - cluster_pos[label]);
        }
        runs[p] = st;
        offs[p] = len;  // length for now
        mine += static_cast<int>(len);
    }
    int total;
    const int incl = block_inclusive_scan_shared(mine, scratch, &total);
    int run = incl - mine;
    for (int p = p0; p < p0 + per && p < nprobe; ++p) {
        const uint32_t len = offs[p];
        offs[p] = static_cast<uint32_t>(run);
        run += static_cast<int>(len);
    }
    if (threadIdx.x == 0) offs[nprobe] = static_cast<uint32_t>(total);
    __syncthreads();
    // A thread's visits increase by blockDim.x, so its run index only moves
    // forward (runs average over a hundred visits: one or two steps per
    // visit). Positions of kGroup visits are found first and their document
    // ids loaded together.
    constexpr int kGroup = 8;
    int first, end;
    part_range(total, part, parts, first, end);
    if (first >= end) return;
    int lo = run_of(offs, nprobe, static_cast<uint32_t>(first));
    for (int vb = first + static_cast<int>(threadIdx.x); vb < end; vb += kGroup * static_cast<int>(blockDim.x)) {
        uint64_t pos[kGroup];
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const int v = vb + u * static_cast<int>(blockDim.x);
            pos[u] = 0;
            if (v < end) {
                while (offs[lo + 1] <= static_cast<uint32_t>(v)) ++lo;
                pos[u] = static_cast<uint64_t>(runs[lo]) + (static_cast<uint32_t>(v) - offs[lo]);
            }
        }
        int32_t doc[kGroup];
#pragma unroll
        for (int u = 0; u < kGroup; ++u) doc[u] = doc_clu[pos[u]];
#pragma unroll
        for (int u = 0; u < kGroup; ++u)
            if (vb + u * static_cast<int>(blockDim.x) < end && doc[u] >= 0 && doc[u] < num_docs) f(pos[u], doc[u]);
    }
}

}  // namespace

__global__ __launch_bounds__(256) void cand_count_kernel(const uint32_t* __restrict__ labels, int q_base, int qs,
                                                         int nprobe, const uint64_t* __restrict__ cluster_pos,
                                                         const int32_t* __restrict__ doc_clu, int64_t n_clusters,
                                                         int64_t num_docs, int blog, int nbk, int parts,
                                                         uint32_t* __restrict__ vcnt) {
    extern __shared__ uint32_t hist[];  // [nbk]
    __shared__ uint32_t runs[kMaxProbe];
    __shared__ uint32_t offs[kMaxProbe + 1];
    __shared__ int scratch[17];
    int qq, i, part;
    if (!cand_block(blockIdx.x, qs, parts, qq, i, part)) return;
    for (int t = threadIdx.x; t < nbk; t += blockDim.x) hist[t] = 0u;
    __syncthreads();
    const uint32_t* lab = labels + (static_cast<size_t>(q_base + qq) * kQ + i) * nprobe;
    for_each_visit(lab, nprobe, cluster_pos, doc_clu, n_clusters, num_docs, runs, offs, scratch, part, parts,
                   [&](uint64_t, int32_t doc) { atomicAdd(&hist[doc >> blog], 1u); });
    __syncthreads();
    const size_t bs = static_cast<size_t>(kQ) * parts;  // entries per bucket
    uint32_t* out = vcnt + static_cast<size_t>(qq) * nbk * bs + static_cast<size_t>(i) * parts + part;
    for (int b = threadIdx.x; b < nbk; b += blockDim.x) out[static_cast<size_t>(b) * bs] = hist[b];
}

namespace {

// Exclusive scan, in place, of the counts v[a, b) (as uint4) by the block,
// from `base`; returns the sum of the range. Wave w takes a contiguous part
// of the range, 64 consecutive uint4 per step so that every load and store is
// coalesced: pass 1 sums it (kU steps' loads in flight), a block scan of the
// lanes' sums gives each wave its start, and pass 2 rewrites the part as
// exclusive prefixes with a wave scan per step. Called by every thread.
__device__ int scan_counts(uint4* __restrict__ v, int a, int b, uint32_t base, int* scratch) {
    constexpr int kU = 4;
    const int nw = static_cast<int>(blockDim.x) / kWave;
    const int lane = lane_id();
    const int seg = (b - a + nw - 1) / nw;
    const int s0 = min(b, a + wave_id() * seg);
    const int s1 = min(b, s0 + seg);
    int mine = 0;
    for (int j = s0 + lane; j < s1; j += kU * kWave) {
        uint4 x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) x[u] = j + u * kWave < s1 ? v[j + u * kWave] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int u = 0; u < kU; ++u) mine += static_cast<int>(x[u].x + x[u].y + x[u].z + x[u].w);
    }
    int total;
    const int incl = block_inclusive_scan_shared(mine, scratch, &total);
    uint32_t carry = base + static_cast<uint32_t>(__builtin_amdgcn_readlane(incl - mine, 0));
    for (int j = s0; j < s1; j += kU * kWave) {
        uint4 x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int idx = j + u * kWave + lane;
            x[u] = idx < s1 ? v[idx] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int idx = j + u * kWave + lane;
            const int t = static_cast<int>(x[u].x + x[u].y + x[u].z + x[u].w);
            const int wi = wave_inclusive_scan(t);
            const uint32_t p = carry + static_cast<uint32_t>(wi - t), q = p + x[u].x, r = q + x[u].y, w = r + x[u].z;
            if (idx < s1) v[idx] = make_uint4(p, q, r, w);
            carry += static_cast<uint32_t>(__builtin_amdgcn_readlane(wi, kWave - 1));
        }
    }
    return total;
}

// Range [a, b) of segment sg of nseg over n4 uint4.
__device__ __forceinline__ void count_segment(int n4, int nseg, int sg, int& a, int& b) {
    const int per = (n4 + nseg - 1) / nseg;
    a = min(n4, sg * per);
    b = min(n4, a + per);
}

}  // namespace

// Per query: exclusive scan of the [bucket][token][part] visit counts in
// place, the total into vtot; a total above the record capacity raises
// kErrCandOverflow. Every bucket's records thus form one slice, starting at
// the offset of its (token 0, part 0).
__global__ __launch_bounds__(1024) void cand_offsets_kernel(uint32_t* __restrict__ vcnt, int nbk, int parts, int qs,
                                                            int64_t vcap, uint32_t* __restrict__ vtot,
                                                            uint32_t* __restrict__ err) {
    __shared__ int scratch[17];
    const int qq = blockIdx.x;
    if (qq >= qs) return;
    const int n = nbk * kQ * parts;  // a multiple of 32
    uint4* v = reinterpret_cast<uint4*>(vcnt + static_cast<size_t>(qq) * n);
    const int total = scan_counts(v, 0, n / 4, 0u, scratch);
    if (threadIdx.x == 0) {
        vtot[qq] = static_cast<uint32_t>(total);
        if (total > vcap) atomicOr(err, kErrCandOverflow);
    }
}

// The same scan for small sub-batches, with each query's counts split into
// nseg segments over nseg blocks (one CU moves a query's 0.5 MB of counts at
// about 0.1 TB/s). First each segment's sum, into the first nseg words of
// the query's record area (the visit records overwrite it later).
__global__ __launch_bounds__(256) void cand_offsets_part_kernel(const uint32_t* __restrict__ vcnt, int nbk, int parts,
                                                                int nseg, uint2* __restrict__ rec, int64_t vcap) {
    __shared__ int scratch[17];
    const int qq = blockIdx.y, sg = blockIdx.x;
    const int n4 = nbk * kQ * parts / 4;
    int a, b;
    count_segment(n4, nseg, sg, a, b);
    const uint4* v = reinterpret_cast<const uint4*>(vcnt) + static_cast<size_t>(qq) * n4;
    constexpr int kU = 4;
    const int step = static_cast<int>(blockDim.x);
    int mine = 0;
    for (int j = a + static_cast<int>(threadIdx.x); j < b; j += kU * step) {
        uint4 x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) x[u] = j + u * step < b ? v[j + u * step] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int u = 0; u < kU; ++u) mine += static_cast<int>(x[u].x + x[u].y + x[u].z + x[u].w);
    }
    int total;
    (void)block_inclusive_scan_shared(mine, scratch, &total);
    if (threadIdx.x == 0) reinterpret_cast<uint32_t*>(rec + static_cast<size_t>(qq) * vcap)[sg] = static_cast<uint32_t>(total);
}

// Then each segment's scan from the sum of the segments before it (nseg at
// most 64); the last segment's block writes the total into vtot.
__global__ __launch_bounds__(256) void cand_offsets_seg_kernel(uint32_t* __restrict__ vcnt, int nbk, int parts,
                                                               int nseg, const uint2* __restrict__ rec, int64_t vcap,
                                                               uint32_t* __restrict__ vtot,
                                                               uint32_t* __restrict__ err) {
    __shared__ int scratch[17];
    __shared__ int s_base;
    const int qq = blockIdx.y, sg = blockIdx.x;
    const int n4 = nbk * kQ * parts / 4;
    if (threadIdx.x < kWave) {
        const uint32_t* part = reinterpret_cast<const uint32_t*>(rec + static_cast<size_t>(qq) * vcap);
        const int x = static_cast<int>(threadIdx.x) < sg ? static_cast<int>(part[threadIdx.x]) : 0;
        const int before = wave_inclusive_scan(x);
        if (threadIdx.x == kWave - 1) s_base = before;
    }
    __syncthreads();
    const int base = s_base;
    int a, b;
    count_segment(n4, nseg, sg, a, b);
    uint4* v = reinterpret_cast<uint4*>(vcnt) + static_cast<size_t>(qq) * n4;
    const int total = base + scan_counts(v, a, b, static_cast<uint32_t>(base), scratch);
    if (sg == nseg - 1 && threadIdx.x == 0) {
        vtot[qq] = static_cast<uint32_t>(total);
        if (total > vcap) atomicOr(err, kErrCandOverflow);
    }
}

// One record per visit: {(doc mod 2^blog) << 5 | token, est1 bits}, with
// est1 = (sum over the 32 chunks of lut[c][nibble_c] - cb1) * f1 as in
// kernels.cu:361-379 (chunks summed in ascending order).
__global__ __launch_bounds__(256) void cand_emit_kernel(
    const uint32_t* __restrict__ labels, int q_base, int qs, int nprobe, const uint64_t* __restrict__ cluster_pos,
    const uint8_t* __restrict__ codes_clu, const float* __restrict__ f1_clu, const int32_t* __restrict__ doc_clu,
    int64_t n_clusters, int64_t num_docs, const float* __restrict__ lut, const float* __restrict__ cb1, int blog,
    int nbk, int parts, const uint32_t* __restrict__ vcnt, uint2* __restrict__ rec, int64_t vcap) {
    extern __shared__ uint32_t ctr[];  // [nbk] next free slot of each bucket
    __shared__ float llut[kChunks * kLut];
    __shared__ uint32_t runs[kMaxProbe];
    __shared__ uint32_t offs[kMaxProbe + 1];
    __shared__ int scratch[17];
    int qq, i, part;
    if (!cand_block(blockIdx.x, qs, parts, qq, i, part)) return;
    const int q = q_base + qq;
    for (int t = threadIdx.x; t < kChunks * kLut; t += blockDim.x)
        llut[t] = lut[static_cast<size_t>(q) * kLutPerQuery + static_cast<size_t>(i) * (kChunks * kLut) + t];
    const size_t bs = static_cast<size_t>(kQ) * parts;  // entries per bucket
    const uint32_t* off = vcnt + static_cast<size_t>(qq) * nbk * bs + static_cast<size_t>(i) * parts + part;
    for (int b = threadIdx.x; b < nbk; b += blockDim.x) ctr[b] = off[static_cast<size_t>(b) * bs];
    __syncthreads();
    const float cb = cb1[q * kQ + i];
    uint2* rq = rec + static_cast<size_t>(qq) * vcap;
    const uint32_t* lab = labels + (static_cast<size_t>(q) * kQ + i) * nprobe;
    for_each_visit(lab, nprobe, cluster_pos, doc_clu, n_clusters, num_docs, runs, offs, scratch, part, parts,
                   [&](uint64_t pos, int32_t doc) {
        const uint4 code = *reinterpret_cast<const uint4*>(codes_clu + pos * kCodeBytes);
        float ip = 0.0f;
#pragma unroll
        for (int c = 0; c < kChunks; ++c) ip += llut[c * kLut + code_nibble(code, c)];
        const float e = (ip - cb) * f1_clu[pos];
        const uint32_t slot = atomicAdd(&ctr[doc >> blog], 1u);
        if (slot < vcap)
            rq[slot] = make_uint2((static_cast<uint32_t>(doc & ((1 << blog) - 1)) << 5) | static_cast<uint32_t>(i),
                                  __float_as_uint(e));
    });
}

// The same records, written through an LDS staging area: the visits are
// taken in chunks of kStageVisits, counted per bucket, placed in LDS in
// bucket order and then written with consecutive threads on consecutive
// addresses of each bucket's slice (one run of about kStageVisits / nbk
// records per bucket and chunk instead of scattered 8-byte writes). For
// indexes of at most kStagedMaxBuckets buckets.
__global__ __launch_bounds__(256) void cand_emit_staged_kernel(
    const uint32_t* __restrict__ labels, int q_base, int qs, int nprobe, const uint64_t* __restrict__ cluster_pos,
    const uint8_t* __restrict__ codes_clu, const float* __restrict__ f1_clu, const int32_t* __restrict__ doc_clu,
    int64_t n_clusters, int64_t num_docs, const float* __restrict__ lut, const float* __restrict__ cb1, int blog,
    int nbk, int parts, const uint32_t* __restrict__ vcnt, uint2* __restrict__ rec, int64_t vcap) {
    extern __shared__ uint32_t dyn[];               // [nbk] ctr, [nbk] bcnt, [nprobe] runs, [nprobe + 1] offs
    uint32_t* ctr = dyn;                            // next free slot of each bucket's slice
    uint32_t* bcnt = dyn + nbk;                     // records of the chunk per bucket, then run starts
    uint32_t* runs = dyn + 2 * nbk;
    uint32_t* offs = dyn + 2 * nbk + nprobe;
    __shared__ uint2 stage[kStageVisits];
    __shared__ uint16_t sbucket[kStageVisits];
    __shared__ float llut[kChunks * kLut];
    __shared__ int scratch[17];
    int qq, i, part;
    if (!cand_block(blockIdx.x, qs, parts, qq, i, part)) return;
    const int q = q_base + qq;
    for (int t = threadIdx.x; t < kChunks * kLut; t += blockDim.x)
        llut[t] = lut[static_cast<size_t>(q) * kLutPerQuery + static_cast<size_t>(i) * (kChunks * kLut) + t];
    const size_t bs = static_cast<size_t>(kQ) * parts;  // entries per bucket
    const uint32_t* off = vcnt + static_cast<size_t>(qq) * nbk * bs + static_cast<size_t>(i) * parts + part;
    for (int b = threadIdx.x; b < nbk; b += blockDim.x) {
        ctr[b] = off[static_cast<size_t>(b) * bs];
        bcnt[b] = 0u;
    }
    // run bounds and their prefix (as in for_each_visit)
    const uint32_t* lab = labels + (static_cast<size_t>(q) * kQ + i) * nprobe;
    const int per = (nprobe + static_cast<int>(blockDim.x) - 1) / static_cast<int>(blockDim.x);
    const int p0 = static_cast<int>(threadIdx.x) * per;
    int mine = 0;
    for (int p = p0; p < p0 + per && p < nprobe; ++p) {
        const uint32_t label = lab[p];
        uint32_t len = 0, st = 0;
        if (label < static_cast<uint64_t>(n_clusters)) {
            st = static_cast<uint32_t>(cluster_pos[label]);
            len = static_cast<uint32_t>(cluster_pos[label + 1] - cluster_pos[label]);
        }
        runs[p] = st;
        offs[p] = len;
        mine += static_cast<int>(len);
    }
    int total;
    const int incl = block_inclusive_scan_shared(mine, scratch, &total);
    int run = incl - mine;
    for (int p = p0; p < p0 + per && p < nprobe; ++p) {
        const uint32_t len = offs[p];
        offs[p] = static_cast<uint32_t>(run);
        run += static_cast<int>(len);
    }
    if (threadIdx.x == 0) offs[nprobe] = static_cast<uint32_t>(total);
    __syncthreads();
    const float cb = cb1[q * kQ + i];
    uint2* rq = rec + static_cast<size_t>(qq) * vcap;
    constexpr int kPer = kStageVisits / 256;
    constexpr int kGroup = 8;  // visits whose loads are issued together
    static_assert(kPer % kGroup == 0, "whole groups per chunk");
    int first, end;  // this part's visits
    part_range(total, part, parts, first, end);
    // run of this thread's visit: only moves forward
    int lo = first < end ? run_of(offs, nprobe, static_cast<uint32_t>(first)) : 0;
    for (int v0 = first; v0 < end; v0 += kStageVisits) {
        const int n = end - v0 < kStageVisits ? end - v0 : kStageVisits;
        uint32_t key[kPer], est[kPer], local[kPer];
#pragma unroll
        for (int j0 = 0; j0 < kPer; j0 += kGroup) {
            uint64_t pos[kGroup];
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                const int v = v0 + static_cast<int>(threadIdx.x) + 256 * (j0 + u);
                pos[u] = 0;
                if (v < v0 + n) {
                    while (offs[lo + 1] <= static_cast<uint32_t>(v)) ++lo;
                    pos[u] = static_cast<uint64_t>(runs[lo]) + (static_cast<uint32_t>(v) - offs[lo]);
                }
            }
            // unconditional loads (position 0 stands in past the chunk)
            int32_t dv[kGroup];
            uint4 cv[kGroup];
            float fv[kGroup];
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                dv[u] = doc_clu[pos[u]];
                cv[u] = *reinterpret_cast<const uint4*>(codes_clu + pos[u] * kCodeBytes);
                fv[u] = f1_clu[pos[u]];
            }
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                const int j = j0 + u;
                const int v = v0 + static_cast<int>(threadIdx.x) + 256 * j;
                key[j] = 0xFFFFFFFFu;
                const int32_t doc = dv[u];
                if (v < v0 + n && doc >= 0 && doc < num_docs) {
                    float ip = 0.0f;
#pragma unroll
                    for (int c = 0; c < kChunks; ++c) ip += llut[c * kLut + code_nibble(cv[u], c)];
                    const float e = (ip - cb) * fv[u];
                    key[j] = static_cast<uint32_t>(doc);
                    est[j] = __float_as_uint(e);
                    local[j] = atomicAdd(&bcnt[doc >> blog], 1u);
                }
            }
        }
        __syncthreads();
        // bucket run starts within the chunk (exclusive scan of bcnt); m
        // records in the chunk
        int m;
        {
            const int bper = (nbk + static_cast<int>(blockDim.x) - 1) / static_cast<int>(blockDim.x);
            const int b0 = static_cast<int>(threadIdx.x) * bper;
            int sm = 0;
            for (int b = b0; b < b0 + bper && b < nbk; ++b) sm += static_cast<int>(bcnt[b]);
            int tot;
            const int inc = block_inclusive_scan_shared(sm, scratch, &tot);
            int rs = inc - sm;
            for (int b = b0; b < b0 + bper && b < nbk; ++b) {
                const uint32_t c = bcnt[b];
                bcnt[b] = static_cast<uint32_t>(rs);
                rs += static_cast<int>(c);
            }
            m = tot;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            if (key[j] != 0xFFFFFFFFu) {
                const uint32_t b = key[j] >> blog;
                const uint32_t slot = bcnt[b] + local[j];
                stage[slot] = make_uint2(((key[j] & ((1u << blog) - 1u)) << 5) | static_cast<uint32_t>(i), est[j]);
                sbucket[slot] = static_cast<uint16_t>(b);
            }
        }
        __syncthreads();
        // records of the chunk, bucket by bucket
        for (int t = threadIdx.x; t < m; t += blockDim.x) {
            const uint32_t b = sbucket[t];
            const uint32_t dest = ctr[b] + (static_cast<uint32_t>(t) - bcnt[b]);
            if (dest < vcap) rq[dest] = stage[t];
        }
        __syncthreads();
        // advance the slice cursors and clear the chunk counts: the count of
        // bucket b is the distance to the next non-empty run start
        for (int b = threadIdx.x; b < nbk; b += blockDim.x) {
            const uint32_t next = b + 1 < nbk ? bcnt[b + 1] : static_cast<uint32_t>(m);
            ctr[b] += next - bcnt[b];
        }
        __syncthreads();
        for (int b = threadIdx.x; b < nbk; b += blockDim.x) bcnt[b] = 0u;
        __syncthreads();
    }
}

// Value of lane l ^ 1 or l ^ 2 (DPP quad permute kCtl = 0xB1 or 0x4E).
template <int kCtl>
__device__ __forceinline__ int quad_xor(int v) {
    return __builtin_amdgcn_mov_dpp(v, kCtl, 0xF, 0xF, false);
}
__device__ __forceinline__ void group_stats_combine(float& m1, float& m2, uint32_t& arg, float om1, float om2,
                                                    uint32_t oarg) {
    m2 = fmaxf(fminf(m1, om1), fmaxf(m2, om2));
    arg = m1 >= om1 ? arg : oarg;
    m1 = fmaxf(m1, om1);
}
template <int kCtl>
__device__ __forceinline__ void group_stats_quad(float& m1, float& m2, uint32_t& arg, int& cnt) {
    const float om1 = __int_as_float(quad_xor<kCtl>(__float_as_int(m1)));
    const float om2 = __int_as_float(quad_xor<kCtl>(__float_as_int(m2)));
    const uint32_t oarg = static_cast<uint32_t>(quad_xor<kCtl>(static_cast<int>(arg)));
    cnt += quad_xor<kCtl>(cnt);
    group_stats_combine(m1, m2, arg, om1, om2, oarg);
}
// The statistics of a group of gl lanes (a power of two up to 64, aligned
// to gl, uniform over the wave) combined by a lane butterfly, every lane
// ending with them: the largest and second-largest S of the group's
// documents, the doc of the largest and the candidate count. Equal largest
// values make the second equal to them (the doc is then not used). Lanes
// l ^ 1 and l ^ 2 by DPP quad permutes (no LDS), wider by shuffles.
__device__ __forceinline__ void group_stats(int gl, float& m1, float& m2, uint32_t& arg, int& cnt) {
    if (gl > 1) group_stats_quad<0xB1>(m1, m2, arg, cnt);
    if (gl > 2) group_stats_quad<0x4E>(m1, m2, arg, cnt);
    for (int o = 4; o < gl; o <<= 1) {
        const float om1 = __shfl_xor(m1, o, kWave);
        const float om2 = __shfl_xor(m2, o, kWave);
        const uint32_t oarg = static_cast<uint32_t>(__shfl_xor(static_cast<int>(arg), o, kWave));
        cnt += __shfl_xor(cnt, o, kWave);
        group_stats_combine(m1, m2, arg, om1, om2, oarg);
    }
}

// One block per (query, bucket) item; S_cand of every touched document,
// bit for bit the reference's: partial[doc][i] = max(0, max est over token
// i's visits of doc) (kernels.cu:381-396), S = the shuffle-down tree over
// the 32 tokens (kernels.cu:175-204: lane l += lane l + 16, + 8, + 4, + 2,
// + 1), whatever the order of the records.
//   pass A  mask[doc] |= 1 << token for every record; the record that first
//           touches a document sets its bit in `touched`, the one that adds
//           its second distinct token sets its bit in `multi` (read from
//           the value atomicOr returns, so each happens once)
//   scan    a document visited by one token needs no slot: its S is the max
//           of that token's positive estimates (x + 0 = x in the tree), kept
//           in aux[doc]. Documents of c >= 2 tokens get c consecutive LDS
//           slots (token order) at the prefix of their counts in doc order,
//           found by walking the `multi` bitmap
//   pass B  max (as the bits of non-negative floats) of the positive
//           estimates into aux or the slots
//   pass C  S = a + b for two tokens (exact in either order); documents of
//           three or more tokens are listed, and one thread per listed
//           document evaluates the shuffle-down tree over the 32 tokens
// When a bucket's multi-token documents need more slots than LDS holds, the
// slots are processed in chunks of documents whose slot bases fall in one
// kChunkSlots window. An item whose slots fit one chunk (the 8-record
// variant) skips pass C: its wide documents are listed with the slot bases,
// at places the same scan gives, and its two-token sums are taken in the
// output phase. Every per-document step after pass A walks the
// bitmaps rather than all 2^blog documents (each thread a slice of
// 2^blog / 512 documents, or one), and the masks and S values of the
// touched documents are cleared as they are written out, so an item costs
// its records and touched documents only. One scan after pass A gives both
// the slot bases and the output positions.
// Output: the bucket's candidates {doc, S bits} in ascending doc order at the
// start of its record slice, the candidate count, and per 64-document group
// {max S (-1 when empty), offset | count << 16} in gstat and {second-largest
// S (-1 when fewer than two candidates; equal to the max when two share
// it), doc of the max} in gsec, and the top 16 bits of the max's ordered key
// in gkey.
template <int kHeld>
__global__ __launch_bounds__(kReduceThreads, 4) void cand_reduce_kernel(
    const uint32_t* __restrict__ vcnt, const uint32_t* __restrict__ vtot, int blog, int nbk, int bshift, int qs,
    int64_t num_docs, uint2* __restrict__ rec, int64_t vcap, uint32_t* __restrict__ tcount,
    float2* __restrict__ gstat, uint2* __restrict__ gsec, uint16_t* __restrict__ gkey) {
    __shared__ __align__(16) uint32_t mask[kMaxBucketDocs];  // token bits
    __shared__ __align__(16) uint32_t aux[kMaxBucketDocs];   // S bits, or the slot base of a multi-token doc
    __shared__ uint32_t touched[kWords];                  // documents with a record
    __shared__ uint32_t multi[kWords];                    // documents with records of two or more tokens
    __shared__ __align__(16) uint32_t slots[kSlotCap + 1];  // one word past the last slot: see tree_sum32
    __shared__ uint16_t wide[kWideCap];
    __shared__ int chunk_doc[kMaxChunks + 1];             // first document of each chunk
    __shared__ int scratch[32];
    __shared__ int s_nwide;
    // Persistent blocks: item = (query, bucket), bucket fastest; a block
    // takes items blockIdx.x, + gridDim.x, ... and loads the next item's
    // records while it finishes the current one (from the end of pass B for
    // a one-chunk item, in the output phase otherwise).
    const int nitems = nbk * qs;
    int item = static_cast<int>(blockIdx.x);
    if (item >= nitems) return;
    const int stride = static_cast<int>(blockDim.x);
    struct Item {
        int b, qq, r0, r1;
    };
    auto item_of = [&](int it) {
        Item x;
        x.b = it % nbk;
        x.qq = it / nbk;
        const uint32_t* oq = vcnt + (static_cast<size_t>(x.qq) * nbk << bshift);
        x.r0 = static_cast<int>(oq[static_cast<size_t>(x.b) << bshift]);
        const int e = x.b + 1 < nbk ? static_cast<int>(oq[static_cast<size_t>(x.b + 1) << bshift])
                                    : static_cast<int>(vtot[x.qq]);
        x.r1 = e < vcap ? e : static_cast<int>(vcap);
        return x;
    };
    // The first kHeld records of each thread are loaded together and kept
    // in registers for pass B; a bucket with more than kHeld * blockDim.x
    // records reads the rest again.
    auto load_held = [&](const Item& x, uint2 (&h)[kHeld]) {
        const uint2* rq = rec + static_cast<size_t>(x.qq) * vcap;
#pragma unroll
        for (int u = 0; u < kHeld; ++u) {
            const int r = x.r0 + static_cast<int>(threadIdx.x) + u * stride;
            h[u] = r < x.r1 ? rq[r] : make_uint2(0xFFFFFFFFu, 0u);
        }
    };
    Item cur = item_of(item);
    uint2 held[kHeld];
    load_held(cur, held);
    // everything starts cleared once; afterwards each item clears what it
    // touched (bitmap words after the scan, masks and S values in the
    // output phase, the slots after their last read)
    static_assert(kMaxBucketDocs % 4 == 0 && kSlotCap % 4 == 0, "vector clears");
    for (int t = threadIdx.x; t < kMaxBucketDocs / 4; t += blockDim.x) {
        reinterpret_cast<uint4*>(mask)[t] = make_uint4(0u, 0u, 0u, 0u);
        reinterpret_cast<uint4*>(aux)[t] = make_uint4(0u, 0u, 0u, 0u);
    }
    for (int t = threadIdx.x; t < kSlotCap / 4; t += blockDim.x)
        reinterpret_cast<uint4*>(slots)[t] = make_uint4(0u, 0u, 0u, 0u);
    const int tid = static_cast<int>(threadIdx.x);
    const int nb = 1 << blog;  // documents per bucket
    // Per-document steps: thread t takes the dpt consecutive documents from
    // d0 = t dpt (dpt divides 32: a whole or part bitmap word; with fewer
    // documents than threads the last threads take none).
    const int dpt = nb > kReduceThreads ? nb / kReduceThreads : 1;
    const int d0 = tid * dpt;
    const bool has = d0 < nb;
    const int sw = d0 >> 5, ssh = d0 & 31;
    const uint32_t smask = dpt >= 32 ? 0xFFFFFFFFu : (1u << dpt) - 1u;
    const bool word_head = has && ssh == 0;  // clears its bitmap word for the next item
    if (word_head) {
        touched[sw] = 0u;
        multi[sw] = 0u;
    }
    if (tid == 0) s_nwide = 0;
    __syncthreads();
    for (;;) {
    const int b = cur.b;
    const int qq = cur.qq;
    const int r0 = cur.r0;
    const int r1 = cur.r1;
    uint2* rq = rec + static_cast<size_t>(qq) * vcap;
    const int rt = r0 + tid;
    // the next item's record range, read now so that its record loads do
    // not wait on it
    const int next = item + static_cast<int>(gridDim.x);
    Item nxt{0, 0, 0, 0};
    if (next < nitems) nxt = item_of(next);
    // pass A
    auto mark = [&](uint32_t key) {
        const uint32_t d = key >> 5, bit = 1u << (key & 31u);
        const uint32_t old = atomicOr(&mask[d], bit);
        if (old == 0u) {
            atomicOr(&touched[d >> 5], 1u << (d & 31u));
        } else if ((old & bit) == 0u && (old & (old - 1u)) == 0u) {  // its second token
            atomicOr(&multi[d >> 5], 1u << (d & 31u));
        }
    };
#pragma unroll
    for (int u = 0; u < kHeld; ++u)
        if (held[u].x != 0xFFFFFFFFu) mark(held[u].x);
    for (int r = rt + kHeld * stride; r < r1; r += stride) mark(rq[r].x);
    __syncthreads();
    // One scan in doc order gives both the slot bases of the multi-token
    // documents (prefix of their token counts) and the output positions
    // (prefix of the touched documents). Each thread holds its slice's bits,
    // so the word heads clear the bitmaps for the next item once the scan's
    // barriers have passed.
    static_assert(kMaxChunks + 1 <= kReduceThreads, "one chunk start per thread");
    if (tid <= kMaxChunks) chunk_doc[tid] = nb;  // ordered by the scan's barriers
    const uint32_t tbits = has ? (touched[sw] >> ssh) & smask : 0u;
    const uint32_t mbits = has ? (multi[sw] >> ssh) & smask : 0u;
    int mine = 0;
    uint32_t twobits = 0u;  // the slice's documents of exactly two tokens
    for (uint32_t m = mbits; m != 0u; m &= m - 1u) {
        const int j = __ffs(m) - 1;
        const int c = __popc(mask[d0 + j]);
        mine += c;
        if (c == 2) twobits |= 1u << j;
    }
    const int cnt = __popc(tbits);
    const uint32_t wbits0 = mbits & ~twobits;  // documents of three or more tokens
    // the wide documents' count rides in the high half of the touched count
    // (both at most 2^13 per bucket), for the one-chunk path below
    static_assert(kMaxBucketDocs < (1 << 16), "two 16-bit counts in one scan word");
    const int packed = kHeld == 8 ? cnt | (__popc(wbits0) << 16) : cnt;
    int incl = mine, pos = packed;
    int total_slots, total;
    // (the scan's closing barrier is not needed: the next write of scratch
    // is the next item's scan, several barriers on)
    block_inclusive_scan2<false>(incl, pos, scratch, &total_slots, &total);
    pos -= packed;
    const int wpos = pos >> 16;  // the slice's first place in the wide list
    pos &= 0xFFFF;               // the slice's first output position
    const int total_wide = total >> 16;
    total &= 0xFFFF;
    if (word_head) {
        touched[sw] = 0u;
        multi[sw] = 0u;
    }
    // When every slot fits one chunk (as with few multi-token documents per
    // bucket), the wide documents are listed now at the places the scan
    // gave, their trees run right after pass B, and the two-token sums are
    // taken in the output phase: no pass C and one barrier fewer. Only the
    // 8-record variant has this path: the 12-record one (buckets raised by
    // the bucket cap over many records per document) mostly needs several
    // chunks, and its registers would spill there.
    const bool one_chunk = kHeld == 8 && total_slots <= kChunkSlots;
    if (one_chunk) {
        int k = wpos;
        for (uint32_t m = wbits0; m != 0u; m &= m - 1u) wide[k++] = static_cast<uint16_t>(d0 + __ffs(m) - 1);
    }
    {
        // chunk ch = the multi-token documents whose slot base lies in
        // [ch, ch + 1) * kChunkSlots; its first document is the smallest such
        // one. Bases grow by at most kQ <= kChunkSlots per document, so every
        // chunk up to that of the last base has a document.
        int base = incl - mine;
        int prev_chunk = -1;
        for (uint32_t m = mbits; m != 0u; m &= m - 1u) {
            const int d = d0 + __ffs(m) - 1;
            aux[d] = static_cast<uint32_t>(base);
            const int ch = base / kChunkSlots;
            if (ch != prev_chunk && !one_chunk) atomicMin(&chunk_doc[ch], d);
            prev_chunk = ch;
            base += (twobits >> (d - d0)) & 1u ? 2 : __popc(mask[d]);
        }
    }
    // chunk 0 starts at document 0 whatever its first multi-token document
    const int nchunks = total_slots == 0 ? 1 : (total_slots - 1) / kChunkSlots + 1;
    __syncthreads();
    for (int ch = 0; ch < nchunks; ++ch) {
        const int lo = ch == 0 ? 0 : chunk_doc[ch];
        const int hi = ch + 1 == nchunks ? nb : chunk_doc[ch + 1];
        const uint32_t off = static_cast<uint32_t>(ch) * kChunkSlots;
        // pass B: positive estimates of this chunk's multi-token documents,
        // and (in the first chunk) of every one-token document
        auto add = [&](uint2 v) {
            const float e = __uint_as_float(v.y);
            if (v.x == 0xFFFFFFFFu || !(e > 0.0f)) return;
            const uint32_t dl = v.x >> 5;
            const uint32_t m = mask[dl];
            const uint32_t lower = m & ((1u << (v.x & 31u)) - 1u);
            if (m == (m & (0u - m))) {  // one token
                if (ch == 0) atomicMax(&aux[dl], v.y);  // non-negative floats order as their bits
            } else if (static_cast<int>(dl) >= lo && static_cast<int>(dl) < hi) {
                atomicMax(&slots[aux[dl] - off + __popc(lower)], v.y);
            }
        };
#pragma unroll
        for (int u = 0; u < kHeld; ++u) add(held[u]);
        for (int r = rt + kHeld * stride; r < r1; r += stride) add(rq[r]);
        __syncthreads();
        // a one-chunk item no longer reads its held records: the next item's
        // load now, so that the trees and the output phase cover its latency
        if (one_chunk && next < nitems) load_held(nxt, held);
        if (!one_chunk) {
            // pass C: S = a + b for the slice's two-token documents of the
            // chunk (exact in either order); three or more tokens go to the
            // wide list. A document's slots are read by one thread only,
            // which clears them for the next chunk or item (a barrier
            // separates this from the next pass B).
            uint32_t wbits = 0u;
            for (uint32_t m = mbits; m != 0u; m &= m - 1u) {
                const int j = __ffs(m) - 1;
                const int d = d0 + j;
                if (d < lo || d >= hi) continue;
                if ((twobits >> j) & 1u) {
                    const uint32_t sb = aux[d] - off;
                    const float s = __uint_as_float(slots[sb]) + __uint_as_float(slots[sb + 1]);
                    slots[sb] = 0u;
                    slots[sb + 1] = 0u;
                    aux[d] = __float_as_uint(s);
                } else {
                    wbits |= 1u << j;
                }
            }
            append_wide(wbits, d0, wide, &s_nwide);
            __syncthreads();
        }
        const int nw = one_chunk ? total_wide : s_nwide;
        if (nw > 0) {
            // one thread per wide document: the tree in registers
            for (int k = tid; k < nw; k += stride) {
                const int d = wide[k];
                const uint32_t tm = mask[d];
                const uint32_t sb = aux[d] - off;
                aux[d] = __float_as_uint(tree_sum32(slots, sb, tm));
                const uint32_t se = sb + static_cast<uint32_t>(__popc(tm));
                for (uint32_t t = sb; t < se; ++t) slots[t] = 0u;
            }
            __syncthreads();
        }
        // every thread read s_nwide before the barrier after the trees; with
        // no wide document the value stays 0 (one-chunk items do not use it)
        if (!one_chunk && tid == 0) s_nwide = 0;
        if (ch + 1 < nchunks) __syncthreads();
    }
    // (chunked items) the next item's records load during the output phase
    // (the held records are no longer read)
    if (!one_chunk && next < nitems) load_held(nxt, held);
    // compact output in ascending doc order, each thread its slice's
    // touched documents from position pos, straight into the record slice
    // (its records are no longer read). Their masks and S values are read
    // for the last time and cleared for the next item.
    uint2* out = rq + r0;
    float gmax = -1.0f, gsnd = -1.0f;  // the slice's largest and second-largest S
    uint32_t garg = 0u;                // and the doc of the largest
    int k = pos;
    for (uint32_t m = tbits; m != 0u; m &= m - 1u) {
        const int j = __ffs(m) - 1;
        const int d = d0 + j;
        uint32_t sbits = aux[d];
        if (one_chunk && ((twobits >> j) & 1u)) {
            // a two-token document: sbits is its slot base (chunk 0)
            const float s = __uint_as_float(slots[sbits]) + __uint_as_float(slots[sbits + 1]);
            slots[sbits] = 0u;
            slots[sbits + 1] = 0u;
            sbits = __float_as_uint(s);
        }
        aux[d] = 0u;  // a one-token document of the next item starts from +0
        mask[d] = 0u;
        const uint32_t doc = (static_cast<uint32_t>(b) << blog) + static_cast<uint32_t>(d);
        out[k++] = make_uint2(doc, sbits);
        const float sv = __uint_as_float(sbits);
        garg = sv > gmax ? doc : garg;
        gsnd = fmaxf(gsnd, fminf(sv, gmax));
        gmax = fmaxf(gmax, sv);
    }
    // a 64-document group = the slices of 64 / dpt consecutive lanes; the
    // first of them (whose slice starts at the group's first output
    // position) writes the group's statistics
    const int gl = kWave / dpt;
    int gcnt = cnt;
    group_stats(gl, gmax, gsnd, garg, gcnt);
    if (has && (tid & (gl - 1)) == 0) {
        const size_t g = (static_cast<size_t>(qq) * nbk + b) * groups_per_bucket(blog) + d0 / kWave;
        gstat[g] = make_float2(gmax, __uint_as_float(static_cast<uint32_t>(pos) | (static_cast<uint32_t>(gcnt) << 16)));
        gsec[g] = make_uint2(__float_as_uint(gsnd), garg);
        gkey[g] = static_cast<uint16_t>(float_to_ordered(gmax) >> 16);
    }
    if (tid == 0) tcount[static_cast<size_t>(qq) * nbk + b] = static_cast<uint32_t>(total);
    __syncthreads();  // the next item's pass A finds the masks and bitmaps cleared
    if (next >= nitems) break;
    item = next;
    cur = nxt;
    }
}

// The same output for buckets of kDenseDocs = 256 documents, the size taken
// by indexes with many visit records per document (at least 12), where
// nearly every document is visited by many query tokens: a full
// [document][token] table of the clamped maxima replaces the masks, slots
// and chunks. Every record sets its token bit and does one atomicMax (a
// positive estimate, as the bits of a non-negative float) into its cell;
// then thread t < 256 takes document t and evaluates the shuffle-down tree
// over its 32 cells in registers (for o = 16, 8, 4, 2, 1: v[l] += v[l + o]
// for l < o, which is lane 0's side of kernels.cu:195-198; cells of tokens
// that did not visit hold +0). Cells are swizzled (token ^ (doc mod 32)) so
// that a wave reading one cell index of its documents meets at most two of
// them per bank. About four barriers per item instead of the sparse
// kernel's ten or more.
constexpr int kDenseDocs = 256;
template <int kHeld>
__global__ __launch_bounds__(kReduceThreads) void cand_reduce_dense_kernel(
    const uint32_t* __restrict__ vcnt, const uint32_t* __restrict__ vtot, int nbk, int bshift, int qs,
    uint2* __restrict__ rec, int64_t vcap, uint32_t* __restrict__ tcount, float2* __restrict__ gstat,
    uint2* __restrict__ gsec, uint16_t* __restrict__ gkey) {
    __shared__ __align__(16) uint32_t table[kDenseDocs * kQ];
    __shared__ __align__(16) uint32_t mask[kDenseDocs];
    __shared__ int scratch[17];
    const int nitems = nbk * qs;
    int item = static_cast<int>(blockIdx.x);
    if (item >= nitems) return;
    const int stride = static_cast<int>(blockDim.x);
    struct Item {
        int b, qq, r0, r1;
    };
    auto item_of = [&](int it) {
        Item x;
        x.b = it % nbk;
        x.qq = it / nbk;
        const uint32_t* oq = vcnt + (static_cast<size_t>(x.qq) * nbk << bshift);
        x.r0 = static_cast<int>(oq[static_cast<size_t>(x.b) << bshift]);
        const int e = x.b + 1 < nbk ? static_cast<int>(oq[static_cast<size_t>(x.b + 1) << bshift])
                                    : static_cast<int>(vtot[x.qq]);
        x.r1 = e < vcap ? e : static_cast<int>(vcap);
        return x;
    };
    auto load_held = [&](const Item& x, uint2 (&h)[kHeld]) {
        const uint2* rq = rec + static_cast<size_t>(x.qq) * vcap;
#pragma unroll
        for (int u = 0; u < kHeld; ++u) {
            const int r = x.r0 + static_cast<int>(threadIdx.x) + u * stride;
            h[u] = r < x.r1 ? rq[r] : make_uint2(0xFFFFFFFFu, 0u);
        }
    };
    Item cur = item_of(item);
    uint2 held[kHeld];
    load_held(cur, held);
    // cleared once; afterwards each document's cells and mask are cleared
    // when it is written out
    for (int t = threadIdx.x; t < kDenseDocs * kQ / 4; t += blockDim.x)
        reinterpret_cast<uint4*>(table)[t] = make_uint4(0u, 0u, 0u, 0u);
    for (int t = threadIdx.x; t < kDenseDocs; t += blockDim.x) mask[t] = 0u;
    __syncthreads();
    const int tid = static_cast<int>(threadIdx.x);
    for (;;) {
        const int b = cur.b;
        const int qq = cur.qq;
        const int r0 = cur.r0;
        const int r1 = cur.r1;
        uint2* rq = rec + static_cast<size_t>(qq) * vcap;
        const int next = item + static_cast<int>(gridDim.x);
        Item nxt{0, 0, 0, 0};
        if (next < nitems) nxt = item_of(next);
        auto put = [&](uint2 v) {
            if (v.x == 0xFFFFFFFFu) return;
            const uint32_t d = v.x >> 5, tok = v.x & 31u;
            atomicOr(&mask[d], 1u << tok);
            if (__uint_as_float(v.y) > 0.0f) atomicMax(&table[d * kQ + (tok ^ (d & 31u))], v.y);
        };
#pragma unroll
        for (int u = 0; u < kHeld; ++u) put(held[u]);
        for (int r = r0 + tid + kHeld * stride; r < r1; r += stride) put(rq[r]);
        __syncthreads();
        // the next item's records load during the output phase
        if (next < nitems) load_held(nxt, held);
        uint32_t m = 0u;
        float S = 0.0f;
        if (tid < kDenseDocs) {
            m = mask[tid];
            if (m != 0u) {
                float v[kQ];
#pragma unroll
                for (int j = 0; j < kQ; ++j) {
                    uint32_t* cell = &table[tid * kQ + (j ^ (tid & 31))];
                    v[j] = __uint_as_float(*cell);
                    *cell = 0u;
                }
#pragma unroll
                for (int o = kQ / 2; o >= 1; o >>= 1)
#pragma unroll
                    for (int j = 0; j < o; ++j) v[j] += v[j + o];
                S = v[0];
                mask[tid] = 0u;
            }
        }
        const int cnt = m != 0u ? 1 : 0;
        int total;
        const int pos = block_inclusive_scan_shared(cnt, scratch, &total) - cnt;
        if (cnt) rq[r0 + pos] = make_uint2((static_cast<uint32_t>(b) << 8) + static_cast<uint32_t>(tid), __float_as_uint(S));
        // a 64-document group = one wave
        float gmax = cnt ? S : -1.0f, gsnd = -1.0f;
        uint32_t garg = (static_cast<uint32_t>(b) << 8) + static_cast<uint32_t>(tid);
        int gcnt = cnt;
        group_stats(kWave, gmax, gsnd, garg, gcnt);
        const int gpos = __builtin_amdgcn_readfirstlane(pos);
        if (tid < kDenseDocs && lane_id() == 0) {
            const size_t g = (static_cast<size_t>(qq) * nbk + b) * groups_per_bucket(8) + tid / kWave;
            gstat[g] = make_float2(gmax, __uint_as_float(static_cast<uint32_t>(gpos) | (static_cast<uint32_t>(gcnt) << 16)));
            gsec[g] = make_uint2(__float_as_uint(gsnd), garg);
            gkey[g] = static_cast<uint16_t>(float_to_ordered(gmax) >> 16);
        }
        if (tid == 0) tcount[static_cast<size_t>(qq) * nbk + b] = static_cast<uint32_t>(total);
        __syncthreads();  // the next item finds the cells and masks cleared
        if (next >= nitems) break;
        item = next;
        cur = nxt;
    }
}


// Top R = min(k_refine, C) candidates of one query by (S desc, doc asc).
// Any T at or below the R-th largest group maximum bounds the R-th largest
// S from below (each group maximum is the S of a distinct candidate), so the
// candidates with S >= T (found through the groups with maximum >= T)
// contain the answer; they are collected in LDS and sorted. T is the R-th
// largest group maximum with its low 16 bits cleared (two radix passes over
// the groups' 16-bit keys, a quarter of the bytes of their statistics; the
// bin adds the groups within 2^-7 of it). When C fits the list, all are
// collected. Should the collection exceed the list, two radix passes over
// every candidate give T again (the R-th largest S, low 16 bits cleared) and
// the candidates at or above it are collected instead; only if those exceed
// the list too does an exact radix select over every candidate take over.
// Collection is per wave: a ballot over 64 group maxima; a passing group
// with one candidate at or above T is listed from its statistics, the others
// are queued (in LDS, per wave) and their candidates (contiguous, at most 64
// per group) loaded by the whole wave eight groups at a time when the queue
// fills and at the end of the walk. Two 1,024-thread blocks share a CU (LDS), which
// holds only while the kernel uses at most 80 SGPRs per wave, a limit the
// compiler's occupancy model does not apply; amdgpu_num_sgpr keeps it.
template <int kBlog>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_num_sgpr(80))) void select_refine_kernel(
    const uint32_t* __restrict__ vcnt, const uint32_t* __restrict__ tcount, const float2* __restrict__ gstat,
    const uint2* __restrict__ gsec, const uint16_t* __restrict__ gkey, const uint2* __restrict__ rec, int64_t vcap,
    int nbk, int bshift, int q_base, int qs, int k_refine, int list_cap,
    int32_t* __restrict__ ccount, int32_t* __restrict__ rcount, int32_t* __restrict__ rids,
    float* __restrict__ rscore) {
    constexpr int kGpb = groups_per_bucket(kBlog);
    extern __shared__ uint64_t list[];  // [list_cap]
    __shared__ __align__(16) int hist[256];
    __shared__ int scratch[17];
    __shared__ uint32_t s_prefix;
    __shared__ int s_remaining;
    __shared__ int s_n;
    constexpr int kQueue = 64;                  // queued groups per wave
    __shared__ uint2 mqueue[1024 / kWave][kQueue];  // {record offset, count}
    const int qq = blockIdx.x;
    if (qq >= qs) return;
    const int q = q_base + qq;
    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int nwaves = static_cast<int>(blockDim.x) / kWave;
    const uint32_t* tq = tcount + static_cast<size_t>(qq) * nbk;
    const uint32_t* offq = vcnt + (static_cast<size_t>(qq) * nbk << bshift);
    const uint2* rq = rec + static_cast<size_t>(qq) * vcap;
    const float2* gq = gstat + static_cast<size_t>(qq) * nbk * kGpb;
    const uint2* sq = gsec + static_cast<size_t>(qq) * nbk * kGpb;
    int part = 0;
    for (int bb = threadIdx.x; bb < nbk; bb += blockDim.x) part += static_cast<int>(tq[bb]);
    int C;
    (void)block_inclusive_scan_shared(part, scratch, &C);
    const int R = C < k_refine ? C : k_refine;
    if (threadIdx.x == 0) {
        ccount[qq] = C;
        rcount[q] = R;
        s_n = 0;
    }
    if (R == 0) return;
    const bool take_all = C <= list_cap;
    uint32_t T = 0u;
    if (!take_all) {
        const int64_t G = static_cast<int64_t>(nbk) * kGpb;
        const uint16_t* kq = gkey + static_cast<size_t>(qq) * nbk * kGpb;
        T = block_radix_select<true, 2>([&](int64_t g) { return static_cast<uint32_t>(kq[g]) << 16; }, G, R, hist,
                                        &s_prefix, &s_remaining, nullptr);
        // the wave's queued groups, eight at a time: a missing one reads
        // record 0 with count 0, so every load is in bounds and unconditional
        uint2* myq = mqueue[wave];
        int qn = 0;
        auto flush = [&]() {
            wave_lds_sync();
            for (int q0 = 0; q0 < qn; q0 += 8) {
                constexpr int kGroups = 8;
                uint32_t gb[kGroups], gc[kGroups];
#pragma unroll
                for (int u = 0; u < kGroups; ++u) {
                    const uint2 e = q0 + u < qn ? myq[q0 + u] : make_uint2(0u, 0u);
                    gb[u] = e.x;
                    gc[u] = e.y;
                }
                uint2 e[kGroups];
#pragma unroll
                for (int u = 0; u < kGroups; ++u) {
                    const uint32_t j = static_cast<uint32_t>(lane) < gc[u] ? static_cast<uint32_t>(lane) : 0u;
                    e[u] = rq[static_cast<size_t>(gb[u]) + j];
                }
                // the round's places with one LDS atomic for its groups
                uint64_t bal[kGroups];
                int tot = 0;
#pragma unroll
                for (int u = 0; u < kGroups; ++u) {
                    const uint32_t key = float_to_ordered(__uint_as_float(e[u].y));
                    bal[u] = __ballot(static_cast<uint32_t>(lane) < gc[u] && key >= T);
                    tot += __popcll(bal[u]);
                }
                int off = 0;
                if (lane == 0 && tot > 0) off = atomicAdd(&s_n, tot);
                off = __builtin_amdgcn_readlane(off, 0);
#pragma unroll
                for (int u = 0; u < kGroups; ++u) {
                    const int slot = off + lanes_below(bal[u]);
                    if (((bal[u] >> lane) & 1ull) && slot < list_cap)
                        list[slot] = (static_cast<uint64_t>(~float_to_ordered(__uint_as_float(e[u].y))) << 32) |
                                     e[u].x;
                    off += __popcll(bal[u]);
                }
            }
            qn = 0;
            wave_lds_sync();
        };
        // kBatches batches of 64 groups per step of a wave: the groups'
        // {max S, offset | count << 16} and their buckets' record offsets
        // are all loaded before any is tested (most batches have no passing
        // group, so a step costs about one round trip)
        constexpr int kBatches = 4;
        const int64_t step = static_cast<int64_t>(nwaves) * kWave;
        for (int64_t gs = static_cast<int64_t>(wave) * kWave; gs < G; gs += kBatches * step) {
            uint64_t stv[kBatches];
            uint2 secv[kBatches];
            uint32_t boffv[kBatches];
#pragma unroll
            for (int i = 0; i < kBatches; ++i) {
                const int64_t gi = gs + i * step + lane;
                const int64_t g = gi < G ? gi : int64_t{0};
                stv[i] = reinterpret_cast<const uint64_t*>(gq)[g];
                secv[i] = sq[g];
                boffv[i] = offq[static_cast<size_t>(g / kGpb) << bshift];
            }
#pragma unroll
            for (int i = 0; i < kBatches; ++i) asm volatile("" : : "v"(stv[i]), "v"(secv[i].x), "v"(boffv[i]));
#pragma unroll
            for (int i = 0; i < kBatches; ++i) {
                const int64_t g0 = gs + i * step;
                if (g0 >= G) break;
                const uint64_t st = stv[i];
                const uint32_t packed = static_cast<uint32_t>(st >> 32);
                const bool pass = g0 + lane < G && float_to_ordered(__uint_as_float(static_cast<uint32_t>(st))) >= T;
                const uint32_t cnt = pass ? packed >> 16 : 0u;
                // a passing group whose second-largest S is below T holds
                // exactly one candidate at or above T, its maximum: listed
                // from the statistics, without reading its records
                const bool one = cnt != 0u && float_to_ordered(__uint_as_float(secv[i].x)) < T;
                {
                    const int slot = wave_append_slot(&s_n, one);
                    if (one && slot < list_cap)
                        list[slot] = (static_cast<uint64_t>(~float_to_ordered(__uint_as_float(static_cast<uint32_t>(st))))
                                      << 32) |
                                     secv[i].y;
                }
                const uint32_t base = boffv[i] + (packed & 0xFFFFu);
                const bool multi = cnt != 0u && !one;
                const uint64_t mm = __ballot(multi);
                if (mm != 0ull) {
                    const int k = __popcll(mm);
                    if (qn + k > kQueue) flush();
                    if (multi) myq[qn + lanes_below(mm)] = make_uint2(base, cnt);
                    qn += k;
                }
            }
        }
        if (qn > 0) flush();
    } else {
        // every candidate: one bucket per wave, its candidates contiguous
        for (int bb = wave; bb < nbk; bb += nwaves) {
            const int n = static_cast<int>(tq[bb]);
            const size_t base = offq[static_cast<size_t>(bb) << bshift];
            for (int j0 = 0; j0 < n; j0 += kWave) {
                const int j = j0 + lane;
                const uint2 e = rq[base + static_cast<size_t>(j < n ? j : j0)];
                const int slot = wave_append_slot(&s_n, j < n);
                if (j < n) list[slot] = (static_cast<uint64_t>(~float_to_ordered(__uint_as_float(e.y))) << 32) | e.x;
            }
        }
    }
    __syncthreads();
    int n = s_n;
    if (n > list_cap) {
        // too many for the list (few groups, or dense maxima): T from two
        // radix passes over every candidate (the R-th largest S with its low
        // 16 bits cleared, one bucket per wave), then the candidates at or
        // above it, which contain the answer and usually fit
        uint32_t prefix = 0, pmask = 0;
        int remaining = R;
        for (int shift = 24; shift >= 16; shift -= 8) {
            for (int t = threadIdx.x; t < 256; t += blockDim.x) hist[t] = 0;
            __syncthreads();
            for (int bb = wave; bb < nbk; bb += nwaves) {
                const int cntb = static_cast<int>(tq[bb]);
                const size_t base = offq[static_cast<size_t>(bb) << bshift];
                for (int j0 = 0; j0 < cntb; j0 += kWave) {
                    const int j = j0 + lane;
                    const uint32_t key = float_to_ordered(__uint_as_float(rq[base + (j < cntb ? j : j0)].y));
                    wave_hist_add(hist, j < cntb && (key & pmask) == prefix, (key >> shift) & 255u);
                }
            }
            __syncthreads();
            radix_pick_bin<true>(hist, prefix, shift, remaining, &s_prefix, &s_remaining);
            __syncthreads();
            prefix = s_prefix;
            remaining = s_remaining;
            pmask |= 255u << shift;
            __syncthreads();
        }
        if (threadIdx.x == 0) s_n = 0;
        __syncthreads();
        for (int bb = wave; bb < nbk; bb += nwaves) {
            const int cntb = static_cast<int>(tq[bb]);
            const size_t base = offq[static_cast<size_t>(bb) << bshift];
            for (int j0 = 0; j0 < cntb; j0 += kWave) {
                const int j = j0 + lane;
                const uint2 e = rq[base + (j < cntb ? j : j0)];
                const uint32_t key = float_to_ordered(__uint_as_float(e.y));
                const bool sel = j < cntb && key >= prefix;
                const int slot = wave_append_slot(&s_n, sel);
                if (sel && slot < list_cap) list[slot] = (static_cast<uint64_t>(~key) << 32) | e.x;
            }
        }
        __syncthreads();
        n = s_n;
    }
    if (n > list_cap) {
        // exact path: R-th largest S over every candidate, all keys above it,
        // and the first ties in ascending doc order
        int need;
        uint32_t Tx;
        // walk buckets directly for the histogram passes
        uint32_t prefix = 0, pmask = 0;
        int remaining = R;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int t = threadIdx.x; t < 256; t += blockDim.x) hist[t] = 0;
            __syncthreads();
            for (int bb = 0; bb < nbk; ++bb) {
                const int cnt = static_cast<int>(tq[bb]);
                const int64_t base = offq[static_cast<size_t>(bb) << bshift];
                for (int j = threadIdx.x; j < cnt; j += blockDim.x) {
                    const uint32_t key = float_to_ordered(__uint_as_float(rq[base + j].y));
                    if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
                }
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                int cum = 0, sel = 0;
                for (int h = 255; h >= 0; --h) {
                    if (cum + hist[h] >= remaining) {
                        sel = h;
                        break;
                    }
                    cum += hist[h];
                }
                s_prefix = prefix | (static_cast<uint32_t>(sel) << shift);
                s_remaining = remaining - cum;
            }
            __syncthreads();
            prefix = s_prefix;
            remaining = s_remaining;
            pmask |= 255u << shift;
            __syncthreads();
        }
        Tx = prefix;
        need = remaining;
        int tie_carry = 0, out_carry = 0;
        for (int bb = 0; bb < nbk; ++bb) {
            const int cnt = static_cast<int>(tq[bb]);
            const int64_t base = offq[static_cast<size_t>(bb) << bshift];
            for (int j0 = 0; j0 < cnt; j0 += blockDim.x) {
                const int j = j0 + static_cast<int>(threadIdx.x);
                uint2 e = make_uint2(0u, 0u);
                uint32_t key = 0u;
                if (j < cnt) {
                    e = rq[base + j];
                    key = float_to_ordered(__uint_as_float(e.y));
                }
                const int is_eq = (j < cnt && key == Tx) ? 1 : 0;
                int tot;
                const int tie_incl = block_inclusive_scan_shared(is_eq, scratch, &tot);
                const int tie_rank = tie_carry + tie_incl - is_eq;
                tie_carry += tot;
                const int sel = (j < cnt && (key > Tx || (is_eq && tie_rank < need))) ? 1 : 0;
                const int pos_incl = block_inclusive_scan_shared(sel, scratch, &tot);
                const int pos = out_carry + pos_incl - sel;
                out_carry += tot;
                if (sel && pos < list_cap) list[pos] = (static_cast<uint64_t>(~key) << 32) | e.x;
            }
        }
        n = R;
    }
    // at least one key per thread (the list holds at least 4,096)
    const int sort_n = max(pow2_at_least_dev(n < 2 ? 2 : n), static_cast<int>(blockDim.x));
    for (int t = n + threadIdx.x; t < sort_n; t += blockDim.x) list[t] = ~0ull;
    __syncthreads();
    block_sort_u64(list, sort_n);
    for (int t = threadIdx.x; t < R; t += blockDim.x) {
        const uint64_t v = list[t];
        rids[static_cast<size_t>(q) * k_refine + t] = static_cast<int32_t>(v & 0xFFFFFFFFu);
        if (rscore) rscore[static_cast<size_t>(q) * k_refine + t] = ordered_to_float(~static_cast<uint32_t>(v >> 32));
    }
}

// Dense candidate list of each query (ascending doc IDs and S_cand) for
// traces: at most cap entries per query.
__global__ __launch_bounds__(256) void cand_compact_kernel(const uint32_t* __restrict__ vcnt,
                                                           const uint32_t* __restrict__ tcount,
                                                           const uint2* __restrict__ rec, int64_t vcap, int nbk,
                                                           int bstride, int qs, int64_t cap,
                                                           int32_t* __restrict__ cand, float* __restrict__ score) {
    const int qq = blockIdx.x;
    if (qq >= qs) return;
    const uint32_t* tq = tcount + static_cast<size_t>(qq) * nbk;
    const uint32_t* offq = vcnt + static_cast<size_t>(qq) * nbk * bstride;
    const uint2* rq = rec + static_cast<size_t>(qq) * vcap;
    int64_t k = 0;
    for (int bb = 0; bb < nbk && k < cap; ++bb) {
        const int64_t cnt = tq[bb];
        const int64_t base = offq[static_cast<size_t>(bb) * bstride];
        for (int64_t j = threadIdx.x; j < cnt && k + j < cap; j += blockDim.x) {
            const uint2 e = rq[base + j];
            cand[static_cast<size_t>(qq) * cap + k + j] = static_cast<int32_t>(e.x);
            score[static_cast<size_t>(qq) * cap + k + j] = __uint_as_float(e.y);
        }
        k += cnt;
    }
}

// ---- launchers ----

int cand_buckets(int64_t num_docs, int blog) {
    return static_cast<int>((num_docs + (int64_t{1} << blog) - 1) >> blog);
}

// Documents per bucket = 2^blog: the largest in [kMinBucketLog2,
// kMaxBucketLog2] whose expected records per item (rho per document, rho =
// 32 nprobe N / (K M) for a uniform probe) fit 8 per reduce thread, then
// raised until the staged emit's per-bucket LDS counters suffice. Such
// items mostly fit one slot chunk and take the reduce's one-chunk path;
// items raised past 8 records per thread take the 12-record reduce
// (kReduceHeldMax). At 1M documents (rho 0.69) 4,096-document buckets beat
// 8,192 with 12 records per thread: the reduce is 1.0 ms faster, the visit
// records 0.64 ms slower (more, shorter bucket runs).
CandShape cand_shape(int64_t num_docs, int64_t n_tokens, int64_t n_clusters, int nprobe) {
    const double rho = static_cast<double>(kQ) * nprobe * static_cast<double>(n_tokens) /
                       (static_cast<double>(std::max<int64_t>(1, n_clusters)) *
                        static_cast<double>(std::max<int64_t>(1, num_docs)));
    int blog = kMaxBucketLog2;
    while (blog > kMinBucketLog2 && rho * static_cast<double>(int64_t{1} << blog) > 8.0 * kReduceThreads)
        --blog;
    while (blog < kMaxBucketLog2 && cand_buckets(num_docs, blog) > kStagedMaxBuckets) ++blog;
    const int held = rho * static_cast<double>(int64_t{1} << blog) <= 8.0 * kReduceThreads ? 8 : kReduceHeldMax;
    return {blog, held};
}

int select_list_cap(int k_refine) {
    const int want = pow2_at_least(2 * (k_refine < 2048 ? 2048 : k_refine));
    return want < 16384 ? want : 16384;
}

// The select kernel of a bucket size 2^blog, blog in [kMinBucketLog2, kMaxBucketLog2].
static const void* select_refine_fn(int blog) {
    switch (blog) {
        case 8: return reinterpret_cast<const void*>(select_refine_kernel<8>);
        case 9: return reinterpret_cast<const void*>(select_refine_kernel<9>);
        case 10: return reinterpret_cast<const void*>(select_refine_kernel<10>);
        case 11: return reinterpret_cast<const void*>(select_refine_kernel<11>);
        case 12: return reinterpret_cast<const void*>(select_refine_kernel<12>);
        default: return reinterpret_cast<const void*>(select_refine_kernel<13>);
    }
}
static_assert(kMinBucketLog2 == 8 && kMaxBucketLog2 == 13, "one select kernel per bucket size");

hipError_t configure_candidate_kernels(int nbk, int k_refine) {
    hipError_t e = hipSuccess;
    if (nbk * 4 > 60 * 1024) {
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(cand_count_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, nbk * 4);
        if (e != hipSuccess) return e;
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(cand_emit_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, nbk * 4);
        if (e != hipSuccess) return e;
    }
    const int sel_shm = select_list_cap(k_refine) * 8;
    if (sel_shm > 60 * 1024) {
        for (int blog = kMinBucketLog2; blog <= kMaxBucketLog2 && e == hipSuccess; ++blog)
            e = hipFuncSetAttribute(select_refine_fn(blog), hipFuncAttributeMaxDynamicSharedMemorySize, sel_shm);
    }
    return e;
}

// Visit ranges per (query, token) in the count and emit kernels of a
// sub-batch of qs queries: doubled, up to kMaxParts, while their grids stay
// within two blocks per CU and the visit counts of qs x parts queries fit
// the candidate state (which holds wqs queries). One query at docs2m takes
// 16 parts: 512 blocks instead of 32 on one XCD.
constexpr int kMaxParts = 16;
int cand_parts(int qs, int num_cus, int wqs) {
    int p = 1;
    while (p < kMaxParts && static_cast<int64_t>(qs) * kQ * p <= num_cus && static_cast<int64_t>(qs) * p * 2 <= wqs)
        p *= 2;
    return p;
}

// Segments per query of the visit-count scan: one block per query while the
// sub-batch fills a quarter of the CUs, else up to 64 segments of at least
// 256 uint4 each, so that the sub-batch takes about one block per CU (their
// sums sit in the first words of each query's record area).
static int offsets_segments(int qs, int num_cus, int n4, int64_t vcap) {
    if (static_cast<int64_t>(qs) * 4 > num_cus) return 1;
    int nseg = std::min(64, num_cus / std::max(qs, 1));
    nseg = std::min<int64_t>(nseg, std::min<int64_t>(n4 / 256, 2 * vcap));
    return nseg >= 4 ? nseg : 1;
}

static int cand_grid(int qs, int parts) { return (qs >= 8 ? (qs + 7) / 8 * 8 : qs) * kQ * parts; }

static int log2_of(int p) {
    int l = 0;
    while ((1 << l) < p) ++l;
    return l;
}

template <int kBlog>
static void launch_select(hipStream_t s, const CandidateArgs& a, int bshift, int q_base, int qs, int cap) {
    hipLaunchKernelGGL(select_refine_kernel<kBlog>, dim3(qs), dim3(1024), static_cast<size_t>(cap) * 8, s, a.vcnt,
                       a.tcount, a.gstat, a.gsec, a.gkey, a.rec, a.vcap, a.nbk, bshift, q_base, qs, a.k_refine, cap,
                       a.ccount, a.rcount, a.rids, a.rscore);
}

hipError_t launch_candidates(hipStream_t s, const CandidateArgs& a, int q_base, int qs, int phase) {
    hipError_t e = hipSuccess;
    const size_t shm = static_cast<size_t>(a.nbk) * 4;
    // every phase of a sub-batch derives the same parts from (qs, CUs, wqs)
    const int parts = cand_parts(qs, a.num_cus, a.wqs);
    const int bshift = log2_of(kQ * parts);  // visit counts per bucket: 1 << bshift
    const int grid = cand_grid(qs, parts);
    switch (phase) {
        case 0:
            hipLaunchKernelGGL(cand_count_kernel, dim3(grid), dim3(256), shm, s, a.labels, q_base, qs, a.nprobe,
                               a.cluster_pos, a.doc_clu, a.n_clusters, a.num_docs, a.blog, a.nbk, parts, a.vcnt);
            break;
        case 1: {
            const int nseg = offsets_segments(qs, a.num_cus, a.nbk * kQ * parts / 4, a.vcap);
            if (nseg > 1) {
                hipLaunchKernelGGL(cand_offsets_part_kernel, dim3(nseg, qs), dim3(256), 0, s, a.vcnt, a.nbk, parts,
                                   nseg, a.rec, a.vcap);
                hipLaunchKernelGGL(cand_offsets_seg_kernel, dim3(nseg, qs), dim3(256), 0, s, a.vcnt, a.nbk, parts,
                                   nseg, a.rec, a.vcap, a.vtot, a.err);
            } else {
                hipLaunchKernelGGL(cand_offsets_kernel, dim3(qs), dim3(1024), 0, s, a.vcnt, a.nbk, parts, qs, a.vcap,
                                   a.vtot, a.err);
            }
        } break;
        case 2:
            if (a.nbk <= kStagedMaxBuckets) {
                const size_t dshm = (static_cast<size_t>(2 * a.nbk) + 2 * a.nprobe + 1) * 4;
                hipLaunchKernelGGL(cand_emit_staged_kernel, dim3(grid), dim3(256), dshm, s, a.labels, q_base, qs,
                                   a.nprobe, a.cluster_pos, a.codes_clu, a.f1_clu, a.doc_clu, a.n_clusters, a.num_docs,
                                   a.lut, a.cb1, a.blog, a.nbk, parts, a.vcnt, a.rec, a.vcap);
                break;
            }
            hipLaunchKernelGGL(cand_emit_kernel, dim3(grid), dim3(256), shm, s, a.labels, q_base, qs, a.nprobe,
                               a.cluster_pos, a.codes_clu, a.f1_clu, a.doc_clu, a.n_clusters, a.num_docs, a.lut, a.cb1,
                               a.blog, a.nbk, parts, a.vcnt, a.rec, a.vcap);
            break;
        case 3:
        {
            // two resident blocks per CU (LDS), each walking its items
            const int64_t items = static_cast<int64_t>(a.nbk) * qs;
            const int rgrid = static_cast<int>(std::min<int64_t>(items, int64_t{2} * std::max(a.num_cus, 1)));
            static_assert(kDenseDocs == 1 << kMinBucketLog2, "the dense reduce takes the smallest buckets");
            if (a.blog == kMinBucketLog2) {
                const int dgrid = static_cast<int>(std::min<int64_t>(items, int64_t{2} * std::max(a.num_cus, 1)));
                if (a.held <= 8)
                    hipLaunchKernelGGL(cand_reduce_dense_kernel<8>, dim3(dgrid), dim3(kReduceThreads), 0, s, a.vcnt,
                                       a.vtot, a.nbk, bshift, qs, a.rec, a.vcap, a.tcount, a.gstat, a.gsec, a.gkey);
                else
                    hipLaunchKernelGGL(cand_reduce_dense_kernel<kReduceHeldMax>, dim3(dgrid), dim3(kReduceThreads), 0,
                                       s, a.vcnt, a.vtot, a.nbk, bshift, qs, a.rec, a.vcap, a.tcount, a.gstat,
                                       a.gsec, a.gkey);
            } else if (a.held <= 8)
                hipLaunchKernelGGL(cand_reduce_kernel<8>, dim3(rgrid), dim3(kReduceThreads), 0, s, a.vcnt, a.vtot,
                                   a.blog, a.nbk, bshift, qs, a.num_docs, a.rec, a.vcap, a.tcount, a.gstat, a.gsec,
                                   a.gkey);
            else
                hipLaunchKernelGGL(cand_reduce_kernel<kReduceHeldMax>, dim3(rgrid), dim3(kReduceThreads), 0, s, a.vcnt,
                                   a.vtot, a.blog, a.nbk, bshift, qs, a.num_docs, a.rec, a.vcap, a.tcount, a.gstat,
                                   a.gsec, a.gkey);
        }
            break;
        case 4: {
            const int cap = select_list_cap(a.k_refine);
            switch (a.blog) {
                case 8: launch_select<8>(s, a, bshift, q_base, qs, cap); break;
                case 9: launch_select<9>(s, a, bshift, q_base, qs, cap); break;
                case 10: launch_select<10>(s, a, bshift, q_base, qs, cap); break;
                case 11: launch_select<11>(s, a, bshift, q_base, qs, cap); break;
                case 12: launch_select<12>(s, a, bshift, q_base, qs, cap); break;
                case 13: launch_select<13>(s, a, bshift, q_base, qs, cap); break;
                default: return hipErrorInvalidValue;
            }
            break;
        }
        default:
            return hipErrorInvalidValue;
    }
    e = hipGetLastError();
    return e;
}

hipError_t launch_cand_compact(hipStream_t s, const CandidateArgs& a, int qs, int64_t cap, int32_t* cand,
                               float* score) {
    const int bstride = kQ * cand_parts(qs, a.num_cus, a.wqs);
    hipLaunchKernelGGL(cand_compact_kernel, dim3(qs), dim3(256), 0, s, a.vcnt, a.tcount, a.rec, a.vcap, a.nbk, bstride,
                       qs, cap, cand, score);
    return hipGetLastError();
}

int pow2_at_least(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

}  // namespace chimera
