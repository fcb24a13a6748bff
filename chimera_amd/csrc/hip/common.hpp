// Shared constants and wave64 helpers for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace chimera {

constexpr int kDim = 128;        // PADDED_DIM (config.cuh:7)
constexpr int kQ = 32;           // Q_DOCLEN (config.cuh:8)
constexpr int kChunks = 32;      // 4-bit chunks of a 128-bit code (config.cuh:17-18)
constexpr int kLut = 16;         // entries per chunk
constexpr int kLutPerQuery = kQ * kChunks * kLut;  // 16384 floats = 64 KB
constexpr int kWave = 64;
constexpr int kCodeBytes = 16;   // one-bit code bytes
// candidate stage: documents per bucket, 2^blog with blog chosen per index
// in [kMinBucketLog2, kMaxBucketLog2] (LDS is sized for the largest)
constexpr int kMaxBucketLog2 = 13;
constexpr int kMinBucketLog2 = 8;
constexpr int kMaxBucketDocs = 1 << kMaxBucketLog2;
// 64-document groups per bucket of 2^blog documents
__host__ __device__ constexpr int groups_per_bucket(int blog) { return 1 << (blog - 6); }

// Float <-> totally ordered unsigned key (ascending key == ascending float).
__device__ __forceinline__ uint32_t float_to_ordered(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ordered_to_float(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(u);
}

__device__ __forceinline__ int pow2_at_least_dev(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// Set bits of a wave mask below this lane (a lane's rank among the set lanes).
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// Slot of this lane in an LDS list for the lanes with `sel`, taken with one
// atomic per wave on *counter (slots in lane order). Called by the whole wave.
__device__ __forceinline__ int wave_append_slot(int* counter, bool sel) {
    const uint64_t m = __ballot(sel);
    if (m == 0ull) return 0;
    int base = 0;
    if ((threadIdx.x & (kWave - 1)) == 0) base = atomicAdd(counter, __popcll(m));
    return __builtin_amdgcn_readlane(base, 0) + lanes_below(m);  // lane 0's value, no LDS round trip
}

// max(v of lane l, v of lane l ^ 16) and max(v of lane l, v of lane l ^ 32)
// through the gfx950 lane-swap instructions (VALU, no LDS traffic): the swap
// returns the lane's own value and its partner's, in some order.
__device__ __forceinline__ float wave_max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// v + (v of lane l + kOff) inside the lane's row of 16 lanes (a DPP row
// shift; lanes whose partner lies past the row add 0): one step of a
// shuffle-down sum tree over 16 lanes.
template <int kOff>
__device__ __forceinline__ float row_add_down(float v) {
    static_assert(kOff >= 1 && kOff <= 15, "row shift");
    const int o = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x100 + kOff, 0xF, 0xF, true);
    return v + __int_as_float(o);
}

// Orders LDS traffic between the lanes of one wave (no block barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
__device__ __forceinline__ int wave_id() { return static_cast<int>(threadIdx.x) / kWave; }

// Nibble c of a 128-bit code held as four little-endian 32-bit words
// (kernels.cu:361-373: word c/8, shift 4*(c%8)).
__device__ __forceinline__ int code_nibble(const uint4& w, int c) {
    const uint32_t word = (c < 8) ? w.x : (c < 16) ? w.y : (c < 24) ? w.z : w.w;
    return static_cast<int>((word >> (4 * (c & 7))) & 0xFu);
}

// Error bits reported through the context's device flag word.
enum : uint32_t {
    kErrCandOverflow = 1u << 1,    // more candidate documents than the bound
    kErrRefineCap = 1u << 2,       // refined selection exceeded its capacity
    kErrFullbitCap = 1u << 3,      // full-bit selection exceeded its capacity
};

}  // namespace chimera

namespace chimera {

// Inclusive prefix sum over the 64 lanes of a wave. DPP row shifts by 1, 2,
// 4 and 8 give the sum within each row of 16 lanes (a lane whose source lies
// outside its row adds the `old` operand, 0), then each row adds the totals
// of the rows before it, read from lanes 15, 31 and 47. Every lane of the
// wave must be active.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(v, 15);
    const int r1 = __builtin_amdgcn_readlane(v, 31);
    const int r2 = __builtin_amdgcn_readlane(v, 47);
    const int row = lane_id() >> 4;
    return v + (row == 0 ? 0 : row == 1 ? r0 : row == 2 ? r0 + r1 : r0 + r1 + r2);
}

// Inclusive scan of one int per thread over the block (blockDim a multiple of
// 64, at most 1024): the wave scan above, the wave totals through LDS, and
// each wave adds those of the waves before it. Every thread of the block
// must call it; *total receives the block sum. It ends with a barrier (the
// next call may rewrite scratch).
__device__ inline int block_inclusive_scan_shared(int v, int* scratch /*[17]*/, int* total) {
    const int w = wave_id();
    const int nw = static_cast<int>(blockDim.x) / kWave;
    v = wave_inclusive_scan(v);
    if (lane_id() == kWave - 1) scratch[w] = v;
    __syncthreads();
    int before = 0, sum = 0;
    for (int k = 0; k < nw; ++k) {
        const int t = scratch[k];
        before += k < w ? t : 0;
        sum += t;
    }
    *total = sum;
    __syncthreads();
    return v + before;
}

// Two inclusive scans over the block at the cost of one (the same waves,
// one barrier for both sets of wave totals): a and b become their inclusive
// prefixes, *ta and *tb the block sums. scratch holds 32 ints. Every thread
// of the block must call it; it ends with a barrier (kClose) that lets the
// next call rewrite scratch, which a caller with other barriers in between
// may leave out.
template <bool kClose = true>
__device__ inline void block_inclusive_scan2(int& a, int& b, int* scratch /*[32]*/, int* ta, int* tb) {
    const int w = wave_id();
    const int nw = static_cast<int>(blockDim.x) / kWave;
    a = wave_inclusive_scan(a);
    b = wave_inclusive_scan(b);
    if (lane_id() == kWave - 1) {
        scratch[w] = a;
        scratch[16 + w] = b;
    }
    __syncthreads();
    int pa = 0, pb = 0, sa = 0, sb = 0;
    for (int k = 0; k < nw; ++k) {
        const int x = scratch[k], y = scratch[16 + k];
        pa += k < w ? x : 0;
        pb += k < w ? y : 0;
        sa += x;
        sb += y;
    }
    *ta = sa;
    *tb = sb;
    if (kClose) __syncthreads();
    a += pa;
    b += pb;
}

// Bitonic sort of keys[0, n) ascending (n a power of two) by the whole block.
__device__ inline void block_bitonic_sort_u64(uint64_t* keys, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < n / 2; t += blockDim.x) {
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
}

// The value of lane (lane ^ M) of the wave, M a power of two below 64: DPP
// quad permutations for 1 and 2, a bitmask swizzle (within 32 lanes, no LDS
// access) for 4, 8 and 16, a bpermute for 32.
template <int M>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    static_assert(M >= 1 && M < kWave && (M & (M - 1)) == 0, "a lane bit");
    const int x = static_cast<int>(v);
    if constexpr (M == 1) return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
    else if constexpr (M == 2) return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
    else if constexpr (M < 32) return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(x, (M << 10) | 0x1F));
    else return static_cast<uint32_t>(__shfl_xor(x, M, kWave));
}

// The bitonic stages of strides S, S / 2, ..., 1 that lie below `size` (the
// length of the sequences being merged), for keys K t .. K t + K - 1 of thread
// t: partners in one thread compare in registers, partners in one wave
// (stride S >= K) exchange through lane t ^ S / K. Compile-time strides, so
// each exchange is one instruction of the right kind.
template <int K, int S>
__device__ __forceinline__ void bitonic_wave_stages(uint64_t (&r)[K], int t, int size) {
    if (S < size) {
        if constexpr (S < K) {
#pragma unroll
            for (int j = 0; j < K; ++j) {
                if ((j & S) != 0) continue;
                const bool asc = ((K * t + j) & size) == 0;
                const uint64_t x = r[j], y = r[j | S];
                if ((x > y) == asc) {
                    r[j] = y;
                    r[j | S] = x;
                }
            }
        } else {
            constexpr int m = S / K;
            const bool keep_min = ((t & m) == 0) == ((t & (size / K)) == 0);
#pragma unroll
            for (int j = 0; j < K; ++j) {
                const uint32_t lo = lane_xor<m>(static_cast<uint32_t>(r[j]));
                const uint32_t hi = lane_xor<m>(static_cast<uint32_t>(r[j] >> 32));
                const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
                r[j] = keep_min == (o < r[j]) ? o : r[j];
            }
        }
    }
    if constexpr (S > 1) bitonic_wave_stages<K, S / 2>(r, t, size);
}

// Ascending bitonic sort of n = K * (threads of the group) keys, thread t of
// the group holding keys [K t, K t + K) in r on entry and on exit. Strides of
// at least K * 64 (partners in other waves) go through lds (n keys) with a
// barrier (kBlock: the group is the block; otherwise it is one wave and such
// strides do not occur); the smaller ones stay in registers and lane
// exchanges (bitonic_wave_stages). Every thread of the group calls it.
template <int K, bool kBlock>
__device__ __forceinline__ void sort_keys_regs(uint64_t (&r)[K], uint64_t* lds, int n, int t) {
    static_assert((K & (K - 1)) == 0, "K a power of two");
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size / 2; stride >= K * kWave; stride >>= 1) {
#pragma unroll
            for (int j = 0; j < K; ++j) lds[K * t + j] = r[j];
            if (kBlock) __syncthreads(); else wave_lds_sync();
            const bool keep_min = (((K * t) & stride) == 0) == (((K * t) & size) == 0);
            uint64_t o[K];
#pragma unroll
            for (int j = 0; j < K; ++j) o[j] = lds[(K * t + j) ^ stride];
#pragma unroll
            for (int j = 0; j < K; ++j) r[j] = keep_min == (o[j] < r[j]) ? o[j] : r[j];
            if (kBlock) __syncthreads(); else wave_lds_sync();
        }
        bitonic_wave_stages<K, K * kWave / 2>(r, t, size);
    }
}

// One merge level of block_merge_sort_keys. Lane l of wave w holds the keys
// at sorted positions 64 K w + 64 j + l (j < K; all in one run of length L,
// as a wave's K * 64 keys are), so for each j the wave's 64 searches cover
// neighbouring keys and their deep steps read neighbouring LDS words (no
// bank conflicts; with K consecutive keys per lane they lay K words apart).
// Each key moves to its index in its run plus its rank in the partner run:
// the keys below it when in the first run of the pair, at or below it when
// in the second, so equal keys keep their order and each place is taken
// once. The searches (log2 L + 1 LDS reads each, branch-free) advance four at
// a time, so four reads are in flight per step. Ends with a barrier.
template <int K, int L>
__device__ __forceinline__ void merge_level(uint64_t* keys, const uint64_t (&r)[K], int t) {
    const int lane = t & (kWave - 1);
    const int p0 = K * (t - lane) + lane;  // position of key j: p0 + 64 j
    const int run = p0 / L;
    const int base = (run & ~1) * L;
    const bool second = (run & 1) != 0;
    const uint64_t* other = keys + base + (second ? 0 : L);
    // at most four searches at a time: the 1,024-thread kernels stay within
    // the 64 VGPRs of two blocks per CU
    constexpr int kG = K < 4 ? K : 4;
    int c[K];
#pragma unroll
    for (int j0 = 0; j0 < K; j0 += kG) {
#pragma unroll
        for (int j = j0; j < j0 + kG; ++j) c[j] = 0;
#pragma unroll
        for (int step = L / 2; step >= 1; step >>= 1) {
            uint64_t e[kG];
#pragma unroll
            for (int j = 0; j < kG; ++j) e[j] = other[c[j0 + j] + step - 1];
#pragma unroll
            for (int j = 0; j < kG; ++j) c[j0 + j] += (e[j] < r[j0 + j] || (second && e[j] == r[j0 + j])) ? step : 0;
        }
        uint64_t e[kG];
#pragma unroll
        for (int j = 0; j < kG; ++j) e[j] = other[c[j0 + j]];
#pragma unroll
        for (int j = 0; j < kG; ++j) c[j0 + j] += (e[j] < r[j0 + j] || (second && e[j] == r[j0 + j])) ? 1 : 0;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < K; ++j) keys[base + p0 + kWave * j - run * L + c[j]] = r[j];
    __syncthreads();
}

// Ascending merge sort of keys[0, n) in LDS by a 1,024-thread block, n = K *
// 1,024: each wave sorts its K * 64 keys in registers (sort_keys_regs, lane
// exchanges only, K consecutive keys per lane), then four merge levels (runs
// of 64 K to 512 K keys, each length a compile-time constant) place every key
// by binary search in the partner run, with lane l of a wave taking every
// 64th of its keys. A level costs log2 L + 1 LDS reads per key and two
// barriers, against the bitonic network's 8-byte reads and writes of every
// key in each of its log2(n) (log2(n) + 1) / 2 stages. Ends with a barrier.
template <int K>
__device__ __forceinline__ void block_merge_sort_keys(uint64_t* keys) {
    const int t = static_cast<int>(threadIdx.x);
    const int lane = t & (kWave - 1);
    uint64_t r[K];
#pragma unroll
    for (int j = 0; j < K; ++j) r[j] = keys[K * t + j];
    // the wave's K * 64 keys: strides below K * 64 only, so no LDS stage
    sort_keys_regs<K, false>(r, keys, K * kWave, lane);
#pragma unroll
    for (int j = 0; j < K; ++j) keys[K * t + j] = r[j];
    __syncthreads();
    const int p0 = K * (t - lane) + lane;
    auto reload = [&]() {
#pragma unroll
        for (int j = 0; j < K; ++j) r[j] = keys[p0 + kWave * j];
    };
    reload();
    merge_level<K, K * kWave>(keys, r, t);
    reload();
    merge_level<K, 2 * K * kWave>(keys, r, t);
    reload();
    merge_level<K, 4 * K * kWave>(keys, r, t);
    reload();
    merge_level<K, 8 * K * kWave>(keys, r, t);
}

// Ascending sort of keys[0, n) in LDS by the whole block, n = K * blockDim.x
// (a power of two): each thread loads its K consecutive keys, sorts with
// sort_keys_regs (keys doubling as its exchange area) and stores them back;
// ends with a barrier.
template <int K>
__device__ __forceinline__ void block_sort_keys(uint64_t* keys, int n) {
    const int t = static_cast<int>(threadIdx.x);
    uint64_t r[K];
#pragma unroll
    for (int j = 0; j < K; ++j) r[j] = keys[K * t + j];
    sort_keys_regs<K, true>(r, keys, n, t);
#pragma unroll
    for (int j = 0; j < K; ++j) keys[K * t + j] = r[j];
    __syncthreads();
}

// Ascending sort of keys[0, n) in LDS by the block (n a power of two, keys
// valid and stable before the call; ends with a barrier), for n = 1, 2, 4
// or 8 times blockDim.x: with 1,024 threads (16 waves, four merge levels)
// the merge sort over wave-sorted runs, which measured faster there
// (4,096 keys: the full-bit selection 0.18 -> 0.16 ms per batch at docs2m,
// 0.08 ms with compile-time levels and lane-strided keys); with fewer
// threads the bitonic network in registers and lane exchanges.
// Other n take the LDS bitonic network.
__device__ __forceinline__ void block_sort_u64(uint64_t* keys, int n) {
    const int per = n / static_cast<int>(blockDim.x);
    if (per * static_cast<int>(blockDim.x) == n && blockDim.x % kWave == 0) {
        if (blockDim.x == 1024) {
            switch (per) {
                case 1: block_merge_sort_keys<1>(keys); return;
                case 2: block_merge_sort_keys<2>(keys); return;
                case 4: block_merge_sort_keys<4>(keys); return;
                case 8: block_merge_sort_keys<8>(keys); return;
                default: break;
            }
        } else {
            switch (per) {
                case 1: block_sort_keys<1>(keys, n); return;
                case 2: block_sort_keys<2>(keys, n); return;
                case 4: block_sort_keys<4>(keys, n); return;
                case 8: block_sort_keys<8>(keys, n); return;
                default: break;
            }
        }
    }
    block_bitonic_sort_u64(keys, n);
}

// One histogram add per lane (act: the lane has a key under the prefix),
// combined for the lanes that share the first active lane's digit. Called
// by every lane of the wave.
__device__ __forceinline__ void wave_hist_add(int* hist, bool act, uint32_t digit) {
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const uint64_t live = __ballot(act);
    if (live == 0ull) return;
    const int leader = __ffsll(static_cast<long long>(live)) - 1;
    // the leader's digit through a scalar register (no LDS round trip)
    const uint32_t d0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(digit), leader));
    const uint64_t same = __ballot(act && digit == d0);
    if (lane == leader) atomicAdd(&hist[d0], __popcll(same));
    if (act && digit != d0) atomicAdd(&hist[digit], 1);
}

// After a pass's histogram: wave 0 finds the bin holding position rem in
// scan order and publishes the extended prefix and the remaining count.
template <bool kDescending>
__device__ __forceinline__ void radix_pick_bin(const int* hist, uint32_t prefix, int shift, int rem,
                                               uint32_t* s_prefix, int* s_rem) {
    if (threadIdx.x >= kWave) return;
    const int L = static_cast<int>(threadIdx.x);
    int hv[4];
    if (kDescending) {
        const int4 h = *reinterpret_cast<const int4*>(&hist[252 - 4 * L]);
        hv[0] = h.w;
        hv[1] = h.z;
        hv[2] = h.y;
        hv[3] = h.x;
    } else {
        const int4 h = *reinterpret_cast<const int4*>(&hist[4 * L]);
        hv[0] = h.x;
        hv[1] = h.y;
        hv[2] = h.z;
        hv[3] = h.w;
    }
    const int own = hv[0] + hv[1] + hv[2] + hv[3];
    const int incl = wave_inclusive_scan(own);
    const int excl = incl - own;
    // at least rem keys share the prefix, so exactly one lane holds the
    // digit; the last lane covers an (impossible) short count
    if ((excl < rem && incl >= rem) || (L == kWave - 1 && incl < rem)) {
        int cum = excl, qd = 0;
        while (qd < 3 && cum + hv[qd] < rem) {
            cum += hv[qd];
            ++qd;
        }
        const int bin = kDescending ? 255 - (4 * L + qd) : 4 * L + qd;
        *s_prefix = prefix | (static_cast<uint32_t>(bin) << shift);
        *s_rem = rem - cum;
    }
}

// Radix select over the n keys key_at(0..n-1), 8 bits per pass, most
// significant digit first: the key T holding position `count` (1-based) in
// ascending order (kDescending: descending), and through *need the number
// of keys equal to T that complete the first `count`. With kPasses < 4 only
// the leading 8 kPasses bits are resolved: the result is that key with its
// remaining bits cleared (a lower bound of it) and *need is not meaningful.
// Called by every thread of the block with the same arguments (blockDim.x a
// multiple of the wave size, n > 0); hist is 256 ints of LDS (16-byte
// aligned), s_prefix and s_rem LDS scalars. Each lane reads four keys
// before adding them, so four loads are in flight; key_at is only called
// with indexes below n. Histogram adds are combined per wave for the lanes
// that share the first active lane's digit (most keys share their leading
// digits), and wave 0 finds each pass's digit with a prefix sum over the
// bins (lane L holds four consecutive bins in scan order).
template <bool kDescending, int kPasses = 4, typename KeyAt>
__device__ uint32_t block_radix_select(KeyAt key_at, int64_t n, int count, int* hist, uint32_t* s_prefix,
                                       int* s_rem, int* need) {
    static_assert(kPasses >= 1 && kPasses <= 4, "8-bit digits of a 32-bit key");
    constexpr int kUnroll = 4;
    uint32_t prefix = 0, pmask = 0;
    int rem = count;
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int64_t wave_base = static_cast<int64_t>(threadIdx.x) - lane;
    const int64_t step = blockDim.x;
    for (int shift = 24; shift >= 32 - 8 * kPasses; shift -= 8) {
        for (int t = threadIdx.x; t < 256; t += blockDim.x) hist[t] = 0;
        __syncthreads();
        for (int64_t base = wave_base; base < n; base += kUnroll * step) {
            uint32_t key[kUnroll];
            bool in[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t idx = base + u * step + lane;
                in[u] = idx < n;
                key[u] = key_at(in[u] ? idx : int64_t{0});
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
                wave_hist_add(hist, in[u] && (key[u] & pmask) == prefix, (key[u] >> shift) & 255u);
        }
        __syncthreads();
        radix_pick_bin<kDescending>(hist, prefix, shift, rem, s_prefix, s_rem);
        __syncthreads();
        prefix = *s_prefix;
        rem = *s_rem;
        pmask |= 255u << shift;
        __syncthreads();
    }
    if (need) *need = rem;
    return prefix;
}

// Key of 0-based rank `rank` (ascending) among the n keys key_at(0..n-1);
// requires rank < n.
template <typename KeyAt>
__device__ uint32_t block_radix_select_u32(KeyAt key_at, int n, int rank, int* hist, uint32_t* s_prefix,
                                           int* s_rem) {
    return block_radix_select<false>(key_at, static_cast<int64_t>(n), rank + 1, hist, s_prefix, s_rem, nullptr);
}

}  // namespace chimera
