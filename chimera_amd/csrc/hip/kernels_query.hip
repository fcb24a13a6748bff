// Query-side kernels: FhtKac rotation + QueryState + one-bit LUT, the exact
// centroid probe, centroid norms and code unpacking.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "rotate.hpp"

namespace chimera {

// One wave per (query, token) row. Lane l holds elements l and l + 64.
// Rotation: rotator.hpp:281-334. QueryState: chimera_index_internal.cuh:58-64
// (sequential sum). LUT: kernels.cu:402-428, written as [q][c][e][i].
__global__ __launch_bounds__(256) void rotate_lut_kernel(const float* __restrict__ queries, int nq, int dim,
                                                         const uint8_t* __restrict__ flips, float fac, int ex_bits,
                                                         float* __restrict__ rot, float* __restrict__ cb1,
                                                         float* __restrict__ cbex, float* __restrict__ lut) {
    __shared__ float row[4][kDim];
    __shared__ uint8_t fl[4 * kDim / 8];
    const int l = lane_id();
    const int w = wave_id();
    if (threadIdx.x < 4 * kDim / 8) fl[threadIdx.x] = flips[threadIdx.x];
    __syncthreads();
    const int r = blockIdx.x * 4 + w;
    const bool valid = r < nq * kQ;
    const float* src = queries + static_cast<size_t>(valid ? r : 0) * dim;
    float x0 = (valid && l < dim) ? src[l] : 0.0f;
    float x1 = (valid && l + 64 < dim) ? src[l + 64] : 0.0f;
    fht_kac_rotate(x0, x1, fl, fac, dim >= kDim, l);  // trunc_dim == padded_dim when dim == 128
    row[w][l] = x0;
    row[w][l + 64] = x1;
    __syncthreads();
    if (!valid) return;
    if (rot) {
        rot[static_cast<size_t>(r) * kDim + l] = x0;
        rot[static_cast<size_t>(r) * kDim + l + 64] = x1;
    }
    if (l == 0) {
        float s = 0.0f;
        for (int j = 0; j < kDim; ++j) s = s + row[w][j];
        if (cb1) cb1[r] = s * ((1 << 1) - 1) / 2.0f;
        if (cbex) cbex[r] = s * ((1 << (ex_bits + 1)) - 1) / 2.0f;
    }
    if (lut) {
        const int q = r / kQ;
        const int i = r % kQ;
        float* out = lut + static_cast<size_t>(q) * kLutPerQuery + static_cast<size_t>(i) * (kChunks * kLut);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int idx = l + 64 * k;
            const int c = idx >> 4;
            const int e = idx & 15;
            float s = 0.0f;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if ((e >> b) & 1) s += row[w][c * 4 + b];
            out[c * kLut + e] = s;
        }
    }
}

// |c|^2 by sequential fmaf (the probe score's norm term).
__global__ void centroid_norms_kernel(const float* __restrict__ c, int64_t k, float* __restrict__ norms) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= k) return;
    const float* v = c + i * kDim;
    float s = 0.0f;
    for (int j = 0; j < kDim; ++j) s = __fmaf_rn(v[j], v[j], s);
    norms[i] = s;
}

namespace {

// Ascending bitonic sort of `rows` independent LDS arrays of n (power of two)
// 64-bit keys, by all threads of the block.
__device__ void bitonic_sort_rows(uint64_t* buf, int rows, int n) {
    const int total = rows * (n / 2);
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size / 2; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < total; t += blockDim.x) {
                const int rr = t / (n / 2);
                const int p = t % (n / 2);
                const int i = 2 * p - (p & (stride - 1));
                const int j = i + stride;
                uint64_t* b = buf + static_cast<size_t>(rr) * n;
                const bool up = ((i & size) == 0);
                const uint64_t a = b[i], c = b[j];
                if ((a > c) == up) {
                    b[i] = c;
                    b[j] = a;
                }
            }
            __syncthreads();
        }
    }
}

}  // namespace

namespace {

// Exact top-nprobe of ROWS rows (q: [ROWS][128] in LDS, written before the
// call) over centroids [c0, c1): every centroid's score |c|^2 - 2<q,c>
// (sequential fmaf over the 128 dims, as the oracle). Candidates below the
// running threshold go to the row's LDS buffer buf[rr * cap ...], which is
// sorted by (ordered score << 32 | id) and cut back to nprobe whenever the
// next tile could overflow it, and once at the end: the first nprobe entries
// of each row are then its best keys in order (~0 past the range's size).
template <int ROWS>
__device__ void exact_rows_topk(const float* q, const float* __restrict__ centroids, const float* __restrict__ norms,
                                int64_t c0, int64_t c1, int nprobe, int cap, uint64_t* buf, int* cnt, uint32_t* thr) {
    if (threadIdx.x < ROWS) {
        cnt[threadIdx.x] = 0;
        thr[threadIdx.x] = 0xFFFFFFFFu;
    }
    __syncthreads();
    for (int64_t tile = c0; tile < c1; tile += blockDim.x) {
        const int64_t c = tile + threadIdx.x;
        if (c < c1) {
            const float4* cv = reinterpret_cast<const float4*>(centroids + c * kDim);
            float acc[ROWS];
#pragma unroll
            for (int rr = 0; rr < ROWS; ++rr) acc[rr] = 0.0f;
            for (int j4 = 0; j4 < kDim / 4; ++j4) {
                const float4 v = cv[j4];
#pragma unroll
                for (int rr = 0; rr < ROWS; ++rr) {
                    const float* qr = q + rr * kDim + 4 * j4;
                    acc[rr] = __fmaf_rn(qr[0], v.x, acc[rr]);
                    acc[rr] = __fmaf_rn(qr[1], v.y, acc[rr]);
                    acc[rr] = __fmaf_rn(qr[2], v.z, acc[rr]);
                    acc[rr] = __fmaf_rn(qr[3], v.w, acc[rr]);
                }
            }
            const float nrm = norms[c];
#pragma unroll
            for (int rr = 0; rr < ROWS; ++rr) {
                const float score = nrm - 2.0f * acc[rr];
                const uint32_t key = float_to_ordered(score);
                if (key < thr[rr]) {
                    const int pos = atomicAdd(&cnt[rr], 1);
                    buf[static_cast<size_t>(rr) * cap + pos] = (static_cast<uint64_t>(key) << 32) | static_cast<uint32_t>(c);
                }
            }
        }
        __syncthreads();
        bool need = false;
#pragma unroll
        for (int rr = 0; rr < ROWS; ++rr) need |= cnt[rr] > cap - static_cast<int>(blockDim.x);
        if (need || tile + blockDim.x >= c1) {
            for (int t = threadIdx.x; t < ROWS * cap; t += blockDim.x) {
                const int rr = t / cap;
                if ((t % cap) >= cnt[rr]) buf[t] = ~0ull;
            }
            __syncthreads();
            bitonic_sort_rows(buf, ROWS, cap);
            if (threadIdx.x < ROWS) {
                const int rr = threadIdx.x;
                if (cnt[rr] >= nprobe) {
                    cnt[rr] = nprobe;
                    thr[rr] = static_cast<uint32_t>(buf[static_cast<size_t>(rr) * cap + nprobe - 1] >> 32);
                }
            }
            __syncthreads();
        }
    }
    if (c0 >= c1) {  // an empty range has no keys
        for (int t = threadIdx.x; t < ROWS * cap; t += blockDim.x) buf[t] = ~0ull;
        __syncthreads();
    }
}

}  // namespace

// Exact probe: for ROWS rotated query vectors per block, the nprobe
// centroids with the smallest score (ties to the lower id), nearest first.
// With row_flag, only blocks that hold a flagged row work; with gate, not
// even those while *gate <= gate_cap (the split kernels below have taken
// the flagged rows).
template <int ROWS>
__global__ __launch_bounds__(256) void probe_exact_kernel(const float* __restrict__ rot, int nrows,
                                                          const float* __restrict__ centroids,
                                                          const float* __restrict__ norms, int64_t k, int nprobe,
                                                          int cap, uint32_t* __restrict__ labels,
                                                          const uint32_t* __restrict__ row_flag,
                                                          const uint32_t* __restrict__ gate, int gate_cap) {
    extern __shared__ __align__(16) unsigned char smem[];
    if (gate && *gate <= static_cast<uint32_t>(gate_cap)) return;
    if (row_flag) {
        bool any = false;
        for (int rr = 0; rr < ROWS; ++rr)
            if (blockIdx.x * ROWS + rr < nrows && row_flag[blockIdx.x * ROWS + rr]) any = true;
        if (!any) return;
    }
    uint64_t* buf = reinterpret_cast<uint64_t*>(smem);                       // [ROWS][cap]
    float* q = reinterpret_cast<float*>(buf + static_cast<size_t>(ROWS) * cap);  // [ROWS][128]
    __shared__ int cnt[ROWS];
    __shared__ uint32_t thr[ROWS];  // ordered score threshold
    const int row0 = blockIdx.x * ROWS;
    for (int t = threadIdx.x; t < ROWS * kDim; t += blockDim.x) {
        const int rr = t / kDim;
        q[t] = (row0 + rr < nrows) ? rot[static_cast<size_t>(row0 + rr) * kDim + (t % kDim)] : 0.0f;
    }
    exact_rows_topk<ROWS>(q, centroids, norms, 0, k, nprobe, cap, buf, cnt, thr);
    for (int t = threadIdx.x; t < ROWS * nprobe; t += blockDim.x) {
        const int rr = t / nprobe;
        const int p = t % nprobe;
        if (row0 + rr < nrows)
            labels[static_cast<size_t>(row0 + rr) * nprobe + p] =
                static_cast<uint32_t>(buf[static_cast<size_t>(rr) * cap + p] & 0xFFFFFFFFu);
    }
}

// The flagged rows in a list: list[f] for f < min(*nflag, list_cap), in no
// particular order (each row's result is independent of it); *nflag is the
// full count (cleared by the caller).
__global__ __launch_bounds__(256) void probe_flag_list_kernel(const uint32_t* __restrict__ row_flag, int nrows,
                                                              uint32_t* __restrict__ list, uint32_t* __restrict__ nflag,
                                                              int list_cap) {
    const int row = static_cast<int>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= nrows || !row_flag[row]) return;
    const uint32_t f = atomicAdd(nflag, 1u);
    if (f < static_cast<uint32_t>(list_cap)) list[f] = static_cast<uint32_t>(row);
}

// Split exact probe of the listed rows: block (s, g) scores flagged rows
// g * ROWS .. g * ROWS + ROWS - 1 against centroids [s * chunk, (s + 1) *
// chunk) and writes their best nprobe keys of that range (~0-padded) to
// partial[(f * splits + s) * nprobe ...]. Does nothing when more than
// list_cap rows are flagged (the row-block kernel takes them all).
template <int ROWS>
__global__ __launch_bounds__(256) void probe_exact_split_kernel(const float* __restrict__ rot,
                                                                const float* __restrict__ centroids,
                                                                const float* __restrict__ norms, int64_t k,
                                                                int nprobe, int cap, const uint32_t* __restrict__ list,
                                                                const uint32_t* __restrict__ nflag, int list_cap,
                                                                int64_t chunk, int splits,
                                                                uint64_t* __restrict__ partial) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nf = *nflag;
    const int f0 = static_cast<int>(blockIdx.y) * ROWS;
    if (nf > static_cast<uint32_t>(list_cap) || static_cast<uint32_t>(f0) >= nf) return;
    uint64_t* buf = reinterpret_cast<uint64_t*>(smem);                       // [ROWS][cap]
    float* q = reinterpret_cast<float*>(buf + static_cast<size_t>(ROWS) * cap);  // [ROWS][128]
    __shared__ int cnt[ROWS];
    __shared__ uint32_t thr[ROWS];
    for (int t = threadIdx.x; t < ROWS * kDim; t += blockDim.x) {
        const int rr = t / kDim;
        const uint32_t f = static_cast<uint32_t>(f0 + rr);
        q[t] = f < nf ? rot[static_cast<size_t>(list[f]) * kDim + (t % kDim)] : 0.0f;
    }
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t c1 = c0 + chunk < k ? c0 + chunk : k;
    exact_rows_topk<ROWS>(q, centroids, norms, c0 < k ? c0 : k, c1, nprobe, cap, buf, cnt, thr);
    for (int t = threadIdx.x; t < ROWS * nprobe; t += blockDim.x) {
        const int rr = t / nprobe;
        const int p = t % nprobe;
        if (static_cast<uint32_t>(f0 + rr) < nf)
            partial[(static_cast<size_t>(f0 + rr) * splits + blockIdx.x) * nprobe + p] =
                buf[static_cast<size_t>(rr) * cap + p];
    }
}

// Labels of listed row f from its splits' keys: all splits * nprobe keys
// sorted in LDS (sort_n, a power of two, entries past them ~0), the first
// nprobe ids written. One block per list entry.
__global__ __launch_bounds__(256) void probe_exact_merge_kernel(const uint32_t* __restrict__ list,
                                                                const uint32_t* __restrict__ nflag, int list_cap,
                                                                const uint64_t* __restrict__ partial, int splits,
                                                                int nprobe, int sort_n, uint32_t* __restrict__ labels) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint64_t* keys = reinterpret_cast<uint64_t*>(smem);  // [sort_n]
    const uint32_t nf = *nflag;
    const uint32_t f = blockIdx.x;
    if (nf > static_cast<uint32_t>(list_cap) || f >= nf) return;
    const int n = splits * nprobe;
    for (int t = threadIdx.x; t < sort_n; t += blockDim.x)
        keys[t] = t < n ? partial[static_cast<size_t>(f) * n + t] : ~0ull;
    __syncthreads();
    bitonic_sort_rows(keys, 1, sort_n);
    const size_t row = list[f];
    for (int p = threadIdx.x; p < nprobe; p += blockDim.x)
        labels[row * nprobe + p] = static_cast<uint32_t>(keys[p] & 0xFFFFFFFFu);
}

// ---- W-bit unpack (space.hpp:604-801 layouts) ----

// Dimension j of a packed 128-dim W-bit code.
__device__ __forceinline__ uint32_t unpack_dim(const uint8_t* p, int width, int j) {
    switch (width) {
        case 1:
            return (p[j >> 3] >> (j & 7)) & 1u;
        case 2: {
            const int b = j >> 4, o = j & 15;
            return (p[4 * b + (o & 3)] >> (2 * (o >> 2))) & 3u;
        }
        case 4: {
            const int b = j >> 4, o = j & 15;
            return (p[8 * b + (o & 7)] >> (4 * (o >> 3))) & 15u;
        }
        case 6: {
            const int b = j >> 4, o = j & 15;
            const uint8_t* q = p + 12 * b;
            const uint32_t lo = (q[o & 7] >> (4 * (o >> 3))) & 15u;
            const uint32_t hi = (q[8 + (o & 3)] >> (2 * (o >> 2))) & 3u;
            return lo | (hi << 4);
        }
        case 8:
            return p[j];
        default: {  // 3, 5, 7
            const int bytes = 8 * width;
            const uint8_t* q = p + (j >> 6) * bytes;
            const int o = j & 63;
            uint32_t low;
            if (width == 3) {
                low = (q[o & 15] >> (2 * (o >> 4))) & 3u;
            } else if (width == 5) {
                low = (q[16 * (o >> 5) + (o & 15)] >> (4 * ((o >> 4) & 1))) & 15u;
            } else {
                if (o < 48) {
                    low = q[o] & 63u;
                } else {
                    const int m = o - 48;
                    low = (q[m] >> 6) | ((q[16 + m] >> 6) << 2) | ((q[32 + m] >> 6) << 4);
                }
            }
            const uint8_t* top = q + bytes - 8;
            const int bit = 8 * (o & 7) + (o >> 3);  // dimension i + b -> bit 8b + i/8
            const uint32_t t = (top[bit >> 3] >> (bit & 7)) & 1u;
            return low | (t << (width - 1));
        }
    }
}

__global__ void unpack_codes_kernel(int width, const uint8_t* __restrict__ packed, int64_t n,
                                    uint8_t* __restrict__ raw) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * kDim) return;
    const int64_t v = t / kDim;
    const int j = static_cast<int>(t % kDim);
    raw[t] = static_cast<uint8_t>(unpack_dim(packed + v * 16 * width, width, j));
}

// ---- host launchers ----

hipError_t configure_query_kernels(int nprobe) {
    const int cap = probe_buffer_cap(nprobe);
    const int rows = cap <= 1024 ? 8 : 2;
    const int shm = rows * cap * 8 + rows * kDim * 4;
    if (shm <= 64 * 1024) return hipSuccess;
    const void* whole = rows == 8 ? reinterpret_cast<const void*>(probe_exact_kernel<8>)
                                  : reinterpret_cast<const void*>(probe_exact_kernel<2>);
    const void* split = rows == 8 ? reinterpret_cast<const void*>(probe_exact_split_kernel<8>)
                                  : reinterpret_cast<const void*>(probe_exact_split_kernel<2>);
    const hipError_t e = hipFuncSetAttribute(whole, hipFuncAttributeMaxDynamicSharedMemorySize, shm);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(split, hipFuncAttributeMaxDynamicSharedMemorySize, shm);
}

hipError_t launch_rotate_lut(hipStream_t s, const float* queries, int nq, int dim, const uint8_t* flips,
                             int ex_bits, float* rot, float* cb1, float* cbex, float* lut) {
    const int rows = nq * kQ;
    const int trunc = dim >= kDim ? kDim : 64;
    const float fac = 1.0F / sqrtf(static_cast<float>(trunc));
    hipLaunchKernelGGL(rotate_lut_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, queries, nq, dim, flips, fac,
                       ex_bits, rot, cb1, cbex, lut);
    return hipGetLastError();
}

hipError_t launch_centroid_norms(hipStream_t s, const float* c, int64_t k, float* norms) {
    hipLaunchKernelGGL(centroid_norms_kernel, dim3(static_cast<unsigned>((k + 255) / 256)), dim3(256), 0, s, c, k,
                       norms);
    return hipGetLastError();
}

int probe_buffer_cap(int nprobe) {
    int cap = 512;
    while (cap < nprobe + 256) cap <<= 1;
    return cap;
}

static hipError_t launch_probe_exact_impl(hipStream_t s, const float* rot, int nrows, const float* centroids,
                                          const float* norms, int64_t k, int nprobe, uint32_t* labels,
                                          const uint32_t* row_flag, const uint32_t* gate, int gate_cap) {
    const int cap = probe_buffer_cap(nprobe);
    if (cap <= 1024) {
        constexpr int R = 8;
        const size_t shm = static_cast<size_t>(R) * cap * 8 + R * kDim * 4;
        hipLaunchKernelGGL(probe_exact_kernel<R>, dim3((nrows + R - 1) / R), dim3(256), shm, s, rot, nrows,
                           centroids, norms, k, nprobe, cap, labels, row_flag, gate, gate_cap);
    } else {
        constexpr int R = 2;
        const size_t shm = static_cast<size_t>(R) * cap * 8 + R * kDim * 4;
        hipLaunchKernelGGL(probe_exact_kernel<R>, dim3((nrows + R - 1) / R), dim3(256), shm, s, rot, nrows,
                           centroids, norms, k, nprobe, cap, labels, row_flag, gate, gate_cap);
    }
    return hipGetLastError();
}

hipError_t launch_probe_exact(hipStream_t s, const float* rot, int nrows, const float* centroids,
                              const float* norms, int64_t k, int nprobe, uint32_t* labels) {
    return launch_probe_exact_impl(s, rot, nrows, centroids, norms, k, nprobe, labels, nullptr, nullptr, 0);
}

int exact_fallback_splits(int nprobe) {
    return std::max(1, std::min(64, kExactPartialKeys / std::max(1, nprobe)));
}

hipError_t launch_probe_exact_flagged(hipStream_t s, const float* rot, int nrows, const float* centroids,
                                      const float* norms, int64_t k, int nprobe, const uint32_t* row_flag,
                                      uint32_t* labels, const ExactFallback& fb) {
    if (nrows <= 0) return hipSuccess;
    if (fb.list == nullptr || fb.list_cap <= 0 || nprobe > kExactPartialKeys)
        return launch_probe_exact_impl(s, rot, nrows, centroids, norms, k, nprobe, labels, row_flag, nullptr, 0);
    hipError_t e = launch_fill_u32(s, fb.nflag, 1, 0u);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(probe_flag_list_kernel, dim3((nrows + 255) / 256), dim3(256), 0, s, row_flag, nrows, fb.list,
                       fb.nflag, fb.list_cap);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // up to list_cap flagged rows: every centroid split of every ROWS of
    // them in its own block, then one merge block per row (grids for at most
    // nrows flagged rows: a one-query batch launches 32 merge blocks, not 512)
    const int listed = std::min(fb.list_cap, nrows);
    const int splits = exact_fallback_splits(nprobe);
    const int64_t chunk = (k + splits - 1) / splits;
    const int cap = probe_buffer_cap(nprobe);
    if (cap <= 1024) {
        constexpr int R = 8;
        const size_t shm = static_cast<size_t>(R) * cap * 8 + R * kDim * 4;
        hipLaunchKernelGGL(probe_exact_split_kernel<R>, dim3(splits, (listed + R - 1) / R), dim3(256), shm, s,
                           rot, centroids, norms, k, nprobe, cap, fb.list, fb.nflag, fb.list_cap, chunk, splits,
                           fb.partial);
    } else {
        constexpr int R = 2;
        const size_t shm = static_cast<size_t>(R) * cap * 8 + R * kDim * 4;
        hipLaunchKernelGGL(probe_exact_split_kernel<R>, dim3(splits, (listed + R - 1) / R), dim3(256), shm, s,
                           rot, centroids, norms, k, nprobe, cap, fb.list, fb.nflag, fb.list_cap, chunk, splits,
                           fb.partial);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    int sort_n = 2;
    while (sort_n < splits * nprobe) sort_n <<= 1;
    hipLaunchKernelGGL(probe_exact_merge_kernel, dim3(listed), dim3(256), static_cast<size_t>(sort_n) * 8, s,
                       fb.list, fb.nflag, fb.list_cap, fb.partial, splits, nprobe, sort_n, labels);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // more flagged rows than the list holds: the row-block kernel
    return launch_probe_exact_impl(s, rot, nrows, centroids, norms, k, nprobe, labels, row_flag, fb.nflag,
                                   fb.list_cap);
}

hipError_t launch_unpack_codes(hipStream_t s, int width, const uint8_t* packed, int64_t n, uint8_t* raw) {
    const int64_t total = n * kDim;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(unpack_codes_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s,
                       width, packed, n, raw);
    return hipGetLastError();
}

}  // namespace chimera
