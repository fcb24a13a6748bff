// Query-side kernels: FhtKac rotation + QueryState + one-bit LUT, the exact
// centroid probe, centroid norms and code unpacking.
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

// Exact probe: for ROWS rotated query vectors per block, every centroid's
// score |c|^2 - 2<q,c> (sequential fmaf over the 128 dims, as the oracle) and
// the nprobe smallest (score, id) pairs, nearest first. Candidates below the
// running threshold go to a per-row LDS buffer that is sorted and cut back to
// nprobe whenever it could overflow.
template <int ROWS>
__global__ __launch_bounds__(256) void probe_exact_kernel(const float* __restrict__ rot, int nrows,
                                                          const float* __restrict__ centroids,
                                                          const float* __restrict__ norms, int64_t k, int nprobe,
                                                          int cap, uint32_t* __restrict__ labels,
                                                          const uint32_t* __restrict__ row_flag) {
    extern __shared__ __align__(16) unsigned char smem[];
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
    if (threadIdx.x < ROWS) {
        cnt[threadIdx.x] = 0;
        thr[threadIdx.x] = 0xFFFFFFFFu;
    }
    __syncthreads();
    for (int64_t tile = 0; tile < k; tile += blockDim.x) {
        const int64_t c = tile + threadIdx.x;
        if (c < k) {
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
        if (need || tile + blockDim.x >= k) {
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
    for (int t = threadIdx.x; t < ROWS * nprobe; t += blockDim.x) {
        const int rr = t / nprobe;
        const int p = t % nprobe;
        if (row0 + rr < nrows)
            labels[static_cast<size_t>(row0 + rr) * nprobe + p] =
                static_cast<uint32_t>(buf[static_cast<size_t>(rr) * cap + p] & 0xFFFFFFFFu);
    }
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
    if (rows == 8)
        return hipFuncSetAttribute(reinterpret_cast<const void*>(probe_exact_kernel<8>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, shm);
    return hipFuncSetAttribute(reinterpret_cast<const void*>(probe_exact_kernel<2>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, shm);
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
                                          const uint32_t* row_flag) {
    const int cap = probe_buffer_cap(nprobe);
    if (cap <= 1024) {
        constexpr int R = 8;
        const size_t shm = static_cast<size_t>(R) * cap * 8 + R * kDim * 4;
        hipLaunchKernelGGL(probe_exact_kernel<R>, dim3((nrows + R - 1) / R), dim3(256), shm, s, rot, nrows,
                           centroids, norms, k, nprobe, cap, labels, row_flag);
    } else {
        constexpr int R = 2;
        const size_t shm = static_cast<size_t>(R) * cap * 8 + R * kDim * 4;
        hipLaunchKernelGGL(probe_exact_kernel<R>, dim3((nrows + R - 1) / R), dim3(256), shm, s, rot, nrows,
                           centroids, norms, k, nprobe, cap, labels, row_flag);
    }
    return hipGetLastError();
}

hipError_t launch_probe_exact(hipStream_t s, const float* rot, int nrows, const float* centroids,
                              const float* norms, int64_t k, int nprobe, uint32_t* labels) {
    return launch_probe_exact_impl(s, rot, nrows, centroids, norms, k, nprobe, labels, nullptr);
}

hipError_t launch_probe_exact_flagged(hipStream_t s, const float* rot, int nrows, const float* centroids,
                                      const float* norms, int64_t k, int nprobe, const uint32_t* row_flag,
                                      uint32_t* labels) {
    return launch_probe_exact_impl(s, rot, nrows, centroids, norms, k, nprobe, labels, row_flag);
}

hipError_t launch_unpack_codes(hipStream_t s, int width, const uint8_t* packed, int64_t n, uint8_t* raw) {
    const int64_t total = n * kDim;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(unpack_codes_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s,
                       width, packed, n, raw);
    return hipGetLastError();
}

}  // namespace chimera
