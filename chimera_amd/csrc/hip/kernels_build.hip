// Index build on the GPU (build_index.cu:258-363, quantization.cpp:32-193,
// ivf_pg.cpp:110-126): rotation and one-bit / full-code encoding of every
// token, the cluster-ordered layout and the per-cluster document runs.
// The arithmetic mirrors the host encoder operation for operation (the same
// fused multiply-adds, the same sequential sums, the same event order in
// best_rescale_factor) so both builds produce identical bytes.
#include "common.hpp"
#include "kernels.hpp"
#include "rotate.hpp"

#include <hipcub/hipcub.hpp>

namespace chimera {

namespace {

__constant__ float kTightStart[9] = {0.F, 0.15F, 0.20F, 0.52F, 0.59F, 0.71F, 0.75F, 0.77F, 0.81F};

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor_u64(v, m);
        v = o < v ? o : v;
    }
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
    return v;
}

// Byte o of the W-bit packing of 128 raw codes (packing_rabitqplus_code,
// pack_excode.hpp; the host pack_codes states the same layouts).
__device__ uint8_t pack_byte(const uint8_t* r, int W, int o) {
    switch (W) {
        case 2: {
            const uint8_t* b = r + 16 * (o >> 2);
            const int m = o & 3;
            return static_cast<uint8_t>((b[m] & 3) | (b[4 + m] & 3) << 2 | (b[8 + m] & 3) << 4 | (b[12 + m] & 3) << 6);
        }
        case 4: {
            const uint8_t* b = r + 16 * (o >> 3);
            const int m = o & 7;
            return static_cast<uint8_t>((b[m] & 15) | (b[8 + m] & 15) << 4);
        }
        case 6: {
            const uint8_t* b = r + 16 * (o / 12);
            const int m = o % 12;
            if (m < 8) return static_cast<uint8_t>((b[m] & 15) | (b[8 + m] & 15) << 4);
            const int k = m - 8;
            return static_cast<uint8_t>(((b[k] >> 4) & 3) | ((b[4 + k] >> 4) & 3) << 2 | ((b[8 + k] >> 4) & 3) << 4 |
                                        ((b[12 + k] >> 4) & 3) << 6);
        }
        case 8:
            return r[o];
        default: {  // 3, 5, 7: 64-dimension blocks, top bits in the last u64
            const int bb = 8 * W;
            const uint8_t* b = r + 64 * (o / bb);
            const int m = o % bb;
            const int low = W - 1;
            if (m >= bb - 8) {
                const int k = m - (bb - 8);
                int v = 0;
#pragma unroll
                for (int g = 0; g < 8; ++g) v |= ((b[8 * g + k] >> low) & 1) << g;
                return static_cast<uint8_t>(v);
            }
            if (W == 3)
                return static_cast<uint8_t>((b[m] & 3) | (b[16 + m] & 3) << 2 | (b[32 + m] & 3) << 4 |
                                            (b[48 + m] & 3) << 6);
            if (W == 5) {
                if (m < 16) return static_cast<uint8_t>((b[m] & 15) | (b[16 + m] & 15) << 4);
                const int k = m - 16;
                return static_cast<uint8_t>((b[32 + k] & 15) | (b[48 + k] & 15) << 4);
            }
            const int part = m >> 4;  // W == 7
            const int k = m & 15;
            return static_cast<uint8_t>((b[16 * part + k] & 63) | ((b[48 + k] >> (2 * part)) & 3) << 6);
        }
    }
}

}  // namespace

// One wave per token (grid-stride over blocks of 4 tokens). Lane l holds
// rotated elements l and l + 64; for the rescale sweep it owns dimensions
// 2l and 2l + 1 so that equal event times resolve to the lower dimension as
// std::priority_queue over (t, id) pairs does (quantization.cpp:62-119).
__global__ __launch_bounds__(256) void encode_tokens_kernel(const float* __restrict__ emb, int64_t n, int dim,
                                                            const uint8_t* __restrict__ flips, float fac,
                                                            int ex_bits, uint8_t* __restrict__ codes1,
                                                            float* __restrict__ f1, uint8_t* __restrict__ full,
                                                            float* __restrict__ fF, uint32_t* __restrict__ status) {
    __shared__ float srow[4][kDim];
    __shared__ float sabs[4][kDim];
    __shared__ uint8_t sraw[4][kDim];
    __shared__ uint8_t fl[4 * kDim / 8];
    const int l = lane_id();
    const int w = wave_id();
    if (threadIdx.x < 4 * kDim / 8) fl[threadIdx.x] = flips[threadIdx.x];
    __syncthreads();
    const int top = (1 << ex_bits) - 1;
    const int W = ex_bits + 1;
    const bool pow2 = dim >= kDim;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * 4; base < n; base += stride) {
        const int64_t t = base + w;
        if (t >= n) continue;  // wave-uniform
        const float* src = emb + t * dim;
        float x0 = l < dim ? src[l] : 0.0f;
        float x1 = l + 64 < dim ? src[l + 64] : 0.0f;
        fht_kac_rotate(x0, x1, fl, fac, pow2, l);
        srow[w][l] = x0;
        srow[w][l + 64] = x1;

        // one-bit code: bit j of the little-endian 128-bit word is o'_j > 0
        const uint64_t m0 = __ballot(x0 > 0.0f);
        const uint64_t m1 = __ballot(x1 > 0.0f);
        if (l == 0) {
            uint4 v;
            v.x = static_cast<uint32_t>(m0);
            v.y = static_cast<uint32_t>(m0 >> 32);
            v.z = static_cast<uint32_t>(m1);
            v.w = static_cast<uint32_t>(m1 >> 32);
            reinterpret_cast<uint4*>(codes1)[t] = v;
        }
        wave_lds_sync();
        // lane 0: <x_u - 1/2, o'> ; lane 1: |o'|^2 ; both in dimension order
        float acc = 0.0f;
        if (l < 2) {
            for (int j = 0; j < kDim; ++j) {
                const float r = srow[w][j];
                const float x = (l == 0) ? ((r > 0.0f ? 1.0f : 0.0f) - 0.5F) : r;
                acc = __fmaf_rn(x, r, acc);
            }
        }
        const float ip1 = __shfl(acc, 0, kWave);
        const float sq = __shfl(acc, 1, kWave);
        if (l == 0) f1[t] = 1.0F / ip1;
        const float norm = sqrtf(sq);
        const float a0 = norm > 0.0f ? fabsf(x0 / norm) : fabsf(x0);
        const float a1 = norm > 0.0f ? fabsf(x1 / norm) : fabsf(x1);
        sabs[w][l] = a0;
        sabs[w][l + 64] = a1;
        const float max_o = wave_max_f32(fmaxf(a0, a1));
        const bool finite = __ballot(!(isfinite(x0) && isfinite(x1))) == 0ull;
        uint8_t* out = full + t * (16 * W);
        if (!finite || !(max_o > 0.0f) || !isfinite(max_o)) {
            // zero or non-finite token: the rescale search is undefined
            if (l == 0) {
                atomicOr(status, 1u);
                fF[t] = 0.0f;
            }
            for (int o = l; o < 16 * W; o += kWave) out[o] = 0;
            wave_lds_sync();
            continue;
        }
        wave_lds_sync();

        // best_rescale_factor (quantization.cpp:62-119)
        const double t_end = static_cast<double>(top + 10) / static_cast<double>(max_o);
        const double t_start = t_end * static_cast<double>(kTightStart[ex_bits]);
        const float oa = sabs[w][2 * l];
        const float ob = sabs[w][2 * l + 1];
        int ca = static_cast<int>(fma(t_start, static_cast<double>(oa), 1e-5));
        int cb = static_cast<int>(fma(t_start, static_cast<double>(ob), 1e-5));
        double den = static_cast<double>(kDim) * 0.25 + static_cast<double>(wave_sum_i32(ca * ca + ca + cb * cb + cb));
        double num = 0.0;
        if (l == 0) {
            for (int i = 0; i < kDim; ++i) {
                const double o = static_cast<double>(sabs[w][i]);
                const int c = static_cast<int>(fma(t_start, o, 1e-5));
                num = fma(static_cast<double>(c) + 0.5, o, num);
            }
        }
        num = __shfl(num, 0, kWave);
        double ta = static_cast<double>(ca + 1) / static_cast<double>(oa);
        double tb = static_cast<double>(cb + 1) / static_cast<double>(ob);
        bool pa = true, pb = true;
        double max_ip = 0.0, tbest = 0.0;
        const int max_events = kDim * (top + 2) + 1;
        int it = 0;
        for (; it < max_events; ++it) {
            const uint64_t ka = pa ? static_cast<uint64_t>(__double_as_longlong(ta)) : ~0ull;
            const uint64_t kb = pb ? static_cast<uint64_t>(__double_as_longlong(tb)) : ~0ull;
            const bool sel_b = kb < ka;
            const uint64_t key = sel_b ? kb : ka;
            const uint64_t kmin = wave_min_u64(key);
            if (kmin == ~0ull) break;
            const int win = __builtin_ctzll(__ballot(key == kmin));
            const int u = __shfl((sel_b ? cb : ca) + 1, win, kWave);
            const float o = __shfl(sel_b ? ob : oa, win, kWave);
            const double cur_t = __longlong_as_double(static_cast<long long>(kmin));
            den += static_cast<double>(2 * u);
            num += static_cast<double>(o);
            const double cur_ip = num / sqrt(den);
            if (cur_ip > max_ip) {
                max_ip = cur_ip;
                tbest = cur_t;
            }
            if (l == win) {
                bool keep = false;
                double tn = 0.0;
                if (u < top) {
                    tn = static_cast<double>(u + 1) / static_cast<double>(o);
                    keep = tn < t_end;
                }
                if (sel_b) {
                    cb = u;
                    pb = keep;
                    if (keep) tb = tn;
                } else {
                    ca = u;
                    pa = keep;
                    if (keep) ta = tn;
                }
            }
        }
        if (it == max_events && l == 0) atomicOr(status, 2u);

        // quantize_ex + total code (quantization.cpp:121-193)
        int e0 = static_cast<int>(fma(tbest, static_cast<double>(a0), 1e-5));
        int e1 = static_cast<int>(fma(tbest, static_cast<double>(a1), 1e-5));
        e0 = e0 > top ? top : e0;
        e1 = e1 > top ? top : e1;
        if (x0 < 0.0f) e0 = (~e0) & top;
        if (x1 < 0.0f) e1 = (~e1) & top;
        sraw[w][l] = static_cast<uint8_t>(e0 + ((x0 >= 0.0f ? 1 : 0) << ex_bits));
        sraw[w][l + 64] = static_cast<uint8_t>(e1 + ((x1 >= 0.0f ? 1 : 0) << ex_bits));
        wave_lds_sync();
        if (l == 0) {
            const float cbf = -(static_cast<float>(1 << ex_bits) - 0.5F);
            float ip = 0.0f;
            for (int j = 0; j < kDim; ++j) ip = __fmaf_rn(static_cast<float>(sraw[w][j]) + cbf, srow[w][j], ip);
            fF[t] = 1.0F / ip;
        }
        for (int o = l; o < 16 * W; o += kWave) out[o] = pack_byte(sraw[w], W, o);
        wave_lds_sync();
    }
}

// Rows src[ids[r]] (dim floats) zero-padded to 128, optionally rotated.
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ src, int dim,
                                                          const int64_t* __restrict__ ids, int64_t nrows,
                                                          const uint8_t* __restrict__ flips, float fac, int rotate,
                                                          float* __restrict__ out) {
    __shared__ uint8_t fl[4 * kDim / 8];
    const int l = lane_id();
    if (threadIdx.x < 4 * kDim / 8) fl[threadIdx.x] = rotate ? flips[threadIdx.x] : 0;
    __syncthreads();
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + wave_id();
    if (r >= nrows) return;
    const float* s = src + (ids ? ids[r] : r) * dim;
    float x0 = l < dim ? s[l] : 0.0f;
    float x1 = l + 64 < dim ? s[l + 64] : 0.0f;
    if (rotate) fht_kac_rotate(x0, x1, fl, fac, dim >= kDim, l);
    out[r * kDim + l] = x0;
    out[r * kDim + l + 64] = x1;
}

__global__ void iota_u32_kernel(uint32_t* __restrict__ v, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) v[i] = static_cast<uint32_t>(i);
}

// cluster_pos[c] = first position of cluster c in the sorted assignments.
__global__ void cluster_bounds_kernel(const uint32_t* __restrict__ sorted, int64_t n, int64_t k,
                                      uint64_t* __restrict__ cluster_pos) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (c > k) return;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (static_cast<int64_t>(sorted[mid]) < c) lo = mid + 1; else hi = mid;
    }
    cluster_pos[c] = static_cast<uint64_t>(lo);
}

__global__ void token_doc_kernel(const int32_t* __restrict__ doc_ptrs, int64_t m, int32_t* __restrict__ token_doc) {
    const int64_t d = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (d >= m) return;
    for (int32_t t = doc_ptrs[d]; t < doc_ptrs[d + 1]; ++t) token_doc[t] = static_cast<int32_t>(d);
}

// reorder_by_cluster (build_index.cu:328-363)
__global__ void reorder_kernel(const uint32_t* __restrict__ inv, int64_t n, const uint8_t* __restrict__ codes_tok,
                               const float* __restrict__ f1_tok, const int32_t* __restrict__ token_doc,
                               uint8_t* __restrict__ codes_clu, float* __restrict__ f1_clu,
                               int32_t* __restrict__ doc_clu) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const uint32_t t = inv[p];
    reinterpret_cast<uint4*>(codes_clu)[p] = reinterpret_cast<const uint4*>(codes_tok)[t];
    f1_clu[p] = f1_tok[t];
    doc_clu[p] = token_doc[t];
}

// Number of runs of equal document ids inside each cluster.
__global__ void cluster_runs_kernel(const uint64_t* __restrict__ cluster_pos, const int32_t* __restrict__ doc_clu,
                                    int64_t k, uint32_t* __restrict__ runs) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (c >= k) return;
    uint32_t r = 0;
    for (uint64_t p = cluster_pos[c]; p < cluster_pos[c + 1]; ++p)
        if (p == cluster_pos[c] || doc_clu[p] != doc_clu[p - 1]) ++r;
    runs[c] = r;
}

// ---- launchers ----

namespace {
unsigned blocks_for(int64_t n, int per) { return static_cast<unsigned>((n + per - 1) / per); }
}  // namespace

hipError_t launch_encode_tokens(hipStream_t s, const float* emb, int64_t n, int dim, const uint8_t* flips,
                                int ex_bits, int num_cus, uint8_t* codes1, float* f1, uint8_t* full, float* fF,
                                uint32_t* status) {
    if (n == 0) return hipSuccess;
    const int trunc = dim >= kDim ? kDim : 64;
    const float fac = 1.0F / sqrtf(static_cast<float>(trunc));
    const int64_t want = static_cast<int64_t>(num_cus) * 32;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((n + 3) / 4, want));
    hipLaunchKernelGGL(encode_tokens_kernel, dim3(grid), dim3(256), 0, s, emb, n, dim, flips, fac, ex_bits, codes1,
                       f1, full, fF, status);
    return hipGetLastError();
}

hipError_t launch_gather_rows(hipStream_t s, const float* src, int dim, const int64_t* ids, int64_t nrows,
                              const uint8_t* flips, bool rotate, float* out) {
    if (nrows == 0) return hipSuccess;
    const int trunc = dim >= kDim ? kDim : 64;
    const float fac = 1.0F / sqrtf(static_cast<float>(trunc));
    hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_for(nrows, 4)), dim3(256), 0, s, src, dim, ids, nrows, flips,
                       fac, rotate ? 1 : 0, out);
    return hipGetLastError();
}

hipError_t launch_sort_assignments(hipStream_t s, const uint32_t* labels, int64_t n, int64_t k, uint32_t* keys_out,
                                   uint32_t* vals_in, uint32_t* vals_out, void* temp, size_t* temp_bytes) {
    int end_bit = 1;
    while ((int64_t{1} << end_bit) < k) ++end_bit;
    if (temp == nullptr)
        return hipcub::DeviceRadixSort::SortPairs(nullptr, *temp_bytes, labels, keys_out, vals_in, vals_out,
                                                  static_cast<int>(n), 0, end_bit, s);
    hipLaunchKernelGGL(iota_u32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, vals_in, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return hipcub::DeviceRadixSort::SortPairs(temp, *temp_bytes, labels, keys_out, vals_in, vals_out,
                                              static_cast<int>(n), 0, end_bit, s);
}

hipError_t launch_layout(hipStream_t s, const uint32_t* sorted_keys, const uint32_t* inv, int64_t n, int64_t k,
                         const int32_t* doc_ptrs, int64_t m, const uint8_t* codes_tok, const float* f1_tok,
                         int32_t* token_doc, uint64_t* cluster_pos, uint8_t* codes_clu, float* f1_clu,
                         int32_t* doc_clu, uint32_t* runs) {
    hipLaunchKernelGGL(cluster_bounds_kernel, dim3(blocks_for(k + 1, 256)), dim3(256), 0, s, sorted_keys, n, k,
                       cluster_pos);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(token_doc_kernel, dim3(blocks_for(m, 256)), dim3(256), 0, s, doc_ptrs, m, token_doc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(reorder_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, inv, n, codes_tok, f1_tok, token_doc,
                       codes_clu, f1_clu, doc_clu);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(cluster_runs_kernel, dim3(blocks_for(k, 256)), dim3(256), 0, s, cluster_pos, doc_clu, k, runs);
    return hipGetLastError();
}

}  // namespace chimera
