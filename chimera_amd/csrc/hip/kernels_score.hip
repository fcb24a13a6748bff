// Document scoring for a batch of queries:
//   refine        one-bit MaxSim S1 of the refined documents
//                 (kernels.cu:430-575, fused; no [32 x T] intermediate)
//   chunk_select  the documents rescored at full precision
//                 (search_impl.cu:341-494)
//   fullbit       full-bit MaxSim SF (search_impl.cu:510-574, replacing the
//                 AVX-512 CPU loop)
//   final_topk    top-k by SF, ties to the larger doc ID (search_impl.cu:409,496-500)
#include "common.hpp"
#include "kernels.hpp"

#include <cfloat>
#include <type_traits>

namespace chimera {

namespace {

__device__ __forceinline__ uint32_t unpack_dim_w(const uint8_t* p, int width, int j) {
    switch (width) {
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
            return ((q[o & 7] >> (4 * (o >> 3))) & 15u) | (((q[8 + (o & 3)] >> (2 * (o >> 2))) & 3u) << 4);
        }
        case 8:
            return p[j];
        case 1:
            return (p[j >> 3] >> (j & 7)) & 1u;
        default: {
            const int bytes = 8 * width;
            const uint8_t* q = p + (j >> 6) * bytes;
            const int o = j & 63;
            uint32_t low;
            if (width == 3) {
                low = (q[o & 15] >> (2 * (o >> 4))) & 3u;
            } else if (width == 5) {
                low = (q[16 * (o >> 5) + (o & 15)] >> (4 * ((o >> 4) & 1))) & 15u;
            } else if (o < 48) {
                low = q[o] & 63u;
            } else {
                const int m = o - 48;
                low = (q[m] >> 6) | ((q[16 + m] >> 6) << 2) | ((q[32 + m] >> 6) << 4);
            }
            const int bit = 8 * (o & 7) + (o >> 3);
            return low | (((q[bytes - 8 + (bit >> 3)] >> (bit & 7)) & 1u) << (width - 1));
        }
    }
}

}  // namespace

constexpr int kRefineDocsPerBlock = 64;

// Exact LUT form of the one-bit MaxSim: one wave per document; lane i (and
// i + 32, for the odd tokens) holds query token i. The LUT sits in LDS as
// [chunk][entry][token], so a wave's 32 lookups for one chunk hit 32
// consecutive words. Arithmetic order is the reference's: 32 chunk entries
// summed in order, (ip - cb1) * f, max from -FLT_MAX, shuffle-down tree.
__global__ __launch_bounds__(256) void refine_lut_kernel(const float* __restrict__ lut, const float* __restrict__ cb1,
                                                         const int32_t* __restrict__ rcount,
                                                         const int32_t* __restrict__ rids, int k_refine,
                                                         const int32_t* __restrict__ doc_ptrs,
                                                         const uint8_t* __restrict__ codes_tok,
                                                         const float* __restrict__ f1_tok, float* __restrict__ s1) {
    extern __shared__ float llut[];  // [32*16*32]
    const int q = blockIdx.x;
    const int r0 = blockIdx.y * kRefineDocsPerBlock;
    const int R = rcount[q];
    if (r0 >= R) return;
    // the query's LUT ([token][chunk][entry] in memory) transposed into LDS
    // as [chunk][entry][token]
    const float* src = lut + static_cast<size_t>(q) * kLutPerQuery;
    for (int t = threadIdx.x; t < kLutPerQuery; t += blockDim.x)
        llut[(t % (kChunks * kLut)) * kQ + t / (kChunks * kLut)] = src[t];
    __syncthreads();
    const int l = lane_id();
    const int i = l & 31;
    const int half = l >> 5;
    const float cb = cb1[q * kQ + i];
    const int r_end = min(r0 + kRefineDocsPerBlock, R);
    for (int r = r0 + wave_id(); r < r_end; r += blockDim.x / kWave) {
        const int doc = rids[static_cast<size_t>(q) * k_refine + r];
        const int start = doc_ptrs[doc];
        const int end = doc_ptrs[doc + 1];
        float m = -FLT_MAX;
        for (int t = start + half; t < end; t += 2) {
            const uint4 code = *reinterpret_cast<const uint4*>(codes_tok + static_cast<size_t>(t) * kCodeBytes);
            const float f = f1_tok[t];
            float ip = 0.0f;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) ip += llut[(c * kLut + code_nibble(code, c)) * kQ + i];
            m = fmaxf(m, (ip - cb) * f);
        }
        m = fmaxf(m, __shfl_xor(m, 32, kWave));
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) m = m + __shfl_down(m, off, kWave);
        if (l == 0) s1[static_cast<size_t>(q) * k_refine + r] = m;
    }
}

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kRefineMfmaDocsPerBlock = 256;  // at most: 64 per wave of a 256-thread block
static_assert(kRefineMfmaDocsPerBlock / 4 <= kWave, "one document per lane");

// One-bit MaxSim on the matrix cores. For a tile of 16 doc tokens the 32
// one-bit inner products per token are D[16 x 32] = A[16 x 128] * B[128 x 32]
// with A the code bits (0/1 in fp16) and B the rotated query scaled per
// token by a power of two and split into fp16 hi + lo parts; both products
// accumulate into one fp32 accumulator (v_mfma_f32_16x16x32_f16: A lane l
// holds row l%16, k (l/16)*8..+7; B lane l holds column l%16; D lane l holds
// rows (l/16)*4..+3 of column l%16). The split keeps the error of ip near
// 2^-22 of the largest query component; the estimate, the max over tokens
// and the shuffle-down sum over query tokens follow kernels.cu:497-575.
__global__ __launch_bounds__(256) void refine_mfma_kernel(const float* __restrict__ rot,
                                                          const float* __restrict__ cb1,
                                                          const int32_t* __restrict__ rcount,
                                                          const int32_t* __restrict__ rids, int k_refine,
                                                          const int32_t* __restrict__ doc_ptrs,
                                                          const uint8_t* __restrict__ codes_tok,
                                                          const float* __restrict__ f1_tok, float* __restrict__ s1,
                                                          int docs_per_block) {
    // code byte -> 8 fp16 of 0/1 (bit j -> element j), eight copies: lane l
    // reads copy l % 8, so the eight lanes of one 16-byte LDS read cycle use
    // eight different bank groups whatever bytes they look up
    __shared__ uint4 byte2half[256 * 8];
    __shared__ float fstage[4][64];  // per wave: factors of the group on the matrix cores (token tb + lane)
    const int q = blockIdx.x;
    const int r0 = blockIdx.y * docs_per_block;
    const int R = rcount[q];
    if (r0 >= R) return;
    const int l = lane_id();
    for (uint32_t t = threadIdx.x; t < 256u * 8u; t += blockDim.x) {
        const uint32_t e = t >> 3;
        uint32_t hw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            hw[j] = (((e >> (2 * j)) & 1u) ? 0x3C00u : 0u) | (((e >> (2 * j + 1)) & 1u) ? 0x3C000000u : 0u);
        byte2half[t] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    }

    // query operands [kk][half][hi/lo], straight from global memory. Lane
    // group g supplies, in k step kk, the 8 dimensions of code byte 4g + kk
    // (dimensions 32g + 8kk .. +7): one 32-bit word of the code per lane, and
    // a 16-token tile is one contiguous 256-byte read. The four lanes that
    // share a query token c (or 16 + c) hold its 128 dimensions between them,
    // so its largest |component| is their max, and the power-of-two scale
    // 2^s puts it in [512, 1024).
    const int g = l >> 4;   // k group within a 32-wide k step
    const int c = l & 15;   // column (query token within a half) / row (doc token)
    const float* qsrc = rot + static_cast<size_t>(q) * kQ * kDim;
    float qv[2][4][8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int e4 = 0; e4 < 2; ++e4) {
                const float4 v =
                    *reinterpret_cast<const float4*>(qsrc + (16 * h + c) * kDim + 32 * g + 8 * kk + 4 * e4);
                qv[h][kk][4 * e4 + 0] = v.x;
                qv[h][kk][4 * e4 + 1] = v.y;
                qv[h][kk][4 * e4 + 2] = v.z;
                qv[h][kk][4 * e4 + 3] = v.w;
            }
    float inv_scale[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float mx = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(qv[h][kk][e]));
        mx = wave_max_xor32(wave_max_xor16(mx));
        int ex = 0;
        frexpf(mx > 0.0f ? mx : 1.0f, &ex);
        inv_scale[h] = ldexpf(1.0f, ex - 10);
    }
    half8_t bq[4][2][2];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float sc = 1.0f / inv_scale[h];  // a power of two: v * sc is v / 2^-s exactly
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = qv[h][kk][e] * sc;
                const _Float16 hi = static_cast<_Float16>(v);
                bq[kk][h][0][e] = hi;
                bq[kk][h][1][e] = static_cast<_Float16>(v - static_cast<float>(hi));
            }
        }
    const float is0 = inv_scale[0], is1 = inv_scale[1];
    __syncthreads();  // the byte table is complete
    const float cb0 = cb1[q * kQ + c], cb1v = cb1[q * kQ + 16 + c];
    const uint32_t* words = reinterpret_cast<const uint32_t*>(codes_tok);
    const uint4* b2h = byte2half + (l & 7);
    float* fw = fstage[wave_id()];

    // The wave's documents are r0 + w, r0 + w + nw, ... (at most
    // docs_per_block / nw <= 64: one per lane).
    // Their ids and token ranges are loaded once, one per lane, and the wave
    // walks their tokens as one stream of 64-token groups (four 16-token
    // tiles). Three groups are in flight ahead of the one on the matrix
    // cores; a group is one code word per lane and tile plus one factor per
    // lane (token tb + lane), broadcast to the rows through LDS. Rows past a
    // document's end read the tokens after it (the arrays hold
    // kRefinePadTokens more) and are masked. The wave index is a scalar, so
    // the cursors and the groups' base addresses stay in scalar registers.
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int nw = blockDim.x / kWave;
    const int r_end = min(r0 + docs_per_block, R);
    const int ndocs = r0 + w < r_end ? (r_end - (r0 + w) + nw - 1) / nw : 0;
    if (ndocs == 0) return;
    int my_start = 0, my_end = 0;
    if (l < ndocs) {
        const int doc = rids[static_cast<size_t>(q) * k_refine + r0 + w + nw * l];
        my_start = doc_ptrs[doc];
        my_end = doc_ptrs[doc + 1];
    }
    constexpr int kTiles = 4;
    struct Cursor {
        int d, tb, start, end;
    };
    struct Group {
        uint32_t w[kTiles];
        float f;
    };
    auto advance = [&](const Cursor& cu) {
        Cursor n = cu;
        n.tb = cu.tb + 16 * kTiles;
        if (n.tb >= cu.end) {
            n.d = cu.d + 1;
            const int idx = n.d < ndocs ? n.d : 0;
            n.start = __builtin_amdgcn_readlane(my_start, idx);
            n.end = __builtin_amdgcn_readlane(my_end, idx);
            n.tb = n.start;
        }
        return n;
    };
    // The five loads of a group are issued unconditionally (groups past the
    // wave's last document read token 0's), so the compiler can count them
    // in order across the ring: the group's first token as a scalar base,
    // the lanes' offsets as loop constants.
    auto load = [&](const Cursor& cu, Group& gr) {
        const int64_t tb = cu.d < ndocs ? cu.tb : 0;
        const uint32_t* wq = words + tb * 4;
#pragma unroll
        for (int u = 0; u < kTiles; ++u) gr.w[u] = wq[static_cast<uint32_t>((16 * u + c) * 4 + g)];
        gr.f = (f1_tok + tb)[static_cast<uint32_t>(l)];
    };
    // A tile's LDS traffic (four byte lookups, four factor shuffles) is
    // issued one tile ahead of its matrix-core work, so its latency hides
    // behind the previous tile.
    struct TileIn {
        uint4 a[4];
        float f[4];
    };
    auto fetch_tile = [&](uint32_t word, float fgroup, int u, TileIn& ti) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) ti.a[kk] = b2h[((word >> (8 * kk)) & 0xFFu) * 8];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) ti.f[rr] = fw[16 * u + 4 * g + rr];
    };
    // The accumulators start at -cb1 * 2^s, so they end at (ip - cb1) * 2^s;
    // with the factor f > 0 and the power of two 2^-s common to a query
    // token's column, max over rows of (ip - cb1) * f is 2^-s times the max
    // of acc * f, and the scale is applied once per document (finalize).
    const float cbs0 = -cb0 / is0, cbs1 = -cb1v / is1;
    auto run_tile = [&](const TileIn& ti, float& m0v, float& m1v, auto full, int rows_left) {
        float4_t acc0 = {cbs0, cbs0, cbs0, cbs0}, acc1 = {cbs1, cbs1, cbs1, cbs1};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            half8_t a;
            __builtin_memcpy(&a, &ti.a[kk], sizeof(a));
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][0][0], acc0, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][0][1], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][1][0], acc1, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][1][1], acc1, 0, 0, 0);
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (decltype(full)::value || 4 * g + rr < rows_left) {
                m0v = fmaxf(m0v, acc0[rr] * ti.f[rr]);
                m1v = fmaxf(m1v, acc1[rr] * ti.f[rr]);
            }
        }
    };
    auto compute = [&](const Group& gr, const Cursor& cu, float& m0v, float& m1v) {
        // the group's factors go through the wave's LDS row: a tile's rows
        // read theirs back as four consecutive words
        fw[l] = gr.f;
        wave_lds_sync();
        TileIn tin[2];
        if (cu.tb + 16 * kTiles <= cu.end) {
            fetch_tile(gr.w[0], gr.f, 0, tin[0]);
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                if (u + 1 < kTiles) fetch_tile(gr.w[u + 1], gr.f, u + 1, tin[(u + 1) & 1]);
                run_tile(tin[u & 1], m0v, m1v, std::true_type{}, 16);
            }
        } else {
            // the document's last group: whole tiles unmasked, then the one
            // tile that crosses its end (its rows past the end see word 0)
            auto word_of = [&](int u) {
                const int tt = cu.tb + 16 * u;
                return tt + c < cu.end ? gr.w[u] : 0u;
            };
            fetch_tile(word_of(0), gr.f, 0, tin[0]);
#pragma unroll
            for (int u = 0; u < kTiles; ++u) {
                const int tt = cu.tb + 16 * u;
                if (tt >= cu.end) break;
                if (u + 1 < kTiles && tt + 16 < cu.end) fetch_tile(word_of(u + 1), gr.f, u + 1, tin[(u + 1) & 1]);
                if (tt + 16 <= cu.end)
                    run_tile(tin[u & 1], m0v, m1v, std::true_type{}, 16);
                else
                    run_tile(tin[u & 1], m0v, m1v, std::false_type{}, cu.end - tt);
            }
        }
    };
    float m0 = -FLT_MAX, m1 = -FLT_MAX;
    auto finalize = [&](int d) {
        // max over the four lane groups, then the sum over the 32 query
        // tokens by the shuffle-down tree 8, 4, 2, 1 (lane-swap and DPP
        // steps: no LDS round trips)
        const float a0 = wave_max_xor32(wave_max_xor16(m0)) * is0;
        const float a1 = wave_max_xor32(wave_max_xor16(m1)) * is1;
        float sum = a0 + a1;  // tokens c and c + 16
        sum = row_add_down<8>(sum);
        sum = row_add_down<4>(sum);
        sum = row_add_down<2>(sum);
        sum = row_add_down<1>(sum);
        if (l == 0) s1[static_cast<size_t>(q) * k_refine + r0 + w + nw * d] = sum;
        m0 = -FLT_MAX;
        m1 = -FLT_MAX;
    };
    // one step on ring slot (G, C): C is the group on the matrix cores, Cn
    // the next one, Cf the furthest loaded; the slot is then refilled with
    // the group after Cf. The loop below is unrolled by the ring size so each
    // slot keeps its registers and no in-flight load is copied.
    auto step = [&](Group& G, Cursor& C, const Cursor& Cn, const Cursor& Cf) {
        compute(G, C, m0, m1);
        if (Cn.d != C.d) finalize(C.d);
        C = advance(Cf);
        load(C, G);
    };
    Cursor c0{0, 0, 0, 0};
    c0.start = __builtin_amdgcn_readlane(my_start, 0);
    c0.end = __builtin_amdgcn_readlane(my_end, 0);
    c0.tb = c0.start;
    Cursor c1 = advance(c0);
    Cursor c2 = advance(c1);
    Group g0{}, g1{}, g2{};
    load(c0, g0);
    load(c1, g1);
    load(c2, g2);
    while (true) {
        if (c0.d >= ndocs) break;
        step(g0, c0, c1, c2);
        if (c1.d >= ndocs) break;
        step(g1, c1, c2, c0);
        if (c2.d >= ndocs) break;
        step(g2, c2, c0, c1);
    }
}

namespace {

__device__ __forceinline__ uint32_t lds32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
// rotate right by n mod 32 (v_alignbit_b32): with n = b - c (mod 32) and
// b, c < 8, bit b of every byte lands at bit c of the same byte
__device__ __forceinline__ uint32_t rotr(uint32_t x, uint32_t n) { return __builtin_amdgcn_alignbit(x, x, n); }

// The W-bit code values of one token for the four k steps of a 16-token
// tile, in the packing layouts of pack_excode.hpp (unpacked as
// space.hpp:604-801): v[kk][0] holds elements 0..3 of lane group g's A
// operand in step kk, v[kk][1] elements 4..7, one value per byte. Which
// dimension element e of (kk, g) carries is code_dim<W>: each lane takes
// whole 32-bit words of the packed code, so that a word (with a word of the
// top bit plane, rotated so the plane's bit lands in place) gives four
// values by a mask or two. The query operand is laid out by the same
// code_dim, so each product pairs a code value with its own dimension.
//   W = 2, 8: dimension 32 kk + 8 g + e (the layouts' own order)
//   W = 4, 6: 16-dimension group G = 2 kk + g/2, word h = g % 2 of its
//             nibble bytes: low nibbles are dimensions 16 G + 4 h + i, high
//             nibbles 16 G + 8 + 4 h + i
//   W = 3, 5: 64-dimension block kk / 2, word g of its low part: the values
//             of dimensions 32 (kk % 2) + 4 g + i and 32 (kk % 2) + 16 + 4 g + i
//   W = 7:    8-dimension groups in their order, the two groups per block
//             whose low bits sit in bits 6-7 of three bytes all in step 3
template <int W>
__device__ __forceinline__ int code_dim(int kk, int g, int e) {
    if constexpr (W == 2 || W == 8) {
        return 32 * kk + 8 * g + e;
    } else if constexpr (W == 4 || W == 6) {
        const int G = 2 * kk + (g >> 1), h = g & 1;
        return 16 * G + 4 * h + (e < 4 ? e : 8 + e - 4);
    } else if constexpr (W == 3 || W == 5) {
        return 64 * (kk >> 1) + 32 * (kk & 1) + 4 * g + (e < 4 ? e : 16 + e - 4);
    } else {
        const int n = 4 * kk + g;
        const int blk = kk < 3 ? n / 6 : g >> 1;
        const int grp = kk < 3 ? n % 6 : 6 + (g & 1);
        return 64 * blk + 8 * grp + e;
    }
}

template <int W>
__device__ __forceinline__ void code_values(const uint8_t* p, int g, uint32_t (&v)[4][2]) {
    constexpr uint32_t k2 = 0x03030303u, k4 = 0x0F0F0F0Fu;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        if constexpr (W == 8) {
            v[kk][0] = lds32(p + 32 * kk + 8 * g);
            v[kk][1] = lds32(p + 32 * kk + 8 * g + 4);
        } else if constexpr (W == 2) {  // per 16 dims 4 bytes: byte m bits 2k.. = dim 4k + m
            const uint32_t w = lds32(p + 8 * kk + 4 * (g >> 1));
            const int h = g & 1;
            v[kk][0] = (w >> (4 * h)) & k2;
            v[kk][1] = (w >> (4 * h + 2)) & k2;
        } else if constexpr (W == 4) {  // per 16 dims 8 bytes: byte m = dim m | dim 8 + m << 4
            const uint32_t w = lds32(p + 8 * (2 * kk + (g >> 1)) + 4 * (g & 1));
            v[kk][0] = w & k4;
            v[kk][1] = (w >> 4) & k4;
        } else if constexpr (W == 6) {  // per 16 dims the 8 nibble bytes, then 4 bytes of bits 4-5
            const uint8_t* q = p + 12 * (2 * kk + (g >> 1));  // (byte m bits 2k.. = dim 4k + m)
            const uint32_t w = lds32(q + 4 * (g & 1));
            const uint32_t t = lds32(q + 8);
            const int h = g & 1;
            v[kk][0] = (w & k4) | ((t << (4 - 2 * h)) & 0x30303030u);
            v[kk][1] = ((w >> 4) & k4) | ((t >> (2 * h)) & 0x30303030u);
        } else if constexpr (W == 5) {  // per 64 dims: bytes 16s + m = dim 32s + m | dim 32s + 16 + m << 4,
            const uint8_t* q = p + 40 * (kk >> 1);  // then the top bits (byte j bit b = dim 8b + j)
            const int s = kk & 1;
            const uint32_t w = lds32(q + 16 * s + 4 * g);
            const uint32_t t = lds32(q + 32 + 4 * (g & 1));
            const uint32_t b = static_cast<uint32_t>(4 * s + (g >> 1));
            v[kk][0] = (w & k4) | (rotr(t, b - 4u) & 0x10101010u);
            v[kk][1] = ((w >> 4) & k4) | (rotr(t, b - 2u) & 0x10101010u);
        } else if constexpr (W == 3) {  // per 64 dims: bytes m bits 2k.. = dim 16k + m, then the top bits
            const uint8_t* q = p + 24 * (kk >> 1);
            const int s = kk & 1;
            const uint32_t w = lds32(q + 4 * g);
            const uint32_t t = lds32(q + 16 + 4 * (g & 1));
            const uint32_t b = static_cast<uint32_t>(4 * s + (g >> 1));
            v[kk][0] = ((w >> (4 * s)) & k2) | (rotr(t, b - 2u) & 0x04040404u);
            v[kk][1] = ((w >> (4 * s + 2)) & k2) | (rotr(t, b) & 0x04040404u);
        } else {  // W = 7, per 64 dims: bytes 0..47 bits 0-5 = dims 0..47; dims 48..63 in bits 6-7 of
                  // bytes j, 16 + j, 32 + j (two bits each); then the top bits
            if (kk < 3) {
                const int n = 4 * kk + g;
                const uint8_t* q = p + 56 * (n / 6);
                const int grp = n % 6;
                const uint32_t r = static_cast<uint32_t>(grp - 6);
                v[kk][0] = (lds32(q + 8 * grp) & 0x3F3F3F3Fu) | (rotr(lds32(q + 48), r) & 0x40404040u);
                v[kk][1] = (lds32(q + 8 * grp + 4) & 0x3F3F3F3Fu) | (rotr(lds32(q + 52), r) & 0x40404040u);
            } else {
                const uint8_t* q = p + 56 * (g >> 1);
                const uint32_t r = static_cast<uint32_t>(g & 1);  // group 6 + (g & 1): top bit b - 6
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int c = 8 * (g & 1) + 4 * h;
                    v[kk][h] = ((lds32(q + c) >> 6) & k2) | ((lds32(q + c + 16) >> 4) & 0x0C0C0C0Cu) |
                               ((lds32(q + c + 32) >> 2) & 0x30303030u) | (rotr(lds32(q + 48 + 4 * h), r) & 0x40404040u);
                }
            }
        }
    }
}

// Eight byte values (< 256) to eight exact fp16 denormals (bits 0x00xx,
// value xx * 2^-24): one byte permute per two values, no arithmetic.
// Products with them and their sums are the ordinary encoding's scaled by
// 2^-24 up to the matrix cores' fp32 rounding; the accumulators start at
// 2^-24 times their value and the scale is undone once per document.
__device__ __forceinline__ half8_t bytes_to_denormals(uint32_t lo, uint32_t hi) {
    uint32_t u[4];
    u[0] = __builtin_amdgcn_perm(lo, lo, 0x0C010C00u);
    u[1] = __builtin_amdgcn_perm(lo, lo, 0x0C030C02u);
    u[2] = __builtin_amdgcn_perm(hi, hi, 0x0C010C00u);
    u[3] = __builtin_amdgcn_perm(hi, hi, 0x0C030C02u);
    half8_t h;
    __builtin_memcpy(&h, u, sizeof(h));
    return h;
}

}  // namespace

constexpr int kFullbitMfmaDocsPerBlock = 32;  // at most: 8 per wave

__device__ __forceinline__ __attribute__((address_space(3))) void* to_lds(void* p) {
    return (__attribute__((address_space(3))) void*)(p);
}

// s_waitcnt vmcnt(n), expcnt and lgkmcnt not waited on (vmcnt in bits
// [3:0] and [15:14])
constexpr int waitcnt_vmcnt(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

// Full-bit MaxSim on the matrix cores. For a tile of 16 doc tokens,
// D[16 x 32] = A[16 x 128] * B[128 x 32] with A the W-bit code values (fp16
// denormals, exact) and B the rotated query scaled per token by a power of
// two and split into fp16 hi + lo, as in the one-bit refine (lane layout of
// v_mfma_f32_16x16x32_f16 above; lane group g supplies dimensions
// code_dim<W>(kk, g, 0..7) in k step kk). Products are exact and accumulate
// in fp32, so ip = <c, q> carries the split's error (about 2^-22 of the
// largest query component per term) and fp32 rounding, like the reference's
// fp32 AVX-512 sums. Estimate, max and the sum over query tokens follow
// search_impl.cu:538-572: (ip - cbex) * f, max over tokens, max[m] +
// max[m+16], then a 8,4,2,1 tree.
//
// A wave walks its documents (j0 + w, j0 + w + 4, ...) as one stream of
// 16-token tiles. A tile's codes (16 * 16W contiguous bytes in token order)
// and its 16 factors go from global memory straight into LDS
// (global_load_lds, no registers on the way) into one of four slots of the
// wave, three tiles ahead of the tile on the matrix cores; the slots are
// separately declared arrays and the loop is unrolled by four, so each
// slot's reads depend only on its own loads, which an explicit vmcnt wait
// covers. Rows past a document's end are left out of the max.
template <int W>
__global__ __launch_bounds__(256) void fullbit_mfma_kernel(const float* __restrict__ rot,
                                                           const float* __restrict__ cbex,
                                                           const int32_t* __restrict__ fcount,
                                                           const int32_t* __restrict__ fids, int fb_cap,
                                                           const int32_t* __restrict__ doc_ptrs,
                                                           const uint8_t* __restrict__ full_codes,
                                                           const float* __restrict__ full_factors,
                                                           float* __restrict__ fscores, int docs_per_block) {
    constexpr int kCodeBytes = 256 * W;             // 16 tokens x 16W bytes
    constexpr int kSlot = kCodeBytes + 64;          // + 16 factors
    constexpr int kCodeLoads = (16 * W + 63) / 64;  // 16-byte loads of a wave per tile
    constexpr int kTileLoads = kCodeLoads + 1;
    constexpr int kWaves = 4;
    __shared__ __align__(16) uint8_t ring0[kWaves][kSlot];
    __shared__ __align__(16) uint8_t ring1[kWaves][kSlot];
    __shared__ __align__(16) uint8_t ring2[kWaves][kSlot];
    __shared__ __align__(16) uint8_t ring3[kWaves][kSlot];
    const int q = blockIdx.x;
    const int j0 = blockIdx.y * docs_per_block;
    const int nf = fcount[q];
    if (j0 >= nf) return;
    const int l = lane_id();
    const int g = l >> 4;
    const int c = l & 15;
    // The query operand straight from global memory (no LDS copy, which
    // leaves the LDS to the tile ring): lane (g, c) loads the 32 dimensions
    // code_dim<W>(kk, g, .) of query tokens c and 16 + c, four consecutive
    // ones per 16-byte load. Each token's largest |component| is the max
    // over the four lanes that share c; its power-of-two scale puts it in
    // [512, 1024).
    float qv[2][4][8];
    const float* qsrc = rot + static_cast<size_t>(q) * kQ * kDim;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int e4 = 0; e4 < 2; ++e4) {
                const float4 v =
                    *reinterpret_cast<const float4*>(qsrc + (16 * h + c) * kDim + code_dim<W>(kk, g, 4 * e4));
                qv[h][kk][4 * e4 + 0] = v.x;
                qv[h][kk][4 * e4 + 1] = v.y;
                qv[h][kk][4 * e4 + 2] = v.z;
                qv[h][kk][4 * e4 + 3] = v.w;
            }
    float inv_scale[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float mx = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(qv[h][kk][e]));
        mx = wave_max_xor32(wave_max_xor16(mx));
        int ex = 0;
        frexpf(mx > 0.0f ? mx : 1.0f, &ex);
        inv_scale[h] = ldexpf(1.0f, ex - 10);
    }
    half8_t bq[4][2][2];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float sc = 1.0f / inv_scale[h];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = qv[h][kk][e] * sc;
                const _Float16 hi = static_cast<_Float16>(v);
                bq[kk][h][0][e] = hi;
                bq[kk][h][1][e] = static_cast<_Float16>(v - static_cast<float>(hi));
            }
        }
    // The accumulators start at -cbex * 2^s * 2^-24, so with the code values
    // as denormals (x * 2^-24) they end at (ip - cbex) * 2^s * 2^-24; with
    // f > 0 and 2^-s common to a query token's column, the max over rows of
    // (ip - cbex) * f is 2^(24 - s) times the max of acc * f (scale applied
    // per document; every factor is a power of two).
    const float is0 = inv_scale[0] * 0x1p24f, is1 = inv_scale[1] * 0x1p24f;
    const float cb0 = cbex[q * kQ + c], cb1v = cbex[q * kQ + 16 + c];
    const float cbs0 = -cb0 / is0, cbs1 = -cb1v / is1;

    // the wave index as a scalar, so that the cursors, the buffer bases and
    // the LDS slots below stay in scalar registers
    const int w = __builtin_amdgcn_readfirstlane(wave_id());
    const int j_end = min(j0 + docs_per_block, nf);
    const int ndocs = j0 + w < j_end ? (j_end - (j0 + w) + kWaves - 1) / kWaves : 0;
    if (ndocs == 0) return;
    int my_start = 0, my_end = 0;
    if (l < ndocs) {
        const int doc = fids[static_cast<size_t>(q) * fb_cap + j0 + w + kWaves * l];
        my_start = doc_ptrs[doc];
        my_end = doc_ptrs[doc + 1];
    }
    struct Cursor {
        int d, t0, start, end;
    };
    auto advance = [&](const Cursor& cu) {
        Cursor n = cu;
        n.t0 = cu.t0 + 16;
        if (n.t0 >= cu.end) {
            n.d = cu.d + 1;
            const int idx = n.d < ndocs ? n.d : 0;
            n.start = __builtin_amdgcn_readlane(my_start, idx);
            n.end = __builtin_amdgcn_readlane(my_end, idx);
            n.t0 = n.start;
        }
        return n;
    };
    // exactly kTileLoads load instructions per tile, each with active lanes;
    // the tile's first token as a scalar base and the lanes' offsets as loop
    // constants (the arrays hold kFullbitPadTokens tokens past the last one,
    // so a tile that crosses the end stays in bounds)
    auto fetch = [&](const Cursor& cu, uint8_t* slot) {
        const int64_t t0 = cu.d < ndocs ? cu.t0 : 0;
        const uint8_t* codes = full_codes + t0 * (16 * W);
#pragma unroll
        for (int i = 0; i < kCodeLoads; ++i) {
            constexpr int kLastLanes = 16 * W - 64 * (kCodeLoads - 1);
            if (i + 1 < kCodeLoads || kLastLanes == 64 || l < kLastLanes)
                __builtin_amdgcn_global_load_lds(codes + static_cast<uint32_t>(1024 * i + 16 * l),
                                                 to_lds(slot + 1024 * i), 16, 0, 0);
        }
        if (l < 16)
            __builtin_amdgcn_global_load_lds(full_factors + t0 + static_cast<uint32_t>(l), to_lds(slot + kCodeBytes), 4,
                                             0, 0);
    };
    float m0 = -FLT_MAX, m1 = -FLT_MAX;
    auto compute = [&](const Cursor& cu, const uint8_t* slot) {
        uint32_t cv[4][2];
        code_values<W>(slot + c * (16 * W), g, cv);
        const float4 f4 = *reinterpret_cast<const float4*>(slot + kCodeBytes + 16 * g);
        const float fr[4] = {f4.x, f4.y, f4.z, f4.w};
        // rows past the document's end hold the next tokens' codes (finite);
        // the epilogue leaves them out of the max
        float4_t acc0 = {cbs0, cbs0, cbs0, cbs0}, acc1 = {cbs1, cbs1, cbs1, cbs1};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const half8_t a = bytes_to_denormals(cv[kk][0], cv[kk][1]);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][0][0], acc0, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][0][1], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][1][0], acc1, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[kk][1][1], acc1, 0, 0, 0);
        }
        if (cu.t0 + 16 <= cu.end) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                m0 = fmaxf(m0, acc0[rr] * fr[rr]);
                m1 = fmaxf(m1, acc1[rr] * fr[rr]);
            }
        } else {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                if (cu.t0 + 4 * g + rr < cu.end) {
                    m0 = fmaxf(m0, acc0[rr] * fr[rr]);
                    m1 = fmaxf(m1, acc1[rr] * fr[rr]);
                }
            }
        }
    };
    auto finalize = [&](int d) {
        const float a0 = wave_max_xor32(wave_max_xor16(m0)) * is0;
        const float a1 = wave_max_xor32(wave_max_xor16(m1)) * is1;
        float sum = a0 + a1;  // query tokens c and c + 16, then the 8, 4, 2, 1 tree
        sum = row_add_down<8>(sum);
        sum = row_add_down<4>(sum);
        sum = row_add_down<2>(sum);
        sum = row_add_down<1>(sum);
        if (l == 0) fscores[static_cast<size_t>(q) * fb_cap + j0 + w + kWaves * d] = sum;
        m0 = -FLT_MAX;
        m1 = -FLT_MAX;
    };
    // one step on slot S: its tile C has landed once at most the loads of the
    // three tiles issued after it are outstanding; then the slot is refilled
    // with the tile after the furthest one (Cf)
    auto step = [&](uint8_t* S, Cursor& C, const Cursor& Cn, const Cursor& Cf) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vmcnt(3 * kTileLoads));
        compute(C, S);
        if (Cn.d != C.d) finalize(C.d);
        C = advance(Cf);
        fetch(C, S);
    };
    Cursor c0{0, 0, 0, 0};
    c0.start = __builtin_amdgcn_readlane(my_start, 0);
    c0.end = __builtin_amdgcn_readlane(my_end, 0);
    c0.t0 = c0.start;
    Cursor c1 = advance(c0);
    Cursor c2 = advance(c1);
    Cursor c3 = advance(c2);
    uint8_t* s0 = ring0[w];
    uint8_t* s1 = ring1[w];
    uint8_t* s2 = ring2[w];
    uint8_t* s3 = ring3[w];
    fetch(c0, s0);
    fetch(c1, s1);
    fetch(c2, s2);
    fetch(c3, s3);
    while (true) {
        if (c0.d >= ndocs) break;
        step(s0, c0, c1, c3);
        if (c1.d >= ndocs) break;
        step(s1, c1, c2, c0);
        if (c2.d >= ndocs) break;
        step(s2, c2, c3, c1);
        if (c3.d >= ndocs) break;
        step(s3, c3, c0, c2);
    }
    // the ring's last loads land before the wave ends
    __builtin_amdgcn_s_waitcnt(waitcnt_vmcnt(0));
}

// Chunked full-bit selection (search_impl.cu:341-494): chunks are contiguous
// slices of the refined list; after chunk c the top min(F(c+1)/n_ch, F, end_c)
// documents by S1 among the first end_c refined documents are selected. The
// union over chunks is scored. Ties: lower refined index first.
__global__ __launch_bounds__(1024) void chunk_select_kernel(const float* __restrict__ s1,
                                                            const int32_t* __restrict__ rcount,
                                                            const int32_t* __restrict__ rids, int k_refine,
                                                            int k_full_bit, int num_chunks, int sort_cap,
                                                            int fb_cap, int32_t* __restrict__ fcount,
                                                            int32_t* __restrict__ fids, uint32_t* __restrict__ err) {
    extern __shared__ uint64_t keys[];  // [sort_cap], then sel flags
    uint8_t* sel = reinterpret_cast<uint8_t*>(keys + sort_cap);
    __shared__ int scratch[17];
    const int q = blockIdx.x;
    const int R = rcount[q];
    if (R == 0) {
        if (threadIdx.x == 0) fcount[q] = 0;
        return;
    }
    const float* sq = s1 + static_cast<size_t>(q) * k_refine;
    for (int t = threadIdx.x; t < sort_cap; t += blockDim.x) {
        keys[t] = t < R ? (static_cast<uint64_t>(~float_to_ordered(sq[t])) << 32) | static_cast<uint32_t>(t) : ~0ull;
        sel[t] = 0;
    }
    __syncthreads();
    block_sort_u64(keys, sort_cap);
    const int F = min(k_full_bit, R);
    const int nch = min(num_chunks, R);
    const int cs = (R + nch - 1) / nch;
    // The chunks' walks by wave 0 alone (64 sorted keys per step, ranks by
    // ballot, no block barriers): chunk c marks the first tgt keys in sorted
    // order whose refined index lies below its end.
    if (wave_id() == 0) {
        const int l = lane_id();
        const uint64_t below = (1ull << l) - 1ull;
        for (int c = 0; c < nch; ++c) {
            const int end = min((c + 1) * cs, R);
            const int tgt = min(static_cast<int>(static_cast<int64_t>(F) * (c + 1) / nch), min(F, end));
            int carry = 0;
            for (int base = 0; base < R && carry < tgt; base += kWave) {
                const int s = base + l;
                const int r = s < R ? static_cast<int>(keys[s] & 0xFFFFFFFFu) : 0;
                const bool mark = s < R && r < end;
                const uint64_t bal = __ballot(mark);
                if (mark && carry + __popcll(bal & below) < tgt) sel[r] = 1;
                carry += __popcll(bal);
            }
        }
    }
    __syncthreads();
    // the selected documents in refined order: thread t takes the per
    // consecutive refined indices from t * per, one block scan of the counts
    const int per = (R + static_cast<int>(blockDim.x) - 1) / static_cast<int>(blockDim.x);
    const int r0 = static_cast<int>(threadIdx.x) * per;
    int mine = 0;
    for (int r = r0; r < r0 + per && r < R; ++r) mine += sel[r];
    int tot;
    int pos = block_inclusive_scan_shared(mine, scratch, &tot) - mine;
    for (int r = r0; r < r0 + per && r < R; ++r) {
        if (!sel[r]) continue;
        if (pos < fb_cap) {
            fids[static_cast<size_t>(q) * fb_cap + pos] = rids[static_cast<size_t>(q) * k_refine + r];
        } else {
            atomicOr(err, kErrFullbitCap);
        }
        ++pos;
    }
    if (threadIdx.x == 0) fcount[q] = min(tot, fb_cap);
}

constexpr int kFullbitDocsPerBlock = 16;

// Full-bit MaxSim with the reference's float order (search_impl.cu:538-572,
// gemv_batch8_avx512): per query token, 16 fma chains over dims m, m+16, ...,
// reduced 8,4,2,1; (ip - cbex) * f; max from -inf; the 32 maxima summed as
// max[m] + max[m+16] then reduced 8,4,2,1. One wave per document; lanes 0-31
// take even tokens, 32-63 odd tokens; codes are unpacked into LDS once per
// token pair and read back as broadcasts.
__global__ __launch_bounds__(256) void fullbit_kernel(const float* __restrict__ rot, const float* __restrict__ cbex,
                                                      const int32_t* __restrict__ fcount,
                                                      const int32_t* __restrict__ fids, int fb_cap,
                                                      const int32_t* __restrict__ doc_ptrs,
                                                      const uint8_t* __restrict__ full_codes,
                                                      const float* __restrict__ full_factors, int width,
                                                      float* __restrict__ fscores) {
    __shared__ float dec[4][2][kDim];
    const int q = blockIdx.x;
    const int j0 = blockIdx.y * kFullbitDocsPerBlock;
    const int nf = fcount[q];
    if (j0 >= nf) return;
    const int l = lane_id();
    const int w = wave_id();
    const int i = l & 31;
    const int half = l >> 5;
    float qv[kDim];
    const float4* qsrc = reinterpret_cast<const float4*>(rot + (static_cast<size_t>(q) * kQ + i) * kDim);
#pragma unroll
    for (int j4 = 0; j4 < kDim / 4; ++j4) {
        const float4 v = qsrc[j4];
        qv[4 * j4 + 0] = v.x;
        qv[4 * j4 + 1] = v.y;
        qv[4 * j4 + 2] = v.z;
        qv[4 * j4 + 3] = v.w;
    }
    const float cb = cbex[q * kQ + i];
    const size_t stride = static_cast<size_t>(16 * width);
    const int j_end = min(j0 + kFullbitDocsPerBlock, nf);
    for (int j = j0 + w; j < j_end; j += blockDim.x / kWave) {
        const int doc = fids[static_cast<size_t>(q) * fb_cap + j];
        const int start = doc_ptrs[doc];
        const int end = doc_ptrs[doc + 1];
        float mx = -INFINITY;
        for (int t = start; t < end; t += 2) {
            // unpack tokens t and t+1: lane decodes dims 4*(l&31) .. +3 of token t + half
            const int tt = t + half;
            if (tt < end) {
                const uint8_t* p = full_codes + static_cast<size_t>(tt) * stride;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int dim = 4 * i + k;
                    dec[w][half][dim] = static_cast<float>(unpack_dim_w(p, width, dim));
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (tt < end) {
                const float* d = dec[w][half];
                float p16[16];
#pragma unroll
                for (int m = 0; m < 16; ++m) p16[m] = 0.0f;
#pragma unroll
                for (int s = 0; s < kDim / 16; ++s)
#pragma unroll
                    for (int m = 0; m < 16; ++m) p16[m] = __fmaf_rn(d[16 * s + m], qv[16 * s + m], p16[m]);
#pragma unroll
                for (int off = 8; off >= 1; off >>= 1)
#pragma unroll
                    for (int m = 0; m < off; ++m) p16[m] = p16[m] + p16[m + off];
                const float combined = (p16[0] - cb) * full_factors[tt];
                mx = fmaxf(mx, combined);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        float s = mx + __shfl_down(mx, 16, kWave);  // lanes 0..15: max[m] + max[m+16]
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) s = s + __shfl_down(s, off, kWave);
        if (l == 0) fscores[static_cast<size_t>(q) * fb_cap + j] = s;
    }
}

// Final top-k (one 1,024-thread block per query): sort (SF, doc) descending.
__global__ __launch_bounds__(1024) void final_topk_kernel(const int32_t* __restrict__ fcount,
                                                         const int32_t* __restrict__ fids,
                                                         const float* __restrict__ fscores, int fb_cap,
                                                         int sort_cap, int k, int64_t* __restrict__ out_ids,
                                                         float* __restrict__ out_scores,
                                                         int32_t* __restrict__ out_counts) {
    extern __shared__ uint64_t keys[];
    const int q = blockIdx.x;
    const int cnt = fcount[q];
    const int n = cnt < 0 ? 0 : (cnt < fb_cap ? cnt : fb_cap);
    for (int t = threadIdx.x; t < sort_cap; t += blockDim.x) {
        // ascending sort of ~(score, doc) == descending (score, doc)
        keys[t] = t < n ? ~((static_cast<uint64_t>(float_to_ordered(fscores[static_cast<size_t>(q) * fb_cap + t])) << 32) |
                            static_cast<uint32_t>(fids[static_cast<size_t>(q) * fb_cap + t]))
                        : ~0ull;
    }
    __syncthreads();
    block_sort_u64(keys, sort_cap);
    const int kk = min(k, n);
    for (int t = threadIdx.x; t < k; t += blockDim.x) {
        if (t < kk) {
            const uint64_t v = ~keys[t];
            out_ids[static_cast<size_t>(q) * k + t] = static_cast<int64_t>(static_cast<uint32_t>(v & 0xFFFFFFFFu));
            if (out_scores) out_scores[static_cast<size_t>(q) * k + t] = ordered_to_float(static_cast<uint32_t>(v >> 32));
        } else {
            out_ids[static_cast<size_t>(q) * k + t] = -1;
            if (out_scores) out_scores[static_cast<size_t>(q) * k + t] = 0.0f;
        }
    }
    if (threadIdx.x == 0) out_counts[q] = kk;
}

// ---- launchers ----

hipError_t configure_score_kernels(int k_refine, int fb_cap) {
    hipError_t e = hipSuccess;
    const int cs_shm = pow2_at_least(k_refine < 2 ? 2 : k_refine) * 9;
    if (cs_shm > 64 * 1024)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(chunk_select_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, cs_shm);
    if (e != hipSuccess) return e;
    const int fin_shm = pow2_at_least(fb_cap < 2 ? 2 : fb_cap) * 8;
    if (fin_shm > 64 * 1024)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(final_topk_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, fin_shm);
    return e;
}

hipError_t configure_kernels(int nbk, int nprobe, int k_refine, int fb_cap) {
    hipError_t e = configure_query_kernels(nprobe);
    if (e != hipSuccess) return e;
    e = configure_candidate_kernels(nbk, k_refine);
    if (e != hipSuccess) return e;
    return configure_score_kernels(k_refine, fb_cap);
}

hipError_t launch_refine_lut(hipStream_t s, int nq, int k_refine, const float* lut, const float* cb1,
                             const int32_t* rcount, const int32_t* rids, const int32_t* doc_ptrs,
                             const uint8_t* codes_tok, const float* f1_tok, float* s1) {
    const dim3 grid(nq, (k_refine + kRefineDocsPerBlock - 1) / kRefineDocsPerBlock);
    hipLaunchKernelGGL(refine_lut_kernel, grid, dim3(256), kLutPerQuery * sizeof(float), s, lut, cb1, rcount, rids,
                       k_refine, doc_ptrs, codes_tok, f1_tok, s1);
    return hipGetLastError();
}

// Documents per block: the most (a multiple of 4 waves) that still gives a
// small batch at least 4 blocks per CU, down to min_dpb; large batches keep
// max_dpb (each block first stages its query).
static int score_docs_per_block(int nq, int n_docs, int num_cus, int max_dpb, int min_dpb) {
    int dpb = max_dpb;
    while (dpb > min_dpb && static_cast<int64_t>(nq) * ((n_docs + dpb - 1) / dpb) < 4 * static_cast<int64_t>(num_cus))
        dpb /= 2;
    return dpb;
}

hipError_t launch_refine_mfma(hipStream_t s, int nq, int k_refine, const float* rot, const float* cb1,
                              const int32_t* rcount, const int32_t* rids, const int32_t* doc_ptrs,
                              const uint8_t* codes_tok, const float* f1_tok, float* s1, int num_cus) {
    const int dpb = score_docs_per_block(nq, k_refine, num_cus, kRefineMfmaDocsPerBlock, 16);
    const dim3 grid(nq, (k_refine + dpb - 1) / dpb);
    hipLaunchKernelGGL(refine_mfma_kernel, grid, dim3(256), 0, s, rot, cb1, rcount, rids, k_refine, doc_ptrs,
                       codes_tok, f1_tok, s1, dpb);
    return hipGetLastError();
}

hipError_t launch_chunk_select(hipStream_t s, int nq, const float* s1, const int32_t* rcount, const int32_t* rids,
                               int k_refine, int k_full_bit, int num_chunks, int fb_cap, int32_t* fcount,
                               int32_t* fids, uint32_t* err) {
    const int sort_cap = pow2_at_least(k_refine < 2 ? 2 : k_refine);
    const size_t shm = static_cast<size_t>(sort_cap) * 9;
    hipLaunchKernelGGL(chunk_select_kernel, dim3(nq), dim3(1024), shm, s, s1, rcount, rids, k_refine, k_full_bit,
                       num_chunks, sort_cap, fb_cap, fcount, fids, err);
    return hipGetLastError();
}

hipError_t launch_fullbit(hipStream_t s, int nq, const float* rot, const float* cbex, const int32_t* fcount,
                          const int32_t* fids, int fb_cap, const int32_t* doc_ptrs, const uint8_t* full_codes,
                          const float* full_factors, int width, float* fscores) {
    const dim3 grid(nq, (fb_cap + kFullbitDocsPerBlock - 1) / kFullbitDocsPerBlock);
    hipLaunchKernelGGL(fullbit_kernel, grid, dim3(256), 0, s, rot, cbex, fcount, fids, fb_cap, doc_ptrs, full_codes,
                       full_factors, width, fscores);
    return hipGetLastError();
}

hipError_t launch_fullbit_mfma(hipStream_t s, int nq, const float* rot, const float* cbex, const int32_t* fcount,
                               const int32_t* fids, int fb_cap, const int32_t* doc_ptrs, const uint8_t* full_codes,
                               const float* full_factors, int width, float* fscores, int num_cus) {
    const int dpb = score_docs_per_block(nq, fb_cap, num_cus, kFullbitMfmaDocsPerBlock, 4);
    const dim3 grid(nq, (fb_cap + dpb - 1) / dpb);
#define CHIMERA_FULLBIT_MFMA(WW)                                                                                   \
    case WW:                                                                                                       \
        hipLaunchKernelGGL(fullbit_mfma_kernel<WW>, grid, dim3(256), 0, s, rot, cbex, fcount, fids, fb_cap, doc_ptrs, \
                           full_codes, full_factors, fscores, dpb);                                                \
        break;
    switch (width) {
        CHIMERA_FULLBIT_MFMA(2)
        CHIMERA_FULLBIT_MFMA(3)
        CHIMERA_FULLBIT_MFMA(4)
        CHIMERA_FULLBIT_MFMA(5)
        CHIMERA_FULLBIT_MFMA(6)
        CHIMERA_FULLBIT_MFMA(7)
        CHIMERA_FULLBIT_MFMA(8)
        default:
            return hipErrorInvalidValue;
    }
#undef CHIMERA_FULLBIT_MFMA
    return hipGetLastError();
}

hipError_t launch_final_topk(hipStream_t s, int nq, const int32_t* fcount, const int32_t* fids,
                             const float* fscores, int fb_cap, int k, int64_t* out_ids, float* out_scores,
                             int32_t* out_counts) {
    // at least one key per thread of the 1,024-thread block (its merge sort)
    const int sort_cap = std::max(pow2_at_least(fb_cap < 2 ? 2 : fb_cap), 1024);
    hipLaunchKernelGGL(final_topk_kernel, dim3(nq), dim3(1024), static_cast<size_t>(sort_cap) * 8, s, fcount, fids,
                       fscores, fb_cap, sort_cap, k, out_ids, out_scores, out_counts);
    return hipGetLastError();
}

}  // namespace chimera
