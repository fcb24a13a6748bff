// FhtKac rotation of one 128-float row by one wave64 (rotator.hpp:281-334,
// fht_avx.cpp:396-591): lane l holds elements l and l + 64.
#pragma once

#include "common.hpp"

namespace chimera {

// One butterfly stage with stride h < 64 across the lanes of a wave: the
// lower element of each pair becomes a + b and the upper a - b (FFHT runs
// stages 1, 2, 4, ... in that order).
__device__ __forceinline__ float butterfly_lanes(float x, int h, int l) {
    const float p = __shfl_xor(x, h, kWave);
    return (l & h) ? (p - x) : (x + p);
}

__device__ __forceinline__ float fwht64_lanes(float x, int l) {
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) x = butterfly_lanes(x, h, l);
    return x;
}

// Element j changes sign when bit j % 8 of byte j / 8 of the round's 16
// flip bytes is set (rotator.hpp:129-172).
__device__ __forceinline__ float flip_sign(float x, const uint8_t* f, int j) {
    return ((f[j >> 3] >> (j & 7)) & 1u) ? -x : x;
}

// Rotates (x0, x1) = elements (l, l + 64) in place. `flips` holds the 64
// flip bytes (4 rounds x 16), `fac` = 1/sqrtf(trunc_dim), `pow2` is
// trunc_dim == 128 (dim == 128); otherwise the KAC-walk variant with the
// final 0.25 scale runs.
__device__ __forceinline__ void fht_kac_rotate(float& x0, float& x1, const uint8_t* flips, float fac, bool pow2,
                                               int l) {
#pragma unroll
    for (int round = 0; round < 4; ++round) {
        const uint8_t* f = flips + round * (kDim / 8);
        x0 = flip_sign(x0, f, l);
        x1 = flip_sign(x1, f, l + 64);
        if (pow2) {
            x0 = fwht64_lanes(x0, l);
            x1 = fwht64_lanes(x1, l);
            const float a = x0, b = x1;  // stride-64 stage, last
            x0 = a + b;
            x1 = a - b;
            x0 = x0 * fac;
            x1 = x1 * fac;
        } else {
            if (round & 1) {
                x1 = fwht64_lanes(x1, l) * fac;
            } else {
                x0 = fwht64_lanes(x0, l) * fac;
            }
            const float a = x0, b = x1;  // kacs_walk
            x0 = a + b;
            x1 = a - b;
        }
    }
    if (!pow2) {
        x0 = x0 * 0.25F;
        x1 = x1 * 0.25F;
    }
}

}  // namespace chimera
