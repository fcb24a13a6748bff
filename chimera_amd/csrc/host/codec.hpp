// Host-side codec for the Chimera index: the FhtKac rotation, the RaBitQ
// one-bit and (1+ex_bits)-bit encoders, and the packed W-bit code layouts.
//
// Behaviour follows the reference:
//   rotation      cpp/third_party/rabitqlib/utils/rotator.hpp:129-334
//   encoders      cpp/src/quantization.cpp:32-193
//   W-bit packing cpp/third_party/rabitqlib/quantization/pack_excode.hpp:13-297
//   W-bit unpack  cpp/third_party/rabitqlib/utils/space.hpp:604-801
// The code here is scalar C++; the search-time rotation runs on the GPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <istream>
#include <ostream>
#include <vector>

namespace Chimera {
namespace host {

constexpr size_t kPaddedDim = 128;   // PADDED_DIM (config.cuh:7)
constexpr size_t kQueryLen = 32;     // Q_DOCLEN (config.cuh:8)
constexpr size_t kFlipBytes = 4 * kPaddedDim / 8;  // rotator.hpp:224

// FhtKac rotator: four rounds of sign flip, unnormalised Walsh-Hadamard
// transform and 1/sqrt(trunc_dim) scaling (rotator.hpp:281-334).
class FhtKacRotator {
  public:
    FhtKacRotator() = default;
    // Flip bytes drawn from std::mt19937 seeded through std::seed_seq with
    // the two 32-bit halves of `seed`, as rotator.hpp:46-52,183-189,230-237.
    FhtKacRotator(size_t dim, size_t padded_dim, uint64_t seed);
    // Flip bytes given explicitly (as read from doc_1bit.bin).
    FhtKacRotator(size_t dim, size_t padded_dim, const uint8_t* flips);

    void rotate(const float* src, float* dst) const;
    void load(std::istream& in);
    void save(std::ostream& out) const;

    size_t dim() const { return dim_; }
    size_t padded_dim() const { return padded_dim_; }
    size_t trunc_dim() const { return trunc_dim_; }
    float scale() const { return fac_; }
    const std::vector<uint8_t>& flips() const { return flip_; }

  private:
    void init_transform();
    size_t dim_ = 0;
    size_t padded_dim_ = 0;
    size_t trunc_dim_ = 0;
    float fac_ = 0.f;
    std::vector<uint8_t> flip_;
};

// In-place unnormalised Walsh-Hadamard transform, butterfly stages with
// stride 1, 2, 4, ... in that order (the order of FFHT helper_float_6/7).
void fwht_inplace(float* x, size_t n);

// One-bit code: bit j of the 128-bit little-endian word is (x_j > 0);
// factor = 1 / sum_j (b_j - 1/2) x_j (quantization.cpp:47-60).
void encode_one_bit(const float* rotated, size_t dim, uint64_t* code, float* factor);

// best_rescale_factor (quantization.cpp:62-119), double precision.
double best_rescale_factor(const float* o_abs, size_t dim, size_t ex_bits);

// Per-dimension ex code in [0, 2^ex_bits) with negative dims inverted
// (quantization.cpp:121-146).
void quantize_ex(const float* rotated, uint8_t* ex_code, size_t dim, size_t ex_bits);

// Full code c_j = ex_j + ((x_j >= 0) << ex_bits), packed at W = 1 + ex_bits;
// factor = 1 / sum_j (c_j - (2^ex_bits - 1/2)) x_j (quantization.cpp:168-193).
void encode_full_code(const float* rotated, size_t dim, size_t ex_bits,
                      uint8_t* packed, float* factor);

// Packed byte count of one W-bit code of `dim` dimensions.
inline size_t packed_bytes(size_t dim, size_t width) { return dim * width / 8; }

// Pack raw per-dimension codes (values < 2^width) into the W-bit layout
// (pack_excode.hpp:13-297). dim must be a multiple of 64 for W in {3,5,7}
// and of 16 otherwise.
void pack_codes(const uint8_t* raw, uint8_t* packed, size_t dim, size_t width);

// Inverse of pack_codes: the integer each unpack_fxu{W} of space.hpp
// converts to float.
void unpack_codes(const uint8_t* packed, uint8_t* raw, size_t dim, size_t width);

}  // namespace host
}  // namespace Chimera
