// C entry points over the reference's own host-only sources, compiled by
// oracle/Makefile from the files as they lie under the reference tree into
// oracle/_ref/libchimera_ref.so. TEST INFRASTRUCTURE ONLY: used to pin the
// oracle and this build's host codec with known answers, and as the
// reference CPU full-bit baseline in bench.py.
//
// Wrapped reference code:
//   rabitqlib::choose_rotator / choose_rotator_with_seed, FhtKacRotator
//       cpp/third_party/rabitqlib/utils/rotator.hpp:174-398
//   Chimera::encode_one_bit / quantize_ex / encode_full_code / best_rescale_factor
//       cpp/src/quantization.cpp:47-193
//   packing_rabitqplus_code   cpp/third_party/rabitqlib/quantization/pack_excode.hpp:274-297
//   select_excode_unpackfunc  cpp/third_party/rabitqlib/utils/space.hpp:790-801
//   gemv_batch8_avx512        cpp/third_party/rabitqlib/utils/space.hpp:806-850
// ref_full_bit_scores restates the loop of compute_full_bit_scores
// (cpp/src/search_impl.cu:510-574, a member of a .cu file that cannot be
// compiled on its own) around the reference's unpack and GEMV kernels.

#include <immintrin.h>

#include <cstdint>
#include <cstring>
#include <fstream>
#include <limits>
#include <memory>
#include <string>

#include "chimera/quantization.hpp"
#include "rabitqlib/quantization/pack_excode.hpp"
#include "rabitqlib/utils/rotator.hpp"
#include "rabitqlib/utils/space.hpp"

namespace {
constexpr size_t kPadded = 128;
constexpr size_t kQ = 32;
}  // namespace

extern "C" {

int ref_rotator_flips(uint64_t seed, int32_t dim, const char* tmp_path, uint8_t* flips_out) {
    std::unique_ptr<rabitqlib::Rotator<float>> r(rabitqlib::choose_rotator_with_seed<float>(
        static_cast<size_t>(dim), rabitqlib::RotatorType::FhtKacRotator, kPadded, seed));
    {
        std::ofstream out(tmp_path, std::ios::binary | std::ios::trunc);
        r->save(out);
    }
    std::ifstream in(tmp_path, std::ios::binary);
    in.read(reinterpret_cast<char*>(flips_out), 4 * kPadded / 8);
    return in ? 0 : 1;
}

int ref_rotate(int32_t dim, const uint8_t* flips, const char* tmp_path, const float* src, int32_t count,
               float* dst) {
    {
        std::ofstream out(tmp_path, std::ios::binary | std::ios::trunc);
        out.write(reinterpret_cast<const char*>(flips), 4 * kPadded / 8);
    }
    std::unique_ptr<rabitqlib::Rotator<float>> r(
        rabitqlib::choose_rotator<float>(static_cast<size_t>(dim), rabitqlib::RotatorType::FhtKacRotator, kPadded));
    std::ifstream in(tmp_path, std::ios::binary);
    r->load(in);
    if (!in) return 1;
    for (int32_t i = 0; i < count; ++i) r->rotate(src + static_cast<size_t>(i) * dim, dst + static_cast<size_t>(i) * kPadded);
    return 0;
}

void ref_encode_one_bit(const float* rotated, uint64_t* code, float* factor) {
    Chimera::encode_one_bit(rotated, kPadded, code, factor);
}

void ref_quantize_ex(const float* rotated, int32_t ex_bits, uint8_t* ex_code) {
    Chimera::quantize_ex(rotated, ex_code, kPadded, static_cast<size_t>(ex_bits));
}

double ref_best_rescale_factor(const float* o_abs, int32_t ex_bits) {
    return Chimera::best_rescale_factor(o_abs, kPadded, static_cast<size_t>(ex_bits));
}

void ref_encode_full_code(const float* rotated, int32_t ex_bits, uint8_t* packed, float* factor) {
    Chimera::encode_full_code(rotated, kPadded, static_cast<size_t>(ex_bits), packed, factor);
}

void ref_pack(const uint8_t* raw, int32_t width, uint8_t* packed) {
    rabitqlib::quant::rabitq_impl::ex_bits::packing_rabitqplus_code(raw, packed, kPadded, static_cast<size_t>(width));
}

void ref_unpack(const uint8_t* packed, int32_t width, float* out) {
    alignas(64) float tmp[kPadded];
    rabitqlib::select_excode_unpackfunc(static_cast<size_t>(width))(packed, tmp, kPadded);
    std::memcpy(out, tmp, sizeof(tmp));
}

void ref_gemv32(const float* queries, const float* decoded, float* out) {
    alignas(64) float dec[kPadded];
    alignas(64) float res[kQ];
    std::memcpy(dec, decoded, sizeof(dec));
    rabitqlib::gemv_batch8_avx512(queries, dec, res, kQ, kPadded);
    std::memcpy(out, res, sizeof(res));
}

// search_impl.cu:510-574 for `count` documents of one query. rotated is the
// [32,128] rotated query, cbex its 32 cbex_sumq values, doc_ptrs the [M+1]
// prefix of doc_lens, codes/factors the token-order full codes.
void ref_full_bit_scores(const float* rotated, const float* cbex, const int32_t* doc_ptrs, const uint8_t* codes,
                         const float* factors, int32_t ex_bits, const int32_t* docs, int32_t count, float* out) {
    const size_t stride = kPadded * (1 + static_cast<size_t>(ex_bits)) / 8;
    auto unpack = rabitqlib::select_excode_unpackfunc(1 + static_cast<size_t>(ex_bits));
    alignas(64) float cbex_arr[kQ];
    std::memcpy(cbex_arr, cbex, sizeof(cbex_arr));
#pragma omp parallel for schedule(dynamic, 1)
    for (int32_t i = 0; i < count; ++i) {
        const int32_t doc = docs[i];
        const size_t start = static_cast<size_t>(doc_ptrs[doc]);
        const size_t n_tok = static_cast<size_t>(doc_ptrs[doc + 1]) - start;
        alignas(64) float decoded[kPadded];
        alignas(64) float full_ip[kQ];
        alignas(64) float max_ts[kQ];
        const __m512 neg_inf = _mm512_set1_ps(-std::numeric_limits<float>::infinity());
        for (size_t j = 0; j < kQ; j += 16) _mm512_store_ps(&max_ts[j], neg_inf);
        for (size_t t = 0; t < n_tok; ++t) {
            const size_t tid = start + t;
            unpack(codes + tid * stride, decoded, kPadded);
            rabitqlib::gemv_batch8_avx512(rotated, decoded, full_ip, kQ, kPadded);
            const __m512 f = _mm512_set1_ps(factors[tid]);
            for (size_t j = 0; j < kQ; j += 16) {
                const __m512 c = _mm512_mul_ps(_mm512_sub_ps(_mm512_load_ps(&full_ip[j]), _mm512_load_ps(&cbex_arr[j])), f);
                _mm512_store_ps(&max_ts[j], _mm512_max_ps(_mm512_load_ps(&max_ts[j]), c));
            }
        }
        __m512 sum = _mm512_load_ps(&max_ts[0]);
        for (size_t j = 16; j < kQ; j += 16) sum = _mm512_add_ps(sum, _mm512_load_ps(&max_ts[j]));
        out[i] = _mm512_reduce_add_ps(sum);
    }
}

}  // extern "C"
