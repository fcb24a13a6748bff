#include "codec.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <queue>
#include <random>
#include <stdexcept>
#include <string>
#include <utility>

namespace Chimera {
namespace host {

namespace {

size_t floor_log2(size_t x) {
    size_t r = 0;
    while (x > 1) {
        ++r;
        x >>= 1;
    }
    return r;
}

// Element j of `data` changes sign when bit (j % 8) of flip[j / 8] is set
// (rotator.hpp:129-172 reads the bytes as little-endian 16-bit masks).
void flip_sign(const uint8_t* flip, float* data, size_t n) {
    for (size_t j = 0; j < n; ++j) {
        if ((flip[j >> 3] >> (j & 7)) & 1u) {
            uint32_t bits;
            std::memcpy(&bits, &data[j], 4);
            bits ^= 0x80000000u;
            std::memcpy(&data[j], &bits, 4);
        }
    }
}

void rescale(float* data, size_t n, float s) {
    for (size_t j = 0; j < n; ++j) data[j] = data[j] * s;
}

// x[i], x[i + len/2] <- x + y, x - y  (rotator.hpp:267-279)
void kacs_walk(float* data, size_t len) {
    const size_t half = len / 2;
    for (size_t i = 0; i < half; ++i) {
        const float x = data[i];
        const float y = data[i + half];
        data[i] = x + y;
        data[i + half] = x - y;
    }
}

}  // namespace

void fwht_inplace(float* x, size_t n) {
    for (size_t h = 1; h < n; h <<= 1) {
        for (size_t i = 0; i < n; i += 2 * h) {
            for (size_t j = i; j < i + h; ++j) {
                const float a = x[j];
                const float b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
        }
    }
}

FhtKacRotator::FhtKacRotator(size_t dim, size_t padded_dim, uint64_t seed)
    : dim_(dim), padded_dim_(padded_dim), flip_(4 * padded_dim / 8) {
    std::seed_seq seq{static_cast<uint32_t>(seed & 0xFFFFFFFFu),
                      static_cast<uint32_t>(seed >> 32)};
    std::mt19937 gen(seq);
    std::uniform_int_distribution<int> dist(0, 255);
    for (auto& b : flip_) b = static_cast<uint8_t>(dist(gen));
    init_transform();
}

FhtKacRotator::FhtKacRotator(size_t dim, size_t padded_dim, const uint8_t* flips)
    : dim_(dim), padded_dim_(padded_dim), flip_(flips, flips + 4 * padded_dim / 8) {
    init_transform();
}

void FhtKacRotator::init_transform() {
    if (padded_dim_ % 64 != 0 || dim_ == 0 || dim_ > padded_dim_) {
        throw std::invalid_argument("FhtKac rotator needs 0 < dim <= padded_dim, padded_dim % 64 == 0");
    }
    const size_t lg = floor_log2(dim_);
    if (lg < 6 || lg > 11) {
        throw std::invalid_argument("FhtKac rotator supports 64 <= dim < 4096");
    }
    trunc_dim_ = size_t{1} << lg;
    fac_ = 1.0F / std::sqrt(static_cast<float>(trunc_dim_));
}

void FhtKacRotator::load(std::istream& in) {
    flip_.assign(4 * padded_dim_ / 8, 0);
    in.read(reinterpret_cast<char*>(flip_.data()), static_cast<std::streamsize>(flip_.size()));
}

void FhtKacRotator::save(std::ostream& out) const {
    out.write(reinterpret_cast<const char*>(flip_.data()), static_cast<std::streamsize>(flip_.size()));
}

void FhtKacRotator::rotate(const float* src, float* dst) const {
    std::memcpy(dst, src, sizeof(float) * dim_);
    std::fill(dst + dim_, dst + padded_dim_, 0.0f);
    const size_t stride = padded_dim_ / 8;  // flip bytes per round
    if (trunc_dim_ == padded_dim_) {
        for (int r = 0; r < 4; ++r) {
            flip_sign(flip_.data() + r * stride, dst, padded_dim_);
            fwht_inplace(dst, trunc_dim_);
            rescale(dst, trunc_dim_, fac_);
        }
        return;
    }
    const size_t start = padded_dim_ - trunc_dim_;
    for (int r = 0; r < 4; ++r) {
        flip_sign(flip_.data() + r * stride, dst, padded_dim_);
        float* seg = (r & 1) ? dst + start : dst;
        fwht_inplace(seg, trunc_dim_);
        rescale(seg, trunc_dim_, fac_);
        kacs_walk(dst, padded_dim_);
    }
    rescale(dst, padded_dim_, 0.25F);
}

void encode_one_bit(const float* rotated, size_t dim, uint64_t* code, float* factor) {
    for (size_t w = 0; w < dim / 64; ++w) code[w] = 0;
    float ip = 0.0f;
    for (size_t j = 0; j < dim; ++j) {
        const int b = rotated[j] > 0 ? 1 : 0;
        code[j / 64] |= static_cast<uint64_t>(b) << (j % 64);
        ip = std::fma(static_cast<float>(b) - 0.5F, rotated[j], ip);
    }
    *factor = 1.0F / ip;
}

double best_rescale_factor(const float* o_abs, size_t dim, size_t ex_bits) {
    static const float kTightStart[9] = {0.F, 0.15F, 0.20F, 0.52F, 0.59F, 0.71F, 0.75F, 0.77F, 0.81F};
    constexpr double kEps = 1e-5;
    constexpr int kNEnum = 10;
    const double max_o = *std::max_element(o_abs, o_abs + dim);
    const double t_end = static_cast<double>(((1 << ex_bits) - 1) + kNEnum) / max_o;
    const double t_start = t_end * kTightStart[ex_bits];

    std::vector<int> cur(dim);
    double sqr_denominator = static_cast<double>(dim) * 0.25;
    double numerator = 0;
    for (size_t i = 0; i < dim; ++i) {
        const int c = static_cast<int>(std::fma(t_start, static_cast<double>(o_abs[i]), kEps));
        cur[i] = c;
        sqr_denominator += c * c + c;
        numerator = std::fma(c + 0.5, static_cast<double>(o_abs[i]), numerator);
    }
    std::priority_queue<std::pair<double, size_t>, std::vector<std::pair<double, size_t>>,
                        std::greater<>> next_t;
    for (size_t i = 0; i < dim; ++i) {
        next_t.emplace(static_cast<double>(cur[i] + 1) / o_abs[i], i);
    }
    double max_ip = 0;
    double t = 0;
    while (!next_t.empty()) {
        const double cur_t = next_t.top().first;
        const size_t id = next_t.top().second;
        next_t.pop();
        cur[id]++;
        const int u = cur[id];
        sqr_denominator += 2 * u;
        numerator += o_abs[id];
        const double cur_ip = numerator / std::sqrt(sqr_denominator);
        if (cur_ip > max_ip) {
            max_ip = cur_ip;
            t = cur_t;
        }
        if (u < (1 << ex_bits) - 1) {
            const double t_next = static_cast<double>(u + 1) / o_abs[id];
            if (t_next < t_end) next_t.emplace(t_next, id);
        }
    }
    return t;
}

void quantize_ex(const float* rotated, uint8_t* ex_code, size_t dim, size_t ex_bits) {
    float sq = 0.0f;
    for (size_t j = 0; j < dim; ++j) sq = std::fma(rotated[j], rotated[j], sq);
    const float norm = std::sqrt(sq);
    std::vector<float> abs_data(dim);
    for (size_t j = 0; j < dim; ++j) {
        abs_data[j] = norm > 0.0f ? std::fabs(rotated[j] / norm) : std::fabs(rotated[j]);
    }
    constexpr double kEps = 1e-5;
    const double t = best_rescale_factor(abs_data.data(), dim, ex_bits);
    const int top = (1 << ex_bits) - 1;
    for (size_t j = 0; j < dim; ++j) {
        int c = static_cast<int>(std::fma(t, static_cast<double>(abs_data[j]), kEps));
        if (c > top) c = top;
        ex_code[j] = static_cast<uint8_t>(c);
    }
    for (size_t j = 0; j < dim; ++j) {
        if (rotated[j] < 0) ex_code[j] = static_cast<uint8_t>((~ex_code[j]) & top);
    }
}

void encode_full_code(const float* rotated, size_t dim, size_t ex_bits,
                      uint8_t* packed, float* factor) {
    std::vector<uint8_t> ex_code(dim);
    quantize_ex(rotated, ex_code.data(), dim, ex_bits);
    std::vector<uint8_t> total(dim);
    const float cb = -(static_cast<float>(1 << ex_bits) - 0.5F);
    float ip = 0.0f;
    for (size_t j = 0; j < dim; ++j) {
        const int c = static_cast<int>(ex_code[j]) + ((rotated[j] >= 0 ? 1 : 0) << ex_bits);
        total[j] = static_cast<uint8_t>(c);
        ip = std::fma(static_cast<float>(c) + cb, rotated[j], ip);
    }
    *factor = 1.0F / ip;
    pack_codes(total.data(), packed, dim, 1 + ex_bits);
}

void pack_codes(const uint8_t* raw, uint8_t* out, size_t dim, size_t width) {
    switch (width) {
        case 1:
            for (size_t b = 0; b < dim; b += 16, raw += 16, out += 2) {
                uint16_t v = 0;
                for (int i = 0; i < 16; ++i) v |= static_cast<uint16_t>(raw[i] & 1) << i;
                out[0] = static_cast<uint8_t>(v & 0xFF);
                out[1] = static_cast<uint8_t>(v >> 8);
            }
            return;
        case 2:
            for (size_t b = 0; b < dim; b += 16, raw += 16, out += 4)
                for (int m = 0; m < 4; ++m)
                    out[m] = static_cast<uint8_t>((raw[m] & 3) | (raw[4 + m] & 3) << 2 |
                                                  (raw[8 + m] & 3) << 4 | (raw[12 + m] & 3) << 6);
            return;
        case 4:
            for (size_t b = 0; b < dim; b += 16, raw += 16, out += 8)
                for (int m = 0; m < 8; ++m)
                    out[m] = static_cast<uint8_t>((raw[m] & 15) | (raw[8 + m] & 15) << 4);
            return;
        case 6:
            for (size_t b = 0; b < dim; b += 16, raw += 16, out += 12) {
                for (int m = 0; m < 8; ++m)
                    out[m] = static_cast<uint8_t>((raw[m] & 15) | (raw[8 + m] & 15) << 4);
                for (int m = 0; m < 4; ++m)
                    out[8 + m] = static_cast<uint8_t>(((raw[m] >> 4) & 3) | ((raw[4 + m] >> 4) & 3) << 2 |
                                                      ((raw[8 + m] >> 4) & 3) << 4 |
                                                      ((raw[12 + m] >> 4) & 3) << 6);
            }
            return;
        case 8:
            std::memcpy(out, raw, dim);
            return;
        case 3:
        case 5:
        case 7: {
            // 64-dimension blocks: low bits in byte lanes, the top bit of
            // dimension i + b (i in {0,8,...,56}) at bit 8*b + i/8 of a u64.
            const size_t low_bits = width - 1;
            const size_t block_bytes = 64 * width / 8;
            for (size_t b = 0; b < dim; b += 64, raw += 64, out += block_bytes) {
                if (width == 3) {
                    for (int m = 0; m < 16; ++m)
                        out[m] = static_cast<uint8_t>((raw[m] & 3) | (raw[16 + m] & 3) << 2 |
                                                      (raw[32 + m] & 3) << 4 | (raw[48 + m] & 3) << 6);
                } else if (width == 5) {
                    for (int m = 0; m < 16; ++m) {
                        out[m] = static_cast<uint8_t>((raw[m] & 15) | (raw[16 + m] & 15) << 4);
                        out[16 + m] = static_cast<uint8_t>((raw[32 + m] & 15) | (raw[48 + m] & 15) << 4);
                    }
                } else {
                    for (int m = 0; m < 16; ++m) {
                        out[m] = static_cast<uint8_t>((raw[m] & 63) | (raw[48 + m] & 3) << 6);
                        out[16 + m] = static_cast<uint8_t>((raw[16 + m] & 63) | ((raw[48 + m] >> 2) & 3) << 6);
                        out[32 + m] = static_cast<uint8_t>((raw[32 + m] & 63) | ((raw[48 + m] >> 4) & 3) << 6);
                    }
                }
                uint64_t top = 0;
                for (int i = 0; i < 64; i += 8)
                    for (int k = 0; k < 8; ++k)
                        top |= static_cast<uint64_t>((raw[i + k] >> low_bits) & 1) << (8 * k + i / 8);
                std::memcpy(out + block_bytes - 8, &top, 8);
            }
            return;
        }
        default:
            throw std::invalid_argument("pack_codes: width must be in [1, 8], got " + std::to_string(width));
    }
}

void unpack_codes(const uint8_t* in, uint8_t* raw, size_t dim, size_t width) {
    switch (width) {
        case 1:
            for (size_t b = 0; b < dim; b += 16, raw += 16, in += 2) {
                const uint16_t v = static_cast<uint16_t>(in[0] | (in[1] << 8));
                for (int i = 0; i < 16; ++i) raw[i] = (v >> i) & 1;
            }
            return;
        case 2:
            for (size_t b = 0; b < dim; b += 16, raw += 16, in += 4)
                for (int k = 0; k < 4; ++k)
                    for (int m = 0; m < 4; ++m) raw[4 * k + m] = (in[m] >> (2 * k)) & 3;
            return;
        case 4:
            for (size_t b = 0; b < dim; b += 16, raw += 16, in += 8)
                for (int m = 0; m < 8; ++m) {
                    raw[m] = in[m] & 15;
                    raw[8 + m] = in[m] >> 4;
                }
            return;
        case 6:
            for (size_t b = 0; b < dim; b += 16, raw += 16, in += 12) {
                for (int m = 0; m < 8; ++m) {
                    raw[m] = in[m] & 15;
                    raw[8 + m] = in[m] >> 4;
                }
                for (int k = 0; k < 4; ++k)
                    for (int m = 0; m < 4; ++m)
                        raw[4 * k + m] = static_cast<uint8_t>(raw[4 * k + m] | (((in[8 + m] >> (2 * k)) & 3) << 4));
            }
            return;
        case 8:
            std::memcpy(raw, in, dim);
            return;
        case 3:
        case 5:
        case 7: {
            const size_t low_bits = width - 1;
            const size_t block_bytes = 64 * width / 8;
            for (size_t b = 0; b < dim; b += 64, raw += 64, in += block_bytes) {
                if (width == 3) {
                    for (int k = 0; k < 4; ++k)
                        for (int m = 0; m < 16; ++m) raw[16 * k + m] = (in[m] >> (2 * k)) & 3;
                } else if (width == 5) {
                    for (int m = 0; m < 16; ++m) {
                        raw[m] = in[m] & 15;
                        raw[16 + m] = in[m] >> 4;
                        raw[32 + m] = in[16 + m] & 15;
                        raw[48 + m] = in[16 + m] >> 4;
                    }
                } else {
                    for (int m = 0; m < 16; ++m) {
                        raw[m] = in[m] & 63;
                        raw[16 + m] = in[16 + m] & 63;
                        raw[32 + m] = in[32 + m] & 63;
                        raw[48 + m] = static_cast<uint8_t>((in[m] >> 6) | ((in[16 + m] >> 6) << 2) |
                                                           ((in[32 + m] >> 6) << 4));
                    }
                }
                uint64_t top;
                std::memcpy(&top, in + block_bytes - 8, 8);
                for (int i = 0; i < 64; i += 8)
                    for (int k = 0; k < 8; ++k)
                        raw[i + k] = static_cast<uint8_t>(raw[i + k] | (((top >> (8 * k + i / 8)) & 1) << low_bits));
            }
            return;
        }
        default:
            throw std::invalid_argument("unpack_codes: width must be in [1, 8], got " + std::to_string(width));
    }
}

}  // namespace host
}  // namespace Chimera
