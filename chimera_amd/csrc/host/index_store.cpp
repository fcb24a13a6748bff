#include "index_store.hpp"

#include "codec.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <random>
#include <sstream>
#include <stdexcept>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace Chimera {
namespace host {

namespace {


std::ofstream open_out(const std::string& path) {
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    if (!out.is_open()) throw std::runtime_error("Failed to open output file: " + path);
    return out;
}

void finish_out(std::ofstream& out, const std::string& path) {
    out.flush();
    if (!out) throw std::runtime_error("Failed to write output file: " + path);
}

template <typename T>
void write_vec(std::ofstream& out, const std::vector<T>& v) {
    out.write(reinterpret_cast<const char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
}

template <typename T>
bool read_vec(std::istream& in, std::vector<T>& v, size_t count) {
    v.resize(count);
    in.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(count * sizeof(T)));
    return static_cast<bool>(in);
}

// ---- numpy .npy blobs (format version 1.0/2.0) ----

std::string npy_header(size_t rows, size_t cols) {
    std::ostringstream dict;
    dict << "{'descr': '<f4', 'fortran_order': False, 'shape': (" << rows << ", " << cols << "), }";
    std::string h = dict.str();
    const size_t unpadded = 10 + h.size() + 1;
    const size_t padded = (unpadded + 63) / 64 * 64;
    h.append(padded - unpadded, ' ');
    h.push_back('\n');
    std::string out("\x93NUMPY\x01\x00", 8);
    const uint16_t len = static_cast<uint16_t>(h.size());
    out.push_back(static_cast<char>(len & 0xFF));
    out.push_back(static_cast<char>(len >> 8));
    return out + h;
}

struct NpyBlob {
    std::string descr;
    bool fortran = false;
    std::vector<size_t> shape;
    size_t data_offset = 0;
};

bool parse_npy_at(const std::vector<char>& buf, size_t pos, NpyBlob& blob) {
    static const char kMagic[6] = {'\x93', 'N', 'U', 'M', 'P', 'Y'};
    if (pos + 10 > buf.size() || std::memcmp(buf.data() + pos, kMagic, 6) != 0) return false;
    const uint8_t major = static_cast<uint8_t>(buf[pos + 6]);
    size_t hlen = 0, hstart = 0;
    if (major == 1) {
        hlen = static_cast<uint8_t>(buf[pos + 8]) | (static_cast<uint8_t>(buf[pos + 9]) << 8);
        hstart = pos + 10;
    } else if (major == 2 || major == 3) {
        if (pos + 12 > buf.size()) return false;
        uint32_t l;
        std::memcpy(&l, buf.data() + pos + 8, 4);
        hlen = l;
        hstart = pos + 12;
    } else {
        return false;
    }
    if (hstart + hlen > buf.size()) return false;
    const std::string h(buf.data() + hstart, hlen);
    auto field = [&](const char* key) -> size_t { return h.find(key); };
    const size_t d = field("'descr'");
    const size_t s = field("'shape'");
    const size_t f = field("'fortran_order'");
    if (d == std::string::npos || s == std::string::npos) return false;
    const size_t q1 = h.find('\'', h.find(':', d) + 1);
    const size_t q2 = h.find('\'', q1 + 1);
    if (q1 == std::string::npos || q2 == std::string::npos) return false;
    blob.descr = h.substr(q1 + 1, q2 - q1 - 1);
    blob.fortran = f != std::string::npos && h.compare(h.find(':', f) + 1, 5, " True") == 0;
    const size_t p1 = h.find('(', s);
    const size_t p2 = h.find(')', p1);
    if (p1 == std::string::npos || p2 == std::string::npos) return false;
    blob.shape.clear();
    std::string dims = h.substr(p1 + 1, p2 - p1 - 1);
    std::stringstream ss(dims);
    std::string tok;
    while (std::getline(ss, tok, ',')) {
        const size_t a = tok.find_first_not_of(' ');
        if (a == std::string::npos) continue;
        blob.shape.push_back(static_cast<size_t>(std::stoull(tok.substr(a))));
    }
    blob.data_offset = hstart + hlen;
    return true;
}

void save_centroids(const std::string& path, const std::vector<float>& rotated, size_t n_clusters) {
    auto out = open_out(path);
    const std::string h = npy_header(n_clusters, kPaddedDim);
    out.write(h.data(), static_cast<std::streamsize>(h.size()));
    write_vec(out, rotated);
    finish_out(out, path);
}

// Reads the float32 [n_clusters, 128] array from this build's file or from
// the dataset blob a cuVS CAGRA serialization carries after its graph blob.
std::vector<float> load_centroids(const std::string& path, size_t n_clusters) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error("Failed to open centroid file: " + path);
    const std::streamoff size = in.tellg();
    std::vector<char> buf(static_cast<size_t>(size));
    in.seekg(0);
    in.read(buf.data(), size);
    if (!in) throw std::runtime_error("Failed to read centroid file: " + path);
    for (size_t pos = 0; pos + 10 <= buf.size(); ++pos) {
        if (buf[pos] != '\x93') continue;
        NpyBlob blob;
        if (!parse_npy_at(buf, pos, blob)) continue;
        if (blob.descr == "<f4" && !blob.fortran && blob.shape.size() == 2 &&
            blob.shape[0] == n_clusters && blob.shape[1] == kPaddedDim &&
            blob.data_offset + n_clusters * kPaddedDim * sizeof(float) <= buf.size()) {
            std::vector<float> c(n_clusters * kPaddedDim);
            std::memcpy(c.data(), buf.data() + blob.data_offset, c.size() * sizeof(float));
            return c;
        }
    }
    throw std::runtime_error("No float32 [" + std::to_string(n_clusters) +
                             ", 128] centroid array found in " + path);
}

}  // namespace

size_t validate_build_inputs(size_t num_floats, size_t dimension,
                             const std::vector<int32_t>& doc_lens, size_t n_clusters,
                             size_t ex_bits) {
    if (dimension < 64 || dimension > kPaddedDim) {
        throw std::invalid_argument("Embedding dimension must be in [64, " + std::to_string(kPaddedDim) + "]");
    }
    if (num_floats == 0 || num_floats % dimension != 0) {
        throw std::invalid_argument("Embedding storage must contain a non-empty whole number of vectors");
    }
    const size_t n = num_floats / dimension;
    if (n > static_cast<size_t>(std::numeric_limits<int>::max())) {
        throw std::invalid_argument("Embedding count exceeds the int32 index format limit");
    }
    if (n_clusters == 0 || n_clusters > n) {
        throw std::invalid_argument("n_clusters must be between 1 and the number of embeddings");
    }
    if (ex_bits < 1 || ex_bits > 7) {
        throw std::invalid_argument("ex_bits must be in [1, 7] so full codes fit in 2-8 bits per dimension");
    }
    if (doc_lens.empty()) throw std::invalid_argument("doc_lens must not be empty");
    size_t tokens = 0;
    for (const int32_t len : doc_lens) {
        if (len <= 0) throw std::invalid_argument("Every document length must be positive");
        const size_t l = static_cast<size_t>(len);
        if (tokens > n || l > n - tokens) {
            throw std::invalid_argument("Document lengths exceed the number of embeddings");
        }
        tokens += l;
    }
    if (tokens != n) throw std::invalid_argument("Document lengths do not sum to the number of embeddings");
    return n;
}

std::vector<size_t> sample_centroid_ids(size_t num_embeddings, size_t n_clusters) {
    std::vector<size_t> ids(n_clusters);
    for (size_t i = 0; i < n_clusters; ++i) ids[i] = i;
    std::mt19937_64 gen(kCentroidSampleSeed);
    for (size_t index = n_clusters; index < num_embeddings; ++index) {
        std::uniform_int_distribution<size_t> dist(0, index);
        const size_t pos = dist(gen);
        if (pos < n_clusters) ids[pos] = index;
    }
    return ids;
}

std::vector<uint32_t> assign_nearest(const float* x, size_t n, const float* c, size_t k, size_t dim) {
    std::vector<float> cT(dim * k);
    std::vector<float> norms(k);
    for (size_t j = 0; j < k; ++j) {
        float s = 0.f;
        for (size_t t = 0; t < dim; ++t) {
            const float v = c[j * dim + t];
            s = std::fma(v, v, s);
            cT[t * k + j] = v;
        }
        norms[j] = s;
    }
    std::vector<uint32_t> out(n);
#pragma omp parallel
    {
        std::vector<float> acc(k);
#pragma omp for schedule(dynamic, 64)
        for (int64_t r = 0; r < static_cast<int64_t>(n); ++r) {
            std::fill(acc.begin(), acc.end(), 0.f);
            const float* xr = x + static_cast<size_t>(r) * dim;
            for (size_t t = 0; t < dim; ++t) {
                const float xv = xr[t];
                const float* row = cT.data() + t * k;
                for (size_t j = 0; j < k; ++j) acc[j] = std::fma(xv, row[j], acc[j]);
            }
            uint32_t best = 0;
            float best_d = norms[0] - 2.f * acc[0];
            for (size_t j = 1; j < k; ++j) {
                const float dj = norms[j] - 2.f * acc[j];
                if (dj < best_d) {
                    best_d = dj;
                    best = static_cast<uint32_t>(j);
                }
            }
            out[static_cast<size_t>(r)] = best;
        }
    }
    return out;
}

std::vector<int32_t> make_doc_ptrs(const std::vector<int32_t>& doc_lens, size_t n) {
    if (doc_lens.empty()) throw std::runtime_error("Chimera index has no documents");
    std::vector<int32_t> ptrs(doc_lens.size() + 1, 0);
    for (size_t i = 0; i < doc_lens.size(); ++i) {
        if (doc_lens[i] <= 0 || ptrs[i] > std::numeric_limits<int>::max() - doc_lens[i]) {
            throw std::runtime_error("Invalid document lengths in Chimera index");
        }
        ptrs[i + 1] = ptrs[i] + doc_lens[i];
    }
    if (static_cast<size_t>(ptrs.back()) != n) {
        throw std::runtime_error("Document lengths do not match the number of indexed embeddings");
    }
    return ptrs;
}

void finish_index_layout(IndexData& idx, const std::vector<uint32_t>& assignments) {
    const size_t n = idx.n;
    // IVF_PG::build_from_assignments: counting sort, token ids ascending
    // within each cluster (ivf_pg.cpp:110-126).
    idx.cluster_pos.assign(idx.n_clusters + 1, 0);
    for (size_t i = 0; i < n; ++i) ++idx.cluster_pos[assignments[i] + 1];
    for (size_t c = 0; c < idx.n_clusters; ++c) idx.cluster_pos[c + 1] += idx.cluster_pos[c];
    idx.inv_list.resize(n);
    std::vector<uint64_t> write = idx.cluster_pos;
    for (size_t i = 0; i < n; ++i) idx.inv_list[write[assignments[i]]++] = static_cast<uint32_t>(i);

    idx.doc_ptrs = make_doc_ptrs(idx.doc_lens, n);
    std::vector<int32_t> token_doc(n);
    for (size_t dd = 0; dd < idx.doc_lens.size(); ++dd)
        for (int32_t t = idx.doc_ptrs[dd]; t < idx.doc_ptrs[dd + 1]; ++t) token_doc[t] = static_cast<int32_t>(dd);

    // reorder_by_cluster (build_index.cu:328-363)
    idx.clustered_codes.resize(n * kCodeBytes);
    idx.clustered_factors.resize(n);
    idx.clustered_doc_ids.resize(n);
    idx.token_to_cluster_pos.resize(n);
    const uint8_t* src = reinterpret_cast<const uint8_t*>(idx.one_bit_codes.data());
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < static_cast<int64_t>(n); ++p) {
        const uint32_t tok = idx.inv_list[static_cast<size_t>(p)];
        std::memcpy(idx.clustered_codes.data() + static_cast<size_t>(p) * kCodeBytes, src + static_cast<size_t>(tok) * kCodeBytes, kCodeBytes);
        idx.clustered_factors[p] = idx.one_bit_factors[tok];
        idx.clustered_doc_ids[p] = token_doc[tok];
        idx.token_to_cluster_pos[tok] = static_cast<uint32_t>(p);
    }
}

IndexData build_index(const float* embeddings, size_t num_embeddings, size_t dimension,
                      const std::vector<int32_t>& doc_lens, size_t n_clusters, size_t ex_bits) {
    validate_build_inputs(num_embeddings * dimension, dimension, doc_lens, n_clusters, ex_bits);
    IndexData idx;
    idx.n = num_embeddings;
    idx.d = dimension;
    idx.n_clusters = n_clusters;
    idx.ex_bits = ex_bits;
    idx.doc_lens = doc_lens;

    const std::vector<size_t> sampled = sample_centroid_ids(num_embeddings, n_clusters);
    std::vector<float> centroids(n_clusters * dimension);
    for (size_t c = 0; c < n_clusters; ++c)
        std::memcpy(centroids.data() + c * dimension, embeddings + sampled[c] * dimension, dimension * sizeof(float));
    const std::vector<uint32_t> assignments =
        assign_nearest(embeddings, num_embeddings, centroids.data(), n_clusters, dimension);

    const FhtKacRotator rot(dimension, kPaddedDim, kRotatorSeed);
    idx.flips = rot.flips();
    idx.rotated_centroids.resize(n_clusters * kPaddedDim);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < static_cast<int64_t>(n_clusters); ++c)
        rot.rotate(centroids.data() + static_cast<size_t>(c) * dimension, idx.rotated_centroids.data() + static_cast<size_t>(c) * kPaddedDim);

    const size_t full_bytes = kPaddedDim * (1 + ex_bits) / 8;
    idx.one_bit_codes.resize(num_embeddings * 2);
    idx.one_bit_factors.resize(num_embeddings);
    idx.full_bit_codes.resize(num_embeddings * full_bytes);
    idx.full_bit_factors.resize(num_embeddings);
#pragma omp parallel
    {
        std::vector<float> r(kPaddedDim);
#pragma omp for schedule(static)
        for (int64_t row = 0; row < static_cast<int64_t>(num_embeddings); ++row) {
            const size_t i = static_cast<size_t>(row);
            rot.rotate(embeddings + i * dimension, r.data());
            encode_one_bit(r.data(), kPaddedDim, idx.one_bit_codes.data() + 2 * i, &idx.one_bit_factors[i]);
            encode_full_code(r.data(), kPaddedDim, ex_bits, idx.full_bit_codes.data() + i * full_bytes,
                             &idx.full_bit_factors[i]);
        }
    }
    finish_index_layout(idx, assignments);
    return idx;
}

void save_index(const IndexData& idx, const std::string& index_dir) {
    std::error_code ec;
    std::filesystem::create_directories(index_dir, ec);
    if (ec) throw std::runtime_error("Failed to create index directory " + index_dir + ": " + ec.message());
    const std::array<const char*, 6> names = {"doclens.bin", "doc_1bit.bin", "doc_full.bin",
                                              "cluster_1bit.bin", "ivf.bin", "centroids.carga"};
    for (const char* name : names) {
        const auto p = (std::filesystem::path(index_dir) / name).string();
        ec.clear();
        std::filesystem::remove(p, ec);
        if (ec) throw std::runtime_error("Failed to remove stale index output " + p + ": " + ec.message());
    }
    const std::filesystem::path dir(index_dir);
    {
        const auto p = (dir / "doclens.bin").string();
        auto out = open_out(p);
        const int32_t count = static_cast<int32_t>(idx.doc_lens.size());
        out.write(reinterpret_cast<const char*>(&count), sizeof(count));
        write_vec(out, idx.doc_lens);
        finish_out(out, p);
    }
    save_centroids((dir / "centroids.carga").string(), idx.rotated_centroids, idx.n_clusters);
    {
        const auto p = (dir / "ivf.bin").string();
        auto out = open_out(p);
        const uint64_t n = idx.inv_list.size();
        out.write(reinterpret_cast<const char*>(&n), sizeof(n));
        write_vec(out, idx.inv_list);
        write_vec(out, idx.cluster_pos);
        finish_out(out, p);
    }
    {
        const auto p = (dir / "doc_1bit.bin").string();
        auto out = open_out(p);
        const IndexHeader h{idx.n, idx.d, idx.n_clusters, idx.ex_bits, kPaddedDim};
        out.write(reinterpret_cast<const char*>(&h), sizeof(h));
        write_vec(out, idx.flips);
        write_vec(out, idx.one_bit_codes);
        write_vec(out, idx.one_bit_factors);
        write_vec(out, idx.full_bit_factors);
        finish_out(out, p);
    }
    {
        const auto p = (dir / "doc_full.bin").string();
        auto out = open_out(p);
        write_vec(out, idx.full_bit_codes);
        finish_out(out, p);
    }
    {
        const auto p = (dir / "cluster_1bit.bin").string();
        auto out = open_out(p);
        write_vec(out, idx.clustered_codes);
        write_vec(out, idx.clustered_factors);
        write_vec(out, idx.clustered_doc_ids);
        write_vec(out, idx.token_to_cluster_pos);
        finish_out(out, p);
    }
}

IndexData load_index(const std::string& index_dir, size_t nprobe) {
    const std::filesystem::path dir(index_dir);
    if (!std::filesystem::is_directory(dir)) {
        throw std::runtime_error("Chimera index directory does not exist: " + index_dir);
    }
    IndexData idx;
    const auto one_bit_path = (dir / "doc_1bit.bin").string();
    std::ifstream inf(one_bit_path, std::ios::binary);
    IndexHeader h{};
    inf.read(reinterpret_cast<char*>(&h), sizeof(h));
    // chimera_index.cu:82-105
    if (!inf || h.num_embeddings == 0 ||
        h.num_embeddings > static_cast<uint64_t>(std::numeric_limits<int>::max()) ||
        h.dimension < 64 || h.dimension > kPaddedDim || h.num_clusters == 0 ||
        h.num_clusters > h.num_embeddings || h.ex_bits < 1 || h.ex_bits > 7) {
        throw std::runtime_error("Invalid Chimera index header: " + one_bit_path);
    }
    if (nprobe > h.num_clusters) throw std::invalid_argument("nprobe must not exceed the number of clusters");
    if (h.padded_dimension != kPaddedDim) {
        throw std::runtime_error("Index file padded_dim=" + std::to_string(h.padded_dimension) +
                                 " does not match compiled PADDED_DIM=" + std::to_string(kPaddedDim));
    }
    idx.n = h.num_embeddings;
    idx.d = h.dimension;
    idx.n_clusters = h.num_clusters;
    idx.ex_bits = h.ex_bits;
    if (!read_vec(inf, idx.flips, kFlipBytes)) throw std::runtime_error("Failed to read rotator from " + one_bit_path);
    const size_t n = idx.n;
    if (!read_vec(inf, idx.one_bit_codes, n * 2) || !read_vec(inf, idx.one_bit_factors, n) ||
        !read_vec(inf, idx.full_bit_factors, n)) {
        throw std::runtime_error("Failed to read quantized payload from " + one_bit_path);
    }
    {
        const auto p = (dir / "doc_full.bin").string();
        std::ifstream in(p, std::ios::binary);
        if (!read_vec(in, idx.full_bit_codes, n * idx.full_code_bytes())) {
            throw std::runtime_error("Failed to read full-code payload from " + p);
        }
    }
    {
        const auto p = (dir / "ivf.bin").string();
        std::ifstream in(p, std::ios::binary);
        uint64_t nl = 0;
        in.read(reinterpret_cast<char*>(&nl), sizeof(nl));
        if (!in || nl != n || !read_vec(in, idx.inv_list, nl) || !read_vec(in, idx.cluster_pos, idx.n_clusters + 1)) {
            throw std::runtime_error("Failed to read IVF lists from " + p);
        }
        if (idx.cluster_pos.front() != 0 || idx.cluster_pos.back() != n ||
            !std::is_sorted(idx.cluster_pos.begin(), idx.cluster_pos.end())) {
            throw std::runtime_error("Invalid IVF cluster offsets in " + p);
        }
    }
    idx.rotated_centroids = load_centroids((dir / "centroids.carga").string(), idx.n_clusters);
    idx.doc_lens = load_doclens((dir / "doclens.bin").string());
    {
        const auto p = (dir / "cluster_1bit.bin").string();
        const size_t expect = n * (kCodeBytes + sizeof(float) + sizeof(int32_t) + sizeof(uint32_t));
        std::ifstream in(p, std::ios::binary | std::ios::ate);
        if (!in || in.tellg() < 0 || static_cast<size_t>(in.tellg()) != expect) {
            throw std::runtime_error("Invalid clustered index payload: " + p);
        }
        in.seekg(0);
        if (!read_vec(in, idx.clustered_codes, n * kCodeBytes) || !read_vec(in, idx.clustered_factors, n) ||
            !read_vec(in, idx.clustered_doc_ids, n) || !read_vec(in, idx.token_to_cluster_pos, n)) {
            throw std::runtime_error("Failed to read clustered index: " + p);
        }
    }
    idx.doc_ptrs = make_doc_ptrs(idx.doc_lens, n);
    return idx;
}

namespace {

std::ifstream open_in(const std::string& f) {
    std::ifstream in(f, std::ios::binary);
    if (!in.is_open()) throw std::runtime_error("Failed to open input file: " + f);
    return in;
}

template <typename T>
T read_one(std::ifstream& in, const std::string& f) {
    T v{};
    in.read(reinterpret_cast<char*>(&v), sizeof(v));
    if (!in) throw std::runtime_error("Failed to read input file: " + f);
    return v;
}

template <typename T>
void read_all(std::ifstream& in, std::vector<T>& v, const std::string& f) {
    in.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
    if (!in) throw std::runtime_error("Failed to read input file: " + f);
}

}  // namespace

std::vector<float> load_data(size_t& num_embeddings, size_t& d, const std::string& f) {
    auto in = open_in(f);
    const int32_t cnt = read_one<int32_t>(in, f);
    const int32_t dim = read_one<int32_t>(in, f);
    if (cnt <= 0 || dim <= 0) throw std::runtime_error("Embedding header contains non-positive dimensions: " + f);
    num_embeddings = static_cast<size_t>(cnt);
    d = static_cast<size_t>(dim);
    std::vector<float> v(num_embeddings * d);
    read_all(in, v, f);
    return v;
}

std::vector<float> load_query(size_t& q_doclen, size_t& num_q, size_t& d, const std::string& f) {
    auto in = open_in(f);
    const int32_t nq = read_one<int32_t>(in, f);
    const int32_t ql = read_one<int32_t>(in, f);
    const int32_t dim = read_one<int32_t>(in, f);
    if (nq <= 0 || ql <= 0 || dim <= 0) throw std::runtime_error("Query header contains non-positive dimensions: " + f);
    num_q = static_cast<size_t>(nq);
    q_doclen = static_cast<size_t>(ql);
    d = static_cast<size_t>(dim);
    std::vector<float> v(num_q * q_doclen * d);
    read_all(in, v, f);
    return v;
}

std::vector<int32_t> load_doclens(const std::string& f) {
    auto in = open_in(f);
    const int32_t cnt = read_one<int32_t>(in, f);
    if (cnt <= 0) throw std::runtime_error("Document-length header contains a non-positive count: " + f);
    std::vector<int32_t> v(static_cast<size_t>(cnt));
    read_all(in, v, f);
    return v;
}

}  // namespace host
}  // namespace Chimera
