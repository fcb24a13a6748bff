// Host-side index: in-memory arrays, the on-disk file layout, and the CPU
// index build.
//
// File layout is the reference's, byte for byte, for doclens.bin,
// doc_1bit.bin, doc_full.bin, cluster_1bit.bin and ivf.bin
// (build_index.cu:380-390,503-557; ivf_pg.cpp:136-164). centroids.carga is a
// cuVS CAGRA serialization in the reference (ivf_pg.cpp:67-74); this build
// writes the rotated centroids as a numpy .npy blob behind a short header and
// reads either that or the float32 [n_clusters, 128] dataset blob of a cuVS
// file.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace Chimera {
namespace host {

constexpr uint64_t kCentroidSampleSeed = 42;  // build_index.cu:36
constexpr uint64_t kRotatorSeed = 42;         // build_index.cu:37
constexpr size_t kCodeBytes = 16;             // one-bit code bytes per token (PADDED_DIM / 8)

struct IndexHeader {  // chimera_index.cuh:75-81
    uint64_t num_embeddings;
    uint64_t dimension;
    uint64_t num_clusters;
    uint64_t ex_bits;
    uint64_t padded_dimension;
};
static_assert(sizeof(IndexHeader) == 40, "IndexHeader must be 40 bytes");

struct IndexData {
    size_t n = 0;           // token embeddings
    size_t d = 0;           // input dimension
    size_t n_clusters = 0;
    size_t ex_bits = 0;
    std::vector<uint8_t> flips;              // rotator flip bytes [64]
    std::vector<uint64_t> one_bit_codes;     // token order [n * 2]
    std::vector<float> one_bit_factors;      // token order [n]
    std::vector<float> full_bit_factors;     // token order [n]
    std::vector<uint8_t> full_bit_codes;     // token order [n * 16 * (1 + ex_bits)]
    // cluster_1bit.bin, in file order:
    std::vector<uint8_t> clustered_codes;    // [n * 16]
    std::vector<float> clustered_factors;    // [n]
    std::vector<int32_t> clustered_doc_ids;  // [n]
    std::vector<uint32_t> token_to_cluster_pos;  // [n] token order
    // ivf.bin
    std::vector<uint32_t> inv_list;          // cluster position -> token id
    std::vector<uint64_t> cluster_pos;       // [n_clusters + 1]
    // doclens.bin
    std::vector<int32_t> doc_lens;
    std::vector<int32_t> doc_ptrs;           // [num_docs + 1]
    // centroids.carga
    std::vector<float> rotated_centroids;    // [n_clusters * 128]

    size_t num_docs() const { return doc_lens.size(); }
    size_t full_code_bytes() const { return 16 * (1 + ex_bits); }
};

// validate_build_inputs (build_index.cu:75-126): same checks, messages and
// std::invalid_argument; returns N.
size_t validate_build_inputs(size_t num_floats, size_t dimension,
                             const std::vector<int32_t>& doc_lens, size_t n_clusters,
                             size_t ex_bits);

// chimera_index::build (build_index.cu:394-501) on the CPU: reservoir-sampled
// centroids (mt19937_64 seed 42), exact nearest-centroid assignment, FhtKac
// rotator (seed 42), encode, counting-sort IVF lists, reorder by cluster.
IndexData build_index(const float* embeddings, size_t num_embeddings, size_t dimension,
                      const std::vector<int32_t>& doc_lens, size_t n_clusters, size_t ex_bits);

// Reservoir sampling of centroid token ids (build_index.cu:159-184).
std::vector<size_t> sample_centroid_ids(size_t num_embeddings, size_t n_clusters);

// Index of the nearest centroid by |c|^2 - 2<x,c> in fp32, ties to the lower
// index, for every row of x [n, dim] against c [k, dim].
std::vector<uint32_t> assign_nearest(const float* x, size_t n, const float* c, size_t k,
                                     size_t dim);

// Derives the IVF lists, token order codes and the clustered arrays from the
// per-token data already in `idx` (build_index.cu:305-363, ivf_pg.cpp:110-126).
void finish_index_layout(IndexData& idx, const std::vector<uint32_t>& assignments);

// doc_ptrs from doc_lens with the checks of set_doc_mapping (utils.cu:458-475).
std::vector<int32_t> make_doc_ptrs(const std::vector<int32_t>& doc_lens, size_t n);

void save_index(const IndexData& idx, const std::string& index_dir);
// nprobe > 0 also rejects nprobe > n_clusters right after the header, where
// the reference checks it (std::invalid_argument, chimera_index.cu:94-96).
IndexData load_index(const std::string& index_dir, size_t nprobe = 0);

// io.cpp:53-108 raw loaders (embeddings.bin, queries.bin, doclens.bin).
std::vector<float> load_data(size_t& num_embeddings, size_t& d, const std::string& filename);
std::vector<float> load_query(size_t& q_doclen, size_t& num_q, size_t& d,
                              const std::string& filename);
std::vector<int32_t> load_doclens(const std::string& filename);

}  // namespace host
}  // namespace Chimera
