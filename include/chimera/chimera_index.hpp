// Chimera C++ library API for MI355X.
//
// Same class, method names, argument meaning, defaults and exception types
// as the reference's public header cpp/include/chimera/chimera_index.cuh:26-159.
// The vendor runtime headers are not included here: device work goes through
// the C ABI declared in chimera_hip.h.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace Chimera {

// chimera_index.cuh:26-32. `cagra_itopk_size` is accepted and validated but
// has no effect: the centroid probe is exact.
struct SearchOptions {
    int nprobe = 128;
    int k_refine = 3000;
    int k_full_bit = 300;
    int cagra_itopk_size = 150;
    int num_chunks = 5;
};

// chimera_index.cuh:43-159.
class chimera_index {
  public:
    chimera_index();
    ~chimera_index();

    // build_index.cu:394-501. Embeddings [N, dimension] row-major, token rows
    // of one document contiguous; doc_lens sums to N.
    void build(const std::vector<float>& embeddings, size_t dimension,
               const std::vector<int>& doc_lens, size_t n_clusters, size_t ex_bits,
               const SearchOptions& options = {});

    // search_impl.cu:40-70. query is [32, d] fp32; returns up to k document
    // IDs in descending score order.
    std::vector<size_t> search(const std::vector<float>& query, size_t k);
    std::vector<size_t> search(const float* query, size_t query_size, size_t k);

    // Batched search: `queries` is [num_queries, 32, d]; one device call for
    // the whole batch. Results equal num_queries calls of search().
    std::vector<std::vector<size_t>> search_batch(const float* queries, size_t num_queries,
                                                  size_t query_size, size_t k);

    // build_index.cu:503-557 / chimera_index.cu:54-173.
    void save(const std::string& index_dir) const;
    void load(const std::string& index_dir, const SearchOptions& options = {});

    chimera_index(const chimera_index&) = delete;
    chimera_index& operator=(const chimera_index&) = delete;

    // Introspection used by the bindings and tests.
    size_t num_embeddings() const;
    size_t dimension() const;
    size_t num_clusters() const;
    size_t ex_bits() const;
    size_t num_docs() const;
    const SearchOptions& options() const;

    struct Impl;

  private:
    std::unique_ptr<Impl> impl_;
};

}  // namespace Chimera
