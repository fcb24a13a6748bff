// Host view of one index for the oracle and the CPU baseline (test
// infrastructure): the arrays of the index files, as chimera_index::load
// reads them (chimera_index.cu:54-173).
#pragma once

#include <cstdint>

extern "C" {

struct oracle_index {
    int64_t n, dim, n_clusters, ex_bits, num_docs;
    const int32_t* doc_ptrs;
    const uint64_t* cluster_pos;
    const uint8_t* clustered_codes;
    const float* clustered_factors;
    const int32_t* clustered_doc_ids;
    const uint32_t* token_to_cluster_pos;
    const uint8_t* full_codes;
    const float* full_factors;
    const float* rotated_centroids;
    const uint8_t* flips;
};

}  // extern "C"
