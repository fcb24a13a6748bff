// Chimera::chimera_index on MI355X: host index handling in C++, every search
// through the C ABI of libchimera_hip.so.
//
// Method contracts follow the reference:
//   build   build_index.cu:394-501     search  search_impl.cu:40-70
//   save    build_index.cu:503-557     load    chimera_index.cu:54-173
// including which exception type each failure raises and its message.
#include "chimera/chimera_index.hpp"

#include "chimera_hip.h"
#include "codec.hpp"
#include "index_store.hpp"

#include <algorithm>
#include <cstdlib>
#include <filesystem>
#include <stdexcept>
#include <string>

namespace Chimera {

namespace {

constexpr int32_t kDefaultMaxBatch = 1024;

void validate_search_options(const SearchOptions& o) {  // chimera_index.cu:27-36
    if (o.nprobe <= 0 || o.k_refine <= 0 || o.k_full_bit <= 0 || o.cagra_itopk_size <= 0 || o.num_chunks <= 0) {
        throw std::invalid_argument("All Chimera search options must be positive");
    }
    if (o.k_full_bit > o.k_refine) throw std::invalid_argument("k_full_bit must not exceed k_refine");
}

[[noreturn]] void throw_status(int code, const char* what) {
    std::string msg = chimera_last_error();
    if (msg.empty()) msg = what;
    if (code == CHIMERA_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void check(int code, const char* what) {
    if (code != CHIMERA_OK) throw_status(code, what);
}

int32_t max_batch_setting() {
    if (const char* v = std::getenv("CHIMERA_MAX_BATCH")) {
        const long b = std::strtol(v, nullptr, 10);
        if (b > 0 && b <= 65536) return static_cast<int32_t>(b);
    }
    return kDefaultMaxBatch;
}

}  // namespace

struct chimera_index::Impl {
    host::IndexData idx;
    SearchOptions options;
    bool has_index = false;
    bool search_ready = false;
    chimera_ctx* ctx = nullptr;
    int32_t max_batch = 0;

    ~Impl() { release(); }

    void release() noexcept {
        if (ctx) chimera_destroy(ctx);
        ctx = nullptr;
        search_ready = false;
    }

    void reset() noexcept {
        release();
        idx = host::IndexData{};
        has_index = false;
    }

    void initialize_search_state() {  // chimera_index.cu:175-248
        if (search_ready) return;
        if (!has_index) throw std::runtime_error("Cannot initialize an empty Chimera index");
        if (static_cast<size_t>(options.nprobe) > idx.n_clusters) {
            throw std::invalid_argument("nprobe must not exceed the number of clusters");
        }
        const int n_dev = chimera_device_count();
        if (n_dev < 0) throw std::runtime_error(chimera_last_error());
        if (n_dev == 0) throw std::runtime_error("No HIP device is available");
        check(chimera_create(&ctx, 0), "chimera_create");
        chimera_index_desc d{};
        d.num_embeddings = idx.n;
        d.dimension = idx.d;
        d.num_clusters = idx.n_clusters;
        d.ex_bits = idx.ex_bits;
        d.num_docs = idx.num_docs();
        d.doc_ptrs = idx.doc_ptrs.data();
        d.cluster_pos = idx.cluster_pos.data();
        d.clustered_codes = idx.clustered_codes.data();
        d.clustered_factors = idx.clustered_factors.data();
        d.clustered_doc_ids = idx.clustered_doc_ids.data();
        d.token_to_cluster_pos = idx.token_to_cluster_pos.data();
        d.full_codes = idx.full_bit_codes.data();
        d.full_factors = idx.full_bit_factors.data();
        d.rotated_centroids = idx.rotated_centroids.data();
        d.rotator_flips = idx.flips.data();
        chimera_search_options o{options.nprobe, options.k_refine, options.k_full_bit, options.cagra_itopk_size,
                                 options.num_chunks};
        max_batch = max_batch_setting();
        check(chimera_upload_index(ctx, &d, &o, max_batch), "chimera_upload_index");
        search_ready = true;
    }

    // Sampling and the rotator seed on the host (build_index.cu:159-184,
    // rotator.hpp:183-189), everything else on the device; the host copy of
    // the index is kept for save() as the reference keeps its host vectors.
    void build_on_device(const float* embeddings, size_t n, size_t dimension, const std::vector<int32_t>& lens,
                         size_t n_clusters, size_t ex_bits) {
        if (static_cast<size_t>(options.nprobe) > n_clusters) {
            throw std::invalid_argument("nprobe must not exceed the number of clusters");
        }
        const std::vector<size_t> sampled = host::sample_centroid_ids(n, n_clusters);
        const std::vector<int64_t> ids(sampled.begin(), sampled.end());
        const host::FhtKacRotator rot(dimension, host::kPaddedDim, host::kRotatorSeed);
        check(chimera_create(&ctx, 0), "chimera_create");
        void* d_emb = nullptr;
        const size_t bytes = n * dimension * sizeof(float);
        check(chimera_device_alloc(ctx, &d_emb, bytes), "chimera_device_alloc");
        chimera_search_options o{options.nprobe, options.k_refine, options.k_full_bit, options.cagra_itopk_size,
                                 options.num_chunks};
        max_batch = max_batch_setting();
        int r = chimera_copy_to_device(ctx, d_emb, embeddings, bytes);
        if (r == CHIMERA_OK)
            r = chimera_build_index_device(ctx, static_cast<const float*>(d_emb), n, dimension, lens.data(), lens.size(),
                                           n_clusters, ex_bits, ids.data(), rot.flips().data(), &o, max_batch);
        const std::string msg = r == CHIMERA_OK ? std::string() : std::string(chimera_last_error());
        (void)chimera_device_free(ctx, d_emb);
        if (r != CHIMERA_OK) {
            if (r == CHIMERA_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
            throw std::runtime_error(msg);
        }
        host::IndexData& x = idx;
        x.n = n;
        x.d = dimension;
        x.n_clusters = n_clusters;
        x.ex_bits = ex_bits;
        x.flips = rot.flips();
        x.doc_lens = lens;
        x.doc_ptrs.assign(lens.size() + 1, 0);
        for (size_t i = 0; i < lens.size(); ++i) x.doc_ptrs[i + 1] = x.doc_ptrs[i] + lens[i];
        x.one_bit_codes.resize(n * 2);
        x.one_bit_factors.resize(n);
        x.full_bit_factors.resize(n);
        x.full_bit_codes.resize(n * x.full_code_bytes());
        x.clustered_codes.resize(n * host::kCodeBytes);
        x.clustered_factors.resize(n);
        x.clustered_doc_ids.resize(n);
        x.token_to_cluster_pos.resize(n);
        x.inv_list.resize(n);
        x.cluster_pos.resize(n_clusters + 1);
        x.rotated_centroids.resize(n_clusters * host::kPaddedDim);
        chimera_index_host h{};
        h.cluster_pos = x.cluster_pos.data();
        h.inv_list = x.inv_list.data();
        h.token_to_cluster_pos = x.token_to_cluster_pos.data();
        h.one_bit_codes = reinterpret_cast<uint8_t*>(x.one_bit_codes.data());
        h.one_bit_factors = x.one_bit_factors.data();
        h.full_codes = x.full_bit_codes.data();
        h.full_factors = x.full_bit_factors.data();
        h.clustered_codes = x.clustered_codes.data();
        h.clustered_factors = x.clustered_factors.data();
        h.clustered_doc_ids = x.clustered_doc_ids.data();
        h.rotated_centroids = x.rotated_centroids.data();
        check(chimera_download_index(ctx, &h), "chimera_download_index");
        has_index = true;
        search_ready = true;
    }

    void ensure_ready() {
        if (!has_index) throw std::runtime_error("Cannot search an empty Chimera index");
        if (!search_ready) {
            try {
                initialize_search_state();
            } catch (...) {
                reset();
                throw;
            }
        }
    }

    // Full-bit scoring never yields more documents than this, so larger k
    // values return the same lists.
    int32_t effective_k(size_t k) const {
        const size_t cap = static_cast<size_t>(std::max(options.k_refine, 1));
        return static_cast<int32_t>(std::min(k, cap));
    }

    std::vector<std::vector<size_t>> run(const float* queries, size_t nq, size_t k) {
        std::vector<std::vector<size_t>> out(nq);
        const int32_t kk = effective_k(k);
        std::vector<int64_t> ids;
        std::vector<int32_t> counts;
        for (size_t b = 0; b < nq; b += static_cast<size_t>(max_batch)) {
            const int32_t n = static_cast<int32_t>(std::min(nq - b, static_cast<size_t>(max_batch)));
            ids.assign(static_cast<size_t>(n) * kk, -1);
            counts.assign(static_cast<size_t>(n), 0);
            check(chimera_search(ctx, queries + b * host::kQueryLen * idx.d, n, kk, ids.data(), nullptr,
                                 counts.data()),
                  "chimera_search");
            for (int32_t q = 0; q < n; ++q) {
                auto& r = out[b + static_cast<size_t>(q)];
                r.reserve(static_cast<size_t>(counts[q]));
                for (int32_t j = 0; j < counts[q]; ++j) r.push_back(static_cast<size_t>(ids[static_cast<size_t>(q) * kk + j]));
            }
        }
        return out;
    }
};

chimera_index::chimera_index() : impl_(std::make_unique<Impl>()) {}
chimera_index::~chimera_index() = default;

void chimera_index::build(const std::vector<float>& embeddings, size_t dimension, const std::vector<int>& doc_lens,
                          size_t n_clusters, size_t ex_bits, const SearchOptions& options) {
    const std::vector<int32_t> lens(doc_lens.begin(), doc_lens.end());
    const size_t n = host::validate_build_inputs(embeddings.size(), dimension, lens, n_clusters, ex_bits);
    const int n_dev = chimera_device_count();
    if (n_dev < 0) throw std::runtime_error(chimera_last_error());
    if (n_dev == 0) throw std::runtime_error("No HIP device is available");
    impl_->reset();
    impl_->options = options;
    validate_search_options(options);
    try {
        impl_->build_on_device(embeddings.data(), n, dimension, lens, n_clusters, ex_bits);
    } catch (...) {
        impl_->reset();
        throw;
    }
}

std::vector<size_t> chimera_index::search(const std::vector<float>& query, size_t k) {
    return search(query.data(), query.size(), k);
}

std::vector<size_t> chimera_index::search(const float* query, size_t query_size, size_t k) {
    if (!impl_->has_index) throw std::runtime_error("Cannot search an empty Chimera index");
    if (query == nullptr || query_size != host::kQueryLen * impl_->idx.d) {
        throw std::invalid_argument("A Chimera query must have shape [" + std::to_string(host::kQueryLen) + ", " +
                                    std::to_string(impl_->idx.d) + "]");
    }
    if (k == 0) throw std::invalid_argument("k must be positive");
    impl_->ensure_ready();
    return impl_->run(query, 1, k).front();
}

std::vector<std::vector<size_t>> chimera_index::search_batch(const float* queries, size_t num_queries,
                                                             size_t query_size, size_t k) {
    if (!impl_->has_index) throw std::runtime_error("Cannot search an empty Chimera index");
    if ((queries == nullptr && num_queries > 0) || query_size != host::kQueryLen * impl_->idx.d) {
        throw std::invalid_argument("A Chimera query must have shape [" + std::to_string(host::kQueryLen) + ", " +
                                    std::to_string(impl_->idx.d) + "]");
    }
    if (k == 0) throw std::invalid_argument("k must be positive");
    if (num_queries == 0) return {};
    impl_->ensure_ready();
    return impl_->run(queries, num_queries, k);
}

void chimera_index::save(const std::string& index_dir) const {
    if (!impl_->has_index) throw std::runtime_error("Cannot save an empty Chimera index");
    host::save_index(impl_->idx, index_dir);
}

void chimera_index::load(const std::string& index_dir, const SearchOptions& options) {
    if (!std::filesystem::is_directory(index_dir)) {
        throw std::runtime_error("Chimera index directory does not exist: " + index_dir);
    }
    impl_->reset();
    impl_->options = options;
    validate_search_options(options);
    impl_->idx = host::load_index(index_dir, static_cast<size_t>(options.nprobe));
    impl_->has_index = true;
    try {
        impl_->initialize_search_state();
    } catch (...) {
        impl_->reset();
        throw;
    }
}

size_t chimera_index::num_embeddings() const { return impl_->idx.n; }
size_t chimera_index::dimension() const { return impl_->idx.d; }
size_t chimera_index::num_clusters() const { return impl_->idx.n_clusters; }
size_t chimera_index::ex_bits() const { return impl_->idx.ex_bits; }
size_t chimera_index::num_docs() const { return impl_->idx.num_docs(); }
const SearchOptions& chimera_index::options() const { return impl_->options; }

}  // namespace Chimera
