// pybind11 module `chimera`: the reference's Python surface
// (python/bindings.cpp:19-166) - ChimeraIndex.build / load (static), search,
// save - with the same argument names, defaults, shapes, return types and
// exception mapping (std::invalid_argument -> ValueError, runtime_error ->
// RuntimeError). A [Q, 32, d] query batch is one batched device call instead
// of Q serial calls.
//
// Underscore-prefixed module functions expose the host index arrays and the
// host codec to Python tests; they are not part of the reference surface.
#include "chimera/chimera_index.hpp"
#include "chimera/search_report.hpp"

#include "codec.hpp"
#include "index_store.hpp"

#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

namespace py = pybind11;

namespace {

using Chimera::SearchOptions;
using Chimera::chimera_index;
using FloatArray = py::array_t<float, py::array::c_style>;

SearchOptions search_options(int nprobe, int k_refine, int k_full_bit, int cagra_itopk_size, int num_chunks) {
    return {nprobe, k_refine, k_full_bit, cagra_itopk_size, num_chunks};
}

std::unique_ptr<chimera_index> build(const FloatArray& embeddings, const std::vector<int>& doc_lens,
                                     size_t n_clusters, size_t ex_bits, int nprobe, int k_refine, int k_full_bit,
                                     int cagra_itopk_size, int num_chunks) {
    if (embeddings.ndim() != 2) throw std::invalid_argument("embeddings must have shape [num_embeddings, dimension]");
    std::vector<float> data(embeddings.data(), embeddings.data() + embeddings.size());
    const size_t dim = static_cast<size_t>(embeddings.shape(1));
    auto index = std::make_unique<chimera_index>();
    {
        py::gil_scoped_release release;
        index->build(data, dim, doc_lens, n_clusters, ex_bits,
                     search_options(nprobe, k_refine, k_full_bit, cagra_itopk_size, num_chunks));
    }
    return index;
}

std::unique_ptr<chimera_index> load(const std::string& index_dir, int nprobe, int k_refine, int k_full_bit,
                                    int cagra_itopk_size, int num_chunks) {
    auto index = std::make_unique<chimera_index>();
    {
        py::gil_scoped_release release;
        index->load(index_dir, search_options(nprobe, k_refine, k_full_bit, cagra_itopk_size, num_chunks));
    }
    return index;
}

py::object search(chimera_index& index, const FloatArray& queries, size_t k) {
    if (queries.ndim() != 2 && queries.ndim() != 3) {
        throw std::invalid_argument(
            "queries must have shape [query_length, dimension] or [num_queries, query_length, dimension]");
    }
    const size_t num_queries = queries.ndim() == 3 ? static_cast<size_t>(queries.shape(0)) : 1;
    const size_t query_length = static_cast<size_t>(queries.shape(queries.ndim() - 2));
    const size_t dimension = static_cast<size_t>(queries.shape(queries.ndim() - 1));
    const size_t query_size = query_length * dimension;
    const float* data = queries.data();
    std::vector<std::vector<size_t>> results;
    {
        py::gil_scoped_release release;
        if (queries.ndim() == 2) {
            results.push_back(index.search(data, query_size, k));
        } else {
            results = index.search_batch(data, num_queries, query_size, k);
        }
    }
    if (queries.ndim() == 2) return py::cast(std::move(results.front()));
    return py::cast(std::move(results));
}

void save(const chimera_index& index, const std::string& index_dir) {
    py::gil_scoped_release release;
    index.save(index_dir);
}

template <typename T>
py::array_t<T> to_numpy(const std::vector<T>& v) {
    py::array_t<T> a(static_cast<py::ssize_t>(v.size()));
    if (!v.empty()) std::memcpy(a.mutable_data(), v.data(), v.size() * sizeof(T));
    return a;
}

py::dict index_dict(const Chimera::host::IndexData& x) {
    py::dict d;
    d["num_embeddings"] = x.n;
    d["dimension"] = x.d;
    d["num_clusters"] = x.n_clusters;
    d["ex_bits"] = x.ex_bits;
    d["flips"] = to_numpy(x.flips);
    d["one_bit_codes"] = to_numpy(x.one_bit_codes);
    d["one_bit_factors"] = to_numpy(x.one_bit_factors);
    d["full_bit_factors"] = to_numpy(x.full_bit_factors);
    d["full_bit_codes"] = to_numpy(x.full_bit_codes);
    d["clustered_codes"] = to_numpy(x.clustered_codes);
    d["clustered_factors"] = to_numpy(x.clustered_factors);
    d["clustered_doc_ids"] = to_numpy(x.clustered_doc_ids);
    d["token_to_cluster_pos"] = to_numpy(x.token_to_cluster_pos);
    d["inv_list"] = to_numpy(x.inv_list);
    d["cluster_pos"] = to_numpy(x.cluster_pos);
    d["doc_lens"] = to_numpy(x.doc_lens);
    d["doc_ptrs"] = to_numpy(x.doc_ptrs);
    d["rotated_centroids"] = to_numpy(x.rotated_centroids);
    return d;
}

py::dict build_index_arrays(const FloatArray& embeddings, const std::vector<int32_t>& doc_lens, size_t n_clusters,
                            size_t ex_bits, const std::string& save_dir) {
    if (embeddings.ndim() != 2) throw std::invalid_argument("embeddings must have shape [num_embeddings, dimension]");
    Chimera::host::IndexData x;
    {
        py::gil_scoped_release release;
        x = Chimera::host::build_index(embeddings.data(), static_cast<size_t>(embeddings.shape(0)),
                                       static_cast<size_t>(embeddings.shape(1)), doc_lens, n_clusters, ex_bits);
        if (!save_dir.empty()) Chimera::host::save_index(x, save_dir);
    }
    return index_dict(x);
}

py::dict read_index(const std::string& dir) {
    Chimera::host::IndexData x;
    {
        py::gil_scoped_release release;
        x = Chimera::host::load_index(dir);
    }
    return index_dict(x);
}

FloatArray rotate(const FloatArray& src, const py::array_t<uint8_t, py::array::c_style>& flips) {
    if (src.ndim() != 2) throw std::invalid_argument("src must be [n, dim]");
    if (flips.size() != static_cast<py::ssize_t>(Chimera::host::kFlipBytes)) throw std::invalid_argument("flips must have 64 bytes");
    const size_t n = static_cast<size_t>(src.shape(0)), dim = static_cast<size_t>(src.shape(1));
    Chimera::host::FhtKacRotator rot(dim, Chimera::host::kPaddedDim, flips.data());
    FloatArray out({static_cast<py::ssize_t>(n), static_cast<py::ssize_t>(Chimera::host::kPaddedDim)});
    for (size_t i = 0; i < n; ++i) rot.rotate(src.data() + i * dim, out.mutable_data() + i * Chimera::host::kPaddedDim);
    return out;
}

py::array_t<uint8_t> rotator_flips(uint64_t seed, size_t dim) {
    Chimera::host::FhtKacRotator rot(dim, Chimera::host::kPaddedDim, seed);
    return to_numpy(rot.flips());
}

py::tuple encode_one_bit(const FloatArray& rot) {
    const size_t n = static_cast<size_t>(rot.shape(0));
    py::array_t<uint64_t> codes({static_cast<py::ssize_t>(n), py::ssize_t{2}});
    py::array_t<float> f(static_cast<py::ssize_t>(n));
    for (size_t i = 0; i < n; ++i)
        Chimera::host::encode_one_bit(rot.data() + i * 128, 128, codes.mutable_data() + 2 * i, f.mutable_data() + i);
    return py::make_tuple(codes, f);
}

py::tuple encode_full(const FloatArray& rot, size_t ex_bits) {
    const size_t n = static_cast<size_t>(rot.shape(0));
    const size_t bytes = 16 * (1 + ex_bits);
    py::array_t<uint8_t> codes({static_cast<py::ssize_t>(n), static_cast<py::ssize_t>(bytes)});
    py::array_t<float> f(static_cast<py::ssize_t>(n));
    for (size_t i = 0; i < n; ++i)
        Chimera::host::encode_full_code(rot.data() + i * 128, 128, ex_bits, codes.mutable_data() + i * bytes,
                                        f.mutable_data() + i);
    return py::make_tuple(codes, f);
}

py::array_t<uint8_t> quantize_ex(const FloatArray& rot, size_t ex_bits) {
    const size_t n = static_cast<size_t>(rot.shape(0));
    py::array_t<uint8_t> out({static_cast<py::ssize_t>(n), py::ssize_t{128}});
    for (size_t i = 0; i < n; ++i)
        Chimera::host::quantize_ex(rot.data() + i * 128, out.mutable_data() + i * 128, 128, ex_bits);
    return out;
}

py::array_t<uint8_t> pack(const py::array_t<uint8_t, py::array::c_style>& raw, size_t width) {
    const size_t n = static_cast<size_t>(raw.shape(0));
    const size_t bytes = 16 * width;
    py::array_t<uint8_t> out({static_cast<py::ssize_t>(n), static_cast<py::ssize_t>(bytes)});
    for (size_t i = 0; i < n; ++i) Chimera::host::pack_codes(raw.data() + i * 128, out.mutable_data() + i * bytes, 128, width);
    return out;
}

py::array_t<uint8_t> unpack(const py::array_t<uint8_t, py::array::c_style>& packed, size_t width) {
    const size_t n = static_cast<size_t>(packed.shape(0));
    py::array_t<uint8_t> out({static_cast<py::ssize_t>(n), py::ssize_t{128}});
    for (size_t i = 0; i < n; ++i)
        Chimera::host::unpack_codes(packed.data() + i * 16 * width, out.mutable_data() + i * 128, 128, width);
    return out;
}

}  // namespace

PYBIND11_MODULE(chimera, module) {
    const SearchOptions defaults;
    // measurement helpers of the search command (cpp/apps/utils.cpp:186-290)
    module.def("percentile_ms", &Chimera::percentile_ms, py::arg("sorted_ms"), py::arg("pct"));
    module.def(
        "summarize_query_latencies_ms",
        [](const std::vector<double>& ms) {
            const Chimera::QueryLatencySummary s = Chimera::summarize_query_latencies_ms(ms);
            py::dict d;
            d["mean_ms"] = s.mean_ms;
            d["stddev_ms"] = s.stddev_ms;
            d["min_ms"] = s.min_ms;
            d["p50_ms"] = s.p50_ms;
            d["p90_ms"] = s.p90_ms;
            d["p95_ms"] = s.p95_ms;
            d["p99_ms"] = s.p99_ms;
            d["max_ms"] = s.max_ms;
            return d;
        },
        py::arg("latencies_ms"));
    module.def("read_gt_tsv", &Chimera::read_gt_tsv, py::arg("num_queries"), py::arg("top_k"), py::arg("gt_filename"));
    module.def("compute_recall", &Chimera::compute_recall, py::arg("ground_truth"), py::arg("retrieved"),
               py::arg("top_k"));
    auto index = py::class_<chimera_index>(module, "ChimeraIndex");
    index
        .def_static("build", &build, py::arg("embeddings").noconvert(), py::arg("doc_lens"), py::arg("n_clusters"),
                    py::arg("ex_bits"), py::arg("nprobe") = defaults.nprobe, py::arg("k_refine") = defaults.k_refine,
                    py::arg("k_full_bit") = defaults.k_full_bit,
                    py::arg("cagra_itopk_size") = defaults.cagra_itopk_size,
                    py::arg("num_chunks") = defaults.num_chunks)
        .def("search", &search, py::arg("queries").noconvert(), py::arg("k") = 100)
        .def("save", &save, py::arg("index_dir"))
        .def_static("load", &load, py::arg("index_dir"), py::arg("nprobe") = defaults.nprobe,
                    py::arg("k_refine") = defaults.k_refine, py::arg("k_full_bit") = defaults.k_full_bit,
                    py::arg("cagra_itopk_size") = defaults.cagra_itopk_size,
                    py::arg("num_chunks") = defaults.num_chunks);
    if (py::hasattr(index, "_pybind11_conduit_v1_")) py::delattr(index, "_pybind11_conduit_v1_");

    module.def("_build_index", &build_index_arrays, py::arg("embeddings").noconvert(), py::arg("doc_lens"),
               py::arg("n_clusters"), py::arg("ex_bits"), py::arg("save_dir") = std::string());
    module.def("_read_index", &read_index, py::arg("index_dir"));
    module.def("_rotate", &rotate, py::arg("src").noconvert(), py::arg("flips"));
    module.def("_rotator_flips", &rotator_flips, py::arg("seed"), py::arg("dim") = 128);
    module.def("_encode_one_bit", &encode_one_bit, py::arg("rotated").noconvert());
    module.def("_encode_full", &encode_full, py::arg("rotated").noconvert(), py::arg("ex_bits"));
    module.def("_quantize_ex", &quantize_ex, py::arg("rotated").noconvert(), py::arg("ex_bits"));
    module.def("_pack", &pack, py::arg("raw"), py::arg("width"));
    module.def("_unpack", &unpack, py::arg("packed"), py::arg("width"));
    module.def("_sample_centroid_ids", &Chimera::host::sample_centroid_ids, py::arg("num_embeddings"),
               py::arg("n_clusters"));
    module.def("_best_rescale_factor", [](const FloatArray& o_abs, size_t ex_bits) {
        return Chimera::host::best_rescale_factor(o_abs.data(), static_cast<size_t>(o_abs.size()), ex_bits);
    });
}
