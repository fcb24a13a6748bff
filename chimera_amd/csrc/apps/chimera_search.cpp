// chimera_search: the search command of the reference (cpp/apps/search.cpp,
// flags and checks of cpp/apps/utils.cpp:85-183). It loads an index
// directory, a query file ([int32 count, int32 length, int32 dim] + fp32) and
// a ground-truth TSV, runs `--warmup` queries, then times each of `--nq`
// queries one at a time and prints the reference's two report lines
//   [SEARCH] latency_ms mean=... min=... p50=... p90=... p95=... p99=... max=... stddev=...
//   [SEARCH] recall@k=...            (and recall@10 when k is 100)
// followed by one line for the same queries as a single batched call:
//   [SEARCH] batch queries=N ms=T qps=Q
#include "chimera/chimera_index.hpp"
#include "chimera/search_report.hpp"
#include "index_store.hpp"

#include <algorithm>
#include <chrono>
#include <filesystem>
#include <iomanip>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

using Chimera::SearchOptions;

struct Args {
    int k = 100;
    int nq = -1;
    int warmup = 5;
    std::string query_file, gt_file, index_dir;
    SearchOptions options;
};

struct HelpRequested {};

void usage(const char* prog) {
    const Args d;
    std::cout << "Usage: " << prog << "\n"
              << "  --query <query_embeddings.bin>\n"
              << "  --gt <groundtruth.tsv>\n"
              << "  --index <index_dir>\n"
              << "  [--k <top_k>]                   Final documents returned. Default: " << d.k << "\n"
              << "  [--nq <num_queries>]            Evaluation queries; -1 means all. Default: " << d.nq << "\n"
              << "  [--warmup <num_queries>]        Warmup queries. Default: " << d.warmup << "\n"
              << "  [--nprobe <num_probes>]         IVF clusters probed per query token. Default: "
              << d.options.nprobe << "\n"
              << "  [--k-refine <count>]            Candidates retained after refinement. Default: "
              << d.options.k_refine << "\n"
              << "  [--k-full-bit <count>]          Candidates scored with full-bit codes. Default: "
              << d.options.k_full_bit << "\n"
              << "  [--cagra-itopk-size <count>]    Accepted for compatibility (the probe is exact). Default: "
              << d.options.cagra_itopk_size << "\n"
              << "  [--num-chunks <count>]          Collaborative-scoring chunks. Default: " << d.options.num_chunks
              << "\n";
}

Args parse(int argc, char** argv) {
    if (argc == 1) throw HelpRequested{};
    Args a;
    auto value = [&](int& i, const std::string& flag) -> std::string {
        if (i + 1 >= argc) throw std::runtime_error("Missing value for " + flag);
        return argv[++i];
    };
    for (int i = 1; i < argc; ++i) {
        const std::string f = argv[i];
        if (f == "--help" || f == "-h") throw HelpRequested{};
        if (f == "--query" || f == "-q") {
            a.query_file = value(i, f);
        } else if (f == "--gt" || f == "-g") {
            a.gt_file = value(i, f);
        } else if (f == "--index" || f == "-i") {
            a.index_dir = value(i, f);
        } else if (f == "--k") {
            a.k = std::stoi(value(i, f));
        } else if (f == "--nq") {
            a.nq = std::stoi(value(i, f));
        } else if (f == "--warmup") {
            a.warmup = std::stoi(value(i, f));
        } else if (f == "--nprobe") {
            a.options.nprobe = std::stoi(value(i, f));
        } else if (f == "--k-refine") {
            a.options.k_refine = std::stoi(value(i, f));
        } else if (f == "--k-full-bit") {
            a.options.k_full_bit = std::stoi(value(i, f));
        } else if (f == "--cagra-itopk-size") {
            a.options.cagra_itopk_size = std::stoi(value(i, f));
        } else if (f == "--num-chunks") {
            a.options.num_chunks = std::stoi(value(i, f));
        } else {
            throw std::runtime_error("Unknown argument: " + f);
        }
    }
    if (a.query_file.empty() || a.gt_file.empty() || a.index_dir.empty())
        throw std::runtime_error("Missing required arguments.");
    if (!std::filesystem::is_directory(a.index_dir))
        throw std::runtime_error("--index must point to a Chimera index directory.");
    if (!std::filesystem::exists(std::filesystem::path(a.index_dir) / "doclens.bin"))
        throw std::runtime_error("Missing doclens.bin in --index.");
    if (a.k <= 0) throw std::runtime_error("--k must be > 0");
    if (a.warmup < 0) throw std::runtime_error("--warmup must be >= 0");
    const SearchOptions& o = a.options;
    if (o.nprobe <= 0) throw std::runtime_error("--nprobe must be > 0");
    if (o.k_refine <= 0) throw std::runtime_error("--k-refine must be > 0");
    if (o.k_full_bit <= 0) throw std::runtime_error("--k-full-bit must be > 0");
    if (o.cagra_itopk_size <= 0) throw std::runtime_error("--cagra-itopk-size must be > 0");
    if (o.num_chunks <= 0) throw std::runtime_error("--num-chunks must be > 0");
    if (o.k_full_bit > o.k_refine) throw std::runtime_error("--k-full-bit must not exceed --k-refine");
    return a;
}

}  // namespace

int main(int argc, char** argv) {
    Args args;
    try {
        args = parse(argc, argv);
    } catch (const HelpRequested&) {
        usage(argv[0]);
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "Argument error: " << e.what() << "\n\n";
        usage(argv[0]);
        return 1;
    }
    constexpr size_t kQueryTokens = 32;

    size_t num_q = 0, d = 0, qlen = 0;
    const std::vector<float> queries = Chimera::host::load_query(qlen, num_q, d, args.query_file);
    std::vector<std::vector<size_t>> gt;
    try {
        gt = Chimera::read_gt_tsv(static_cast<int>(num_q), 1000, args.gt_file);
    } catch (const std::exception& e) {
        // the reference's command stops here with status 0
        std::cerr << "Warning: " << e.what() << ". Skipping." << std::endl;
        return 0;
    }
    if (qlen != kQueryTokens) {
        std::cerr << "Query length " << qlen << " does not match compiled Q_DOCLEN=" << kQueryTokens << '\n';
        return 1;
    }
    const int warm = std::min<int>(args.warmup, static_cast<int>(num_q));
    const int runs = args.nq < 0 ? static_cast<int>(num_q) : std::min<int>(args.nq, static_cast<int>(num_q));
    if (runs == 0) {
        std::cerr << "No evaluation queries selected.\n";
        return 1;
    }
    const std::vector<std::vector<size_t>> eval_gt(gt.begin(), gt.begin() + runs);

    Chimera::chimera_index index;
    index.load(args.index_dir, args.options);
    const size_t qsize = kQueryTokens * d;
    for (int i = 0; i < warm; ++i) index.search(queries.data() + static_cast<size_t>(i) * qsize, qsize, args.k);

    std::vector<std::vector<size_t>> results(static_cast<size_t>(runs));
    std::vector<double> ms(static_cast<size_t>(runs));
    for (int i = 0; i < runs; ++i) {
        const auto t0 = std::chrono::high_resolution_clock::now();
        results[i] = index.search(queries.data() + static_cast<size_t>(i) * qsize, qsize, args.k);
        const auto t1 = std::chrono::high_resolution_clock::now();
        ms[i] = std::chrono::duration<double, std::milli>(t1 - t0).count();
    }

    const Chimera::QueryLatencySummary s = Chimera::summarize_query_latencies_ms(ms);
    std::cout << std::fixed << std::setprecision(3) << "[SEARCH] latency_ms mean=" << s.mean_ms
              << " min=" << s.min_ms << " p50=" << s.p50_ms << " p90=" << s.p90_ms << " p95=" << s.p95_ms
              << " p99=" << s.p99_ms << " max=" << s.max_ms << " stddev=" << s.stddev_ms << '\n';
    std::cout << "[SEARCH] recall@" << args.k << '=' << Chimera::compute_recall(eval_gt, results, args.k) << '\n';
    if (args.k == 100) std::cout << "[SEARCH] recall@10=" << Chimera::compute_recall(eval_gt, results, 10) << '\n';

    // the same queries as one batched device call
    const auto b0 = std::chrono::high_resolution_clock::now();
    const std::vector<std::vector<size_t>> batch =
        index.search_batch(queries.data(), static_cast<size_t>(runs), qsize, args.k);
    const auto b1 = std::chrono::high_resolution_clock::now();
    const double bms = std::chrono::duration<double, std::milli>(b1 - b0).count();
    std::cout << std::fixed << std::setprecision(3) << "[SEARCH] batch queries=" << runs << " ms=" << bms
              << " qps=" << (bms > 0.0 ? 1000.0 * runs / bms : 0.0) << '\n';
    return batch.size() == results.size() ? 0 : 1;
}
