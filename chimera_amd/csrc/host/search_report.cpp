// Latency summary, ground-truth reader and recall@k of the search command.
// Semantics: cpp/apps/utils.cpp:186-290 of the reference.
#include "chimera/search_report.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <fstream>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <unordered_set>

namespace Chimera {

double percentile_ms(const std::vector<double>& sorted_ms, double pct) {
    if (sorted_ms.empty()) return 0.0;
    const double p = std::min(100.0, std::max(0.0, pct));
    const double pos = p / 100.0 * static_cast<double>(sorted_ms.size() - 1);
    const size_t below = static_cast<size_t>(std::floor(pos));
    const size_t above = static_cast<size_t>(std::ceil(pos));
    const double t = pos - static_cast<double>(below);
    return sorted_ms[below] * (1.0 - t) + sorted_ms[above] * t;
}

QueryLatencySummary summarize_query_latencies_ms(const std::vector<double>& latencies_ms) {
    QueryLatencySummary s;
    if (latencies_ms.empty()) return s;
    std::vector<double> v(latencies_ms);
    std::sort(v.begin(), v.end());
    double total = 0.0;
    for (double x : v) total += x;
    const double n = static_cast<double>(v.size());
    s.mean_ms = total / n;
    double ss = 0.0;
    for (double x : v) ss += (x - s.mean_ms) * (x - s.mean_ms);
    s.stddev_ms = std::sqrt(ss / n);
    s.min_ms = v.front();
    s.max_ms = v.back();
    s.p50_ms = percentile_ms(v, 50.0);
    s.p90_ms = percentile_ms(v, 90.0);
    s.p95_ms = percentile_ms(v, 95.0);
    s.p99_ms = percentile_ms(v, 99.0);
    return s;
}

std::vector<std::vector<size_t>> read_gt_tsv(int num_queries, int top_k, const std::string& gt_filename) {
    std::vector<std::vector<size_t>> table(static_cast<size_t>(std::max(0, num_queries)),
                                           std::vector<size_t>(static_cast<size_t>(std::max(0, top_k)), SIZE_MAX));
    std::ifstream in(gt_filename);
    if (!in) {
        std::cerr << "Error: Could not open file " << gt_filename << std::endl;
        return table;
    }
    std::string line;
    while (std::getline(in, line)) {
        std::vector<std::string> cols;
        std::stringstream ls(line);
        std::string col;
        while (std::getline(ls, col, '\t')) cols.push_back(col);
        if (cols.size() < 3) {
            std::cerr << "Warning: Skipping malformed line." << std::endl;
            continue;
        }
        const long long qid = std::stoll(cols[0]);
        const unsigned long long doc = std::stoull(cols[1]);
        const long long rank = std::stoll(cols[2]);
        if (rank < 1 || rank > top_k)
            throw std::runtime_error("Rank " + std::to_string(rank) + " exceeds top_k " + std::to_string(top_k));
        if (qid < 0 || qid >= num_queries)
            throw std::runtime_error("Query id " + std::to_string(qid) + " outside [0, " +
                                     std::to_string(num_queries) + ")");
        table[static_cast<size_t>(qid)][static_cast<size_t>(rank - 1)] = static_cast<size_t>(doc);
    }
    return table;
}

double compute_recall(const std::vector<std::vector<size_t>>& ground_truth,
                      const std::vector<std::vector<size_t>>& retrieved, int top_k) {
    if (top_k <= 0) return 0.0;
    long long hits = 0;
    for (size_t i = 0; i < retrieved.size(); ++i) {
        const std::vector<size_t>& r = retrieved[i];
        const size_t rn = std::min(r.size(), static_cast<size_t>(top_k));
        const std::unordered_set<size_t> got(r.begin(), r.begin() + static_cast<std::ptrdiff_t>(rn));
        const std::vector<size_t>& g = ground_truth.at(i);
        const size_t gn = std::min(g.size(), static_cast<size_t>(top_k));
        for (size_t j = 0; j < gn; ++j) hits += got.count(g[j]) ? 1 : 0;
    }
    return static_cast<double>(hits) / (static_cast<double>(retrieved.size()) * top_k);
}

}  // namespace Chimera
