// Measurement helpers of the search command (chimera_search): per-query
// latency summary, ground-truth TSV reader and recall@k, with the meaning the
// reference gives them in cpp/apps/utils.cpp:186-290 and cpp/apps/utils.hpp.
#pragma once

#include <cstddef>
#include <string>
#include <vector>

namespace Chimera {

// utils.hpp:32-41.
struct QueryLatencySummary {
    double mean_ms = 0.0;
    double stddev_ms = 0.0;  // population standard deviation
    double min_ms = 0.0;
    double p50_ms = 0.0;
    double p90_ms = 0.0;
    double p95_ms = 0.0;
    double p99_ms = 0.0;
    double max_ms = 0.0;
};

// utils.cpp:186-197: linear interpolation between the two order statistics
// around pct / 100 * (n - 1) of an ascending list; 0 for an empty list.
double percentile_ms(const std::vector<double>& sorted_ms, double pct);

// utils.cpp:199-224. All fields 0 for an empty list.
QueryLatencySummary summarize_query_latencies_ms(const std::vector<double>& latencies_ms);

// utils.cpp:226-263. Lines "query_id<TAB>doc_id<TAB>rank[<TAB>...]" with
// 1-based ranks fill a [num_queries][top_k] table whose other entries stay
// SIZE_MAX. A file that cannot be opened leaves the table unfilled (a
// message goes to stderr); lines with fewer than three fields are skipped
// with a warning. A rank outside [1, top_k] or a query id outside
// [0, num_queries) throws std::runtime_error (the reference's command exits
// with status 0 on such a rank; chimera_search does the same).
std::vector<std::vector<size_t>> read_gt_tsv(int num_queries, int top_k, const std::string& gt_filename);

// utils.cpp:265-290: sum over the retrieved queries of |gt[i][:k] ∩
// retrieved[i][:k]| divided by (number of retrieved queries * k); 0 for
// k <= 0.
double compute_recall(const std::vector<std::vector<size_t>>& ground_truth,
                      const std::vector<std::vector<size_t>>& retrieved, int top_k);

}  // namespace Chimera
