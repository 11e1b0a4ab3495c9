// Search shape limits (reference include/coraanns/search/parameters.hpp:9-25): query
// chunks of at most 65,535 (the ring record keeps 16-bit query and probe indices) and at
// most 65,536 probes, with the same accept/reject boundaries and exception type.
#pragma once

#include <climits>
#include <cstddef>
#include <stdexcept>

namespace coraanns {

inline constexpr std::size_t default_vanguard_size = 5;
inline constexpr int default_batch_q = 4;
// Default multiplier of the GPU filter's error term (HybridIndex::set_lower_bound_scale).
inline constexpr float default_bound_scale = 1.3f;
inline constexpr float max_bound_scale = 16.0f;
inline constexpr std::size_t max_query_chunk = 65535;
inline constexpr std::size_t max_probe_count = 65536;
// Cross-query reuse groups up to batch-q same-cluster pairs (the reference accepts 1..6);
// larger requests are accepted up to 64 and scanned at most 8 pairs per popcount pass
// (4 with the LUT4 estimator; the matrix-core scans take 16 at a time whatever batch-q is).
inline constexpr int max_batch_q = 64;

inline void validate_search_shape(std::size_t queries, std::size_t topk, std::size_t nprobe,
                                  std::size_t centroids, std::size_t padded_dim) {
    if (queries == 0 || queries > max_query_chunk)
        throw std::invalid_argument("query count must be in [1, 65535]; split larger batches");
    if (topk == 0 || topk > INT_MAX / queries)
        throw std::invalid_argument("topk must be positive and queries * topk must fit an int");
    if (nprobe == 0 || nprobe > max_probe_count || nprobe > centroids)
        throw std::invalid_argument("nprobe must be in [1, min(nlist, 65536)]");
    if (centroids > INT_MAX / queries || padded_dim == 0 || padded_dim > INT_MAX / (queries * 4))
        throw std::invalid_argument("query workspace exceeds kernel indexing limits");
}

}  // namespace coraanns
