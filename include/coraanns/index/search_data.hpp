// Host arrays HybridIndex::load_from_raw_pointers consumes, adapted from an IVF file
// (reference include/coraanns/index/search_data.hpp:14-30, src/index/search_data.cpp:9-127):
// FastScan-packed sign codes unpacked to per-cluster word-major u32 words (dimension
// 32w+l at bit 31-l of word w), AoS short factors, ex-codes compacted to a dense
// [num][padded_dim*ex_bits/8] array (taking over the IVF's ex-data storage), and the
// rotator. The engine builds its GPU tile layout from these arrays.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "coraanns/index/ivf_file.hpp"

namespace coraanns::index {

class SearchData {
  public:
    // include_extended = false keeps only the short codes (exact FP32 refine mode).
    SearchData(IvfFile &source, bool include_extended, int cpu_threads = 0);
    std::vector<float> h_centroids, host_rotator, host_short_factors, host_ex_factors;
    std::vector<uint32_t> host_short_data;
    std::vector<std::size_t> cluster_sizes;
    uint8_t *host_long_codes = nullptr;
    std::size_t max_cluster_size = 0;

  private:
    std::vector<uint8_t> extended_storage_;
};

// Sign bits of one 32-vector FastScan block, restating the unpack of
// search_data.cpp:60-72: byte = codes[(d/8)*32 + (d%8 < 4 ? 0 : 16) + invPerm0[v%16]],
// nibble = v < 16 ? low : high, bit = (nibble >> (3 - d%4)) & 1.
// out: [batch_len][padded_dim/32] words, dimension 32w+l at bit 31-l.
void unpack_fastscan_block(const uint8_t *codes, std::size_t padded_dim, std::size_t batch_len,
                           uint32_t *out_words);

}  // namespace coraanns::index
