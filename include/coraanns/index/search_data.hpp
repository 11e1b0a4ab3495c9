// Host arrays HybridIndex::load_from_raw_pointers consumes, adapted from an IVF file
// (reference include/coraanns/index/search_data.hpp:14-30, src/index/search_data.cpp:9-127):
// FastScan-packed sign codes unpacked to per-cluster word-major u32 words (dimension
// 32w+l at bit 31-l of word w), AoS short factors, ex-codes compacted to a dense
// [num][padded_dim*ex_bits/8] array, and the rotator. The engine builds its GPU tile
// layout from these arrays.
#pragma once

#include <sys/mman.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "coraanns/index/ivf_file.hpp"

namespace coraanns::index {

// Allocator of the multi-GB host arrays that the CPU refinement reads at random (ex-codes,
// ex-factors, ids): blocks of 4 MB and more are 2 MB aligned and marked MADV_HUGEPAGE before
// their first touch, so that where transparent huge pages are in madvise mode the kernel
// backs them with huge pages and a random record read rarely misses the TLB (measured on
// the benchmark host: a config-5-sized consumer run 12.6 -> 8.8 ms). Smaller blocks come from
// operator new. The advice is best effort: without huge pages the memory is ordinary.
template <class T>
class HugePageAllocator {
  public:
    using value_type = T;
    static constexpr std::size_t kHuge = std::size_t{2} << 20, kMin = std::size_t{4} << 20;
    HugePageAllocator() noexcept = default;
    template <class U>
    HugePageAllocator(const HugePageAllocator<U> &) noexcept {}
    T *allocate(std::size_t n) {
        const std::size_t bytes = n * sizeof(T);
        if (bytes < kMin)
            return static_cast<T *>(::operator new(bytes));
        const std::size_t size = (bytes + kHuge - 1) / kHuge * kHuge;
        void *p = std::aligned_alloc(kHuge, size);
        if (!p)
            throw std::bad_alloc();
        (void)madvise(p, size, MADV_HUGEPAGE);
        return static_cast<T *>(p);
    }
    void deallocate(T *p, std::size_t n) noexcept {
        if (n * sizeof(T) < kMin)
            ::operator delete(p);
        else
            std::free(p);
    }
    template <class U>
    bool operator==(const HugePageAllocator<U> &) const noexcept {
        return true;
    }
    template <class U>
    bool operator!=(const HugePageAllocator<U> &) const noexcept {
        return false;
    }
};

template <class T>
using HugeVector = std::vector<T, HugePageAllocator<T>>;

class SearchData {
  public:
    // From an index already in memory (the reference constructor's signature). The
    // ex-codes are compacted in the IVF's own ex-data storage, which SearchData takes over.
    // include_extended = false keeps only the short codes (exact FP32 refine mode).
    SearchData(IvfFile &source, bool include_extended, int cpu_threads = 0);

    // Streaming load straight from an index file: batch data and ex data are read in
    // bounded chunks (a reader thread overlaps the next read with the unpacking of the
    // current chunk), so the peak host memory is the adapted arrays plus two chunks, not
    // the file plus the arrays. header / ids (may be null) receive the file's header and
    // the cluster-order ids.
    static std::unique_ptr<SearchData> load(const std::string &path, bool include_extended,
                                            int cpu_threads = 0, IvfHeader *header = nullptr,
                                            HugeVector<uint32_t> *ids = nullptr);

    std::vector<float> h_centroids, host_rotator, host_short_factors;
    HugeVector<float> host_ex_factors;
    std::vector<uint32_t> host_short_data;
    std::vector<std::size_t> cluster_sizes;
    uint8_t *host_long_codes = nullptr;
    std::size_t max_cluster_size = 0;

  private:
    SearchData() = default;
    std::vector<uint8_t> extended_storage_;  // the IVF's own ex-data, compacted (in-memory constructor)
    HugeVector<uint8_t> extended_huge_;      // streamed load
};

// Sign bits of one 32-vector FastScan block, restating the unpack of
// search_data.cpp:60-72: byte = codes[(d/8)*32 + (d%8 < 4 ? 0 : 16) + invPerm0[v%16]],
// nibble = v < 16 ? low : high, bit = (nibble >> (3 - d%4)) & 1.
// out: [batch_len][padded_dim/32] words, dimension 32w+l at bit 31-l.
void unpack_fastscan_block(const uint8_t *codes, std::size_t padded_dim, std::size_t batch_len,
                           uint32_t *out_words);

}  // namespace coraanns::index
