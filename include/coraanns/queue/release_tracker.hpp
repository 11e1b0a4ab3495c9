// Prefix release of consumed ring chunks (semantics of the reference
// include/coraanns/queue/release_tracker.hpp:14-57): workers claim chunks in any order,
// but Progress::released only advances over a contiguous prefix of completed chunks, so
// the GPU never overwrites a slot a slow worker has not finished. Completion tags hold
// the full logical end position, which distinguishes ring generations.
#pragma once

#include <cstddef>
#include <mutex>
#include <stdexcept>
#include <vector>

#include "coraanns/queue/candidate_queue.hpp"

namespace coraanns::queue {

class ReleaseTracker {
  public:
    ReleaseTracker(Progress &progress, std::size_t capacity, std::size_t chunk_size)
        : progress_(progress), capacity_(capacity), chunk_(chunk_size) {
        const auto pow2 = [](std::size_t v) { return v != 0 && (v & (v - 1)) == 0; };
        if (!pow2(capacity) || !pow2(chunk_size) || chunk_size > capacity)
            throw std::invalid_argument("invalid ring capacity/chunk size");
        end_tag_.assign(capacity / chunk_size, 0);
    }

    Position released() const { return __atomic_load_n(&progress_.released, __ATOMIC_ACQUIRE); }

    // A claim at logical position `start` may be read once its generation is live.
    bool readable_generation(Position start) const { return start < released() + capacity_; }

    // Call after the whole physical chunk has been cleared to the empty pattern.
    void complete(Position start) {
        std::lock_guard<std::mutex> lock(mutex_);
        const std::size_t slots = end_tag_.size();
        end_tag_[(start / chunk_) & (slots - 1)] = start + chunk_;
        Position r = __atomic_load_n(&progress_.released, __ATOMIC_RELAXED);
        const Position before = r;
        while (end_tag_[(r / chunk_) & (slots - 1)] == r + chunk_)
            r += chunk_;
        if (r != before)
            __atomic_store_n(&progress_.released, r, __ATOMIC_RELEASE);
    }

  private:
    Progress &progress_;
    Position capacity_;
    Position chunk_;
    std::vector<Position> end_tag_;
    std::mutex mutex_;
};

}  // namespace coraanns::queue
