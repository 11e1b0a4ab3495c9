// GPU->CPU candidate ring wire format. Byte-compatible with the reference's
// include/coraanns/queue/candidate_queue.hpp:10-55 so that a consumer written against
// the reference reads this engine's ring unchanged: 16-byte Candidate records, a
// 64-byte-aligned Progress block, all-ones bytes marking an empty slot.
#pragma once

#include <cstddef>
#include <cstdint>
#include <type_traits>

namespace coraanns::queue {

// Monotonic logical ring position (64-bit so wraps never alias).
using Position = unsigned long long;
static_assert(sizeof(Position) == 8);

struct alignas(64) Progress {
    alignas(64) Position released = 0;  // written by the CPU: every position below is consumed
    alignas(64) Position produced = 0;  // written by the GPU at completion
    alignas(64) Position spilled = 0;   // records that went through the HBM spill buffer
    alignas(64) int done = 0;           // GPU: produced/spilled are final, ring fully published
    alignas(64) int overflow = 0;       // GPU: spill buffer exhausted (results incomplete)
};
static_assert(sizeof(Progress) == 320);

inline constexpr std::size_t default_capacity = std::size_t{1} << 26;
inline constexpr std::size_t default_spill_capacity = std::size_t{1} << 24;
inline constexpr std::size_t consumer_chunk = 8192;

struct alignas(16) Candidate {
    std::uint16_t query_idx;  // query within the chunk
    std::uint16_t probe_idx;  // probe rank of the cluster for that query
    std::uint32_t gid;        // cluster-order vector index
    float exact_ip;           // 1-bit estimator inner product (<q', b> estimate)
    float low_dist;           // lower bound that passed the GPU filter
};
static_assert(sizeof(Candidate) == 16 && alignof(Candidate) == 16);
static_assert(std::is_trivially_copyable_v<Candidate>);

struct SpillRecord {
    Candidate item;
    Position position;
    Position pad;
};
static_assert(sizeof(SpillRecord) == 32);

}  // namespace coraanns::queue
