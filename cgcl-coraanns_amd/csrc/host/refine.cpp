// CPU refinement: the OpenMP consumer of the GPU->CPU candidate ring.
//
// Semantics of the reference consumer (src/search/cpu_refinement.cpp:71-284):
//  * workers claim chunks of min(8192, capacity) consecutive ring positions from a shared
//    read head; a claim in a later ring generation waits until its generation is live;
//  * a slot is complete when none of its four 32-bit words holds the empty pattern (no
//    field of a published Candidate can be all ones: query < 65535, gid < 2^32-1, and
//    exact_ip / low_dist are finite), so a record is never read half-written even if the
//    16-byte GPU store reaches host memory in pieces; the wait ends at done && position
//    >= produced, or on overflow;
//  * secondary filter: skip when low_dist >= threshold[query];
//  * refine = f_ex_add + g_add + f_ex_rescale * (2^ex * exact_ip + <q', ex_code> + kbxSumq)
//    (or the exact squared L2 distance to the base vector), inserted into the query's
//    sorted top-k under a per-query spinlock; a full top-k publishes its k-th distance as
//    the query's threshold (as an atomic minimum, since the GPU may have lowered it with
//    its seed thresholds), which the GPU filter reads;
//  * a processed chunk is cleared to the empty pattern before its release, and released
//    only as part of a contiguous prefix (ReleaseTracker).
#include "refine.hpp"

#include <immintrin.h>
#include <omp.h>

#include <atomic>
#include <cfloat>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <vector>

#include "coraanns/queue/release_tracker.hpp"

namespace coraanns::detail {

// AVX2: eight dimensions per step (the reference's ip64_fxu7_avx granularity,
// space.hpp:677-761).
float excode_ip7_avx2(const float *q, const uint8_t *packed, std::size_t P) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    constexpr uint64_t kLow6 = 0x3F3F3F3F3F3F3F3Full;
    constexpr uint64_t kOnes = 0x0101010101010101ull;
    for (std::size_t g = 0; g < P; g += 64) {
        const uint8_t *c = packed + g / 64 * 56;
        const float *qq = q + g;
        uint64_t top;
        std::memcpy(&top, c + 48, 8);
        for (int k = 0; k < 8; ++k) {  // dimensions 8k .. 8k+7 of the group
            uint64_t v;
            if (k < 6) {
                std::memcpy(&v, c + 8 * k, 8);
                v &= kLow6;
            } else {
                uint64_t a, b, d;
                const int off = (k - 6) * 8;
                std::memcpy(&a, c + off, 8);
                std::memcpy(&b, c + 16 + off, 8);
                std::memcpy(&d, c + 32 + off, 8);
                v = ((a >> 6) & 0x0303030303030303ull) | ((b >> 4) & 0x0C0C0C0C0C0C0C0Cull) |
                    ((d >> 2) & 0x3030303030303030ull);
            }
            v |= ((top >> k) & kOnes) << 6;
            const __m256 cf = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_cvtsi64_si128((long long)v)));
            if (k & 1)
                acc1 = _mm256_fmadd_ps(cf, _mm256_loadu_ps(qq + 8 * k), acc1);
            else
                acc0 = _mm256_fmadd_ps(cf, _mm256_loadu_ps(qq + 8 * k), acc0);
        }
    }
    const __m256 s = _mm256_add_ps(acc0, acc1);
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(s), _mm256_extractf128_ps(s, 1));
    h = _mm_add_ps(h, _mm_movehl_ps(h, h));
    h = _mm_add_ss(h, _mm_movehdup_ps(h));
    return _mm_cvtss_f32(h);
}

// AVX-512: sixteen dimensions per step. Per 64-dimension group, dimensions 0..47 are the
// low six bits of bytes 0..47, dimensions 48..63 gather their bit pairs from the top two
// bits of bytes j, 16+j and 32+j, and bit 6 of dimension 16i+m (bit 8(m%8) + 2i + m/8 of
// the group's u64 at byte 48) enters as a masked +64 built with pext.
__attribute__((target("avx512f,avx512bw,avx512vl,bmi2"))) float
excode_ip7_avx512(const float *q, const uint8_t *packed, std::size_t P) {
    __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
    const __m512i low6 = _mm512_set1_epi32(0x3F), two = _mm512_set1_epi32(3), c64 = _mm512_set1_epi32(64);
    for (std::size_t g = 0; g < P; g += 64) {
        const uint8_t *c = packed + g / 64 * 56;
        const float *qq = q + g;
        uint64_t top;
        std::memcpy(&top, c + 48, 8);
        const __m512i v0 = _mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i *>(c)));
        const __m512i v1 = _mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i *>(c + 16)));
        const __m512i v2 = _mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i *>(c + 32)));
        __m512i d[4];
        d[0] = _mm512_and_si512(v0, low6);
        d[1] = _mm512_and_si512(v1, low6);
        d[2] = _mm512_and_si512(v2, low6);
        d[3] = _mm512_or_si512(
            _mm512_and_si512(_mm512_srli_epi32(v0, 6), two),
            _mm512_or_si512(_mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(v1, 6), two), 2),
                            _mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(v2, 6), two), 4)));
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = static_cast<uint32_t>(_pext_u64(top, 0x0303030303030303ull << (2 * i)));
            const __mmask16 m = static_cast<__mmask16>(_pext_u32(r, 0x5555u) | (_pext_u32(r, 0xAAAAu) << 8));
            const __m512i code = _mm512_mask_add_epi32(d[i], m, d[i], c64);
            const __m512 prod = _mm512_cvtepi32_ps(code);
            if (i & 1)
                acc1 = _mm512_fmadd_ps(prod, _mm512_loadu_ps(qq + 16 * i), acc1);
            else
                acc0 = _mm512_fmadd_ps(prod, _mm512_loadu_ps(qq + 16 * i), acc0);
        }
    }
    return _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
}

namespace {

using ExcodeIpFn = float (*)(const float *, const uint8_t *, std::size_t);

// AVX-512 when the CPU has it, unless CORA_CPU_ISA=avx2 asks for the AVX2 path.
ExcodeIpFn pick_excode_ip() {
    const char *isa = std::getenv("CORA_CPU_ISA");
    const bool force_avx2 = isa && std::strcmp(isa, "avx2") == 0;
    __builtin_cpu_init();
    if (!force_avx2 && __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("bmi2"))
        return excode_ip7_avx512;
    return excode_ip7_avx2;
}

const ExcodeIpFn g_excode_ip = pick_excode_ip();

}  // namespace

float excode_ip7(const float *q, const uint8_t *packed, std::size_t P) { return g_excode_ip(q, packed, P); }

int excode_ip7_isa() { return g_excode_ip == excode_ip7_avx512 ? 512 : 256; }

namespace {

inline bool slot_complete(const queue::Candidate *slot, queue::Candidate &out) {
    const __m128i v = _mm_load_si128(reinterpret_cast<const __m128i *>(slot));
    const __m128i empty = _mm_set1_epi32(-1);
    if (_mm_movemask_epi8(_mm_cmpeq_epi32(v, empty)) != 0)
        return false;
    _mm_store_si128(reinterpret_cast<__m128i *>(&out), v);
    return true;
}

// Non-temporal clear (the consumed chunk is not read again by this CPU); the fence
// orders the clear before the release that lets the GPU write the slots again.
inline void clear_slots(queue::Candidate *slots, std::size_t n) {
    const __m128i empty = _mm_set1_epi32(-1);
    for (std::size_t i = 0; i < n; ++i)
        _mm_stream_si128(reinterpret_cast<__m128i *>(slots + i), empty);
    _mm_sfence();
}

// Records this many ring positions ahead have their ex-code, ex-factors and id lines
// prefetched: candidates are random accesses into arrays far larger than the caches, and
// their gids are in the ring well before the records are processed.
constexpr std::size_t kPrefetchAhead = 20;

inline void prefetch_record(const queue::Candidate *slot, const RefineArgs &a, std::size_t lc) {
    const uint32_t gid = __atomic_load_n(&slot->gid, __ATOMIC_RELAXED);
    if (gid >= a.num_vectors)  // empty (all ones) or not yet written
        return;
    // every cache line the code touches (112 bytes at a 112-byte stride often span three)
    const uintptr_t first = reinterpret_cast<uintptr_t>(a.long_codes + static_cast<std::size_t>(gid) * lc);
    for (uintptr_t line = first & ~uintptr_t{63}; line < first + lc; line += 64)
        _mm_prefetch(reinterpret_cast<const char *>(line), _MM_HINT_T0);
    _mm_prefetch(reinterpret_cast<const char *>(a.ex_factors + 2 * static_cast<std::size_t>(gid)), _MM_HINT_T0);
    _mm_prefetch(reinterpret_cast<const char *>(a.ids + gid), _MM_HINT_T0);
}

inline float load_threshold(const float *t, std::size_t q) {
    uint32_t bits = __atomic_load_n(reinterpret_cast<const uint32_t *>(t) + q, __ATOMIC_RELAXED);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Publish a query's k-th distance as an atomic minimum: the GPU may have lowered the
// threshold below this consumer's running k-th (seed thresholds), which a plain store
// would undo. With the CPU as the only writer this equals the reference's plain store,
// its k-th only ever decreasing (cpu_refinement.cpp:218,228).
inline void store_threshold(float *t, std::size_t q, float v) {
    uint32_t *slot = reinterpret_cast<uint32_t *>(t) + q;
    uint32_t cur = __atomic_load_n(slot, __ATOMIC_RELAXED);
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    for (;;) {
        float f;
        std::memcpy(&f, &cur, 4);
        if (!(v < f))
            return;
        if (__atomic_compare_exchange_n(slot, &cur, bits, true, __ATOMIC_RELAXED, __ATOMIC_RELAXED))
            return;
    }
}

constexpr std::size_t kRefineChunk = 1024;
static_assert(queue::consumer_chunk % kRefineChunk == 0, "a power of two no larger than the reference's chunk");

struct alignas(64) QuerySlot {
    std::atomic_flag lock = ATOMIC_FLAG_INIT;
    int count = 0;
};

}  // namespace

RefineOut cpu_refine(const RefineArgs &a, std::size_t nq, std::size_t topk, float *h_dists,
                     uint32_t *h_pids) {
    using queue::Position;
    const bool exact = a.base_mapping != nullptr;
    const std::size_t P = a.padded_dim;
    const std::size_t lc = (P * a.ex_bits + 7) / 8;
    const float scale = static_cast<float>(1u << a.ex_bits);
    const std::size_t kstride = (topk + 15) / 16 * 16;
    std::vector<float> td(nq * kstride);
    std::vector<uint32_t> tp(nq * kstride);
    std::unique_ptr<QuerySlot[]> slots(new QuerySlot[nq]);
    const Position capacity = a.capacity, mask = capacity - 1;
    // Consumer chunks of kRefineChunk records rather than the reference's consumer_chunk
    // (8,192): at ~170 ns a record, a thread that takes one of the last 8,192-record chunks
    // would refine for ~1.4 ms after the GPU published its records, the length of the far
    // scan, and end the search after the GPU; smaller chunks spread the last records over
    // all threads. Which thread refines a record changes nothing in the results.
    const Position chunk = std::min<Position>(kRefineChunk, capacity);
    std::atomic<Position> head{0};
    queue::ReleaseTracker tracker(*a.progress, capacity, chunk);
    queue::Progress *pg = a.progress;
    auto done = [&] { return __atomic_load_n(&pg->done, __ATOMIC_ACQUIRE) != 0; };
    auto aborted = [&] { return __atomic_load_n(&pg->overflow, __ATOMIC_ACQUIRE) != 0; };
    auto produced = [&] { return __atomic_load_n(&pg->produced, __ATOMIC_ACQUIRE); };
    std::atomic<std::size_t> refined_total{0};
    const int threads = a.threads > 0 ? a.threads : omp_get_max_threads();

#pragma omp parallel num_threads(threads)
    {
        std::size_t refined = 0;
        bool stop = false;
        while (!stop && !aborted()) {
            const Position start = head.fetch_add(chunk, std::memory_order_relaxed);
            if (done() && start >= produced())
                break;
            if (start >= capacity) {
                while (!tracker.readable_generation(start)) {
                    if (aborted() || (done() && start >= produced())) {
                        stop = true;
                        break;
                    }
                    _mm_pause();
                }
                if (stop)
                    break;
            }
            Position consumed = 0;
            const bool prefetch = !exact && a.num_vectors != 0;
            if (prefetch)
                for (Position i = 0; i < std::min<Position>(kPrefetchAhead, chunk); ++i)
                    prefetch_record(&a.items[(start + i) & mask], a, lc);
            for (Position i = 0; i < chunk; ++i) {
                const Position pos = start + i;
                queue::Candidate *slot = &a.items[pos & mask];
                if (prefetch && i + kPrefetchAhead < chunk)
                    prefetch_record(&a.items[(pos + kPrefetchAhead) & mask], a, lc);
                queue::Candidate rec;
                while (!slot_complete(slot, rec)) {
                    if (aborted() || (done() && pos >= produced())) {
                        stop = true;
                        break;
                    }
                    _mm_pause();
                }
                if (stop)
                    break;
                ++consumed;
                const std::size_t q = rec.query_idx;
                // defensive: the engine produces none of these; a record outside the
                // search's shape would index past the probe and code arrays
                if (q >= nq || rec.probe_idx >= a.nprobe || rec.gid >= a.num_vectors)
                    continue;
                if (a.secondary_filter && rec.low_dist >= load_threshold(a.thresholds, q))
                    continue;
                float dist;
                if (exact) {
                    const uint32_t pid = a.ids[rec.gid];
                    if (pid >= a.base_rows || a.base_dim != a.dim)
                        continue;
                    const float *x = reinterpret_cast<const float *>(
                        a.base_mapping + a.base_offset + static_cast<std::size_t>(pid) * a.base_stride);
                    const float *qv = a.raw_queries + q * a.dim;
                    float s = 0.0f;
#pragma omp simd reduction(+ : s)
                    for (std::size_t d = 0; d < a.dim; ++d) {
                        const float diff = qv[d] - x[d];
                        s += diff * diff;
                    }
                    dist = s;
                } else {
                    const float ip2 = excode_ip7(a.rotated_queries + q * P,
                                                 a.long_codes + static_cast<std::size_t>(rec.gid) * lc, P);
                    const float g_add = a.probe_gadd[q * a.nprobe + rec.probe_idx];
                    const float f_add = a.ex_factors[2 * static_cast<std::size_t>(rec.gid)];
                    const float f_rescale = a.ex_factors[2 * static_cast<std::size_t>(rec.gid) + 1];
                    dist = f_add + g_add + f_rescale * (scale * rec.exact_ip + ip2 + a.kbxsumq[q]);
                }
                ++refined;
                if (dist >= load_threshold(a.thresholds, q))
                    continue;
                QuerySlot &s = slots[q];
                while (s.lock.test_and_set(std::memory_order_acquire))
                    _mm_pause();
                float *d = td.data() + q * kstride;
                uint32_t *p = tp.data() + q * kstride;
                const uint32_t pid = a.ids[rec.gid];
                if (s.count < static_cast<int>(topk)) {
                    int i = s.count - 1;
                    while (i >= 0 && d[i] > dist) {
                        d[i + 1] = d[i];
                        p[i + 1] = p[i];
                        --i;
                    }
                    d[i + 1] = dist;
                    p[i + 1] = pid;
                    if (++s.count == static_cast<int>(topk))
                        store_threshold(a.thresholds, q, d[topk - 1]);
                } else if (dist < d[topk - 1]) {
                    int i = static_cast<int>(topk) - 2;
                    while (i >= 0 && d[i] > dist) {
                        d[i + 1] = d[i];
                        p[i + 1] = p[i];
                        --i;
                    }
                    d[i + 1] = dist;
                    p[i + 1] = pid;
                    store_threshold(a.thresholds, q, d[topk - 1]);
                }
                s.lock.clear(std::memory_order_release);
            }
            if (consumed != 0) {
                clear_slots(&a.items[start & mask], static_cast<std::size_t>(chunk));
                tracker.complete(start);
            }
        }
        refined_total.fetch_add(refined, std::memory_order_relaxed);
    }

    RefineOut out;
    out.produced = produced();
    out.refined = refined_total.load();
    out.aborted = aborted();
    // the results, one query per iteration, over the refinement threads (this runs after the
    // GPU has finished, so it is on the step's critical path)
#pragma omp parallel for num_threads(threads) schedule(static)
    for (std::size_t q = 0; q < nq; ++q) {
        const int n = slots[q].count;
        for (int i = 0; i < static_cast<int>(topk); ++i) {
            h_dists[q * topk + i] = i < n ? td[q * kstride + i] : FLT_MAX;
            h_pids[q * topk + i] = i < n ? tp[q * kstride + i] : 0u;
        }
    }
    return out;
}

}  // namespace coraanns::detail
