// CPU side of the hybrid search: consumer of the GPU->CPU candidate ring.
#pragma once

#include <cstddef>
#include <cstdint>

#include "coraanns/queue/candidate_queue.hpp"

namespace coraanns::detail {

// <q', ex_code> for one 7-bit packed ex-code of P dims (P % 64 == 0): AVX-512 when the
// CPU has it (and CORA_CPU_ISA is not "avx2"), otherwise AVX2.
float excode_ip7(const float *q, const uint8_t *packed, std::size_t P);
float excode_ip7_avx2(const float *q, const uint8_t *packed, std::size_t P);
// vector width of the path excode_ip7 uses: 512 or 256
int excode_ip7_isa();

struct RefineArgs {
    queue::Candidate *items = nullptr;  // host ring
    queue::Progress *progress = nullptr;
    uint64_t capacity = 0;
    float *thresholds = nullptr;        // shared with the GPU filter
    const float *rotated_queries = nullptr;  // [nq][P]
    const float *kbxsumq = nullptr;          // [nq]
    const float *probe_gadd = nullptr;       // [nq][nprobe]
    std::size_t nprobe = 0, padded_dim = 0, ex_bits = 7;
    const uint8_t *long_codes = nullptr;     // [N][P*ex/8]
    const float *ex_factors = nullptr;       // [N][2]
    const uint32_t *ids = nullptr;           // [N]
    std::size_t num_vectors = 0;             // N (bounds the prefetch of upcoming records)
    // exact FP32 refine (reference enable_exact_refine)
    const uint8_t *base_mapping = nullptr;
    std::size_t base_rows = 0, base_dim = 0, base_stride = 0, base_offset = 0;
    const float *raw_queries = nullptr;      // [nq][dim]
    std::size_t dim = 0;
    bool secondary_filter = true;
    bool profile = false;
    int threads = 0;  // <= 0: omp_get_max_threads()
};

struct RefineOut {
    uint64_t produced = 0;
    std::size_t refined = 0;
    bool aborted = false;
};

// Consume the ring until the GPU marks it done (or reports overflow), refining every
// candidate and keeping per-query top-k; writes h_dists/h_pids [nq][topk] padded with
// FLT_MAX / 0 (reference cpu_refinement.cpp:71-284).
RefineOut cpu_refine(const RefineArgs &a, std::size_t nq, std::size_t topk, float *h_dists,
                     uint32_t *h_pids);

}  // namespace coraanns::detail
