// coraanns::HybridIndex: the reference's engine API (hybrid.cuh:18-203) over the GPU
// C-ABI (cora_gpu.h) plus the CPU consumer (refine.cpp).
#include "coraanns/search/hybrid.hpp"

#include <omp.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <stdexcept>
#include <string>

#include "cora_gpu.h"
#include "refine.hpp"

namespace coraanns {
namespace {

std::string engine_error(cora_gpu_engine *e) {
    char buf[512] = {0};
    if (e)
        cora_gpu_last_error(e, buf, sizeof(buf));
    return buf;
}

// Status -> the exception type the reference throws for the same condition.
void check(cora_gpu_engine *e, int rc) {
    if (rc == CORA_OK)
        return;
    const std::string msg = engine_error(e);
    switch (rc) {
    case CORA_ERR_INVALID_ARGUMENT: throw std::invalid_argument(msg);
    case CORA_ERR_LOGIC: throw std::logic_error(msg);
    default: throw std::runtime_error(msg);
    }
}

}  // namespace

HybridIndex::HybridIndex(int device) {
    const int rc = cora_gpu_create(&engine_, device);
    if (rc != CORA_OK)
        throw std::runtime_error("cannot create the GPU engine on device " + std::to_string(device));
}

HybridIndex::~HybridIndex() {
    if (engine_)
        cora_gpu_destroy(engine_);
}

void HybridIndex::set_metric(int metric) {
    if (metric != 0 && metric != 1)
        throw std::invalid_argument("metric must be 0 (L2) or 1 (IP)");
    if (loaded_ && metric != metric_)
        throw std::logic_error("set the metric before loading the index");
    metric_ = metric;
}

void HybridIndex::set_lower_bound_scale(float scale) {
    if (!(scale > 0.0f && scale <= max_bound_scale))
        throw std::invalid_argument("lower-bound scale must be in (0, 16]");
    bound_scale_ = scale;
}

void HybridIndex::set_vanguard_size(std::size_t size) {
    if (workspace_ready_ && std::min(size, ws_max_nprobe_) > ws_vanguard_)
        throw std::logic_error("prepare workspace again before increasing vanguard size");
    vanguard_size_ = size;
}

void HybridIndex::validate_workspace(std::size_t queries, std::size_t topk,
                                     std::size_t nprobe) const {
    if (!workspace_ready_)
        throw std::logic_error("prepare workspace before searching");
    if (queries == 0 || queries > ws_max_queries_ || topk == 0 || topk > ws_max_topk_ ||
        nprobe == 0 || nprobe > ws_max_nprobe_)
        throw std::invalid_argument("search shape exceeds the prepared workspace");
}

void HybridIndex::load_from_raw_pointers(std::size_t num_vecs, std::size_t d, std::size_t p_d,
                                         std::size_t n_centroids, std::size_t ex_b,
                                         const float *h_centroids, const float *h_rotator,
                                         const uint32_t *h_short_data,
                                         const float *h_short_factors, const uint8_t *h_long_code,
                                         const float *h_ex_factors, const uint32_t *h_ids,
                                         const std::size_t *h_cluster_sizes) {
    if (loaded_)
        throw std::logic_error("index already loaded");
    if (!h_ids)
        throw std::invalid_argument("invalid index shape or missing index data");
    static_assert(sizeof(std::size_t) == sizeof(uint64_t));
    check(engine_, cora_gpu_load_index(engine_, num_vecs, d, p_d, n_centroids, ex_b, metric_,
                                       h_centroids, h_rotator, h_short_data, h_short_factors,
                                       reinterpret_cast<const uint64_t *>(h_cluster_sizes)));
    if ((gpu_seed_refine_ || gpu_refine_filter_) && h_long_code && h_ex_factors && ex_b == 7)
        check(engine_, cora_gpu_load_excodes(engine_, h_long_code, h_ex_factors));
    num_vectors_ = num_vecs;
    dim_ = d;
    padded_dim_ = p_d;
    num_centroids_ = n_centroids;
    ex_bits_ = ex_b;
    h_long_codes_ = h_long_code;
    h_ex_factors_ = h_ex_factors;
    h_ids_ = h_ids;
    loaded_ = true;
}

void HybridIndex::set_queue_capacity(std::size_t capacity) {
    if (capacity == 0 || (capacity & (capacity - 1)) != 0 ||
        capacity > SIZE_MAX / sizeof(queue::Candidate))
        throw std::invalid_argument("queue-capacity must be a positive power of two");
    if (workspace_ready_)
        throw std::logic_error("set queue capacity before prepare_workspace");
    check(engine_, cora_gpu_set_queue(engine_, capacity, queue_spill_capacity_));
    queue_capacity_ = capacity;
}

void HybridIndex::set_queue_spill_capacity(std::size_t capacity) {
    if (capacity > SIZE_MAX / sizeof(queue::SpillRecord))
        throw std::invalid_argument("queue-spill-capacity is too large");
    if (workspace_ready_)
        throw std::logic_error("set spill capacity before prepare_workspace");
    check(engine_, cora_gpu_set_queue(engine_, queue_capacity_, capacity));
    queue_spill_capacity_ = capacity;
}

void HybridIndex::prepare_workspace(std::size_t max_queries, std::size_t max_topk,
                                    std::size_t max_nprobe) {
    if (!loaded_)
        throw std::logic_error("load an index before preparing workspace");
    validate_search_shape(max_queries, max_topk, max_nprobe, num_centroids_, padded_dim_);
    workspace_ready_ = false;
    check(engine_, cora_gpu_prepare_workspace(engine_, max_queries, max_topk, max_nprobe,
                                              vanguard_size_));
    ws_max_queries_ = max_queries;
    ws_max_topk_ = max_topk;
    ws_max_nprobe_ = max_nprobe;
    ws_vanguard_ = std::min(vanguard_size_, max_nprobe);
    workspace_ready_ = true;
}

void HybridIndex::free_workspace() noexcept {
    workspace_ready_ = false;
    ws_max_queries_ = ws_max_topk_ = ws_max_nprobe_ = ws_vanguard_ = 0;
    if (engine_)
        cora_gpu_free_workspace(engine_);
}

void HybridIndex::reset_buffer(const float *h_queries, std::size_t num_queries) {
    validate_workspace(num_queries, 1, 1);
    if (!h_queries)
        throw std::invalid_argument("missing queries");
    // The queries go to the engine's pinned staging buffer first, copied by the OpenMP team
    // in parallel, so the upload is one DMA from page-locked memory rather than the runtime's
    // pageable path (~1 MB staged copies with the host copying in between).
    float *stage = nullptr;
    check(engine_, cora_gpu_query_staging(engine_, &stage));
    const std::size_t count = num_queries * dim_;
    if (stage != h_queries) {
        const int threads = cpu_threads_ > 0 ? cpu_threads_ : omp_get_max_threads();
        const std::size_t block = 1u << 16;  // floats per task (256 KiB)
        const std::size_t blocks = (count + block - 1) / block;
#pragma omp parallel for num_threads(threads) schedule(static)
        for (std::size_t b = 0; b < blocks; ++b) {
            const std::size_t o = b * block;
            std::memcpy(stage + o, h_queries + o, std::min(block, count - o) * sizeof(float));
        }
    }
    check(engine_, cora_gpu_reset(engine_, stage, num_queries));
    last_spilled_count_ = 0;
}

void HybridIndex::capture_thresholds(float *out, std::size_t nq) const {
    validate_workspace(nq, 1, 1);
    if (!out)
        throw std::invalid_argument("missing threshold output");
    check(engine_, cora_gpu_capture_thresholds(engine_, out, nq));
}

void HybridIndex::seed_thresholds(const float *in, std::size_t nq) {
    validate_workspace(nq, 1, 1);
    if (!in)
        throw std::invalid_argument("missing threshold input");
    check(engine_, cora_gpu_seed_thresholds(engine_, in, nq));
}

void HybridIndex::record_stats(const cora_search_stats &st, std::size_t refined) {
    last_written_count_ = st.produced;
    last_spilled_count_ = st.spilled;
    last_refined_count_ = refined;
    last_gpu_filter_ms_ = st.filter_ms;
    last_scan_ms_ = st.scan_ms;
    last_scan_bytes_ = st.scan_bytes;
    last_scan_units_ = st.scan_units;
    last_scan_vectors_ = st.scan_vectors;
    last_probe_ms_ = st.probe_ms;
    last_probe_flops_ = st.probe_flops;
    for (int i = 0; i < 3; ++i)
        last_pass_produced_[i] = st.pass_produced[i];
    last_seeded_queries_ = st.seeded_queries;
    last_prefilter_dropped_ = st.prefilter_dropped;
    last_seed_ms_ = st.seed_ms;
    last_recovery_ms_ = st.recovery_ms;
    last_gpu_refined_ = st.gpu_refined;
    last_vanguard_ms_ = st.vanguard_ms;
    last_vanguard_bytes_ = st.vanguard_bytes;
    last_vanguard_lows_ms_ = st.vanguard_lows_ms;
    last_vanguard_lows_bytes_ = st.vanguard_lows_bytes;
    last_vanguard_mode_ = st.vanguard_mode;
    for (int i = 0; i < 4; ++i)
        last_phase_ms_[i] = st.phase_ms[i];
    last_vanguard_refine_ms_ = st.vanguard_refine_ms;
    last_vanguard_refine_bytes_ = st.vanguard_refine_bytes;
}

void HybridIndex::print_profile(const cora_search_stats &st, std::size_t refined) const {
    if (profiling_enabled_) {
        // the reference's phases (hybrid.cu:479, 500, 516, 679-685)
        static const char *const kVanguardMode[] = {"none", "per-pair seed and recovery passes",
                                                     "fused per-query pass",
                                                     "matrix-core lows pass + fused per-query pass"};
        std::printf("[Profile] 0~2. Initial Matrix Math time: %g ms\n", st.phase_ms[0]);
        std::printf("[Profile] 3. Select Top-nprobe Clusters time: %g ms\n", st.phase_ms[1]);
        std::printf("[Profile] 4. Flatten Pairs time: %g ms\n", st.phase_ms[2]);
        std::printf("[Profile] 7~9. Single-Stage Global Task Pool Pipeline (%s) time: %g ms\n",
                    ip_kernel_type_ == KernelType::Lut4Bit ? "LUT_4BIT" : "BITWISE_DECOMP", st.phase_ms[3]);
        std::printf("[Profile] vanguard: %s; GPU filter kernels %g ms\n",
                    kVanguardMode[st.vanguard_mode >= 0 && st.vanguard_mode < 4 ? st.vanguard_mode : 0],
                    st.filter_ms);
        std::printf("------------------------------------------\n");
        std::printf("[Cora-Refine] candidates=%llu refined=%zu refinement_ratio=%.6f\n",
                    static_cast<unsigned long long>(st.produced), refined,
                    st.produced ? static_cast<double>(refined) / static_cast<double>(st.produced)
                                : 0.0);
    }
}

void HybridIndex::search(const float *h_queries, std::size_t num_queries, std::size_t topk,
                         std::size_t nprobe, float *h_final_dists, uint32_t *h_final_pids,
                         int batch_q) {
    validate_workspace(num_queries, topk, nprobe);
    if (!h_queries || !h_final_dists || !h_final_pids || batch_q < 1 || batch_q > max_batch_q)
        throw std::invalid_argument("invalid search buffers or batch-q (expected 1..64)");
    const bool exact = exact_base_mapping_ != nullptr;
    if (!exact && (!h_long_codes_ || !h_ex_factors_))
        throw std::logic_error("extended codes or an exact-refine base are required");
    if (!exact && ex_bits_ != 7)
        throw std::logic_error("CPU refinement supports 7 ex-bits (8-bit RaBitQ) indexes");
    if (exact && metric_ != 0)
        throw std::logic_error("exact FP32 refine supports only L2 indexes");

    cora_search_args args{};
    args.num_queries = static_cast<uint32_t>(num_queries);
    args.topk = static_cast<uint32_t>(topk);
    args.nprobe = static_cast<uint32_t>(nprobe);
    args.batch_q = static_cast<uint32_t>(batch_q);
    args.vanguard = static_cast<uint32_t>(vanguard_size_);
    args.flags = (frozen_thresholds_ ? uint32_t{CORA_FLAG_FROZEN_THRESHOLDS} : 0u) |
                 (gpu_filter_timing_enabled_ || profiling_enabled_ ? uint32_t{CORA_FLAG_FILTER_TIMING}
                                                                   : 0u) |
                 (cross_query_reuse_enabled_ ? uint32_t{CORA_FLAG_CROSS_QUERY_REUSE} : 0u) |
                 (gpu_seed_refine_ && !exact ? 0u : uint32_t{CORA_FLAG_NO_GPU_SEED}) |
                 (gpu_refine_filter_ && !exact ? 0u : uint32_t{CORA_FLAG_NO_GPU_PREFILTER}) |
                 (gpu_final_topk_ && !exact ? uint32_t{CORA_FLAG_GPU_FINAL} : 0u) |
                 (ip_kernel_type_ == KernelType::Lut4Bit ? uint32_t{CORA_FLAG_LUT4} : 0u) | extra_flags_;
    args.bound_scale = bound_scale_;
    last_gpu_filter_ms_ = 0.0f;
    check(engine_, cora_gpu_launch_search(engine_, &args));
    if (args.flags & CORA_FLAG_GPU_FINAL) {
        // the GPU formed the final top-k from its refined distances; no CPU refinement
        cora_search_stats st{};
        const int rc = cora_gpu_sync(engine_, &st);
        record_stats(st, 0);
        if (rc != CORA_OK)
            throw std::runtime_error(engine_error(engine_));
        check(engine_, cora_gpu_final_results(engine_, h_final_dists, h_final_pids));
        // cluster-order indexes to ids: random reads of the ids array (80 MB at 20M vectors),
        // one cache miss each, spread over the refinement threads (the CPU refines nothing here)
        const std::size_t n = num_queries * topk;
        const int threads = cpu_threads_ > 0 ? cpu_threads_ : omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static)
        for (std::size_t i = 0; i < n; ++i)
            h_final_pids[i] = h_final_pids[i] < num_vectors_ ? h_ids_[h_final_pids[i]] : 0u;
        print_profile(st, 0);
        return;
    }

    cora_queue_view view{};
    const float *rq = nullptr, *kb = nullptr, *gadd = nullptr;
    detail::RefineOut out;
    try {
        check(engine_, cora_gpu_queue_view(engine_, &view));
        check(engine_, cora_gpu_wait_host_inputs(engine_, &rq, &kb, &gadd));
        detail::RefineArgs ra;
        ra.items = static_cast<queue::Candidate *>(view.items);
        ra.progress = static_cast<queue::Progress *>(view.progress);
        ra.capacity = view.capacity;
        ra.thresholds = view.thresholds;
        ra.rotated_queries = rq;
        ra.kbxsumq = kb;
        ra.probe_gadd = gadd;
        ra.nprobe = nprobe;
        ra.padded_dim = padded_dim_;
        ra.ex_bits = ex_bits_;
        ra.long_codes = h_long_codes_;
        ra.ex_factors = h_ex_factors_;
        ra.ids = h_ids_;
        ra.num_vectors = num_vectors_;
        ra.base_mapping = exact_base_mapping_;
        ra.base_rows = exact_base_rows_;
        ra.base_dim = exact_base_dim_;
        ra.base_stride = exact_base_row_stride_bytes_;
        ra.base_offset = exact_base_data_offset_bytes_;
        ra.raw_queries = h_queries;
        ra.dim = dim_;
        ra.secondary_filter = cpu_secondary_filter_enabled_;
        ra.profile = profiling_enabled_;
        ra.threads = cpu_threads_;
        out = detail::cpu_refine(ra, num_queries, topk, h_final_dists, h_final_pids);
    } catch (...) {
        if (view.abort_flag)
            __atomic_store_n(view.abort_flag, 1, __ATOMIC_RELEASE);
        cora_search_stats ignored{};
        cora_gpu_sync(engine_, &ignored);
        throw;
    }
    cora_search_stats st{};
    const int rc = cora_gpu_sync(engine_, &st);
    record_stats(st, out.refined);
    if (rc != CORA_OK)
        throw std::runtime_error(engine_error(engine_));
    print_profile(st, out.refined);
}

}  // namespace coraanns
