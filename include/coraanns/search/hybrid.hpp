// coraanns::HybridIndex — GPU filter / CPU refine IVF-RaBitQ search on MI355X.
//
// Drop-in for the reference's include/coraanns/search/hybrid.cuh:18-203: the same public
// method set, argument meaning, ownership rules and exception types, with no HIP, CUDA
// or cuBLAS types in the header. The GPU side is the C-ABI engine in cora_gpu.h; this
// class adds the CPU side: the OpenMP consumer of the candidate ring that refines
// candidates with the 7-bit ex-codes (or an exact FP32 base) and keeps per-query top-k
// (reference src/search/cpu_refinement.cpp:71-284).
//
// Ownership (reference hybrid.cuh:185, docs/ARCHITECTURE.md:34-38): load_from_raw_pointers
// copies centroids, rotator, sign codes and short factors to the GPU and borrows the
// host ex-codes, ex-factors and ids until the engine is destroyed. One search at a time.
#pragma once

#include <cstddef>
#include <cstdint>

#include "coraanns/queue/candidate_queue.hpp"
#include "coraanns/search/parameters.hpp"

struct cora_gpu_engine;
struct cora_search_stats;

namespace coraanns {

enum class KernelType { Lut4Bit, Bitwise };

class HybridIndex {
  public:
    explicit HybridIndex(int device = 0);
    HybridIndex(const HybridIndex &) = delete;
    HybridIndex &operator=(const HybridIndex &) = delete;
    ~HybridIndex();

    void set_profiling(bool enabled) { profiling_enabled_ = enabled; }
    void set_candidate_stats(bool enabled) { candidate_stats_enabled_ = enabled; }
    void set_gpu_filter_timing(bool enabled) { gpu_filter_timing_enabled_ = enabled; }
    void set_cross_query_reuse(bool enabled) { cross_query_reuse_enabled_ = enabled; }
    void set_cpu_secondary_filter(bool enabled) { cpu_secondary_filter_enabled_ = enabled; }

    queue::Position get_last_submitted_count() const { return last_written_count_; }
    queue::Position get_last_spilled_count() const { return last_spilled_count_; }
    void set_queue_capacity(std::size_t capacity);
    void set_queue_spill_capacity(std::size_t capacity);
    std::size_t get_queue_capacity() const { return queue_capacity_; }
    std::size_t get_last_refined_count() const { return last_refined_count_; }
    float get_last_gpu_filter_ms() const { return last_gpu_filter_ms_; }

    void set_vanguard_size(std::size_t size);
    std::size_t get_vanguard_size() const { return vanguard_size_; }

    // Bitwise (the default here): the Bq=8 popcount lower bound (filter_kernels.cuh:79-114),
    // the two-stage exact_ip, the fused vanguard pass and the matrix-core scans.
    // Lut4Bit (the reference's default): its FP16 nibble-LUT estimator
    // (query_kernels.cuh:199-221, filter_kernels.cuh:283-306,586-770) on the per-pair seed,
    // far and recovery passes, the LUT value being the exact_ip refinement uses.
    void set_ip_kernel_type(KernelType t) { ip_kernel_type_ = t; }
    KernelType get_ip_kernel_type() const { return ip_kernel_type_; }

    void prepare_workspace(std::size_t max_queries, std::size_t max_topk, std::size_t max_nprobe);
    void free_workspace() noexcept;
    void reset_buffer(const float *h_queries, std::size_t num_queries);

    void enable_exact_refine(const uint8_t *base_mapping, std::size_t base_rows,
                             std::size_t base_dim, std::size_t row_stride_bytes,
                             std::size_t data_offset_bytes) {
        exact_base_mapping_ = base_mapping;
        exact_base_rows_ = base_rows;
        exact_base_dim_ = base_dim;
        exact_base_row_stride_bytes_ = row_stride_bytes;
        exact_base_data_offset_bytes_ = data_offset_bytes;
    }

    // Host extended codes, factors and IDs are borrowed until this engine is destroyed.
    void load_from_raw_pointers(std::size_t num_vecs, std::size_t d, std::size_t p_d,
                                std::size_t n_centroids, std::size_t ex_b,
                                const float *h_centroids, const float *h_rotator,
                                const uint32_t *h_short_data, const float *h_short_factors,
                                const uint8_t *h_long_code, const float *h_ex_factors,
                                const uint32_t *h_ids, const std::size_t *h_cluster_sizes);

    void capture_thresholds(float *out, std::size_t nq) const;
    void seed_thresholds(const float *in, std::size_t nq);

    void search(const float *h_queries, std::size_t num_queries, std::size_t topk,
                std::size_t nprobe, float *h_final_dists, uint32_t *h_final_pids,
                int batch_q = default_batch_q);

    // ---- extensions of this engine (no counterpart in the reference API) ----
    // Metric of the loaded index: 0 = L2, 1 = inner product (the reference hybrid path is
    // L2-only; IP uses g_add = -<q',c'> as rabitq_cpu does, query.hpp:537-545).
    void set_metric(int metric);
    // Frozen thresholds: the GPU filter reads a snapshot taken at launch (deterministic
    // candidate sets for parity tests).
    void set_frozen_thresholds(bool enabled) { frozen_thresholds_ = enabled; }
    // GPU seed thresholds (default on): load_from_raw_pointers also keeps a copy of the
    // ex-codes and ex-factors in HBM, the vanguard seed pass refines its seeds on the GPU
    // and lowers each query's threshold before the far and recovery passes (live
    // thresholds only). Off: only the CPU tightens thresholds, as in the reference. Set
    // before load_from_raw_pointers to skip the HBM copy.
    void set_gpu_seed_refine(bool enabled) { gpu_seed_refine_ = enabled; }
    // GPU refined pre-filter (default on; uses the same HBM ex-codes): the far and
    // recovery passes drop candidates whose refined distance already exceeds their
    // threshold by more than a rounding bound, which the CPU would discard.
    void set_gpu_refine_filter(bool enabled) { gpu_refine_filter_ = enabled; }
    bool get_gpu_refine_filter() const { return gpu_refine_filter_; }
    // Extra cora_search_flags ORed into every launch (test modes such as
    // CORA_FLAG_GPU_SEED_FROZEN).
    void set_extra_search_flags(uint32_t flags) { extra_flags_ = flags; }
    // Multiplier of the filter's error term, low = est - scale * f_error * g_error
    // (cora_search_args.bound_scale). 1 is the reference Bitwise producer's bound
    // (filter_kernels.cuh:111-114) and gives its candidate sets; the default
    // default_bound_scale widens it so that the vectors whose 1-bit estimate errs beyond
    // the bound's confidence are still refined, which the reference CPU path's running
    // threshold does for the vectors it scans early (ivf.hpp:802-817). Range (0, 16].
    void set_lower_bound_scale(float scale);
    // GPU-final top-k (default off): the GPU forms each query's final top-k from the refined
    // distances it computes on the HBM ex-codes (fused vanguard pass, refined pre-filter) and
    // the CPU refines nothing, for searches the CPU refinement would bound (high top-k).
    // Needs the GPU ex-code stages on, the fused pass's limits (vanguard <= 64, topk <= 128)
    // and live thresholds; ties in the final distance go to the lower cluster-order index.
    void set_gpu_final_topk(bool enabled) { gpu_final_topk_ = enabled; }
    bool get_gpu_final_topk() const { return gpu_final_topk_; }
    float get_lower_bound_scale() const { return bound_scale_; }
    bool get_gpu_seed_refine() const { return gpu_seed_refine_; }
    // CPU refinement threads; 0 = omp_get_max_threads() (the reference always uses the
    // caller's OpenMP setting, cpu_refinement.cpp:110).
    void set_cpu_threads(int threads) { cpu_threads_ = threads < 0 ? 0 : threads; }
    float get_last_scan_ms() const { return last_scan_ms_; }
    uint64_t get_last_scan_bytes() const { return last_scan_bytes_; }
    uint64_t get_last_scan_units() const { return last_scan_units_; }
    uint64_t get_last_scan_vectors() const { return last_scan_vectors_; }
    float get_last_probe_ms() const { return last_probe_ms_; }
    uint64_t get_last_probe_flops() const { return last_probe_flops_; }
    // cumulative candidates after the vanguard seed, far-pair and recovery passes
    uint64_t get_last_pass_produced(int pass) const { return last_pass_produced_[pass]; }
    uint64_t get_last_seeded_queries() const { return last_seeded_queries_; }
    uint64_t get_last_prefilter_dropped() const { return last_prefilter_dropped_; }
    float get_last_seed_ms() const { return last_seed_ms_; }
    float get_last_recovery_ms() const { return last_recovery_ms_; }
    uint64_t get_last_gpu_refined() const { return last_gpu_refined_; }
    float get_last_vanguard_ms() const { return last_vanguard_ms_; }
    uint64_t get_last_vanguard_bytes() const { return last_vanguard_bytes_; }
    float get_last_vanguard_lows_ms() const { return last_vanguard_lows_ms_; }
    // 0 none, 1 per-pair seed and recovery passes, 2 fused per-query pass, 3 lows pass + fused,
    // 4 lows pass + staged pass
    int get_last_vanguard_mode() const { return last_vanguard_mode_; }
    // staged vanguard pass: its grid-wide refinement launches and their algorithmic bytes
    float get_last_vanguard_refine_ms() const { return last_vanguard_refine_ms_; }
    uint64_t get_last_vanguard_refine_bytes() const { return last_vanguard_refine_bytes_; }
    // [Profile] phases (with profiling or GPU filter timing): matrix math, probe select,
    // pair scheduling, scan pipeline including the CPU refinement
    float get_last_phase_ms(int phase) const { return phase >= 0 && phase < 4 ? last_phase_ms_[phase] : 0.0f; }
    uint64_t get_last_vanguard_lows_bytes() const { return last_vanguard_lows_bytes_; }
    cora_gpu_engine *gpu_engine() const { return engine_; }

  private:
    void validate_workspace(std::size_t queries, std::size_t topk, std::size_t nprobe) const;
    void record_stats(const cora_search_stats &st, std::size_t refined);
    void print_profile(const cora_search_stats &st, std::size_t refined) const;

    cora_gpu_engine *engine_ = nullptr;
    int metric_ = 0;
    std::size_t num_vectors_ = 0, dim_ = 0, padded_dim_ = 0, num_centroids_ = 0, ex_bits_ = 0;
    bool loaded_ = false;

    const uint8_t *h_long_codes_ = nullptr;
    const float *h_ex_factors_ = nullptr;
    const uint32_t *h_ids_ = nullptr;

    const uint8_t *exact_base_mapping_ = nullptr;
    std::size_t exact_base_rows_ = 0, exact_base_dim_ = 0;
    std::size_t exact_base_row_stride_bytes_ = 0, exact_base_data_offset_bytes_ = 0;

    bool workspace_ready_ = false;
    std::size_t ws_max_queries_ = 0, ws_max_topk_ = 0, ws_max_nprobe_ = 0, ws_vanguard_ = 0;

    bool profiling_enabled_ = false;
    bool candidate_stats_enabled_ = false;
    bool gpu_filter_timing_enabled_ = false;
    bool cross_query_reuse_enabled_ = true;
    bool cpu_secondary_filter_enabled_ = true;
    bool frozen_thresholds_ = false;
    bool gpu_seed_refine_ = true;
    bool gpu_refine_filter_ = true;
    uint32_t extra_flags_ = 0;
    float bound_scale_ = default_bound_scale;
    bool gpu_final_topk_ = false;
    int cpu_threads_ = 0;
    std::size_t vanguard_size_ = default_vanguard_size;
    KernelType ip_kernel_type_ = KernelType::Bitwise;

    std::size_t queue_capacity_ = queue::default_capacity;
    std::size_t queue_spill_capacity_ = queue::default_spill_capacity;
    queue::Position last_written_count_ = 0;
    queue::Position last_spilled_count_ = 0;
    std::size_t last_refined_count_ = 0;
    float last_gpu_filter_ms_ = 0.0f;
    float last_scan_ms_ = 0.0f;
    uint64_t last_scan_bytes_ = 0, last_scan_units_ = 0, last_scan_vectors_ = 0;
    float last_probe_ms_ = 0.0f;
    uint64_t last_probe_flops_ = 0;
    uint64_t last_pass_produced_[3] = {0, 0, 0};
    uint64_t last_seeded_queries_ = 0;
    uint64_t last_prefilter_dropped_ = 0;
    float last_seed_ms_ = 0.0f, last_recovery_ms_ = 0.0f;
    uint64_t last_gpu_refined_ = 0, last_vanguard_bytes_ = 0;
    float last_vanguard_ms_ = 0.0f;
    uint64_t last_vanguard_lows_bytes_ = 0;
    float last_vanguard_lows_ms_ = 0.0f;
    int last_vanguard_mode_ = 0;
    float last_phase_ms_[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float last_vanguard_refine_ms_ = 0.0f;
    uint64_t last_vanguard_refine_bytes_ = 0;
};

}  // namespace coraanns
