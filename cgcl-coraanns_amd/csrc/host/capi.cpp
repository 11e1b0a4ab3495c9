// C-ABI of libcoraanns (include/cora_host.h).
#include "cora_host.h"

#include <immintrin.h>
#include <omp.h>

#include <atomic>
#include <cfloat>
#include <chrono>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "coraanns/index/ivf_builder.hpp"
#include "coraanns/index/ivf_file.hpp"
#include "coraanns/index/search_data.hpp"
#include "coraanns/queue/candidate_queue.hpp"
#include "coraanns/search/hybrid.hpp"
#include "refine.hpp"

using namespace coraanns;

struct cora_hybrid {
    std::unique_ptr<HybridIndex> index;
};

struct cora_ivf {
    index::IvfHeader header;
    index::HugeVector<uint32_t> ids;
    std::unique_ptr<index::SearchData> data;
};

namespace {

thread_local std::string g_error;

template <class F>
int guarded(F &&f) {
    try {
        f();
        return CORA_OK;
    } catch (const std::invalid_argument &e) {
        g_error = e.what();
        return CORA_ERR_INVALID_ARGUMENT;
    } catch (const std::logic_error &e) {
        g_error = e.what();
        return CORA_ERR_LOGIC;
    } catch (const std::bad_alloc &e) {
        g_error = "out of memory";
        return CORA_ERR_OUT_OF_MEMORY;
    } catch (const std::exception &e) {
        g_error = e.what();
        const std::string m = e.what();
        if (m.find("spill capacity exhausted") != std::string::npos)
            return CORA_ERR_SPILL_EXHAUSTED;
        if (m.find("drain stopped") != std::string::npos)
            return CORA_ERR_QUEUE_STALLED;
        return CORA_ERR_RUNTIME;
    }
}

#define NEED(h)                                          \
    do {                                                 \
        if (!(h)) {                                      \
            g_error = "null handle";                     \
            return CORA_ERR_INVALID_ARGUMENT;            \
        }                                                \
    } while (0)

}  // namespace

extern "C" {

const char *cora_host_last_error(void) { return g_error.c_str(); }

int cora_hybrid_create(cora_hybrid **out, int device) {
    NEED(out);
    *out = nullptr;
    return guarded([&] {
        auto h = std::make_unique<cora_hybrid>();
        h->index = std::make_unique<HybridIndex>(device);
        *out = h.release();
    });
}

int cora_hybrid_destroy(cora_hybrid *h) {
    delete h;
    return CORA_OK;
}

int cora_hybrid_configure(cora_hybrid *h, const cora_hybrid_config *c) {
    NEED(h);
    NEED(c);
    return guarded([&] {
        HybridIndex &x = *h->index;
        x.set_profiling(c->profiling != 0);
        x.set_candidate_stats(c->candidate_stats != 0);
        x.set_gpu_filter_timing(c->gpu_filter_timing != 0);
        x.set_cross_query_reuse(c->cross_query_reuse != 0);
        x.set_cpu_secondary_filter(c->cpu_secondary_filter != 0);
        x.set_vanguard_size(c->vanguard_size);
        if (c->queue_capacity)
            x.set_queue_capacity(c->queue_capacity);
        if (c->queue_spill_capacity != UINT64_MAX)
            x.set_queue_spill_capacity(c->queue_spill_capacity);
        x.set_metric(c->metric);
        x.set_frozen_thresholds(c->frozen_thresholds != 0);
        x.set_cpu_threads(c->cpu_threads);
        x.set_gpu_seed_refine(c->gpu_seed_refine != 0);
        x.set_gpu_refine_filter(c->gpu_refine_filter != 0);
        x.set_extra_search_flags(c->extra_flags);
        if (c->lower_bound_scale != 0.0f)
            x.set_lower_bound_scale(c->lower_bound_scale);
        x.set_gpu_final_topk(c->gpu_final_topk != 0);
        if (c->ip_kernel_type == 1)
            x.set_ip_kernel_type(KernelType::Lut4Bit);
        else if (c->ip_kernel_type == 2)
            x.set_ip_kernel_type(KernelType::Bitwise);
        else if (c->ip_kernel_type != 0)
            throw std::invalid_argument("ip_kernel_type must be 0 (keep), 1 (Lut4Bit) or 2 (Bitwise)");
    });
}

int cora_hybrid_load(cora_hybrid *h, uint64_t num_vecs, uint64_t dim, uint64_t padded_dim,
                     uint64_t n_centroids, uint64_t ex_bits, const float *centroids,
                     const float *rotator, const uint32_t *short_data, const float *short_factors,
                     const uint8_t *long_codes, const float *ex_factors, const uint32_t *ids,
                     const uint64_t *cluster_sizes) {
    NEED(h);
    return guarded([&] {
        h->index->load_from_raw_pointers(num_vecs, dim, padded_dim, n_centroids, ex_bits, centroids,
                                         rotator, short_data, short_factors, long_codes, ex_factors,
                                         ids, reinterpret_cast<const std::size_t *>(cluster_sizes));
    });
}

int cora_hybrid_enable_exact_refine(cora_hybrid *h, const uint8_t *base, uint64_t rows,
                                    uint64_t dim, uint64_t stride, uint64_t offset) {
    NEED(h);
    return guarded([&] { h->index->enable_exact_refine(base, rows, dim, stride, offset); });
}

int cora_hybrid_prepare(cora_hybrid *h, uint64_t max_queries, uint64_t max_topk,
                        uint64_t max_nprobe) {
    NEED(h);
    return guarded([&] { h->index->prepare_workspace(max_queries, max_topk, max_nprobe); });
}

int cora_hybrid_free_workspace(cora_hybrid *h) {
    NEED(h);
    h->index->free_workspace();
    return CORA_OK;
}

int cora_hybrid_reset(cora_hybrid *h, const float *queries, uint64_t nq) {
    NEED(h);
    return guarded([&] { h->index->reset_buffer(queries, nq); });
}

int cora_hybrid_search(cora_hybrid *h, const float *queries, uint64_t nq, uint64_t topk,
                       uint64_t nprobe, float *dists, uint32_t *ids, int batch_q) {
    NEED(h);
    return guarded([&] { h->index->search(queries, nq, topk, nprobe, dists, ids, batch_q); });
}

int cora_hybrid_stats_get(cora_hybrid *h, cora_hybrid_stats *out) {
    NEED(h);
    NEED(out);
    const HybridIndex &x = *h->index;
    out->submitted = x.get_last_submitted_count();
    out->spilled = x.get_last_spilled_count();
    out->refined = x.get_last_refined_count();
    out->gpu_filter_ms = x.get_last_gpu_filter_ms();
    out->scan_ms = x.get_last_scan_ms();
    out->scan_bytes = x.get_last_scan_bytes();
    out->scan_units = x.get_last_scan_units();
    out->scan_vectors = x.get_last_scan_vectors();
    out->probe_ms = x.get_last_probe_ms();
    out->probe_flops = x.get_last_probe_flops();
    for (int i = 0; i < 3; ++i)
        out->pass_produced[i] = x.get_last_pass_produced(i);
    out->seeded_queries = x.get_last_seeded_queries();
    out->prefilter_dropped = x.get_last_prefilter_dropped();
    out->seed_ms = x.get_last_seed_ms();
    out->recovery_ms = x.get_last_recovery_ms();
    out->gpu_refined = x.get_last_gpu_refined();
    out->vanguard_ms = x.get_last_vanguard_ms();
    out->vanguard_bytes = x.get_last_vanguard_bytes();
    out->vanguard_lows_ms = x.get_last_vanguard_lows_ms();
    out->vanguard_lows_bytes = x.get_last_vanguard_lows_bytes();
    out->vanguard_mode = x.get_last_vanguard_mode();
    for (int i = 0; i < 4; ++i)
        out->phase_ms[i] = x.get_last_phase_ms(i);
    out->vanguard_refine_ms = x.get_last_vanguard_refine_ms();
    out->vanguard_refine_bytes = x.get_last_vanguard_refine_bytes();
    return CORA_OK;
}

int cora_hybrid_capture_thresholds(cora_hybrid *h, float *out, uint64_t nq) {
    NEED(h);
    return guarded([&] { h->index->capture_thresholds(out, nq); });
}

int cora_hybrid_seed_thresholds(cora_hybrid *h, const float *in, uint64_t nq) {
    NEED(h);
    return guarded([&] { h->index->seed_thresholds(in, nq); });
}

int cora_hybrid_set_vanguard_size(cora_hybrid *h, uint64_t size) {
    NEED(h);
    return guarded([&] { h->index->set_vanguard_size(size); });
}

cora_gpu_engine *cora_hybrid_gpu(cora_hybrid *h) { return h ? h->index->gpu_engine() : nullptr; }

float cora_hybrid_lower_bound_scale(cora_hybrid *h) { return h ? h->index->get_lower_bound_scale() : 0.0f; }

int cora_ivf_load(const char *path, int include_extended, cora_ivf **out) {
    NEED(path);
    NEED(out);
    *out = nullptr;
    return guarded([&] {
        auto v = std::make_unique<cora_ivf>();
        v->data = index::SearchData::load(path, include_extended != 0, 0, &v->header, &v->ids);
        *out = v.release();
    });
}

int cora_ivf_info_get(const cora_ivf *v, cora_ivf_info *out) {
    NEED(v);
    NEED(out);
    out->num = v->header.num;
    out->dim = v->header.dim;
    out->padded_dim = v->header.padded_dim;
    out->nlist = v->header.nlist;
    out->ex_bits = v->header.ex_bits;
    out->max_cluster = v->data->max_cluster_size;
    out->metric = v->header.metric;
    out->centroid_storage = static_cast<int>(v->header.centroid_storage);
    return CORA_OK;
}

int cora_ivf_arrays_get(const cora_ivf *v, cora_ivf_arrays *out) {
    NEED(v);
    NEED(out);
    const index::SearchData &d = *v->data;
    out->centroids = d.h_centroids.data();
    out->rotator = d.host_rotator.data();
    out->short_data = d.host_short_data.data();
    out->short_factors = d.host_short_factors.data();
    out->long_codes = d.host_long_codes;
    out->ex_factors = d.host_ex_factors.empty() ? nullptr : d.host_ex_factors.data();
    out->ids = v->ids.data();
    out->cluster_sizes = reinterpret_cast<const uint64_t *>(d.cluster_sizes.data());
    return CORA_OK;
}

int cora_ivf_free(cora_ivf *v) {
    delete v;
    return CORA_OK;
}

int cora_build_ivf(const float *rotated_data, const float *rotated_centroids,
                   const uint32_t *assignments, const float *rotator, uint64_t n, uint64_t dim,
                   uint64_t padded_dim, uint64_t nlist, uint64_t ex_bits, int metric, int threads,
                   const char *out_path) {
    NEED(out_path);
    return guarded([&] {
        index::BuildInput in;
        in.rotated_data = rotated_data;
        in.rotated_centroids = rotated_centroids;
        in.assignments = assignments;
        in.rotator = rotator;
        in.n = n;
        in.dim = dim;
        in.padded_dim = padded_dim;
        in.nlist = nlist;
        in.ex_bits = ex_bits;
        in.metric = metric;
        index::build_ivf(in, threads).save(out_path);
    });
}

int cora_build_ivf_gpu(const float *data, const float *rotated_centroids, const uint32_t *assignments,
                       const float *rotator, uint64_t n, uint64_t dim, uint64_t padded_dim, uint64_t nlist,
                       uint64_t ex_bits, int metric, int device, int threads, const char *out_path) {
    NEED(out_path);
    return guarded([&] {
        index::GpuBuildInput in;
        in.data = data;
        in.rotated_centroids = rotated_centroids;
        in.assignments = assignments;
        in.rotator = rotator;
        in.n = n;
        in.dim = dim;
        in.padded_dim = padded_dim;
        in.nlist = nlist;
        in.ex_bits = ex_bits;
        in.metric = metric;
        index::build_ivf_gpu(in, device, threads).save(out_path);
    });
}

int cora_quantize_rows(const float *rows, const float *centroid, uint64_t n, uint64_t P,
                       uint64_t ex_bits, int metric, uint8_t *bits, float *f1, uint8_t *excode,
                       float *f2) {
    NEED(rows);
    NEED(centroid);
    return guarded([&] {
        for (uint64_t i = 0; i < n; ++i) {
            index::quantize_one_bit(rows + i * P, centroid, P, bits + i * P, f1 + 3 * i, metric);
            index::quantize_ex_bits(rows + i * P, centroid, P, ex_bits, excode + i * P, f2 + 2 * i,
                                    metric);
        }
    });
}

int cora_cpu_refine_isa(void) { return detail::excode_ip7_isa(); }

int cora_excode_ip7(const float *q, const uint8_t *packed, uint64_t n, uint64_t P, float *out) {
    NEED(q);
    NEED(packed);
    NEED(out);
    if (P % 64) {
        g_error = "padded dimension must be a multiple of 64";
        return CORA_ERR_INVALID_ARGUMENT;
    }
    for (uint64_t i = 0; i < n; ++i)
        out[i] = detail::excode_ip7(q, packed + i * (P * 7 / 8), P);
    return CORA_OK;
}

// CPU emulation of the device publication protocol (scan.hip publish / finish_kernel):
// each producer thread reserves wave-sized groups of positions with one atomic add, writes
// the slots below the cached write limit (refreshing it from Progress::released when a
// group crosses it) and appends the rest to a spill array; after all producers finish,
// a drain thread republishes spilled records as the consumer releases space and sets
// done. The consumer is the real cpu_refine. Record r of query q has refine distance
// f_ex_add = dist_of(q, r) (f_ex_rescale = 0, g_add = 0), so the expected top-k is known.
int cora_test_ring(cora_ring_test *t, float *dists, uint32_t *ids) {
    NEED(t);
    NEED(dists);
    NEED(ids);
    return guarded([&] {
        using queue::Position;
        if (t->capacity == 0 || (t->capacity & (t->capacity - 1)))
            throw std::invalid_argument("capacity must be a power of two");
        if (t->queries == 0 || t->queries > 65535 || t->topk == 0 || t->producers == 0)
            throw std::invalid_argument("bad ring test shape");
        const std::size_t nq = t->queries, per = t->per_query, N = nq * per;
        const std::size_t P = 64, lc = P * 7 / 8;
        std::vector<float> rq(nq * P, 0.0f), kb(nq, 0.0f), gadd(nq, 0.0f);
        std::vector<uint8_t> codes(std::max<std::size_t>(1, N) * lc, 0);
        std::vector<float> exf(std::max<std::size_t>(1, N) * 2, 0.0f);
        std::vector<uint32_t> pid(std::max<std::size_t>(1, N));
        for (std::size_t g = 0; g < N; ++g) {
            const std::size_t q = g / per, r = g % per;
            exf[2 * g] = 0.01f * static_cast<float>((r * 7919 + q * 31) % (per ? per : 1)) + 1.0f;
            pid[g] = static_cast<uint32_t>(g);
        }
        void *ring_mem = nullptr;
        if (posix_memalign(&ring_mem, 64, t->capacity * sizeof(queue::Candidate)))
            throw std::bad_alloc();
        std::unique_ptr<void, decltype(&free)> ring_guard(ring_mem, &free);
        auto *items = static_cast<queue::Candidate *>(ring_mem);
        std::memset(items, 0xFF, t->capacity * sizeof(queue::Candidate));
        auto progress = std::make_unique<queue::Progress>();
        std::vector<float> thr(nq, FLT_MAX);

        std::atomic<Position> produced{0}, cached_limit{t->capacity}, spill_count{0};
        std::atomic<int> overflow{0};
        std::vector<std::pair<queue::Candidate, Position>> spill(t->spill_capacity);
        std::atomic<std::size_t> next_group{0};
        const std::size_t group = 64;
        auto producer = [&] {
            for (;;) {
                const std::size_t g0 = next_group.fetch_add(group);
                if (g0 >= N)
                    break;
                const std::size_t cnt = std::min(group, N - g0);
                const Position base = produced.fetch_add(cnt);
                Position limit = cached_limit.load();
                if (base + cnt > limit) {
                    const Position fresh =
                        __atomic_load_n(&progress->released, __ATOMIC_ACQUIRE) + t->capacity;
                    Position cur = cached_limit.load();
                    while (cur < fresh && !cached_limit.compare_exchange_weak(cur, fresh)) {
                    }
                    limit = std::max(cur, fresh);
                }
                for (std::size_t i = 0; i < cnt; ++i) {
                    const std::size_t g = g0 + i;
                    queue::Candidate c{static_cast<uint16_t>(g / per), 0, static_cast<uint32_t>(g),
                                       0.0f, 0.0f};
                    const Position pos = base + i;
                    if (pos < limit) {
                        _mm_store_si128(reinterpret_cast<__m128i *>(&items[pos & (t->capacity - 1)]),
                                        _mm_load_si128(reinterpret_cast<const __m128i *>(&c)));
                    } else {
                        const Position s = spill_count.fetch_add(1);
                        if (s < t->spill_capacity)
                            spill[s] = {c, pos};
                        else
                            overflow.store(1);
                    }
                }
            }
        };
        auto drain = [&](std::vector<std::thread> &workers) {
            for (auto &w : workers)
                w.join();
            const Position total = produced.load(), sc = spill_count.load();
            __atomic_store_n(&progress->produced, total, __ATOMIC_RELAXED);
            __atomic_store_n(&progress->spilled, sc, __ATOMIC_RELAXED);
            if (overflow.load()) {
                __atomic_store_n(&progress->overflow, 1, __ATOMIC_RELEASE);
            } else {
                const std::size_t n = std::min<Position>(sc, t->spill_capacity);
                std::vector<char> published(n, 0);
                std::size_t remaining = n;
                const auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(60);
                while (remaining) {
                    const Position limit =
                        __atomic_load_n(&progress->released, __ATOMIC_ACQUIRE) + t->capacity;
                    for (std::size_t i = 0; i < n; ++i) {
                        if (!published[i] && spill[i].second < limit) {
                            _mm_store_si128(
                                reinterpret_cast<__m128i *>(&items[spill[i].second & (t->capacity - 1)]),
                                _mm_load_si128(reinterpret_cast<const __m128i *>(&spill[i].first)));
                            published[i] = 1;
                            --remaining;
                        }
                    }
                    if (std::chrono::steady_clock::now() > deadline) {
                        __atomic_store_n(&progress->overflow, 1, __ATOMIC_RELEASE);
                        break;
                    }
                    std::this_thread::yield();
                }
            }
            __atomic_store_n(&progress->done, 1, __ATOMIC_RELEASE);
        };
        std::vector<std::thread> workers;
        for (uint32_t i = 0; i < t->producers; ++i)
            workers.emplace_back(producer);
        std::thread drainer(drain, std::ref(workers));

        detail::RefineArgs a;
        a.items = items;
        a.progress = progress.get();
        a.capacity = t->capacity;
        a.thresholds = thr.data();
        a.rotated_queries = rq.data();
        a.kbxsumq = kb.data();
        a.probe_gadd = gadd.data();
        a.nprobe = 1;
        a.padded_dim = P;
        a.ex_bits = 7;
        a.long_codes = codes.data();
        a.ex_factors = exf.data();
        a.ids = pid.data();
        a.num_vectors = pid.size();
        a.secondary_filter = t->secondary_filter != 0;
        a.threads = static_cast<int>(t->consumers ? t->consumers : 1);
        const detail::RefineOut out = detail::cpu_refine(a, nq, t->topk, dists, ids);
        drainer.join();
        t->submitted = __atomic_load_n(&progress->produced, __ATOMIC_ACQUIRE);
        t->spilled = __atomic_load_n(&progress->spilled, __ATOMIC_ACQUIRE);
        t->refined = out.refined;
        t->overflow = __atomic_load_n(&progress->overflow, __ATOMIC_ACQUIRE);
        // the ring is left all-empty after a complete consumption
        if (!t->overflow)
            for (Position i = 0; i < t->capacity; ++i)
                if (items[i].gid != UINT32_MAX)
                    throw std::runtime_error("ring slot left non-empty after consumption");
    });
}

}  // extern "C"
