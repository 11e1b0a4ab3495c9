// C-ABI GPU engine (include/cora_gpu.h): owns HBM index residency, the search workspace,
// the host-coherent GPU->CPU candidate ring and the launch sequence of
// HybridIndex::search's GPU side (reference src/search/hybrid.cu:35-689).
#include <float.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <string>
#include <vector>

#include "../../../include/cora_gpu.h"
#include "engine_internal.h"

using namespace cora;

namespace {

constexpr unsigned long long kDrainMaxSeconds = 20;        // drain wait for the CPU consumer
constexpr uint64_t kMaxQueryChunk = 65535;                  // parameters.hpp:12
constexpr uint64_t kMaxProbeCount = 65536;                  // parameters.hpp:13
static_assert(kVanguardStagedMaxTopk == CORA_VANGUARD_STAGED_MAX_TOPK, "staged top-k limit");
// seeds per query the staged vanguard pass refines first: at least 128 and twice the top-k, at
// most 2,048 (their cut is a rank among 4,096 sub-stream minima of the query's group minima)
constexpr uint32_t kVsSeeds = 128;
uint32_t vs_seed_target(uint32_t topk) { return std::min<uint32_t>(2048, std::max<uint32_t>(kVsSeeds, 2 * topk)); }

template <class T>
void dfree(T *&p) {
    if (p)
        (void)hipFree(p);
    p = nullptr;
}

template <class T>
void hfree(T *&p) {
    if (p)
        (void)hipHostFree(p);
    p = nullptr;
}

// Query upload slices (cora_gpu_reset): kUploadSlices of them for 2 kUploadMinRows queries
// or more.
constexpr uint32_t kUploadSlices = 3;
constexpr uint32_t kUploadMinRows = 1024;

}  // namespace

struct cora_gpu_engine {
    int device = 0;
    std::string err;
    unsigned long long wall_clock_khz = 0;  // device wall_clock64() rate
    hipStream_t stream = nullptr, stream_d2h = nullptr;
    // query upload from the pinned staging buffer in slices (cora_gpu_reset): each slice's
    // DMA on stream_h2d signals ev_up[i]; the search prepares and probes a slice's queries as
    // soon as it has landed, while the later slices are still in flight
    hipStream_t stream_h2d = nullptr;
    // pair scheduling and the query order of the fused pass need only the probe indices: they
    // run on stream_aux (forked at ev_fork) beside the probes' exact g_add and join the engine
    // stream at ev_join before the first scan
    hipStream_t stream_aux = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    hipEvent_t ev_up[kUploadSlices] = {};
    hipEvent_t ev_pg[kUploadSlices][2] = {};  // the probe GEMM of each slice (timing)
    uint32_t up_slices = 0, up_row[kUploadSlices + 1] = {};
    uint64_t up_nq = 0;
    uint32_t last_slices = 0;  // slices of the last launched search (0: one pass)
    hipEvent_t ev_prep = nullptr, ev_probe = nullptr, ev_f0 = nullptr, ev_f1 = nullptr,
               ev_s0 = nullptr, ev_s1 = nullptr, ev_p0 = nullptr, ev_p1 = nullptr, ev_v0 = nullptr,
               ev_v1 = nullptr, ev_a0 = nullptr, ev_a1 = nullptr, ev_q0 = nullptr, ev_sched = nullptr,
               ev_done = nullptr;
    hipEvent_t ev_r[4] = {};  // the staged vanguard pass's two refinement launches (timing)
    // index
    bool loaded = false;
    uint64_t N = 0, dim = 0, P = 0, nl = 0, ex_bits = 0, max_cluster = 0, total_tiles = 0;
    int metric = 0;
    uint32_t W = 0, tile_bytes = 0;
    float *d_cent = nullptr, *d_cnorm = nullptr, *d_rot = nullptr;
    uint16_t *d_cent_hl = nullptr;  // split-FP16 centroids [2][nl][P] (coarse-probe GEMM)
    float *d_cscale = nullptr;      // their row scales [nl]
    uint16_t *d_rot_hl = nullptr;   // split-FP16 R^T [2][P][dim] (query rotation GEMM)
    float *d_rtscale = nullptr;     // its row scales [P]
    uint8_t *d_tiles = nullptr;
    ClusterMeta *d_meta = nullptr;
    uint8_t *d_exrec = nullptr;  // optional refinement records [N][ex_record_bytes(P)]
    // queue configuration (hybrid.cuh:105-106)
    uint64_t qcap = 1ull << 26, spill_cap = 1ull << 24;
    // workspace
    bool ws = false;
    uint64_t ws_q = 0, ws_k = 0, ws_np = 0, ws_van = 0, seed_words = 0;
    float *d_raw = nullptr, *d_qrot = nullptr, *d_k1 = nullptr, *d_kb = nullptr,
          *d_qnorm = nullptr, *d_qwidth = nullptr, *d_qwidth2 = nullptr, *d_dist = nullptr, *d_gadd = nullptr,
          *d_gerr = nullptr, *d_thr_snap = nullptr;
    uint32_t *d_planes = nullptr, *d_bcount = nullptr, *d_bcursor = nullptr, *d_boff = nullptr,
             *d_uoff = nullptr, *d_nunits = nullptr, *d_cursor = nullptr, *d_seed = nullptr;
    int32_t *d_pidx = nullptr;
    uint16_t *d_q_hl = nullptr;  // split-FP16 rotated queries [2][max_q][P]
    float *d_qscale = nullptr;
    uint16_t *d_raw_hl = nullptr;  // split-FP16 raw queries [2][max_q][dim]
    float *d_rawscale = nullptr;
    uint32_t *d_qorder = nullptr;  // queries by nearest cluster (fused vanguard pass)
    int8_t *d_qbytes = nullptr;    // [max_q][2][P] qint, qres (MFMA far scan operands)
    uint16_t *d_lut = nullptr;     // [max_q][P/4][16] FP16 nibble tables (LUT4 estimator)
    float *d_lut_margin = nullptr;  // [max_q] |LUT4 - Bitwise estimate| bound (launch_lut_margin)
    float *d_seed_dist = nullptr, *d_seed_low = nullptr, *d_seed_err = nullptr;
    uint4 *d_seed_rec = nullptr;
    float *d_van_lows = nullptr;  // [max_q][vanguard][van_stride] lower bounds of vanguard pairs
    float *d_van_mins = nullptr;  // [max_q][vanguard][van_stride / 4] their group minima (staged pass)
    unsigned long long *d_selbig = nullptr;  // [max_q][2][max_nprobe] probe select scratch, nprobe > 4096
    uint32_t *d_probe_fb = nullptr;          // [1 + max_q] fused probe select: fallback count, rows
    // GPU-final top-k: per-query counts/offsets/cursor, grouped keys [spill_cap], results
    uint32_t *d_fcount = nullptr, *d_foff = nullptr, *d_fcur = nullptr, *d_fidx = nullptr;
    unsigned long long *d_fkeys = nullptr;
    float *d_fdist = nullptr;
    uint64_t van_stride = 0;
    // staged vanguard pass (vanguard_staged.hip): per-query regions of seeds, tier and list,
    // per-query state, counters and the overflow list
    uint32_t *d_vs_seed_pos = nullptr, *d_vs_list_pos = nullptr;
    float2 *d_vs_seed_rd = nullptr, *d_vs_seed_aux = nullptr, *d_vs_list_rd = nullptr, *d_vs_list_aux = nullptr;
    VsQuery *d_vs_qs = nullptr;
    uint4 *d_vs_out = nullptr;
    unsigned long long *d_vs_spread = nullptr;
    uint32_t vs_out_cap = 0;
    unsigned long long *d_vs_ctr = nullptr;
    uint32_t *d_vs_ovf = nullptr;
    uint32_t vs_seed_cap = 0, vs_list_cap = 0;
    Pair *d_pairs = nullptr;
    Unit *d_units = nullptr;
    unsigned long long *d_stats = nullptr;
    unsigned long long *d_btot = nullptr;  // per-block totals of the bucket scan
    bool bcount_zero = false;  // d_bcount is all zero: the last pair scheduling's scan cleared it
    // queue
    uint4 *h_items = nullptr;
    ProgressDev *h_progress = nullptr;
    float *h_thr = nullptr, *h_thr_stage = nullptr;
    float *h_qstage = nullptr;  // pinned query staging [max_q][dim] (cora_gpu_query_staging)
    unsigned long long *h_sync = nullptr;  // pinned: the search's statistics and stall flag (cora_gpu_sync)
    int *h_abort = nullptr;
    unsigned long long *d_produced = nullptr, *d_cached_limit = nullptr, *d_spill_count = nullptr;
    int *d_refresh = nullptr, *d_overflow = nullptr, *d_stalled = nullptr;
    SpillRecord *d_spill = nullptr;
    bool ring_dirty = false;
    bool final_mode = false;  // the launch in flight publishes to HBM (CORA_FLAG_GPU_FINAL)
    // pinned host copies for CPU refinement
    float *h_qrot = nullptr, *h_kb = nullptr, *h_gadd = nullptr;
    // last launch
    bool launched = false;
    cora_search_args last{};
    uint32_t last_depth = 0, last_batch = 1;
    bool last_timing = false, last_fused = false, last_mfma = false, last_van_lows = false, last_final = false;
    bool last_staged = false;  // the vanguard pairs ran in the staged pass
    bool last_fused_probe = false;  // the last search selected its probes in the GEMM epilogue + merge
    int last_vanguard_mode = 0;  // cora_search_stats::vanguard_mode
};

namespace {

// The staged pass can serve top-k above kVanguardMaxTopk at this vanguard depth: its kernels
// are there and its seed and list regions hold every vanguard vector of a query, so no query
// overflows to the one-pass kernel.
bool staged_high_k_ok(const cora_gpu_engine *E, uint32_t flags, uint32_t depth) {
    const uint64_t all = (uint64_t)depth * E->van_stride;
    return depth > 0 && E->d_van_lows && E->d_vs_seed_pos && far_mfma_supported(E->W) &&
           !(flags & CORA_FLAG_NO_VANGUARD_MFMA) && E->vs_seed_cap >= all && E->vs_list_cap >= all;
}

int fail(cora_gpu_engine *e, int code, const std::string &msg) {
    if (e)
        e->err = msg;
    return code;
}

#define HIPCHK(call)                                                                             \
    do {                                                                                         \
        hipError_t e_ = (call);                                                                  \
        if (e_ != hipSuccess)                                                                    \
            return fail(E, CORA_ERR_RUNTIME, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

QueueDev queue_dev(cora_gpu_engine *E) {
    QueueDev q{};
    q.items = E->h_items;
    q.progress = E->h_progress;
    q.capacity = E->qcap;
    q.mask = E->qcap - 1;
    q.produced = E->d_produced;
    q.cached_limit = E->d_cached_limit;
    q.refresh_flag = E->d_refresh;
    q.spill = E->d_spill;
    q.spill_count = E->d_spill_count;
    q.spill_capacity = E->spill_cap;
    q.spill_overflow = E->d_overflow;
    q.abort_flag = E->h_abort;
    q.stalled = E->d_stalled;
    q.final_mode = E->final_mode ? 1 : 0;
    return q;
}

ScanParams scan_params(cora_gpu_engine *E, uint32_t depth, uint32_t keep, bool frozen) {
    ScanParams p{};
    p.tiles = E->d_tiles;
    p.meta = E->d_meta;
    p.qplanes = E->d_planes;
    p.qbytes = E->d_qbytes;
    p.lut = (E->last.flags & CORA_FLAG_LUT4) ? reinterpret_cast<const uint32_t *>(E->d_lut) : nullptr;
    p.lut_margin = E->d_lut_margin;
    p.refine_err = refine_err_scale((uint32_t)E->P);
    p.qwidth = E->d_qwidth;
    p.qwidth2 = E->d_qwidth2;
    p.k1 = E->d_k1;
    p.pgadd = E->d_gadd;
    p.pgerr = E->d_gerr;
    p.pairs = E->d_pairs;
    p.units = E->d_units;
    p.num_units = E->d_nunits;
    p.unit_cursor = E->d_cursor;
    // frozen: the launch snapshot; live: a copy of the host thresholds taken before each pass
    p.thresholds = E->d_thr_snap;
    p.nprobe = E->last.nprobe;
    p.vanguard = depth;
    p.keep = keep;
    p.tile_bytes = E->tile_bytes;
    p.P = (uint32_t)E->P;
    p.seed_words = (uint32_t)E->seed_words;
    p.seed_bits = E->d_seed;
    p.queue = queue_dev(E);
    p.van_lows = E->d_van_lows;
    p.van_stride = (uint32_t)E->van_stride;
    uint32_t buf = 128;  // seed pass buffer: power of two >= keep + one tile
    while (buf < keep + kTileVectors)
        buf <<= 1;
    p.seed_buf = buf;
    return p;
}

void release_queue(cora_gpu_engine *E) {
    hfree(E->h_items);
    hfree(E->h_progress);
    hfree(E->h_thr);
    hfree(E->h_thr_stage);
    hfree(E->h_qstage);
    hfree(E->h_sync);
    hfree(E->h_abort);
    dfree(E->d_produced);
    dfree(E->d_cached_limit);
    dfree(E->d_spill_count);
    dfree(E->d_refresh);
    dfree(E->d_overflow);
    dfree(E->d_stalled);
    dfree(E->d_spill);
}

void release_workspace(cora_gpu_engine *E) {
    if (E->stream)
        (void)hipStreamSynchronize(E->stream);
    if (E->stream_d2h)
        (void)hipStreamSynchronize(E->stream_d2h);
    if (E->stream_h2d)
        (void)hipStreamSynchronize(E->stream_h2d);
    if (E->stream_aux)
        (void)hipStreamSynchronize(E->stream_aux);
    E->up_slices = 0;
    E->ws = false;
    E->launched = false;
    E->ws_q = E->ws_k = E->ws_np = E->ws_van = E->seed_words = 0;
    for (float **p : {&E->d_raw, &E->d_qrot, &E->d_k1, &E->d_kb, &E->d_qnorm, &E->d_qwidth, &E->d_qwidth2,
                      &E->d_dist, &E->d_gadd, &E->d_gerr, &E->d_thr_snap, &E->d_qscale, &E->d_rawscale})
        dfree(*p);
    dfree(E->d_q_hl);
    dfree(E->d_raw_hl);
    for (uint32_t **p : {&E->d_planes, &E->d_bcount, &E->d_bcursor, &E->d_boff, &E->d_uoff,
                         &E->d_nunits, &E->d_cursor, &E->d_seed})
        dfree(*p);
    dfree(E->d_pidx);
    dfree(E->d_qorder);
    dfree(E->d_qbytes);
    dfree(E->d_lut);
    dfree(E->d_lut_margin);
    dfree(E->d_seed_dist);
    dfree(E->d_seed_low);
    dfree(E->d_seed_err);
    dfree(E->d_seed_rec);
    dfree(E->d_van_lows);
    dfree(E->d_van_mins);
    dfree(E->d_vs_seed_pos);
    dfree(E->d_vs_seed_rd);
    dfree(E->d_vs_seed_aux);
    dfree(E->d_vs_list_pos);
    dfree(E->d_vs_list_rd);
    dfree(E->d_vs_list_aux);
    dfree(E->d_vs_qs);
    dfree(E->d_vs_out);
    dfree(E->d_vs_spread);
    dfree(E->d_vs_ctr);
    dfree(E->d_vs_ovf);
    E->vs_seed_cap = E->vs_list_cap = 0;
    dfree(E->d_selbig);
    dfree(E->d_probe_fb);
    dfree(E->d_fcount);
    dfree(E->d_foff);
    dfree(E->d_fcur);
    dfree(E->d_fidx);
    dfree(E->d_fkeys);
    dfree(E->d_fdist);
    E->van_stride = 0;
    dfree(E->d_pairs);
    dfree(E->d_units);
    dfree(E->d_stats);
    dfree(E->d_btot);
    hfree(E->h_qrot);
    hfree(E->h_kb);
    hfree(E->h_gadd);
    release_queue(E);
}

template <class T>
int dalloc(cora_gpu_engine *E, T *&p, size_t count) {
    p = nullptr;
    const hipError_t r = hipMalloc(reinterpret_cast<void **>(&p), std::max<size_t>(1, count) * sizeof(T));
    if (r != hipSuccess) {
        p = nullptr;
        return fail(E, r == hipErrorOutOfMemory ? CORA_ERR_OUT_OF_MEMORY : CORA_ERR_RUNTIME,
                    std::string("hipMalloc: ") + hipGetErrorString(r));
    }
    return CORA_OK;
}

template <class T>
int halloc(cora_gpu_engine *E, T *&p, size_t count, unsigned flags) {
    p = nullptr;
    const hipError_t r =
        hipHostMalloc(reinterpret_cast<void **>(&p), std::max<size_t>(1, count) * sizeof(T), flags);
    if (r != hipSuccess) {
        p = nullptr;
        return fail(E, CORA_ERR_OUT_OF_MEMORY, std::string("hipHostMalloc: ") + hipGetErrorString(r));
    }
    return CORA_OK;
}

#define TRY(x)                  \
    do {                        \
        const int rc_ = (x);    \
        if (rc_ != CORA_OK)     \
            return rc_;         \
    } while (0)

bool is_pow2(uint64_t v) { return v && !(v & (v - 1)); }

// validate_search_shape (reference include/coraanns/search/parameters.hpp:15-25)
int validate_shape(cora_gpu_engine *E, uint64_t q, uint64_t k, uint64_t np) {
    if (q == 0 || q > kMaxQueryChunk)
        return fail(E, CORA_ERR_INVALID_ARGUMENT,
                    "query count must be in [1, 65535]; split larger batches");
    if (k == 0 || k > (uint64_t)INT32_MAX / q)
        return fail(E, CORA_ERR_INVALID_ARGUMENT,
                    "topk must be positive and queries * topk must fit an int");
    if (np == 0 || np > kMaxProbeCount || np > E->nl)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "nprobe must be in [1, min(nlist, 65536)]");
    if (E->nl > (uint64_t)INT32_MAX / q || E->P == 0 || E->P > (uint64_t)INT32_MAX / (q * 4))
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "query workspace exceeds kernel indexing limits");
    if (np > 65536)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "nprobe must be in [1, min(nlist, 65536)]");
    return CORA_OK;
}

}  // namespace

extern "C" {

int cora_gpu_create(cora_gpu_engine **out, int device) {
    if (!out)
        return CORA_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    auto *E = new (std::nothrow) cora_gpu_engine();
    if (!E)
        return CORA_ERR_OUT_OF_MEMORY;
    E->device = device;
    auto init = [&]() -> int {
        HIPCHK(hipSetDevice(device));
        int khz = 0;
        HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device));
        if (khz <= 0)
            return fail(E, CORA_ERR_RUNTIME, "device reports no wall clock rate");
        E->wall_clock_khz = (unsigned long long)khz;
        HIPCHK(hipStreamCreateWithFlags(&E->stream, hipStreamNonBlocking));
        HIPCHK(hipStreamCreateWithFlags(&E->stream_d2h, hipStreamNonBlocking));
        HIPCHK(hipStreamCreateWithFlags(&E->stream_h2d, hipStreamNonBlocking));
        HIPCHK(hipStreamCreateWithFlags(&E->stream_aux, hipStreamNonBlocking));
        HIPCHK(hipEventCreateWithFlags(&E->ev_fork, hipEventDisableTiming));
        HIPCHK(hipEventCreateWithFlags(&E->ev_join, hipEventDisableTiming));
        for (uint32_t i = 0; i < kUploadSlices; ++i) {
            HIPCHK(hipEventCreateWithFlags(&E->ev_up[i], hipEventDisableTiming));
            HIPCHK(hipEventCreate(&E->ev_pg[i][0]));
            HIPCHK(hipEventCreate(&E->ev_pg[i][1]));
        }
        for (hipEvent_t *ev : {&E->ev_prep, &E->ev_probe, &E->ev_f0, &E->ev_f1, &E->ev_s0, &E->ev_s1,
                               &E->ev_p0, &E->ev_p1, &E->ev_v0, &E->ev_v1, &E->ev_a0, &E->ev_a1, &E->ev_q0,
                               &E->ev_sched, &E->ev_done})
            HIPCHK(hipEventCreate(ev));
        for (hipEvent_t &ev : E->ev_r)
            HIPCHK(hipEventCreate(&ev));
        return CORA_OK;
    };
    const int rc = init();
    if (rc != CORA_OK) {
        std::string msg = E->err;
        cora_gpu_destroy(E);
        (void)msg;
        return rc;
    }
    *out = E;
    return CORA_OK;
}

int cora_gpu_destroy(cora_gpu_engine *E) {
    if (!E)
        return CORA_OK;
    (void)hipSetDevice(E->device);
    release_workspace(E);
    dfree(E->d_cent);
    dfree(E->d_cnorm);
    dfree(E->d_cent_hl);
    dfree(E->d_cscale);
    dfree(E->d_rot_hl);
    dfree(E->d_rtscale);
    dfree(E->d_rot);
    dfree(E->d_tiles);
    dfree(E->d_meta);
    dfree(E->d_exrec);
    for (hipEvent_t ev : {E->ev_prep, E->ev_probe, E->ev_f0, E->ev_f1, E->ev_s0, E->ev_s1, E->ev_p0,
                          E->ev_p1, E->ev_v0, E->ev_v1, E->ev_a0, E->ev_a1, E->ev_q0, E->ev_sched, E->ev_done})
        if (ev)
            (void)hipEventDestroy(ev);
    if (E->stream)
        (void)hipStreamDestroy(E->stream);
    for (uint32_t i = 0; i < kUploadSlices; ++i)
        for (hipEvent_t ev : {E->ev_up[i], E->ev_pg[i][0], E->ev_pg[i][1]})
            if (ev)
                (void)hipEventDestroy(ev);
    if (E->stream_d2h)
        (void)hipStreamDestroy(E->stream_d2h);
    if (E->stream_h2d)
        (void)hipStreamDestroy(E->stream_h2d);
    for (hipEvent_t ev : {E->ev_fork, E->ev_join, E->ev_r[0], E->ev_r[1], E->ev_r[2], E->ev_r[3]})
        if (ev)
            (void)hipEventDestroy(ev);
    if (E->stream_aux)
        (void)hipStreamDestroy(E->stream_aux);
    delete E;
    return CORA_OK;
}

int cora_gpu_last_error(const cora_gpu_engine *E, char *buf, size_t n) {
    if (!E || !buf || !n)
        return CORA_ERR_INVALID_ARGUMENT;
    const size_t m = std::min(n - 1, E->err.size());
    memcpy(buf, E->err.data(), m);
    buf[m] = '\0';
    return CORA_OK;
}

int cora_gpu_load_index(cora_gpu_engine *E, uint64_t num_vecs, uint64_t dim, uint64_t padded_dim,
                        uint64_t n_centroids, uint64_t ex_bits, int metric,
                        const float *h_centroids, const float *h_rotator,
                        const uint32_t *h_short_data, const float *h_short_factors,
                        const uint64_t *h_cluster_sizes) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (E->loaded)
        return fail(E, CORA_ERR_LOGIC, "index already loaded");
    if (!num_vecs || num_vecs > UINT32_MAX || !dim || padded_dim < dim || padded_dim % 64 ||
        !n_centroids || ex_bits > 8 || !h_centroids || !h_rotator || !h_short_data ||
        !h_short_factors || !h_cluster_sizes || (metric != CORA_METRIC_L2 && metric != CORA_METRIC_IP))
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "invalid index shape or missing index data");
    if (padded_dim > 1024)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "padded dimension above 1024 is not supported");
    if (n_centroids > UINT32_MAX / 2)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "too many centroids");
    HIPCHK(hipSetDevice(E->device));
    std::vector<ClusterMeta> meta(n_centroids);
    uint64_t count = 0, largest = 0, tiles = 0;
    for (uint64_t c = 0; c < n_centroids; ++c) {
        const uint64_t n = h_cluster_sizes[c];
        if (n > num_vecs - count)
            return fail(E, CORA_ERR_INVALID_ARGUMENT, "cluster sizes exceed index size");
        meta[c] = ClusterMeta{(uint32_t)count, (uint32_t)n, (uint32_t)tiles, 0u};
        count += n;
        largest = std::max(largest, n);
        tiles += (n + kTileVectors - 1) / kTileVectors;
    }

    if (count != num_vecs)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "cluster sizes differ from index size");
    if (tiles > UINT32_MAX)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "index too large for 32-bit tile indices");
    const uint32_t W = (uint32_t)(padded_dim / 32);
    const uint32_t tile_bytes = 256u * W + 768u;
    uint32_t *d_ref = nullptr;
    float *d_reff = nullptr;
    float *d_rt = nullptr;  // R^T, FP32, until split
    auto cleanup = [&]() {
        dfree(d_ref);
        dfree(d_reff);
        dfree(d_rt);
    };
    int rc = CORA_OK;
    do {
        if ((rc = dalloc(E, E->d_meta, n_centroids)) ||
            (rc = dalloc(E, E->d_tiles, std::max<uint64_t>(1, tiles) * tile_bytes)) ||
            (rc = dalloc(E, E->d_cent, n_centroids * padded_dim)) ||
            (rc = dalloc(E, E->d_cnorm, n_centroids)) ||
            (rc = dalloc(E, E->d_cent_hl, 2 * n_centroids * padded_dim)) ||
            (rc = dalloc(E, E->d_cscale, n_centroids)) ||
            (rc = dalloc(E, E->d_rot, dim * padded_dim)) ||
            (rc = dalloc(E, E->d_rot_hl, 2 * dim * padded_dim)) ||
            (rc = dalloc(E, E->d_rtscale, padded_dim)) || (rc = dalloc(E, d_rt, dim * padded_dim)) ||
            (rc = dalloc(E, d_ref, num_vecs * W)) || (rc = dalloc(E, d_reff, num_vecs * 3)))
            break;
        hipError_t r = hipSuccess;
        auto chk = [&](hipError_t x, const char *what) {
            if (x != hipSuccess && r == hipSuccess) {
                r = x;
                E->err = std::string(what) + ": " + hipGetErrorString(x);
            }
        };
        chk(hipMemcpyAsync(E->d_meta, meta.data(), n_centroids * sizeof(ClusterMeta),
                           hipMemcpyHostToDevice, E->stream), "meta upload");
        chk(hipMemcpyAsync(E->d_cent, h_centroids, n_centroids * padded_dim * 4,
                           hipMemcpyHostToDevice, E->stream), "centroid upload");
        chk(hipMemcpyAsync(E->d_rot, h_rotator, dim * padded_dim * 4, hipMemcpyHostToDevice,
                           E->stream), "rotator upload");
        std::vector<float> rt(dim * padded_dim);  // R^T [P][dim]: the rotation GEMM's B rows
        for (uint64_t d = 0; d < dim; ++d)
            for (uint64_t c = 0; c < padded_dim; ++c)
                rt[c * dim + d] = h_rotator[d * padded_dim + c];
        chk(hipMemcpyAsync(d_rt, rt.data(), dim * padded_dim * 4, hipMemcpyHostToDevice, E->stream),
            "rotator upload");
        chk(hipMemcpyAsync(d_ref, h_short_data, num_vecs * W * 4, hipMemcpyHostToDevice, E->stream),
            "code upload");
        chk(hipMemcpyAsync(d_reff, h_short_factors, num_vecs * 12, hipMemcpyHostToDevice, E->stream),
            "factor upload");
        if (r == hipSuccess) {
            launch_repack(d_ref, d_reff, E->d_meta, (uint32_t)n_centroids, W, E->d_tiles, tile_bytes,
                          E->stream);
            launch_row_norms(E->d_cent, (uint32_t)n_centroids, (uint32_t)padded_dim, E->d_cnorm,
                             E->stream);
            launch_split_f16(E->d_cent, (uint32_t)n_centroids, (uint32_t)padded_dim, E->d_cent_hl,
                             E->d_cscale, E->stream);
            launch_split_f16(d_rt, (uint32_t)padded_dim, (uint32_t)dim, E->d_rot_hl, E->d_rtscale, E->stream);
            chk(hipGetLastError(), "repack launch");
            chk(hipStreamSynchronize(E->stream), "index upload");
        }
        if (r != hipSuccess)
            rc = CORA_ERR_RUNTIME;
    } while (0);
    cleanup();
    if (rc != CORA_OK) {
        dfree(E->d_meta);
        dfree(E->d_tiles);
        dfree(E->d_cent);
        dfree(E->d_cnorm);
        dfree(E->d_cent_hl);
        dfree(E->d_cscale);
        dfree(E->d_rot_hl);
        dfree(E->d_rtscale);
        dfree(E->d_rot);
        return rc;
    }
    E->N = num_vecs;
    E->dim = dim;
    E->P = padded_dim;
    E->nl = n_centroids;
    E->ex_bits = ex_bits;
    E->metric = metric;
    E->W = W;
    E->tile_bytes = tile_bytes;
    E->max_cluster = largest;
    E->total_tiles = tiles;
    E->loaded = true;
    return CORA_OK;
}

int cora_gpu_load_excodes(cora_gpu_engine *E, const uint8_t *h_long_codes,
                          const float *h_ex_factors) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->loaded)
        return fail(E, CORA_ERR_LOGIC, "load the index before its ex-codes");
    if (E->d_exrec)
        return fail(E, CORA_ERR_LOGIC, "ex-codes already loaded");
    if (E->ws)
        return fail(E, CORA_ERR_LOGIC, "load ex-codes before prepare_workspace");
    if (!h_long_codes || !h_ex_factors || E->ex_bits != 7)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "GPU ex-codes need 7 ex-bits and both arrays");
    HIPCHK(hipSetDevice(E->device));
    // records built on the device: the ex-codes and factors uploaded in bounded chunks
    // through a staging pair, then the sign codes copied from the tiles
    const uint64_t lc = E->P * 7 / 8;
    const uint64_t chunk = std::max<uint64_t>(1, std::min<uint64_t>(E->N, (256ull << 20) / (lc + 8)));
    uint8_t *st_codes = nullptr;
    float *st_fac = nullptr;
    int rc = dalloc(E, E->d_exrec, E->N * ex_record_bytes((uint32_t)E->P));
    if (rc == CORA_OK)
        rc = dalloc(E, st_codes, chunk * lc);
    if (rc == CORA_OK)
        rc = dalloc(E, st_fac, chunk * 2);
    hipError_t r = hipSuccess;
    for (uint64_t g0 = 0; rc == CORA_OK && r == hipSuccess && g0 < E->N; g0 += chunk) {
        const uint64_t n = std::min(chunk, E->N - g0);
        r = hipMemcpy(st_codes, h_long_codes + g0 * lc, n * lc, hipMemcpyHostToDevice);
        if (r == hipSuccess)
            r = hipMemcpy(st_fac, h_ex_factors + 2 * g0, n * 2 * sizeof(float), hipMemcpyHostToDevice);
        if (r == hipSuccess) {
            launch_ex_record_fill(st_codes, st_fac, g0, (uint32_t)n, (uint32_t)E->P, E->d_exrec, E->stream);
            r = hipGetLastError();
        }
        if (r == hipSuccess)
            r = hipStreamSynchronize(E->stream);  // the staging pair is reused
    }
    if (rc == CORA_OK && r == hipSuccess) {
        launch_ex_record_sign(E->d_meta, (uint32_t)E->nl, E->d_tiles, (uint32_t)E->tile_bytes, (uint32_t)E->W,
                              E->d_exrec, E->stream);
        r = hipGetLastError();
        if (r == hipSuccess)
            r = hipStreamSynchronize(E->stream);
    }
    if (rc == CORA_OK && r != hipSuccess)
        rc = fail(E, CORA_ERR_RUNTIME, std::string("ex-code upload: ") + hipGetErrorString(r));
    dfree(st_codes);
    dfree(st_fac);
    if (rc != CORA_OK)
        dfree(E->d_exrec);
    return rc;
}

int cora_gpu_set_queue(cora_gpu_engine *E, uint64_t capacity, uint64_t spill_capacity) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!is_pow2(capacity) || capacity > (1ull << 40))
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "queue-capacity must be a positive power of two");
    if (spill_capacity > (1ull << 36))
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "queue-spill-capacity is too large");
    if (E->ws)
        return fail(E, CORA_ERR_LOGIC, "set queue capacity before prepare_workspace");
    E->qcap = capacity;
    E->spill_cap = spill_capacity;
    return CORA_OK;
}

int cora_gpu_prepare_workspace(cora_gpu_engine *E, uint64_t max_q, uint64_t max_topk,
                               uint64_t max_nprobe, uint64_t vanguard_size) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->loaded)
        return fail(E, CORA_ERR_LOGIC, "load an index before preparing workspace");
    TRY(validate_shape(E, max_q, max_topk, max_nprobe));
    HIPCHK(hipSetDevice(E->device));
    release_workspace(E);
    const uint64_t nb = 2 * E->nl;
    const uint64_t np = max_q * max_nprobe;
    const uint64_t depth = std::min(vanguard_size, max_nprobe);
    const uint64_t seed_words = (E->max_cluster + 31) / 32;
    auto alloc_all = [&]() -> int {
        TRY(dalloc(E, E->d_raw, max_q * E->dim));
        TRY(dalloc(E, E->d_qrot, max_q * E->P));
        TRY(dalloc(E, E->d_k1, max_q));
        TRY(dalloc(E, E->d_kb, max_q));
        TRY(dalloc(E, E->d_qnorm, max_q));
        TRY(dalloc(E, E->d_qwidth, max_q));
        TRY(dalloc(E, E->d_qwidth2, max_q));
        TRY(dalloc(E, E->d_planes, max_q * 2 * kBq * E->W));
        TRY(dalloc(E, E->d_dist, max_q * E->nl));
        TRY(dalloc(E, E->d_q_hl, 2 * max_q * E->P));
        TRY(dalloc(E, E->d_raw_hl, 2 * max_q * E->dim));
        TRY(dalloc(E, E->d_rawscale, max_q));
        TRY(dalloc(E, E->d_qscale, max_q));
        TRY(dalloc(E, E->d_pidx, np));
        TRY(dalloc(E, E->d_qorder, max_q));
        TRY(dalloc(E, E->d_qbytes, max_q * 2 * E->P));
        TRY(dalloc(E, E->d_lut, max_q * 4 * E->P));
        TRY(dalloc(E, E->d_lut_margin, max_q));
        TRY(dalloc(E, E->d_gadd, np));
        TRY(dalloc(E, E->d_gerr, np));
        TRY(dalloc(E, E->d_bcount, nb));
        E->bcount_zero = false;
        TRY(dalloc(E, E->d_bcursor, nb));
        TRY(dalloc(E, E->d_boff, nb + 1));
        TRY(dalloc(E, E->d_uoff, nb + 1));
        TRY(dalloc(E, E->d_nunits, 2));
        TRY(dalloc(E, E->d_cursor, kNumXcd));
        TRY(dalloc(E, E->d_stats, 11));
        TRY(dalloc(E, E->d_btot, bucket_scan_words((uint32_t)E->nl)));
        TRY(dalloc(E, E->d_pairs, np));
        TRY(dalloc(E, E->d_units, np * unit_splits((uint32_t)E->max_cluster)));
        TRY(dalloc(E, E->d_thr_snap, max_q));
        TRY(dalloc(E, E->d_seed, std::max<uint64_t>(1, max_q * depth * seed_words)));
        if (max_nprobe > (uint64_t)kSelectMaxProbe)
            TRY(dalloc(E, E->d_selbig, max_q * 2 * max_nprobe));
        TRY(dalloc(E, E->d_probe_fb, 1 + max_q));
        if (depth > 0) {
            // a multiple of 256: the fused pass streams a pair's bounds 256 at a time
            E->van_stride = (E->max_cluster + 255) / 256 * 256;
            TRY(dalloc(E, E->d_van_lows, max_q * depth * std::max<uint64_t>(E->van_stride, 1)));
            TRY(dalloc(E, E->d_van_mins, max_q * depth * std::max<uint64_t>(E->van_stride / 4, 1)));
        }
        if (E->d_exrec) {
            TRY(dalloc(E, E->d_fcount, max_q));
            TRY(dalloc(E, E->d_foff, max_q + 1));
            TRY(dalloc(E, E->d_fcur, max_q));
            TRY(dalloc(E, E->d_fidx, max_q * max_topk));
            TRY(dalloc(E, E->d_fdist, max_q * max_topk));
            TRY(dalloc(E, E->d_fkeys, std::max<uint64_t>(1, E->spill_cap)));
            if (depth > 0 && vanguard_staged_supported(E->W)) {
                // the staged vanguard pass: per query, room for about four times its seeds, and
                // for the list sixteen times (at least 4,096); a query whose seeds or list do not
                // fit is left to the one-pass kernel
                const auto up256 = [](uint64_t x) { return (x + 255) / 256 * 256; };
                const uint64_t seeds = vs_seed_target((uint32_t)max_topk);
                uint64_t seed_cap = up256(4 * seeds), list_cap = std::max<uint64_t>(4096, up256(16 * seeds));
                // above the one-pass kernel's top-k only the staged pass serves a query, so its
                // regions hold every vanguard vector and cannot overflow
                if (max_topk > kVanguardMaxTopk) {
                    seed_cap = std::max<uint64_t>(seed_cap, depth * E->van_stride);
                    list_cap = std::max<uint64_t>(list_cap, depth * E->van_stride);
                }
                // CORA_VANGUARD_REGION_CAP: smaller regions (tests of the overflow path)
                if (const char *env = getenv("CORA_VANGUARD_REGION_CAP"))
                    seed_cap = list_cap = std::max<uint64_t>(64, strtoull(env, nullptr, 10));
                E->vs_seed_cap = (uint32_t)seed_cap;
                E->vs_list_cap = (uint32_t)list_cap;
                TRY(dalloc(E, E->d_vs_seed_pos, max_q * seed_cap));
                TRY(dalloc(E, E->d_vs_seed_rd, max_q * seed_cap));
                TRY(dalloc(E, E->d_vs_seed_aux, max_q * seed_cap));
                TRY(dalloc(E, E->d_vs_list_pos, max_q * list_cap));
                TRY(dalloc(E, E->d_vs_list_rd, max_q * list_cap));
                TRY(dalloc(E, E->d_vs_list_aux, max_q * list_cap));
                TRY(dalloc(E, E->d_vs_qs, max_q));
                E->vs_out_cap = (uint32_t)up256(std::max<uint64_t>(256, 4 * max_topk));
                TRY(dalloc(E, E->d_vs_out, max_q * E->vs_out_cap));
                TRY(dalloc(E, E->d_vs_spread, kVsSpread * kVsSpreadWords));
                TRY(dalloc(E, E->d_vs_ctr, kVsCtrWords));
                TRY(dalloc(E, E->d_vs_ovf, max_q));
            }
            const uint64_t slots = max_q * depth * std::max<uint64_t>(max_topk, 20);
            TRY(dalloc(E, E->d_seed_dist, slots));
            TRY(dalloc(E, E->d_seed_low, slots));
            TRY(dalloc(E, E->d_seed_err, slots));
            TRY(dalloc(E, E->d_seed_rec, slots));
        }
        TRY(halloc(E, E->h_qrot, max_q * E->P, hipHostMallocDefault));
        TRY(halloc(E, E->h_kb, max_q, hipHostMallocDefault));
        TRY(halloc(E, E->h_gadd, np, hipHostMallocDefault));
        // ring, progress, thresholds: host-coherent so GPU stores and host stores are seen
        // by the other side while kernels run (reference cudaHostAllocMapped, hybrid.cu:192-199)
        const unsigned coherent = hipHostMallocMapped | hipHostMallocCoherent;
        TRY(halloc(E, E->h_items, E->qcap, coherent));
        TRY(halloc(E, E->h_progress, 1, coherent));
        TRY(halloc(E, E->h_thr, max_q, coherent));
        TRY(halloc(E, E->h_thr_stage, max_q, hipHostMallocDefault));
        TRY(halloc(E, E->h_qstage, max_q * E->dim, hipHostMallocDefault));
        TRY(halloc(E, E->h_sync, 12, hipHostMallocDefault));
        TRY(halloc(E, E->h_abort, 1, coherent));
        TRY(dalloc(E, E->d_produced, 1));
        TRY(dalloc(E, E->d_cached_limit, 1));
        TRY(dalloc(E, E->d_spill_count, 1));
        TRY(dalloc(E, E->d_refresh, 1));
        TRY(dalloc(E, E->d_overflow, 1));
        TRY(dalloc(E, E->d_stalled, 1));
        TRY(dalloc(E, E->d_spill, std::max<uint64_t>(1, E->spill_cap)));
        return CORA_OK;
    };
    const int rc = alloc_all();
    if (rc != CORA_OK) {
        const std::string msg = E->err;
        release_workspace(E);
        E->err = msg;
        return rc;
    }
    memset(E->h_items, 0xFF, E->qcap * sizeof(uint4));
    new (E->h_progress) ProgressDev{};
    for (uint64_t i = 0; i < max_q; ++i)
        E->h_thr[i] = FLT_MAX;
    *E->h_abort = 0;
    launch_queue_reset(queue_dev(E), E->stream);
    HIPCHK(hipGetLastError());
    HIPCHK(hipStreamSynchronize(E->stream));
    E->ws_q = max_q;
    E->ws_k = max_topk;
    E->ws_np = max_nprobe;
    E->ws_van = depth;
    E->seed_words = seed_words;
    E->ring_dirty = false;
    E->ws = true;
    return CORA_OK;
}

int cora_gpu_free_workspace(cora_gpu_engine *E) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    (void)hipSetDevice(E->device);
    release_workspace(E);
    return CORA_OK;
}

int cora_gpu_queue_view(cora_gpu_engine *E, cora_queue_view *out) {
    if (!E || !out)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->ws)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace before searching");
    out->items = E->h_items;
    out->progress = E->h_progress;
    out->capacity = E->qcap;
    out->thresholds = E->h_thr;
    out->abort_flag = E->h_abort;
    return CORA_OK;
}

int cora_gpu_final_results(cora_gpu_engine *E, float *dists, uint32_t *idx) {
    if (!E || !dists || !idx)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->launched || !E->last_final)
        return fail(E, CORA_ERR_LOGIC, "no GPU-final search launched");
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->stream));
    const size_t n = (size_t)E->last.num_queries * E->last.topk;
    HIPCHK(hipMemcpy(dists, E->d_fdist, n * 4, hipMemcpyDeviceToHost));
    HIPCHK(hipMemcpy(idx, E->d_fidx, n * 4, hipMemcpyDeviceToHost));
    return CORA_OK;
}

int cora_gpu_query_staging(cora_gpu_engine *E, float **out) {
    if (!E || !out)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->ws)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace before searching");
    // the caller is about to rewrite the buffer: the last reset's upload must be complete
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->stream_h2d));
    *out = E->h_qstage;
    return CORA_OK;
}

int cora_gpu_reset(cora_gpu_engine *E, const float *h_queries, uint64_t nq) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->ws)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace before searching");
    if (nq == 0 || nq > E->ws_q)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "search shape exceeds the prepared workspace");
    if (!h_queries)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "missing queries");
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->stream));
    HIPCHK(hipStreamSynchronize(E->stream_h2d));
    if (E->ring_dirty) {
        memset(E->h_items, 0xFF, E->qcap * sizeof(uint4));
        E->ring_dirty = false;
    }
    E->up_slices = 0;
    E->up_nq = nq;
    if (h_queries == E->h_qstage && nq >= 2 * kUploadMinRows) {
        // from the pinned staging buffer: three slices of whole 128-row tiles on the H2D
        // stream, the first an eighth of the queries (it lands soonest, and the GPU starts on
        // it), the other two halves of the rest (large enough to fill the GPU in the rotation
        // GEMM); the search waits for each before the kernels that read it
        const auto up128 = [](uint64_t r) { return (r + 127) / 128 * 128; };
        const uint64_t s0 = up128(nq / 8), s1 = s0 + up128((nq - s0) / 2);
        const uint64_t bounds[kUploadSlices + 1] = {0, s0, s1, nq};
        const uint32_t ns = kUploadSlices;
        for (uint32_t i = 0; i < ns; ++i) {
            const uint64_t r0 = bounds[i], r1 = bounds[i + 1];
            E->up_row[i] = (uint32_t)r0;
            E->up_row[i + 1] = (uint32_t)r1;
            HIPCHK(hipMemcpyAsync(E->d_raw + r0 * E->dim, h_queries + r0 * E->dim, (r1 - r0) * E->dim * 4,
                                  hipMemcpyHostToDevice, E->stream_h2d));
            HIPCHK(hipEventRecord(E->ev_up[i], E->stream_h2d));
        }
        E->up_slices = ns;
    } else {
        HIPCHK(hipMemcpyAsync(E->d_raw, h_queries, nq * E->dim * 4, hipMemcpyHostToDevice, E->stream));
    }
    launch_queue_reset(queue_dev(E), E->stream);
    HIPCHK(hipGetLastError());
    new (E->h_progress) ProgressDev{};
    for (uint64_t i = 0; i < nq; ++i)
        E->h_thr[i] = FLT_MAX;
    *E->h_abort = 0;
    E->launched = false;
    // an upload from any other host array is resident in HBM when reset returns (a pageable
    // upload may still be in flight after hipMemcpyAsync returns)
    if (!E->up_slices)
        HIPCHK(hipStreamSynchronize(E->stream));
    return CORA_OK;
}

int cora_gpu_launch_search(cora_gpu_engine *E, const cora_search_args *a) {
    if (!E || !a)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->ws)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace before searching");
    if (a->num_queries == 0 || a->num_queries > E->ws_q || a->topk == 0 || a->topk > E->ws_k ||
        a->nprobe == 0 || a->nprobe > E->ws_np)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "search shape exceeds the prepared workspace");
    if (!(a->bound_scale >= 0.0f && a->bound_scale <= 16.0f))
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "invalid bound scale (expected 0..16; 0 means 1)");
    if (a->batch_q < 1 || a->batch_q > kMaxBatchQArg)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "invalid batch-q (expected 1..64)");
    const uint64_t want_depth = std::min<uint64_t>(a->vanguard, a->nprobe);
    if (want_depth > E->ws_van)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace again before increasing vanguard size");
    // GPU-final top-k: every published record must carry its refined distance, which the
    // fused vanguard pass and the refined pre-filter compute (live thresholds, or the
    // frozen snapshot in its GPU-seeded test mode)
    const bool want_final = (a->flags & CORA_FLAG_GPU_FINAL) != 0;
    const bool lut = (a->flags & CORA_FLAG_LUT4) != 0;
    const uint32_t final_max_topk =
        staged_high_k_ok(E, a->flags, (uint32_t)want_depth) ? kVanguardStagedMaxTopk : kVanguardMaxTopk;
    if (want_final &&
        (!E->d_exrec || !E->d_fkeys ||
         (a->flags & (CORA_FLAG_NO_GPU_SEED | CORA_FLAG_NO_GPU_PREFILTER | CORA_FLAG_PAIR_SEEDS | CORA_FLAG_LUT4)) ||
         ((a->flags & CORA_FLAG_FROZEN_THRESHOLDS) && !(a->flags & CORA_FLAG_GPU_SEED_FROZEN)) ||
         want_depth == 0 || want_depth > kVanguardMaxPairs || a->topk > final_max_topk))
        return fail(E, CORA_ERR_LOGIC,
                    "GPU-final top-k needs the ex-codes in HBM, GPU seed thresholds and the refined "
                    "pre-filter, the fused vanguard pass (vanguard 1..64, topk <= 128, or <= 1024 with "
                    "the staged pass's regions, Bitwise estimator) and live thresholds");
    HIPCHK(hipSetDevice(E->device));
    E->final_mode = want_final;
    E->last_final = want_final;
    const uint32_t nq = a->num_queries, np = a->nprobe;
    const uint32_t keep = std::max<uint32_t>(a->topk, 20u);
    const uint32_t depth = keep <= (uint32_t)kMaxVanguardKeep ? (uint32_t)want_depth : 0u;
    // Cross-query reuse: the far pairs of one cluster are scanned together, batch_q at a time
    // by the popcount kernel, or kMfmaBatchQ at a time by the matrix-core kernel when the
    // padded dimension allows it (the unit size changes only the speed, never the result).
    // The LUT4 estimator (the reference's default Lut4Bit producers) runs the per-pair seed,
    // far and recovery passes of the popcount kernels with the FP16 tables in place of the
    // q-planes, at most kLutMaxBatchQ pairs per pass.
    const bool reuse = (a->flags & CORA_FLAG_CROSS_QUERY_REUSE) != 0;
    // LUT4 on the matrix cores (wide codes): the far scan and the vanguard lows pass filter
    // with Bitwise bounds lowered by the query's LUT4 margin and evaluate the LUT4 bound of
    // the survivors exactly; the vanguard pass is the staged one, refining with the LUT4
    // estimate
    const bool lut_mfma = lut && reuse && far_mfma_lut_supported(E->W) && !(a->flags & CORA_FLAG_NO_MFMA_SCAN);
    const bool mfma_far = (!lut || lut_mfma) && reuse && far_mfma_supported(E->W) &&
                          !(a->flags & CORA_FLAG_NO_MFMA_SCAN);
    const uint32_t batch = mfma_far ? kMfmaBatchQ
                           : reuse  ? std::min<uint32_t>(a->batch_q, lut ? kLutMaxBatchQ : (uint32_t)kMaxBatchQ)
                                    : 1u;
    const bool frozen = (a->flags & CORA_FLAG_FROZEN_THRESHOLDS) != 0;
    const bool timing = (a->flags & CORA_FLAG_FILTER_TIMING) != 0;
    E->last = *a;
    E->ring_dirty = true;  // until cora_gpu_sync sees every produced record released
    E->last_depth = depth;
    E->last_batch = batch;
    E->last_mfma = mfma_far;
    E->last_timing = timing;
    hipStream_t s = E->stream;
    const uint32_t P = (uint32_t)E->P;

    if (want_final)  // no ring: the write limit never binds
        launch_fill_u64(E->d_cached_limit, ~0ull, 1, s);
    // query preparation (hybrid.cu:436-463) and coarse probing (hybrid.cu:465-498)
    const bool split_gemm = !(a->flags & CORA_FLAG_FP32_GEMM);
    const bool split_rot = split_gemm && dist_gemm_f16x3_supported((uint32_t)E->dim, nq, P);
    const bool split_probe = split_gemm && dist_gemm_f16x3_supported(P, nq, E->nl);
    // the fused select keeps its candidates in the distance matrix's memory
    const bool fused_probe = split_probe && !(a->flags & CORA_FLAG_UNFUSED_PROBE) &&
                             fused_probe_supported((uint32_t)E->nl, np) &&
                             fused_probe_scratch_bytes(nq, (uint32_t)E->nl, np) <= (size_t)nq * E->nl * sizeof(float);
    E->last_fused_probe = fused_probe;
    // queries uploaded in slices (cora_gpu_reset): each slice is rotated, prepared and probed
    // by the fused GEMM as soon as it has landed; every other path waits for the whole upload
    const uint32_t ns = E->up_slices && E->up_nq == nq && split_rot && fused_probe && !lut ? E->up_slices : 0u;
    E->last_slices = ns;
    if (!ns)
        for (uint32_t i = 0; i < E->up_slices; ++i)
            HIPCHK(hipStreamWaitEvent(s, E->ev_up[i], 0));
    if (ns) {
        const uint64_t D = E->dim;
        launch_fill_u32(E->d_probe_fb, 0u, 1, s);  // the fallback count (launch_fused_probe_gemm)
        for (uint32_t i = 0; i < ns; ++i) {
            const uint32_t r0 = E->up_row[i], rows = E->up_row[i + 1] - r0;
            HIPCHK(hipStreamWaitEvent(s, E->ev_up[i], 0));
            if (timing && i == 0)
                HIPCHK(hipEventRecord(E->ev_q0, s));
            launch_split_f16_rows(E->d_raw + r0 * D, rows, (uint32_t)D, E->d_raw_hl + r0 * D,
                                  E->d_raw_hl + (nq + r0) * D, E->d_rawscale + r0, s);
            launch_rotate_f16x3_rows(E->d_raw_hl + r0 * D, E->d_raw_hl + (nq + r0) * D, E->d_rawscale + r0,
                                     E->d_rot_hl, E->d_rtscale, rows, (uint32_t)D, P, E->d_qrot + (size_t)r0 * P, s);
            launch_query_prep(E->d_qrot + (size_t)r0 * P, rows, P, (uint32_t)E->ex_bits, E->d_k1 + r0, E->d_kb + r0,
                              E->d_qnorm + r0, E->d_qwidth + r0, E->d_qwidth2 + r0,
                              E->d_planes + (size_t)r0 * 2 * kBq * E->W, E->d_qbytes + (size_t)r0 * 2 * P, s);
            if (i + 1 == ns) {
                HIPCHK(hipEventRecord(E->ev_prep, s));
                HIPCHK(hipStreamWaitEvent(E->stream_d2h, E->ev_prep, 0));
                HIPCHK(hipMemcpyAsync(E->h_qrot, E->d_qrot, (size_t)nq * P * 4, hipMemcpyDeviceToHost,
                                      E->stream_d2h));
                HIPCHK(hipMemcpyAsync(E->h_kb, E->d_kb, (size_t)nq * 4, hipMemcpyDeviceToHost, E->stream_d2h));
            }
            launch_split_f16_rows(E->d_qrot + (size_t)r0 * P, rows, P, E->d_q_hl + (size_t)r0 * P,
                                  E->d_q_hl + (size_t)(nq + r0) * P, E->d_qscale + r0, s);
            if (timing)
                HIPCHK(hipEventRecord(E->ev_pg[i][0], s));
            launch_fused_probe_gemm_rows(E->d_q_hl, E->d_q_hl + (size_t)nq * P, E->d_qscale, E->d_qnorm,
                                         E->d_cent_hl, E->d_cscale, E->d_cnorm, r0, rows, nq, (uint32_t)E->nl, P,
                                         np, E->d_dist, s);
            if (timing)
                HIPCHK(hipEventRecord(E->ev_pg[i][1], s));
        }
    } else {
        if (timing)
            HIPCHK(hipEventRecord(E->ev_q0, s));
        if (split_rot) {
            launch_split_f16(E->d_raw, nq, (uint32_t)E->dim, E->d_raw_hl, E->d_rawscale, s);
            launch_rotate_f16x3(E->d_raw_hl, E->d_rawscale, E->d_rot_hl, E->d_rtscale, nq, (uint32_t)E->dim,
                                P, E->d_qrot, s);
        } else
            launch_rotate(E->d_raw, E->d_rot, E->d_qrot, nq, (uint32_t)E->dim, P, s);
        launch_query_prep(E->d_qrot, nq, P, (uint32_t)E->ex_bits, E->d_k1, E->d_kb, E->d_qnorm,
                          E->d_qwidth, E->d_qwidth2, E->d_planes, E->d_qbytes, s);
        if (lut)
            launch_lut_build(E->d_qrot, nq, P, E->d_lut, s);
        if (lut_mfma)
            launch_lut_margin(E->d_qrot, E->d_planes, E->d_qwidth, nq, P, E->d_lut_margin, s);
        HIPCHK(hipEventRecord(E->ev_prep, s));
        HIPCHK(hipStreamWaitEvent(E->stream_d2h, E->ev_prep, 0));
        HIPCHK(hipMemcpyAsync(E->h_qrot, E->d_qrot, (size_t)nq * P * 4, hipMemcpyDeviceToHost,
                              E->stream_d2h));
        HIPCHK(hipMemcpyAsync(E->h_kb, E->d_kb, (size_t)nq * 4, hipMemcpyDeviceToHost, E->stream_d2h));
        if (timing)
            HIPCHK(hipEventRecord(E->ev_p0, s));
        if (split_probe) {
            launch_split_f16(E->d_qrot, nq, P, E->d_q_hl, E->d_qscale, s);
            if (fused_probe)
                launch_fused_probe_gemm(E->d_q_hl, E->d_qscale, E->d_qnorm, E->d_cent_hl, E->d_cscale, E->d_cnorm,
                                        nq, (uint32_t)E->nl, P, np, E->d_dist, E->d_probe_fb, s);
            else
                launch_dist_gemm_f16x3(E->d_q_hl, E->d_qscale, E->d_qnorm, E->d_cent_hl, E->d_cscale, E->d_cnorm,
                                       nq, (uint32_t)E->nl, P, E->d_dist, s);
        } else
            launch_dist_gemm(E->d_qrot, E->d_qnorm, E->d_cent, E->d_cnorm, nq, (uint32_t)E->nl, P,
                             E->d_dist, s);
    }
    if (timing)
        HIPCHK(hipEventRecord(E->ev_p1, s));
    if (fused_probe)
        launch_fused_probe_select(E->d_q_hl, E->d_qscale, E->d_qnorm, E->d_cent_hl, E->d_cscale, E->d_cnorm, nq,
                                  (uint32_t)E->nl, P, np, E->d_dist, E->d_probe_fb, E->d_pidx, s);
    else if (np > (uint32_t)kSelectMaxProbe)
        launch_select_big(E->d_dist, nq, (uint32_t)E->nl, np, E->d_selbig, E->d_pidx, s);
    else
        launch_select(E->d_dist, nq, (uint32_t)E->nl, np, E->d_pidx, s);
    // GPU ex-code stages (seed thresholds, refined pre-filter): live thresholds only, or
    // the frozen snapshot in the GPU_SEED_FROZEN test mode
    const bool ex_stage_mode = !frozen || (a->flags & CORA_FLAG_GPU_SEED_FROZEN);
    const bool gpu_seed = depth > 0 && E->d_exrec && E->d_seed_dist && ex_stage_mode &&
                          !(a->flags & CORA_FLAG_NO_GPU_SEED);
    const bool prefilter = E->d_exrec && ex_stage_mode && !(a->flags & CORA_FLAG_NO_GPU_PREFILTER);
    // fused per-query vanguard pass (vanguard.hip) unless the reference's per-pair passes
    // are asked for or the shape exceeds its limits
    const bool staged_ok = E->d_van_lows && E->d_vs_seed_pos && far_mfma_supported(E->W) &&
                           !(a->flags & CORA_FLAG_NO_VANGUARD_MFMA);
    const bool lut_staged = lut_mfma && staged_ok;
    // above kVanguardMaxTopk (up to kVanguardStagedMaxTopk) only the staged pass, with regions
    // that hold every vanguard vector
    const bool fused = gpu_seed && (!lut || lut_staged) && !(a->flags & CORA_FLAG_PAIR_SEEDS) && depth <= kVanguardMaxPairs &&
                       (a->topk <= kVanguardMaxTopk ||
                        (a->topk <= kVanguardStagedMaxTopk && staged_high_k_ok(E, a->flags, depth)));
    const bool high_k = a->topk > kVanguardMaxTopk;
    // its lower bounds first on the matrix cores, cluster-major, into the per-pair lows
    // array [nq][depth][van_stride] of the workspace
    // (by default for wide codes whose sign codes and factors exceed the last-level cache, and
    // for any index beyond 1 GiB: a nearly cache-resident index is read cheaply enough by each
    // query's own pass)
    const uint64_t index_bytes = (uint64_t)E->N * (E->P / 8 + 12);
    const bool lows_by_size =
        (index_bytes > kLowsMinIndexBytes && E->P >= kLowsMinDim) || index_bytes > kLowsAnyDimBytes;
    const bool van_lows = fused && depth > 0 && far_mfma_supported(E->W) && E->d_van_lows &&
                          !(a->flags & CORA_FLAG_NO_VANGUARD_MFMA) &&
                          (lows_by_size || (a->flags & CORA_FLAG_VANGUARD_MFMA) || lut || high_k);
    // fork: pair scheduling (and the fused pass's query order) on stream_aux
    HIPCHK(hipEventRecord(E->ev_fork, s));
    HIPCHK(hipStreamWaitEvent(E->stream_aux, E->ev_fork, 0));
    // pair scheduling (hybrid.cu:504-508)
    launch_build_pairs(E->d_pidx, E->d_meta, nq, np, (uint32_t)E->nl, depth, batch,
                       van_lows ? kMfmaBatchQ : 1u, P / 8 + 12, E->d_bcount, E->d_bcursor, E->d_boff,
                       E->d_uoff, E->d_pairs, E->d_units,
                       (uint64_t)nq * np * unit_splits((uint32_t)E->max_cluster), E->d_nunits, E->d_stats,
                       E->d_btot, E->bcount_zero, E->stream_aux);
    E->bcount_zero = true;
    const bool ordered = fused && launch_order_queries(E->d_pidx, nq, np, (uint32_t)E->nl, E->d_qorder,
                                                       E->stream_aux);
    HIPCHK(hipEventRecord(E->ev_join, E->stream_aux));
    launch_probe_refine(E->d_qrot, E->d_cent, E->d_pidx, nq, np, P, E->metric, E->d_gadd,
                        E->d_gerr, a->bound_scale > 0.0f ? a->bound_scale : 1.0f, s);
    HIPCHK(hipEventRecord(E->ev_probe, s));
    HIPCHK(hipStreamWaitEvent(E->stream_d2h, E->ev_probe, 0));
    HIPCHK(hipMemcpyAsync(E->h_gadd, E->d_gadd, (size_t)nq * np * 4, hipMemcpyDeviceToHost,
                          E->stream_d2h));
    HIPCHK(hipStreamWaitEvent(s, E->ev_join, 0));
    if (timing)
        HIPCHK(hipEventRecord(E->ev_sched, s));
    if (frozen) {
        memcpy(E->h_thr_stage, E->h_thr, (size_t)nq * 4);
        HIPCHK(hipMemcpyAsync(E->d_thr_snap, E->h_thr_stage, (size_t)nq * 4, hipMemcpyHostToDevice, s));
    }
    ScanParams p = scan_params(E, depth, keep, frozen);
    if (gpu_seed || prefilter) {
        p.ex_rec = E->d_exrec;
        p.ex_stride = ex_record_bytes((uint32_t)E->P);
        p.qrot = E->d_qrot;
        p.kb = E->d_kb;
    }
    if (gpu_seed) {
        p.seed_dist = E->d_seed_dist;
        p.seed_low = E->d_seed_low;
        p.seed_err = E->d_seed_err;
        p.seed_rec = E->d_seed_rec;
    }
    p.prefilter = prefilter ? 1 : 0;
    p.dropped = E->d_stats + 7;
    VanguardArgs va{};
    // the staged pass (grid-wide refinement) where the lows pass wrote every vanguard bound:
    // for LUT4 and above the one-pass kernel's top-k, or when asked for. The one-pass kernel
    // publishes each query as it ends, so the CPU consumer starts early (measured, config 4:
    // top-10 1.53-1.60M QPS one-pass against 1.50M staged, top-100 988k against 713k, 1.08M
    // both with GPU-final top-k; config 5: 1.33M against 1.16M)
    const bool staged = van_lows && E->d_vs_seed_pos &&
                        (lut || high_k ||
                         ((a->flags & CORA_FLAG_VANGUARD_STAGED) && !(a->flags & CORA_FLAG_VANGUARD_ONE_PASS)));
    p.van_mins = staged ? E->d_van_mins : nullptr;
    E->last_fused = fused && depth > 0;
    E->last_van_lows = van_lows;
    E->last_staged = staged;
    E->last_vanguard_mode = depth == 0 ? 0 : !fused ? 1 : staged ? 4 : van_lows ? 3 : 2;
    if (fused) {
        va.probe_idx = E->d_pidx;
        va.nq = nq;
        va.order = ordered ? E->d_qorder : nullptr;
        va.depth = depth;
        va.topk = a->topk;
        va.thr_out = frozen ? E->d_thr_snap : E->h_thr;
        va.seeded = E->d_stats + 6;
        va.refined = E->d_stats + 8;
        va.lows_ready = van_lows ? 1 : 0;
    }
    launch_fill_u64(E->d_stats + 3, 0ull, 6, s);  // per-pass counters of this launch
    if (timing)
        HIPCHK(hipEventRecord(E->ev_f0, s));
    // live thresholds: each pass reads a copy of the host array taken just before it
    auto snapshot = [&]() {
        if (!frozen)
            launch_snapshot_thresholds(E->h_thr, E->d_thr_snap, nq, s);
    };
    if (depth > 0 && fused) {
        if (van_lows) {
            launch_cursor_init(E->d_cursor, E->d_nunits, 0, s);
            if (timing)
                HIPCHK(hipEventRecord(E->ev_a0, s));
            launch_vanguard_lows(p, E->W, s);
            if (timing)
                HIPCHK(hipEventRecord(E->ev_a1, s));
        }
        snapshot();
        if (timing)
            HIPCHK(hipEventRecord(E->ev_v0, s));
        if (staged) {
            VsArgs vs{};
            vs.seed_pos = E->d_vs_seed_pos;
            vs.seed_rd = E->d_vs_seed_rd;
            vs.seed_aux = E->d_vs_seed_aux;
            vs.list_pos = E->d_vs_list_pos;
            vs.list_rd = E->d_vs_list_rd;
            vs.list_aux = E->d_vs_list_aux;
            vs.seed_cap = E->vs_seed_cap;
            vs.list_cap = E->vs_list_cap;
            vs.qs = E->d_vs_qs;
            vs.out = E->d_vs_out;
            vs.out_cap = E->vs_out_cap;
            vs.spread = E->d_vs_spread;
            vs.ctr = E->d_vs_ctr;
            vs.overflow = E->d_vs_ovf;
            vs.seeds = vs_seed_target(a->topk);
            launch_fill_u64(E->d_vs_ctr, 0ull, kVsCtrWords, s);
            launch_fill_u64(E->d_vs_spread, 0ull, kVsSpread * kVsSpreadWords, s);
            launch_vanguard_staged(p, va, vs, E->W, nq, timing ? E->ev_r[0] : nullptr, timing ? E->ev_r[1] : nullptr,
                                   timing ? E->ev_r[2] : nullptr, timing ? E->ev_r[3] : nullptr, s);
        } else {
            launch_vanguard_query(p, va, E->W, nq, s);
        }
        if (timing)
            HIPCHK(hipEventRecord(E->ev_v1, s));
    } else if (depth > 0) {
        launch_fill_u32(E->d_seed, 0u, (size_t)nq * depth * E->seed_words, s);
        snapshot();
        if (gpu_seed)  // +inf marks seed slots the seed pass leaves unused
            launch_fill_u32(reinterpret_cast<uint32_t *>(E->d_seed_dist), 0x7F800000u,
                            (size_t)nq * depth * keep, s);
        launch_cursor_init(E->d_cursor, E->d_nunits, 0, s);
        launch_vanguard_seed(p, E->W, s);
        if (gpu_seed)
            launch_seed_thresholds(E->d_seed_dist, E->d_seed_low, E->d_seed_err, E->d_seed_rec, nq,
                                   depth * keep, a->topk, frozen ? E->d_thr_snap : E->h_thr,
                                   E->d_stats + 6, queue_dev(E), s);
    }
    launch_copy_u64(E->d_produced, E->d_stats + 3, s);
    launch_cursor_init(E->d_cursor, E->d_nunits, 1, s);
    snapshot();
    if (timing)
        HIPCHK(hipEventRecord(E->ev_s0, s));
    if (mfma_far)
        launch_far_mfma(p, E->W, false, s);
    else
        launch_scan(p, E->W, batch, 0, s);
    if (timing)
        HIPCHK(hipEventRecord(E->ev_s1, s));
    launch_copy_u64(E->d_produced, E->d_stats + 4, s);
    if (depth > 0 && !fused) {
        launch_cursor_init(E->d_cursor, E->d_nunits, 0, s);
        snapshot();
        launch_scan(p, E->W, 1, 1, s);
    }
    launch_copy_u64(E->d_produced, E->d_stats + 5, s);
    if (timing)
        HIPCHK(hipEventRecord(E->ev_f1, s));
    launch_finish(queue_dev(E), kDrainMaxSeconds * 1000ull * E->wall_clock_khz, s);
    if (want_final)
        launch_final_topk(reinterpret_cast<const SpillRecord *>(E->d_spill), E->d_produced, E->spill_cap, nq,
                          a->topk, E->d_fcount, E->d_foff, E->d_fcur, E->d_fkeys, E->d_fdist, E->d_fidx, s);
    HIPCHK(hipGetLastError());
    E->final_mode = false;  // the kernels took their copy of the queue view
    E->launched = true;
    return CORA_OK;
}

int cora_gpu_wait_host_inputs(cora_gpu_engine *E, const float **rq, const float **kb,
                              const float **gadd) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->launched)
        return fail(E, CORA_ERR_LOGIC, "no search launched");
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->stream_d2h));
    if (rq)
        *rq = E->h_qrot;
    if (kb)
        *kb = E->h_kb;
    if (gadd)
        *gadd = E->h_gadd;
    return CORA_OK;
}

int cora_gpu_sync(cora_gpu_engine *E, cora_search_stats *st) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->launched)
        return fail(E, CORA_ERR_LOGIC, "no search launched");
    HIPCHK(hipSetDevice(E->device));
    // the statistics and the stall flag in one round trip: both copies behind the search's
    // kernels on its stream, into pinned memory, and one synchronisation
    HIPCHK(hipMemcpyAsync(E->h_sync, E->d_stats, 11 * sizeof(unsigned long long), hipMemcpyDeviceToHost, E->stream));
    HIPCHK(hipMemcpyAsync(E->h_sync + 11, E->d_stalled, sizeof(int), hipMemcpyDeviceToHost, E->stream));
    HIPCHK(hipStreamSynchronize(E->stream));
    HIPCHK(hipStreamSynchronize(E->stream_d2h));
    unsigned long long stats[11];
    memcpy(stats, E->h_sync, sizeof(stats));
    int stalled = 0;
    memcpy(&stalled, E->h_sync + 11, sizeof(int));
    cora_search_stats out{};
    out.produced = __atomic_load_n(&E->h_progress->produced, __ATOMIC_ACQUIRE);
    out.spilled = __atomic_load_n(&E->h_progress->spilled, __ATOMIC_ACQUIRE);
    const int overflow = __atomic_load_n(&E->h_progress->overflow, __ATOMIC_ACQUIRE);
    out.stalled = stalled;
    out.overflow = overflow && !stalled;
    out.vanguard_mode = E->last_vanguard_mode;
    out.scan_bytes = stats[0];
    out.scan_units = stats[1];
    out.scan_vectors = stats[2];
    out.probe_flops = 2ull * E->last.num_queries * E->P * E->nl;
    for (int i = 0; i < 3; ++i)
        out.pass_produced[i] = stats[3 + i];
    out.seeded_queries = stats[6];
    out.prefilter_dropped = stats[7];
    out.gpu_refined = stats[8];
    // the per-query pass: code + factors of every vanguard vector (or its 4-byte lower bound
    // when the lows pass ran), then P/8 + 7P/8 + 8 per refined one; the lows pass: code +
    // factors of the cluster once per unit read, a 4-byte bound per (vector, vanguard pair)
    // written, and for the staged pass the minimum of each 4 of them
    if (E->last_fused && E->last_van_lows) {
        out.vanguard_bytes = 4 * stats[10] + stats[8] * (E->P + 8);
        out.vanguard_lows_bytes = stats[9] + stats[10] * (E->last_staged ? 5 : 4);
        // staged pass: the refinement launches read each refined vector's record and its pool
        // position and lower bound, and write its result (the one-pass kernel's overflow
        // queries, refined inside that kernel, are counted here too)
        if (E->last_staged)
            out.vanguard_refine_bytes = stats[8] * (E->P + 8 + 24);
    } else if (E->last_fused) {
        out.vanguard_bytes = stats[9] + stats[8] * (E->P + 8);
    }
    if (E->last_timing) {
        HIPCHK(hipEventElapsedTime(&out.filter_ms, E->ev_f0, E->ev_f1));
        HIPCHK(hipEventElapsedTime(&out.scan_ms, E->ev_s0, E->ev_s1));
        if (E->last_slices) {
            // the probe GEMM slice by slice (query preparation runs between them)
            out.probe_ms = 0.0f;
            for (uint32_t i = 0; i < E->last_slices; ++i) {
                float ms = 0.0f;
                HIPCHK(hipEventElapsedTime(&ms, E->ev_pg[i][0], E->ev_pg[i][1]));
                out.probe_ms += ms;
            }
        } else {
            HIPCHK(hipEventElapsedTime(&out.probe_ms, E->ev_p0, E->ev_p1));
        }
        HIPCHK(hipEventElapsedTime(&out.seed_ms, E->ev_f0, E->ev_s0));
        HIPCHK(hipEventElapsedTime(&out.recovery_ms, E->ev_s1, E->ev_f1));
        if (E->last_fused) {
            out.recovery_ms = 0.0f;  // no recovery pass
            HIPCHK(hipEventElapsedTime(&out.vanguard_ms, E->ev_v0, E->ev_v1));
        }
        if (E->last_fused && E->last_van_lows)
            HIPCHK(hipEventElapsedTime(&out.vanguard_lows_ms, E->ev_a0, E->ev_a1));
        if (E->last_staged) {
            float r1 = 0.0f, r2 = 0.0f;
            HIPCHK(hipEventElapsedTime(&r1, E->ev_r[0], E->ev_r[1]));
            HIPCHK(hipEventElapsedTime(&r2, E->ev_r[2], E->ev_r[3]));
            out.vanguard_refine_ms = r1 + r2;
        }
        // the reference's profile phases (hybrid.cu:434-516, 679-681); the last ends now,
        // after the host's refinement, as the reference's stop event does
        HIPCHK(hipEventRecord(E->ev_done, E->stream));
        HIPCHK(hipEventSynchronize(E->ev_done));
        HIPCHK(hipEventElapsedTime(&out.phase_ms[0], E->ev_q0, E->ev_p1));
        HIPCHK(hipEventElapsedTime(&out.phase_ms[1], E->ev_p1, E->ev_probe));
        HIPCHK(hipEventElapsedTime(&out.phase_ms[2], E->ev_probe, E->ev_sched));
        HIPCHK(hipEventElapsedTime(&out.phase_ms[3], E->ev_sched, E->ev_done));
    }
    if (st)
        *st = out;
    // The ring is clean once the consumer has cleared and released every record the GPU
    // produced; otherwise (a consumer that stopped early, an abort) the next reset clears it.
    const unsigned long long released = __atomic_load_n(&E->h_progress->released, __ATOMIC_ACQUIRE);
    E->ring_dirty = !E->last_final && released < out.produced;  // GPU-final: nothing in the ring
    if (overflow || stalled) {
        memset(E->h_items, 0xFF, E->qcap * sizeof(uint4));
        E->ring_dirty = false;
        if (stalled)
            return fail(E, CORA_ERR_QUEUE_STALLED,
                        "candidate queue drain stopped waiting for the CPU consumer");
        return fail(E, CORA_ERR_SPILL_EXHAUSTED,
                    E->last_final ? "GPU-final candidate records exceed the HBM spill capacity; increase "
                                    "--queue-spill-capacity, or reduce --query-chunk."
                                  : "HBM queue spill capacity exhausted; increase --queue-capacity or "
                                    "--queue-spill-capacity, or reduce --query-chunk.");
    }
    return CORA_OK;
}

int cora_gpu_capture_thresholds(cora_gpu_engine *E, float *out, uint64_t nq) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->ws)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace before searching");
    if (nq == 0 || nq > E->ws_q)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "search shape exceeds the prepared workspace");
    if (!out)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "missing threshold output");
    memcpy(out, E->h_thr, nq * 4);
    return CORA_OK;
}

int cora_gpu_seed_thresholds(cora_gpu_engine *E, const float *in, uint64_t nq) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->ws)
        return fail(E, CORA_ERR_LOGIC, "prepare workspace before searching");
    if (nq == 0 || nq > E->ws_q)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "search shape exceeds the prepared workspace");
    if (!in)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "missing threshold input");
    memcpy(E->h_thr, in, nq * 4);
    return CORA_OK;
}

int cora_gpu_index_info(const cora_gpu_engine *E, uint64_t *num_vecs, uint64_t *dim,
                        uint64_t *padded_dim, uint64_t *n_centroids, uint64_t *max_cluster) {
    if (!E)
        return CORA_ERR_INVALID_ARGUMENT;
    if (num_vecs)
        *num_vecs = E->N;
    if (dim)
        *dim = E->dim;
    if (padded_dim)
        *padded_dim = E->P;
    if (n_centroids)
        *n_centroids = E->nl;
    if (max_cluster)
        *max_cluster = E->max_cluster;
    return E->loaded ? CORA_OK : CORA_ERR_LOGIC;
}

int cora_gpu_debug_read(cora_gpu_engine *E, int which, void *dst, uint64_t bytes) {
    if (!E || !dst)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->launched)
        return fail(E, CORA_ERR_LOGIC, "no search launched");
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->stream));
    const uint64_t nq = E->last.num_queries, np = E->last.nprobe;
    const void *src = nullptr;
    uint64_t size = 0;
    switch (which) {
    case CORA_DBG_ROTATED_QUERIES: src = E->d_qrot; size = nq * E->P * 4; break;
    case CORA_DBG_K1XSUMQ: src = E->d_k1; size = nq * 4; break;
    case CORA_DBG_KBXSUMQ: src = E->d_kb; size = nq * 4; break;
    case CORA_DBG_Q_WIDTH: src = E->d_qwidth; size = nq * 4; break;
    case CORA_DBG_Q_PLANES: src = E->d_planes; size = nq * 2 * kBq * E->W * 4; break;
    case CORA_DBG_Q_WIDTH2: src = E->d_qwidth2; size = nq * 4; break;
    case CORA_DBG_LUT:
        if (!(E->last.flags & CORA_FLAG_LUT4))
            return fail(E, CORA_ERR_LOGIC, "debug_read: the last search did not use the LUT4 estimator");
        src = E->d_lut;
        size = nq * E->P * 8;
        break;
    case CORA_DBG_SEED_DIST: {
        const uint64_t keep = std::max<uint64_t>(E->last.topk, 20);
        if (!E->d_seed_dist)
            return fail(E, CORA_ERR_LOGIC, "debug_read: no GPU ex-codes, no seed distances");
        src = E->d_seed_dist;
        size = nq * E->last_depth * keep * 4;
        break;
    }
    case CORA_DBG_VANGUARD_LOWS:
        if (!E->last_van_lows)
            return fail(E, CORA_ERR_LOGIC, "debug_read: the last search ran no vanguard lows pass");
        src = E->d_van_lows;
        size = nq * E->last_depth * E->van_stride * 4;
        break;
    case CORA_DBG_THRESHOLDS: {
        if (bytes != nq * 4)
            return fail(E, CORA_ERR_INVALID_ARGUMENT, "debug_read: size mismatch");
        if (E->last.flags & CORA_FLAG_FROZEN_THRESHOLDS)
            HIPCHK(hipMemcpy(dst, E->d_thr_snap, bytes, hipMemcpyDeviceToHost));
        else
            memcpy(dst, E->h_thr, bytes);
        return CORA_OK;
    }
    case CORA_DBG_PROBE_IDX: src = E->d_pidx; size = nq * np * 4; break;
    case CORA_DBG_PROBE_GADD: src = E->d_gadd; size = nq * np * 4; break;
    case CORA_DBG_PROBE_GERR: src = E->d_gerr; size = nq * np * 4; break;
    case CORA_DBG_PROBE_DIST:
        if (E->last_fused_probe)
            return fail(E, CORA_ERR_LOGIC,
                        "debug_read: the last search selected its probes without the distance matrix "
                        "(CORA_FLAG_UNFUSED_PROBE keeps it)");
        src = E->d_dist;
        size = nq * E->nl * 4;
        break;
    case CORA_DBG_PROBE_FALLBACK:
        if (bytes != (1 + nq) * 4)
            return fail(E, CORA_ERR_INVALID_ARGUMENT, "debug_read: size mismatch");
        if (!E->last_fused_probe) {
            memset(dst, 0, bytes);
            return CORA_OK;
        }
        src = E->d_probe_fb;
        size = (1 + nq) * 4;
        break;
    case CORA_DBG_STAGED_COUNTS:
        if (!E->last_staged)
            return fail(E, CORA_ERR_LOGIC, "debug_read: the last search ran no staged vanguard pass");
        src = E->d_vs_ctr;
        size = 4 * sizeof(unsigned long long);
        break;
    case CORA_DBG_PAIRS: {
        if (bytes != nq * np * 12)
            return fail(E, CORA_ERR_INVALID_ARGUMENT, "debug_read: size mismatch");
        std::vector<Pair> pairs(nq * np);
        HIPCHK(hipMemcpy(pairs.data(), E->d_pairs, pairs.size() * sizeof(Pair), hipMemcpyDeviceToHost));
        int32_t *o = static_cast<int32_t *>(dst);
        for (size_t i = 0; i < pairs.size(); ++i) {
            o[3 * i] = (int32_t)pairs[i].cluster;
            o[3 * i + 1] = (int32_t)(pairs[i].word0 & 0xFFFFu);
            o[3 * i + 2] = (int32_t)(pairs[i].word0 >> 16);
        }
        return CORA_OK;
    }
    default: return fail(E, CORA_ERR_INVALID_ARGUMENT, "debug_read: unknown array");
    }
    if (bytes != size)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "debug_read: size mismatch");
    HIPCHK(hipMemcpy(dst, src, size, hipMemcpyDeviceToHost));
    return CORA_OK;
}

int cora_gpu_debug_dense(cora_gpu_engine *E, int32_t *out_ip, int32_t *out_ip2, float *out_low,
                         uint64_t cap) {
    if (!E || !out_ip || !out_ip2 || !out_low)
        return CORA_ERR_INVALID_ARGUMENT;
    if (!E->launched)
        return fail(E, CORA_ERR_LOGIC, "no search launched");
    const uint64_t need = (uint64_t)E->last.num_queries * E->last.nprobe * E->max_cluster;
    if (cap < need)
        return fail(E, CORA_ERR_INVALID_ARGUMENT, "debug_dense: output too small");
    HIPCHK(hipSetDevice(E->device));
    HIPCHK(hipStreamSynchronize(E->stream));
    int32_t *d_ip = nullptr, *d_ip2 = nullptr;
    float *d_low = nullptr;
    int rc = dalloc(E, d_ip, need);
    if (rc == CORA_OK)
        rc = dalloc(E, d_ip2, need);
    if (rc == CORA_OK)
        rc = dalloc(E, d_low, need);
    if (rc == CORA_OK) {
        ScanParams p = scan_params(E, E->last_depth, 0, true);
        p.dbg_ip = d_ip;
        p.dbg_ip2 = d_ip2;
        p.dbg_low = d_low;
        p.dbg_stride = (uint32_t)E->max_cluster;
        hipError_t r = hipMemcpy(d_ip, out_ip, need * 4, hipMemcpyHostToDevice);
        if (r == hipSuccess)
            r = hipMemcpy(d_ip2, out_ip2, need * 4, hipMemcpyHostToDevice);
        if (r == hipSuccess)
            r = hipMemcpy(d_low, out_low, need * 4, hipMemcpyHostToDevice);
        for (uint32_t set = 0; set < 2 && r == hipSuccess; ++set) {
            // the kernel the search ran: the matrix-core far scan for the far units
            launch_cursor_init(E->d_cursor, E->d_nunits, set, E->stream);
            // the matrix-core kernel for the units it scanned in the search (far units with
            // the matrix-core far scan; vanguard units, of up to 16 pairs, with the lows pass)
            p.dbg_set = set;
            if ((set == 1 && E->last_mfma) || (set == 0 && E->last_van_lows))
                launch_far_mfma(p, E->W, true, E->stream);
            else
                launch_scan_set(p, E->W, 2, set, E->stream);
            r = hipGetLastError();
            if (r == hipSuccess)
                r = hipStreamSynchronize(E->stream);
        }
        if (r == hipSuccess)
            r = hipMemcpy(out_ip, d_ip, need * 4, hipMemcpyDeviceToHost);
        if (r == hipSuccess)
            r = hipMemcpy(out_ip2, d_ip2, need * 4, hipMemcpyDeviceToHost);
        if (r == hipSuccess)
            r = hipMemcpy(out_low, d_low, need * 4, hipMemcpyDeviceToHost);
        if (r != hipSuccess)
            rc = fail(E, CORA_ERR_RUNTIME, std::string("debug_dense: ") + hipGetErrorString(r));
    }
    dfree(d_ip);
    dfree(d_ip2);
    dfree(d_low);
    return rc;
}

}  // extern "C"
