/*
 * cora_gpu.h — C-ABI of the MI355X (gfx950) GPU filter engine for IVF-RaBitQ search.
 *
 * This is the GPU half of the reference's coraanns::HybridIndex
 * (include/coraanns/search/hybrid.cuh:18-203, src/search/hybrid.cu:35-689): index
 * residency in HBM, query preparation, coarse probing, pair scheduling, the RaBitQ
 * 1-bit popcount scan with shared-threshold filtering, and the device side of the
 * GPU->CPU candidate ring (src/search/ring_queue.cuh). The CPU half (ex-code
 * refinement consuming the ring) and the C++ HybridIndex shim live in libcoraanns and
 * call these functions. Plain C types only: no HIP, torch or C++ types cross this ABI.
 *
 * Every entry point returns CORA_OK or one of the CORA_ERR_* codes below; the message
 * of the last failure on an engine is available from cora_gpu_last_error(). The C++
 * shim maps CORA_ERR_INVALID_ARGUMENT -> std::invalid_argument, CORA_ERR_LOGIC ->
 * std::logic_error and everything else -> std::runtime_error, matching the exception
 * types the reference throws (hybrid.cu:88-121,236-237,401-404,669-673;
 * src/search/cuda_error.hpp:8-16).
 *
 * Threading: one search at a time per engine (reference docs/ARCHITECTURE.md:44).
 */
#ifndef CORA_GPU_H
#define CORA_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum cora_status {
    CORA_OK = 0,
    CORA_ERR_INVALID_ARGUMENT = 1,
    CORA_ERR_LOGIC = 2,
    CORA_ERR_RUNTIME = 3,
    CORA_ERR_SPILL_EXHAUSTED = 4,
    CORA_ERR_OUT_OF_MEMORY = 5,
    CORA_ERR_QUEUE_STALLED = 6
};

enum cora_metric { CORA_METRIC_L2 = 0, CORA_METRIC_IP = 1 }; /* rabitqlib MetricType (defines.hpp:65) */

/* Search flags (cora_search_args.flags). */
enum cora_search_flags {
    /* The filter reads a device snapshot of the thresholds taken at launch instead of
     * the live host array the CPU tightens (deterministic candidate sets; the reference
     * has only the live mode, hybrid.cu:251-253). */
    CORA_FLAG_FROZEN_THRESHOLDS = 1u << 0,
    /* Record HIP events around the scan kernels (reference set_gpu_filter_timing,
     * hybrid.cu:538-540,655-657). */
    CORA_FLAG_FILTER_TIMING = 1u << 1,
    /* Cross-query reuse: batch up to batch_q same-cluster pairs per pass
     * (reference set_cross_query_reuse, hybrid.cu:594-597). */
    CORA_FLAG_CROSS_QUERY_REUSE = 1u << 2,
    /* Do not seed thresholds on the GPU even when ex-codes are resident in HBM (the
     * reference's behaviour: only the CPU consumer tightens thresholds). */
    CORA_FLAG_NO_GPU_SEED = 1u << 3,
    /* Test mode: with FROZEN_THRESHOLDS, the GPU seed thresholds lower the launch
     * snapshot, so seeding is deterministic and checkable (CORA_DBG_SEED_DIST,
     * CORA_DBG_THRESHOLDS). */
    CORA_FLAG_GPU_SEED_FROZEN = 1u << 4,
    /* Do not use the refined pre-filter: with ex-codes in HBM the far and recovery passes
     * otherwise drop candidates whose refined distance (the CPU consumer's formula)
     * already exceeds their threshold by more than a rounding bound. */
    CORA_FLAG_NO_GPU_PREFILTER = 1u << 5,
    /* Run the vanguard pairs as the reference does, a per-pair seed pass followed by a
     * recovery pass over each pair, instead of the fused per-query vanguard pass that is
     * used when the ex-codes are resident in HBM (vanguard depth <= 64, topk <= 128, or up to
     * CORA_VANGUARD_STAGED_MAX_TOPK in the staged pass; see CORA_FLAG_VANGUARD_STAGED). */
    CORA_FLAG_PAIR_SEEDS = 1u << 6,
    /* Scan the far pairs with the popcount kernel even where the matrix-core kernel
     * applies (cross-query reuse with padded dimension 64..256, 512, 768 or 1024). */
    CORA_FLAG_NO_MFMA_SCAN = 1u << 7,
    /* Query rotation and coarse-probe distances from the FP32 matrix-core GEMMs instead of
     * the split-FP16 ones (each operand row scaled by a power of two and split into two
     * FP16 rows, three FP16 products per term: at most 3 * 2^-22 relative error per term).
     * Either way the selected probes' g_add / g_error are recomputed in FP32
     * (hybrid.cu:436-440, 465-498). */
    CORA_FLAG_FP32_GEMM = 1u << 8,
    /* Fused vanguard pass: where its lower bounds come from (same candidates either way).
     * By default, when the index's sign codes and factors exceed the last-level cache
     * (256 MB) and the padded dimension is at least 512, or exceed 1 GiB at any padded
     * dimension, they are evaluated first on the
     * matrix cores, cluster-major, in units of up to 16 same-cluster pairs (each cluster read
     * once per unit), and the per-query pass streams them; for a cache-resident index, or
     * narrow codes (P/8 + 12 bytes a vector against 4 bytes of bound), each query evaluating
     * its own clusters inside the per-query pass is faster. NO_VANGUARD_MFMA forces the
     * latter, VANGUARD_MFMA the former. */
    CORA_FLAG_NO_VANGUARD_MFMA = 1u << 9,
    CORA_FLAG_VANGUARD_MFMA = 1u << 10,
    /* GPU-final top-k: the candidates' refined distances, which the fused vanguard pass and
     * the refined pre-filter compute on the HBM ex-codes with the CPU consumer's formula,
     * form the final per-query top-k on the GPU (cora_gpu_final_results); nothing goes to
     * the ring and no CPU refinement runs (the reference's GPU baseline engine refines on
     * the GPU likewise, src/baselines/gpu.cu:630-700). Needs the ex-codes in HBM, the fused
     * vanguard pass (vanguard <= 64, topk <= 128, or <= CORA_VANGUARD_STAGED_MAX_TOPK where
     * the staged pass serves it) and the refined pre-filter. */
    CORA_FLAG_GPU_FINAL = 1u << 11,
    /* LUT4 estimator, the reference's KernelType::Lut4Bit (query_kernels.cuh:199-221,
     * filter_kernels.cuh:283-306,586-770): <q',b> is the FP32 sum of FP16 nibble-table
     * entries (even and odd nibbles in two accumulators), used for the lower bound and handed
     * to refinement as exact_ip. For padded dimension 512, 768 or 1024 with cross-query
     * reuse, the matrix-core lows pass and far scan filter with Bitwise bounds lowered by a
     * per-query bound on |LUT4 - Bitwise| and evaluate the survivors' LUT4 bounds exactly, and
     * the staged vanguard pass refines with the LUT4 estimate; otherwise the per-pair seed,
     * far and recovery passes run with at most 4 same-cluster pairs per pass.
     * Without it the Bitwise estimator runs (Bq=8 popcount bound; two-stage exact_ip). */
    CORA_FLAG_LUT4 = 1u << 12,
    /* Coarse probe through the whole [nq][nlist] distance matrix and a select pass over it.
     * Without it, for 8,192 <= nlist <= 65,536 and nprobe <= 64, or up to 1,024 while the
     * 128-cluster tiles hold at most ~4.5 probes each on average (split-FP16 GEMM), the GEMM's
     * epilogue keeps 8 (16 above nprobe 64) candidate keys per query and 128-cluster tile and
     * a merge selects from them, with the same result; the distance matrix is then not
     * available to CORA_DBG_PROBE_DIST (its memory holds the candidates). */
    CORA_FLAG_UNFUSED_PROBE = 1u << 13,
    /* Fused vanguard pass after the matrix-core lows pass: the one per-query kernel (each
     * query selects, refines and publishes in turn), or the staged pass, whose refinement of
     * every query's candidates runs grid-wide between per-query select and merge stages, with
     * the same rules for what is refined, published and the threshold. By default the staged
     * pass runs with the LUT4 estimator (which only it supports), the one-pass kernel
     * otherwise, whose queries' records reach the CPU consumer as each query ends; these
     * flags choose one (ONE_PASS wins when both are given). Top-k above
     * 128 (up to CORA_VANGUARD_STAGED_MAX_TOPK) is served by the staged pass alone, when the
     * workspace was prepared for it (its per-query regions then hold every vanguard vector)
     * and the matrix-core lows pass applies; otherwise the per-pair passes run. */
    CORA_FLAG_VANGUARD_ONE_PASS = 1u << 14,
    CORA_FLAG_VANGUARD_STAGED = 1u << 15
};
#define CORA_VANGUARD_STAGED_MAX_TOPK 1024

typedef struct cora_gpu_engine cora_gpu_engine;

/* Host view of the GPU->CPU candidate ring. Byte layout of items/progress is
 * coraanns::queue::Candidate[capacity] / coraanns::queue::Progress
 * (include/coraanns/queue/candidate_queue.hpp:10-55). All pointers are host
 * addresses of host-coherent pinned memory the GPU reads and writes. */
typedef struct cora_queue_view {
    void *items;
    void *progress;
    uint64_t capacity;
    float *thresholds; /* [max_queries], read by the GPU filter, written by the CPU */
    int *abort_flag;   /* host sets 1 to stop the queue drain kernel waiting */
} cora_queue_view;

typedef struct cora_search_args {
    uint32_t num_queries;
    uint32_t topk;
    uint32_t nprobe;
    uint32_t batch_q;  /* 1..64 same-cluster pairs per cluster pass with cross-query reuse (the
                          reference accepts 1..6); the popcount scan takes at most 8 per pass
                          (4 with LUT4), the matrix-core scans 16 whatever the value */
    uint32_t vanguard; /* vanguard depth: pairs with probe rank < vanguard are scanned first */
    uint32_t flags;    /* cora_search_flags */
    /* Multiplier of the lower bound's error term: low = est - bound_scale * f_error * g_error.
     * 1 (or 0) is the reference Bitwise producer's bound (filter_kernels.cuh:111-114);
     * above 1 the filter keeps the vectors whose 1-bit estimate errs beyond the bound's
     * confidence, which the reference CPU path's running threshold happens to keep
     * (no counterpart in the reference's GPU interface). Range 0..16. */
    float bound_scale;
} cora_search_args;

typedef struct cora_search_stats {
    uint64_t produced;      /* candidates published (reference Progress::produced) */
    uint64_t spilled;       /* candidates that went through the HBM spill buffer */
    int32_t overflow;       /* spill capacity exhausted */
    int32_t stalled;        /* the drain kernel gave up waiting for ring space */
    float filter_ms;        /* all scan kernels (FILTER_TIMING only) */
    float scan_ms;          /* the far-pair scan kernel alone (FILTER_TIMING only) */
    uint64_t scan_bytes;    /* algorithmic code+factor bytes the far-pair scan read */
    uint64_t scan_units;    /* cluster passes the far-pair scan made */
    uint64_t scan_vectors;  /* vector evaluations (vector x query) of the far-pair scan */
    float probe_ms;         /* coarse-probe distance GEMM alone (FILTER_TIMING only) */
    uint64_t probe_flops;   /* its algorithmic flops, 2 * nq * padded_dim * nlist */
    uint64_t pass_produced[3]; /* candidates published by the end of the vanguard seed,
                                  far-pair and recovery passes (cumulative) */
    uint64_t seeded_queries;   /* queries that received a GPU seed threshold */
    uint64_t prefilter_dropped; /* candidates the refined pre-filter dropped */
    float seed_ms;          /* vanguard seed pass + seed thresholds, or the fused vanguard
                               pass (FILTER_TIMING only) */
    float recovery_ms;      /* vanguard recovery pass (FILTER_TIMING only; 0 when fused) */
    uint64_t gpu_refined;   /* vectors the fused vanguard pass refined on the GPU */
    float vanguard_ms;      /* the fused vanguard pass kernel alone (FILTER_TIMING only) */
    uint64_t vanguard_bytes; /* its algorithmic bytes: code + factor bytes of every vector of
                                every vanguard pair (4 bytes of lower bound each when the
                                matrix-core lows pass ran), plus sign code, ex-code and
                                ex-factor bytes of every vector it refined */
    float vanguard_lows_ms;  /* the matrix-core vanguard lows pass alone (0 when it did not run) */
    uint64_t vanguard_lows_bytes; /* its algorithmic bytes: code + factor bytes of every vector
                                     of the cluster read once per unit of up to 16 pairs, and a
                                     4-byte bound per (vector, vanguard pair) written (5 bytes
                                     with the staged pass's group minima) */
    /* how the vanguard pairs ran: 0 none, 1 the per-pair seed and recovery passes (asked
     * for, no ex-codes in HBM, or beyond the fused pass's limits of 64 vanguard pairs and
     * top-128), 2 the fused per-query pass, 3 the fused pass after the matrix-core lows pass,
     * 4 the staged pass after the matrix-core lows pass */
    int32_t vanguard_mode;
    /* the reference's [Profile] phases (FILTER_TIMING only): query preparation and coarse
     * GEMM, probe selection, pair scheduling, then the scan pipeline up to cora_gpu_sync
     * (including the host's refinement) */
    float phase_ms[4];
    /* staged pass: its two grid-wide refinement launches (FILTER_TIMING only), and their
     * algorithmic bytes: sign code, ex-code and ex-factors of each refined vector, plus its
     * 4-byte position and lower bound read and 16 bytes of result written */
    float vanguard_refine_ms;
    uint64_t vanguard_refine_bytes;
} cora_search_stats;

/* Lifecycle (HybridIndex ctor/dtor, hybrid.cu:35-85). device = HIP ordinal. */
int cora_gpu_create(cora_gpu_engine **out, int device);
int cora_gpu_destroy(cora_gpu_engine *engine);
/* Copies the last error message (NUL-terminated, truncated to n). */
int cora_gpu_last_error(const cora_gpu_engine *engine, char *buf, size_t n);

/* Index upload (HybridIndex::load_from_raw_pointers, hybrid.cu:101-164), GPU arrays only.
 * h_short_data: reference SearchData layout (search_data.cpp:45-82), per-cluster
 * word-major u32 [num_vecs * padded_dim/32], dimension 32w+l at bit 31-l of word w.
 * h_short_factors: f32 [num_vecs][3] (f_add, f_rescale, f_error).
 * h_centroids: f32 [n_centroids][padded_dim] rotated; h_rotator: f32 [dim][padded_dim].
 * The engine repacks the codes into its own tile layout in HBM. */
int cora_gpu_load_index(cora_gpu_engine *engine, uint64_t num_vecs, uint64_t dim,
                        uint64_t padded_dim, uint64_t n_centroids, uint64_t ex_bits, int metric,
                        const float *h_centroids, const float *h_rotator,
                        const uint32_t *h_short_data, const float *h_short_factors,
                        const uint64_t *h_cluster_sizes);

/* Optional HBM copy of the 7-bit ex-codes [num_vecs][padded_dim*7/8] (reference packed
 * layout, pack_excode.hpp:216-265) and ex-factors [num_vecs][2] (no counterpart in the
 * reference, whose ex-codes live on the host only), kept as one refinement record per
 * vector (ex-code, sign code, ex-factors: padded_dim + 16 bytes). With them the GPU
 * refines vanguard vectors with the CPU consumer's formula (cpu_refinement.cpp:183-192),
 * lowers each query's live threshold to a value the CPU would publish after refining
 * them, and drops far candidates the CPU would reject. The CPU still refines every
 * published candidate. Requires ex_bits == 7; call after cora_gpu_load_index. */
int cora_gpu_load_excodes(cora_gpu_engine *engine, const uint8_t *h_long_codes,
                          const float *h_ex_factors);

/* Ring sizing before prepare (HybridIndex::set_queue_capacity / set_queue_spill_capacity,
 * hybrid.cu:166-185). capacity: power of two. */
int cora_gpu_set_queue(cora_gpu_engine *engine, uint64_t capacity, uint64_t spill_capacity);

/* Workspace (HybridIndex::prepare_workspace / free_workspace, hybrid.cu:235-378). */
int cora_gpu_prepare_workspace(cora_gpu_engine *engine, uint64_t max_queries, uint64_t max_topk,
                               uint64_t max_nprobe, uint64_t vanguard_size);
int cora_gpu_free_workspace(cora_gpu_engine *engine);
int cora_gpu_queue_view(cora_gpu_engine *engine, cora_queue_view *out);

/* Per-chunk reset (HybridIndex::reset_buffer, hybrid.cu:380-396): uploads the raw
 * queries f32 [nq][dim], resets device queue counters and the host Progress, and sets the
 * thresholds of the first nq queries to FLT_MAX. Queries already placed in the pinned
 * staging buffer (cora_gpu_query_staging) upload asynchronously, in three slices for
 * nq >= 2,048, and the next search prepares and probes each slice as soon as it has landed;
 * the staging buffer is rewritable after the next cora_gpu_query_staging call, which waits
 * for the upload. Any other host array goes through the runtime's pageable-copy path and
 * is resident when the call returns. */
int cora_gpu_reset(cora_gpu_engine *engine, const float *h_queries, uint64_t nq);
/* The final top-k of a search launched with CORA_FLAG_GPU_FINAL, after cora_gpu_sync:
 * dists [nq][topk] ascending (FLT_MAX pad) and cluster-order vector indexes idx [nq][topk]
 * (0xFFFFFFFF pad; the ids array of load_from_raw_pointers maps them to ids); ties by index. */
int cora_gpu_final_results(cora_gpu_engine *engine, float *dists, uint32_t *idx);
/* Pinned host buffer of [max_q][dim] floats for the queries of the next reset (valid from
 * prepare_workspace to free_workspace); returns once the last reset's upload from it is
 * complete. No counterpart in the reference, which uploads from the caller's pageable
 * array. */
int cora_gpu_query_staging(cora_gpu_engine *engine, float **staging);

/* Enqueue the whole GPU side of HybridIndex::search (hybrid.cu:434-660) and return
 * without waiting: rotation, query factors and Bq=8 quantisation, coarse probing,
 * pair scheduling, vanguard seed scan, far-pair scan, vanguard recovery scan, and the
 * queue drain kernel that publishes produced/spilled and sets Progress::done. */
int cora_gpu_launch_search(cora_gpu_engine *engine, const cora_search_args *args);

/* Wait until the host-side inputs of CPU refinement are in pinned memory
 * (hybrid.cu:663) and return pointers to them: rotated queries f32 [nq][P],
 * kbxSumq f32 [nq], probe g_add f32 [nq][nprobe] (||q'-c'||^2 for L2, -<q',c'> for IP). */
int cora_gpu_wait_host_inputs(cora_gpu_engine *engine, const float **rotated_queries,
                              const float **kbxsumq, const float **probe_gadd);

/* Wait for all GPU work of the search and report its counters (hybrid.cu:667-677).
 * Returns CORA_ERR_SPILL_EXHAUSTED when the spill buffer overflowed (the ring is
 * cleared), CORA_ERR_QUEUE_STALLED when the drain kernel timed out. */
int cora_gpu_sync(cora_gpu_engine *engine, cora_search_stats *stats);

/* Threshold snapshot (HybridIndex::capture_thresholds / seed_thresholds,
 * cpu_refinement.cpp:58-69). */
int cora_gpu_capture_thresholds(cora_gpu_engine *engine, float *out, uint64_t nq);
int cora_gpu_seed_thresholds(cora_gpu_engine *engine, const float *in, uint64_t nq);

/* Index and workspace shape queries. */
int cora_gpu_index_info(const cora_gpu_engine *engine, uint64_t *num_vecs, uint64_t *dim,
                        uint64_t *padded_dim, uint64_t *n_centroids, uint64_t *max_cluster);

/* Inspection for parity tests: copy an internal array of the last launched search to
 * host memory. which: see cora_debug_array. bytes must equal the array size. */
enum cora_debug_array {
    CORA_DBG_ROTATED_QUERIES = 0, /* f32 [nq][P] */
    CORA_DBG_K1XSUMQ = 1,         /* f32 [nq] */
    CORA_DBG_KBXSUMQ = 2,         /* f32 [nq] */
    CORA_DBG_Q_WIDTH = 3,         /* f32 [nq] Bq=8 quantisation step */
    CORA_DBG_Q_PLANES = 4,        /* u32 [nq][16][P/32], dim 32w+l at bit l of word w: planes
                                     0..7 = Bq=8 query qint, 8..15 = quantised residual qres */
    CORA_DBG_PROBE_IDX = 5,       /* i32 [nq][nprobe] ascending distance */
    CORA_DBG_PROBE_GADD = 6,      /* f32 [nq][nprobe] */
    CORA_DBG_PROBE_GERR = 7,      /* f32 [nq][nprobe] */
    CORA_DBG_PAIRS = 8,           /* i32 [npairs][3] (cluster, query, probe), scan order */
    CORA_DBG_Q_WIDTH2 = 9,        /* f32 [nq] residual quantisation step (width / 254) */
    CORA_DBG_SEED_DIST = 10,      /* f32 [nq][vanguard depth][keep] GPU-refined seed distances
                                     (+inf: unused slot); keep = max(topk, 20) */
    CORA_DBG_THRESHOLDS = 11,     /* f32 [nq] thresholds the GPU filter read last (the
                                     snapshot in frozen mode, else the live array) */
    CORA_DBG_PROBE_DIST = 12,     /* f32 [nq][nlist] coarse-probe distance matrix
                                     ||q'||^2 + ||c'||^2 - 2 <q',c'> (searches that selected
                                     from it: CORA_FLAG_UNFUSED_PROBE or outside the fused
                                     select's range) */
    CORA_DBG_VANGUARD_LOWS = 13,  /* f32 [nq][vanguard depth][stride] lower bounds the
                                     matrix-core lows pass wrote (stride = the largest
                                     cluster rounded up to 256; entries past a cluster's
                                     size are undefined) */
    CORA_DBG_LUT = 14,            /* f16 [nq][P/4][16] LUT4 tables (CORA_FLAG_LUT4 searches) */
    CORA_DBG_PROBE_FALLBACK = 15, /* u32 [1 + nq]: the number of queries whose fused probe
                                     select fell back to their distance row, then those
                                     queries (any order); count 0 for an unfused search */
    CORA_DBG_STAGED_COUNTS = 16   /* u64 [4] of the last staged vanguard pass: seeds and
                                     list entries refined, queries whose list needed a second
                                     pass over their bounds, queries left to the one-pass
                                     kernel */
};
int cora_gpu_debug_read(cora_gpu_engine *engine, int which, void *dst, uint64_t bytes);

/* Dense estimator for parity tests: for every (query, probe) pair of the last launched
 * search, evaluate every vector of the probed cluster with the scan kernel's estimator
 * and write ip_int = <b, qint> (i32), the residual inner product <b, qres> (i32) and the
 * low distance (f32) to out_ip / out_ip2 / out_low, laid out [nq][nprobe][max_cluster]
 * (entries past the cluster size are left untouched). After a CORA_FLAG_LUT4 search,
 * out_ip holds the bits of the f32 LUT4 estimate and out_ip2 zero. */
int cora_gpu_debug_dense(cora_gpu_engine *engine, int32_t *out_ip, int32_t *out_ip2,
                         float *out_low, uint64_t capacity_elems);

/* ---- Index-build and evaluation tools (no counterpart in the reference's search path;
 * they replace its offline Faiss k-means, tools/data/train_ivf.py:11-47, and the
 * exhaustive ground-truth tool, tools/data/generate_gt_gpu.py). Host arrays in and out;
 * each call allocates and frees its own device memory on `device`. ---- */
const char *cora_tool_last_error(void);
/* out [n][P] = x [n][dim] . R [dim][P] */
int cora_tool_rotate(const float *x, uint64_t n, uint64_t dim, const float *R, uint64_t P,
                     float *out, int device);
/* Lloyd k-means (squared L2), `iters` iterations from k seeded distinct rows. */
int cora_tool_kmeans(const float *x, uint64_t n, uint64_t dim, uint64_t k, uint32_t iters,
                     uint64_t seed, float *centroids, int device);
/* nearest centroid of every row (ties -> lower centroid id) */
int cora_tool_assign(const float *x, uint64_t n, uint64_t dim, const float *centroids, uint64_t k,
                     uint32_t *assign, int device);
/* exhaustive top-k ids by FP32 distance (metric 0: L2, 1: IP), ascending */
int cora_tool_topk(const float *base, uint64_t nb, const float *queries, uint64_t nq, uint64_t dim,
                   uint64_t k, int metric, uint32_t *ids, int device);
/* RaBitQ quantisation of index rows on the GPU (the index builder's per-row step,
 * rabitq_impl.hpp:76-137 and 276-500 as restated by the host builder, bit-identical to it):
 * rows x [n][dim] are rotated by R [dim][P] on the GPU and quantised against their cluster's
 * rotated centroid (centroids [nlist][P], assign [n]) with 1 sign bit + 7 ex-bits.
 * Outputs per row, in input order: bits [n][P/8] (dimension 8b + j at bit 7 - j of byte b),
 * f1 [n][3] (f_add, f_rescale, f_error), code [n][P] (7-bit ex-code values, complemented
 * for negative residuals), f2 [n][2] (f_add_ex, f_rescale_ex). P % 64 == 0, P <= 1024. */
int cora_tool_quantize(const float *x, uint64_t n, uint64_t dim, const float *R, uint64_t P,
                       const float *centroids, uint64_t nlist, const uint32_t *assign, int metric,
                       uint8_t *bits, float *f1, uint8_t *code, float *f2, int device);

/* cora_tool_assign without any allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops that assign new vectors to clusters, harnesses that forbid hipMalloc). x [n][dim],
 * centroids [k][dim] and assign [n] are DEVICE arrays on `device`, owned by the caller; the
 * norms and distance blocks go to a 16 MiB static device array that each GPU holds until the
 * process ends. Same result as cora_tool_assign (nearest centroid, ties -> lower id). At most
 * CORA_NOALLOC_MAX_CENTROIDS centroids and dimension CORA_NOALLOC_MAX_DIM (else
 * CORA_ERR_INVALID_ARGUMENT). Runs on the null stream and returns when done; calls on one GPU
 * take turns on its scratch array (a per-device lock), so several host threads may call it. */
#define CORA_NOALLOC_MAX_CENTROIDS 1048576
#define CORA_NOALLOC_MAX_DIM 4096
int cora_tool_assign_noalloc(const float *x, uint64_t n, uint64_t dim, const float *centroids, uint64_t k,
                             uint32_t *assign, int device);

#ifdef __cplusplus
}
#endif

#endif /* CORA_GPU_H */
