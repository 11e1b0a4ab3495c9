/*
 * cora_host.h — C-ABI of libcoraanns for FFI callers (Python ctypes in this repository's
 * tests and bench; a cgo/JNI/N-API binding would bind the same symbols).
 *
 * cora_hybrid_* wraps coraanns::HybridIndex (include/coraanns/search/hybrid.hpp), the
 * drop-in for the reference's coraanns::HybridIndex (include/coraanns/search/hybrid.cuh:
 * 18-203); each entry names the reference member it forwards to. cora_ivf_* reads the
 * reference's on-disk IVF format and adapts it like the reference SearchData
 * (src/index/search_data.cpp:9-127). cora_build_ivf writes that format. Status codes are
 * the cora_status values of cora_gpu.h; the message of the last failure on the calling
 * thread is returned by cora_host_last_error(). C++ exceptions never cross this ABI.
 */
#ifndef CORA_HOST_H
#define CORA_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "cora_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cora_hybrid cora_hybrid;
typedef struct cora_ivf cora_ivf;

const char *cora_host_last_error(void);

/* Engine settings applied before load/prepare (HybridIndex setters, hybrid.cuh:121-165). */
typedef struct cora_hybrid_config {
    int profiling;            /* set_profiling */
    int candidate_stats;      /* set_candidate_stats */
    int gpu_filter_timing;    /* set_gpu_filter_timing */
    int cross_query_reuse;    /* set_cross_query_reuse */
    int cpu_secondary_filter; /* set_cpu_secondary_filter */
    uint64_t vanguard_size;   /* set_vanguard_size */
    uint64_t queue_capacity;  /* set_queue_capacity (0 = keep) */
    uint64_t queue_spill_capacity; /* set_queue_spill_capacity (UINT64_MAX = keep) */
    int metric;               /* 0 = L2, 1 = IP */
    int frozen_thresholds;    /* GPU filter reads a snapshot taken at launch */
    int cpu_threads;          /* CPU refinement threads, 0 = omp_get_max_threads() */
    int gpu_seed_refine;      /* set_gpu_seed_refine (HBM ex-codes, GPU seed thresholds) */
    int gpu_refine_filter;    /* set_gpu_refine_filter (GPU refined pre-filter) */
    uint32_t extra_flags;     /* set_extra_search_flags (cora_search_flags test modes) */
    float lower_bound_scale;  /* set_lower_bound_scale (0 = keep) */
    int gpu_final_topk;       /* set_gpu_final_topk */
    int ip_kernel_type;       /* set_ip_kernel_type: 0 = keep, 1 = Lut4Bit, 2 = Bitwise */
} cora_hybrid_config;

typedef struct cora_hybrid_stats {
    uint64_t submitted;  /* get_last_submitted_count */
    uint64_t spilled;    /* get_last_spilled_count */
    uint64_t refined;    /* get_last_refined_count */
    float gpu_filter_ms; /* get_last_gpu_filter_ms */
    float scan_ms;       /* far-pair scan kernel alone */
    uint64_t scan_bytes; /* algorithmic code+factor bytes of the far-pair scan */
    uint64_t scan_units;
    uint64_t scan_vectors;
    float probe_ms;       /* coarse-probe distance GEMM alone */
    uint64_t probe_flops; /* 2 * nq * padded_dim * nlist */
    uint64_t pass_produced[3]; /* cumulative candidates after the seed, far, recovery passes */
    uint64_t seeded_queries;   /* queries given a GPU seed threshold */
    uint64_t prefilter_dropped; /* candidates the GPU refined pre-filter dropped */
    float seed_ms;        /* vanguard seed pass + seed thresholds */
    float recovery_ms;    /* vanguard recovery pass */
    uint64_t gpu_refined; /* vectors the fused vanguard pass refined on the GPU */
    float vanguard_ms;    /* fused vanguard pass kernel alone */
    uint64_t vanguard_bytes; /* its algorithmic bytes */
    float vanguard_lows_ms;  /* matrix-core vanguard lows pass alone */
    uint64_t vanguard_lows_bytes; /* its algorithmic bytes */
    int32_t vanguard_mode;   /* get_last_vanguard_mode */
    float phase_ms[4];       /* get_last_phase_ms */
    float vanguard_refine_ms;       /* staged vanguard pass: its grid-wide refinement launches */
    uint64_t vanguard_refine_bytes; /* their algorithmic bytes */
} cora_hybrid_stats;

int cora_hybrid_create(cora_hybrid **out, int device);                 /* HybridIndex() */
int cora_hybrid_destroy(cora_hybrid *h);                               /* ~HybridIndex() */
int cora_hybrid_configure(cora_hybrid *h, const cora_hybrid_config *c);
/* load_from_raw_pointers (hybrid.cuh:186-190); long codes / ex factors / ids are borrowed */
int cora_hybrid_load(cora_hybrid *h, uint64_t num_vecs, uint64_t dim, uint64_t padded_dim,
                     uint64_t n_centroids, uint64_t ex_bits, const float *centroids,
                     const float *rotator, const uint32_t *short_data, const float *short_factors,
                     const uint8_t *long_codes, const float *ex_factors, const uint32_t *ids,
                     const uint64_t *cluster_sizes);
/* enable_exact_refine (hybrid.cuh:171-178) */
int cora_hybrid_enable_exact_refine(cora_hybrid *h, const uint8_t *base_mapping, uint64_t rows,
                                    uint64_t dim, uint64_t row_stride_bytes,
                                    uint64_t data_offset_bytes);
int cora_hybrid_prepare(cora_hybrid *h, uint64_t max_queries, uint64_t max_topk,
                        uint64_t max_nprobe);                          /* prepare_workspace */
int cora_hybrid_free_workspace(cora_hybrid *h);                        /* free_workspace */
int cora_hybrid_reset(cora_hybrid *h, const float *queries, uint64_t nq); /* reset_buffer */
int cora_hybrid_search(cora_hybrid *h, const float *queries, uint64_t nq, uint64_t topk,
                       uint64_t nprobe, float *dists, uint32_t *ids, int batch_q); /* search */
int cora_hybrid_stats_get(cora_hybrid *h, cora_hybrid_stats *out);
int cora_hybrid_capture_thresholds(cora_hybrid *h, float *out, uint64_t nq);
int cora_hybrid_seed_thresholds(cora_hybrid *h, const float *in, uint64_t nq);
int cora_hybrid_set_vanguard_size(cora_hybrid *h, uint64_t size);
cora_gpu_engine *cora_hybrid_gpu(cora_hybrid *h);
/* get_lower_bound_scale (0 for a null handle). */
float cora_hybrid_lower_bound_scale(cora_hybrid *h);

/* IVF file + SearchData adaptation. */
typedef struct cora_ivf_info {
    uint64_t num, dim, padded_dim, nlist, ex_bits, max_cluster;
    int metric;
    int centroid_storage; /* 0 = embedded in the index, 1 = "<index>.hnsw" sidecar (ivf.hpp:487-520) */
} cora_ivf_info;
typedef struct cora_ivf_arrays {
    const float *centroids;     /* [nlist][P] */
    const float *rotator;       /* [dim][P] */
    const uint32_t *short_data; /* [num * P/32] */
    const float *short_factors; /* [num][3] */
    const uint8_t *long_codes;  /* [num][P*ex/8] (NULL without extended data) */
    const float *ex_factors;    /* [num][2] */
    const uint32_t *ids;        /* [num] */
    const uint64_t *cluster_sizes; /* [nlist] */
} cora_ivf_arrays;
/* IVF::load (ivf.hpp:447-539) + SearchData (search_data.cpp:9-127) in one streaming pass:
 * centroids embedded or from the HNSW sidecar, batch and ex data read in bounded chunks. */
int cora_ivf_load(const char *path, int include_extended, cora_ivf **out);
int cora_ivf_info_get(const cora_ivf *ivf, cora_ivf_info *out);
int cora_ivf_arrays_get(const cora_ivf *ivf, cora_ivf_arrays *out);
int cora_ivf_free(cora_ivf *ivf);

/* Index construction into the reference format from rotated inputs. threads <= 0: all. */
int cora_build_ivf(const float *rotated_data, const float *rotated_centroids,
                   const uint32_t *assignments, const float *rotator, uint64_t n, uint64_t dim,
                   uint64_t padded_dim, uint64_t nlist, uint64_t ex_bits, int metric, int threads,
                   const char *out_path);
/* The same index from raw rows [n][dim]: rotation and RaBitQ quantisation on GPU `device`
 * (cora_tool_quantize), code packing on the host; bit-identical to cora_build_ivf on the
 * GPU-rotated rows (cora_tool_rotate). P <= 1024. */
int cora_build_ivf_gpu(const float *data, const float *rotated_centroids, const uint32_t *assignments,
                       const float *rotator, uint64_t n, uint64_t dim, uint64_t padded_dim, uint64_t nlist,
                       uint64_t ex_bits, int metric, int device, int threads, const char *out_path);
/* RaBitQ codes and factors of n rows against one centroid (for quantizer parity tests):
 * bits u8 [n][P], f1 f32 [n][3], excode u8 [n][P], f2 f32 [n][2]. */
int cora_quantize_rows(const float *rows, const float *centroid, uint64_t n, uint64_t P,
                       uint64_t ex_bits, int metric, uint8_t *bits, float *f1, uint8_t *excode,
                       float *f2);
/* <q', ex_code> of n packed 7-bit codes (the CPU refinement's inner product). */
int cora_excode_ip7(const float *q, const uint8_t *packed, uint64_t n, uint64_t P, float *out);
/* Benchmark data: n rows of a Gaussian mixture, row r = centers[label_r] + sd * z_r
 * (z standard normal), L2-normalised when normalize != 0. Each value is a function of
 * (seed, row, column) only (SplitMix64-hashed counters, Box-Muller), so the output does not
 * depend on threads. dim must be even; labels (u32 [n]) may be NULL. */
int cora_gaussian_mixture(const float *centers, uint64_t n_centers, uint64_t dim, const float *sd,
                          uint64_t n, uint64_t seed, int normalize, int threads, float *out,
                          uint32_t *labels);
/* Vector width of the CPU refinement's inner product: 512 (AVX-512) or 256 (AVX2;
 * forced with CORA_CPU_ISA=avx2 in the environment). */
int cora_cpu_refine_isa(void);

/* Ring protocol check without a GPU: producer threads run the device publication
 * protocol (reserve, cached write limit, HBM-style spill, drain, done) against the real
 * CPU consumer of HybridIndex. Every record carries an analytically known refine
 * distance; returns the consumer's top-k and counters. */
typedef struct cora_ring_test {
    uint64_t capacity, spill_capacity;
    uint32_t producers, consumers, queries, per_query, topk;
    int secondary_filter;
    uint64_t submitted, spilled, refined;
    int overflow;
} cora_ring_test;
int cora_test_ring(cora_ring_test *t, float *dists, uint32_t *ids);

#ifdef __cplusplus
}
#endif

#endif /* CORA_HOST_H */
