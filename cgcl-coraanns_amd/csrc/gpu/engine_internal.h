// Internal declarations shared by the engine's HIP translation units.
//
// HBM layout of the index ("tile layout"): the vectors of each cluster are grouped in
// tiles of 64 (one vector per lane of a wave64). A tile is
//     codes   : ceil(W/4) groups; group g holds words [4g, 4g+4) of all 64 vectors as
//               [lane][4 x u32] (16 B per lane, one 128-bit load per lane per group);
//               when W % 4 == 2 the last group is [lane][2 x u32] (8 B per lane)
//     factors : f_add[64], f_rescale[64], f_error[64] (f32, SoA)
// where W = padded_dim / 32 and dimension 32w+l is bit l of word w (LSB first, the
// order a wave64 ballot produces). Tile bytes = 8*P + 768. Lanes past the end of a
// cluster hold zero codes and are masked by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cora {

constexpr int kTileVectors = 64;
constexpr int kBq = 8;             // query quantisation bits (reference RABITQ_BQ)
constexpr int kMaxBatchQ = 8;      // same-cluster pairs per popcount scan pass
constexpr uint32_t kMaxBatchQArg = 64;  // largest batch-q a search accepts
constexpr int kMaxVanguardKeep = 1024;
constexpr int kSelectMaxProbe = 4096;       // top-nprobe select held in LDS
constexpr uint32_t kNumXcd = 8;
constexpr uint32_t kVanguardMaxPairs = 64;  // fused vanguard pass: vanguard depth limit
constexpr uint32_t kVanguardMaxTopk = 128;  // one-pass vanguard kernel: top-k limit
constexpr uint32_t kVanguardStagedMaxTopk = 1024;  // staged vanguard pass: top-k limit
// the vanguard lows pass runs by default for sign codes + factors beyond MI355X's 256 MB
// last-level cache at a padded dimension of at least kLowsMinDim, and at any dimension beyond
// kLowsAnyDimBytes: a query's own pass reads P/8 + 12 bytes per vanguard vector against the
// lows pass's 4, a saving that pays for the extra pass at P = 768 (config 4: 0.98M -> 1.43M
// QPS) and for a 2.8 GB index at P = 128 (config 5: 1.27M -> 1.33M), not for a nearly
// cache-resident one (config 3, 280 MB: 4.45-4.50M without it, 3.81-3.96M with it; config 2,
// 28 MB: 4.39M against 4.27M)
constexpr uint64_t kLowsMinIndexBytes = 256ull << 20;
constexpr uint32_t kLowsMinDim = 512;
constexpr uint64_t kLowsAnyDimBytes = 1ull << 30;

// Refinement record of one vector (cluster order), ex_record_bytes(P) = P + 16 bytes, so a
// refined vector is one contiguous read: the packed 7-bit ex-code (P*7/8 bytes, 64-dimension
// group g at bytes 56g .. 56g + 55, the reference's packing, pack_excode.hpp:216-265), its sign
// code (P/8 bytes at P*7/8, the tiles' words: dimension 32w+l at bit l of word w), f_add_ex and
// f_rescale_ex at P, and 8 bytes of padding (16-byte aligned records). The readers address it
// through the functions below. (Records with each lane's bytes interleaved in 16-byte chunks,
// per 4-lane split or per 64-dimension group, were measured slower for the refinement kernels
// at P = 768: 1.39 and 1.60 ms against 1.27 ms.)
__host__ __device__ constexpr uint32_t ex_record_bytes(uint32_t P) { return P + 16; }
__host__ __device__ constexpr uint32_t ex_record_groups(uint32_t P) { return P / 64; }
// 8-byte word kk (0..6) of 64-dimension ex-code group g
__host__ __device__ constexpr uint32_t ex_record_group_word(uint32_t P, uint32_t g, uint32_t kk) {
    return 56 * g + 8 * kk;
}
// sign-code word w (words 2g, 2g + 1 hold group g's dimensions, an aligned 8-byte pair)
__host__ __device__ constexpr uint32_t ex_record_sign_word(uint32_t P, uint32_t w) { return P * 7 / 8 + 4 * w; }
__host__ __device__ constexpr uint32_t ex_record_factor_offset(uint32_t P) { return P; }

struct ClusterMeta {
    uint32_t start;      // first global (cluster-order) vector index
    uint32_t n;          // vectors in the cluster
    uint32_t tile_base;  // first tile index
    uint32_t pad;
};

// Tiles one scan unit covers at most (8,192 vectors): a pass over a very large cluster
// is cut into several units so no wave walks it alone. Each unit costs a chain of
// dependent metadata loads before its first tile, so smaller units lose more than
// they balance (16-tile units measured 1.6x slower on a skewed 1M-vector index).
constexpr uint32_t kUnitTiles = 128;

// Units a cluster of n vectors is cut into.
__host__ __device__ inline uint32_t unit_splits(uint32_t n) {
    const uint32_t tiles = (n + kTileVectors - 1) / kTileVectors;
    return tiles ? (tiles + kUnitTiles - 1) / kUnitTiles : 1u;
}

// One scan unit: up to batch_q pairs that probe the same cluster, over the tile range
// [tiles >> 8, (tiles >> 8) + (tiles & 255)) of that cluster.
struct Unit {
    uint32_t cluster;
    uint32_t pair_begin;
    uint32_t count;
    uint32_t tiles;
};

// Scheduled (query, probe) pair: word0 = probe << 16 | query (the Candidate's first
// word), cluster alongside.
struct Pair {
    uint32_t word0;
    uint32_t cluster;
};

// Byte-compatible with coraanns::queue::Progress (fields 64-byte aligned).
struct alignas(64) ProgressDev {
    alignas(64) unsigned long long released;
    alignas(64) unsigned long long produced;
    alignas(64) unsigned long long spilled;
    alignas(64) int done;
    alignas(64) int overflow;
};
static_assert(sizeof(ProgressDev) == 320, "Progress layout");

struct SpillRecord {
    uint4 item;
    unsigned long long position;
    unsigned long long pad;
};

struct QueueDev {
    uint4 *items;                      // host-coherent ring
    ProgressDev *progress;             // host-coherent
    unsigned long long capacity;
    unsigned long long mask;
    unsigned long long *produced;      // HBM reservation counter
    unsigned long long *cached_limit;  // HBM copy of released + capacity
    int *refresh_flag;                 // HBM, one refresher at a time
    SpillRecord *spill;                // HBM
    unsigned long long *spill_count;
    unsigned long long spill_capacity;
    int *spill_overflow;
    int *abort_flag;                   // host-coherent
    int *stalled;                      // HBM
    // GPU-final top-k: records go to spill[position].item (not to the ring) and carry the
    // refined distance in place of exact_ip
    int final_mode;
};

// Bound on the difference between two FP32 evaluations of the refined distance
// (cpu_refinement.cpp:183-192) in any orders of summation, per unit of the magnitude of its
// terms |f_add| + |g_add| + |f_rescale| (128 |exact_ip| + 127 ||q'||_1 + |kb|): each evaluation
// lies within gamma_n = n u / (1 - n u) (u = 2^-24) of the exact value times that magnitude,
// n = P + 8 the longest chain of roundings a term passes (the P multiplications and
// additions of the ex-code dot product, fused or not, and the outer formula's five), so two
// differ by at most 2 gamma_n of it; 2.002 also covers the rounding of the magnitude.
// (P = 128: 1.62e-5, P = 768: 9.26e-5, P = 1024: 1.23e-4.)
__host__ __device__ constexpr float refine_err_scale(uint32_t P) {
    return (float)(2.002 * (P + 8.0) * 0x1p-24 / (1.0 - (P + 8.0) * 0x1p-24));
}

struct ScanParams {
    const uint8_t *tiles;
    const ClusterMeta *meta;
    const uint32_t *qplanes;  // [nq][16][W]: Bq=8 query planes 0..7, residual planes 8..15
    const int8_t *qbytes;     // [nq][2][P]: qint and qres as int8 (MFMA operands)
    // LUT4 estimator (CORA_FLAG_LUT4): per query the FP16 nibble table [P/4][16], 2P u32
    // words; nullptr selects the Bitwise estimator
    const uint32_t *lut;
    // LUT4 with the matrix-core kernels: per query a bound on |LUT4 estimate - Bitwise
    // estimate| over all codes (launch_lut_margin), by which their Bitwise lower bounds are
    // lowered (lut_slack) before the LUT4 bound of the survivors is evaluated exactly
    const float *lut_margin;
    float refine_err;  // refine_err_scale(P): the refined distance's rounding bound per unit of magnitude
    const float *qwidth;      // [nq] Bq=8 step
    const float *qwidth2;     // [nq] residual step (qwidth / 254)
    const float *k1;          // [nq]
    const float *pgadd;       // [nq][nprobe]
    const float *pgerr;       // [nq][nprobe]
    const Pair *pairs;
    const Unit *units;
    const uint32_t *num_units;   // device scalar
    uint32_t *unit_cursor;       // [kNumXcd] dynamic scheduling cursors
    const float *thresholds;     // device copy of the thresholds (snapshot per pass, or the
                                 // launch snapshot in frozen mode)
    uint32_t nprobe;
    uint32_t vanguard;
    uint32_t keep;               // vanguard seed count per pair
    uint32_t tile_bytes;
    uint32_t P;
    uint32_t seed_words;         // u32 words of seed bitmask per vanguard pair
    uint32_t *seed_bits;         // [nq * vanguard][seed_words]
    QueueDev queue;
    // GPU seed refinement (optional: ex_rec == nullptr disables it). The seed pass
    // refines each seed with the HBM copy of the ex-codes exactly as the CPU consumer
    // will (cpu_refinement.cpp:183-192) and records, per seed slot
    // [nq][vanguard][keep], its refined distance, its lower bound and a bound on the
    // rounding difference between this and the CPU's evaluation.
    const uint8_t *ex_rec;       // [N][ex_stride] refinement records (ex_record_bytes)
    uint32_t ex_stride;
    const float *qrot;           // [nq][P] rotated queries
    const float *kb;             // [nq] kbxSumq
    float *seed_dist;            // [nq][vanguard][keep], +inf when unused
    float *seed_low;
    float *seed_err;
    uint4 *seed_rec;             // the seeds' Candidate records, published after the threshold
    // lower bounds of every vector of every vanguard pair, written by the seed pass and
    // read by the recovery pass: [nq][vanguard][van_stride]
    float *van_lows;
    uint32_t van_stride;
    // the smallest lower bound of each group of 4 consecutive vectors of a vanguard pair,
    // written with van_lows by the lows pass when set: [nq][vanguard][van_stride / 4] (+inf for
    // vectors past the cluster's end)
    float *van_mins;
    uint32_t seed_buf;           // seed pass LDS buffer entries (power of two >= keep + 64)
    // refined pre-filter of the far and recovery passes (needs ex_rec)
    int prefilter;
    unsigned long long *dropped;  // records the pre-filter dropped
    // dense debug output
    int32_t *dbg_ip;
    int32_t *dbg_ip2;            // residual inner product <b, qres>
    float *dbg_low;
    uint32_t dbg_stride;         // max cluster size
    uint32_t dbg_set;            // matrix-core dense debug: unit set (0 = vanguard, 1 = far)
};

// Fused vanguard pass (vanguard.hip): one workgroup per query over its vanguard pairs.
// With lows_ready the pass streams the lower bounds the matrix-core pass wrote to
// ScanParams::van_lows instead of evaluating them from the tiles.
struct VanguardArgs {
    const int32_t *probe_idx;      // [nq][nprobe] probed clusters, nearest first
    const uint32_t *order;         // [nq] queries by nearest cluster (nullptr: identity)
    uint32_t nq;
    uint32_t depth;                // vanguard pairs per query (probe ranks 0..depth-1)
    uint32_t topk;
    float *thr_out;                // thresholds lowered by the pass (host-coherent, or the
                                   // frozen snapshot in the test mode)
    unsigned long long *seeded;    // queries whose threshold the pass lowered
    unsigned long long *refined;   // vectors refined on the GPU
    int lows_ready;
    // queries taken from a list whose length is on the device (the staged pass's overflow
    // queries): workgroup b handles list[b] when b < *list_count; nullptr: every query
    const uint32_t *list;
    const unsigned long long *list_count;
};

// Staged vanguard pass (vanguard_staged.hip): the fused pass's work split into per-query
// stages (seed select, threshold and candidate list, merge and publication) and grid-wide
// refinement stages that gather the refinement records of every query at once.
//
// Each query has fixed regions: its seeds (seed_cap entries) and its list (list_cap) of other
// vectors to refine. An entry's position
// is its slot j * van_stride + v in the query's lower-bound rows (pair j, cluster position
// v); the refinement writes rd = {refined distance, rounding bound} and aux = {exact_ip,
// lower bound} beside it.
struct VsQuery {
    uint32_t seed_n, list_n;
    uint32_t cut1;    // seeds: the bounds below thr_in with order key <= cut1
    float thr_in;     // the threshold the pass started from
    float thr;        // the threshold the seeds' refined distances back
    uint32_t dk_key;  // order key of the seeds' topk-th refined distance (~0u: fewer seeds)
    uint32_t flags;   // kVsOverflow: a region was too small; the one-pass kernel takes the query
    uint32_t pub_n;   // records the merge left in the query's out region for publication
    uint32_t pad[4];
};
constexpr uint32_t kVsOverflow = 1;
// counters (VsArgs::ctr): seed entries, list entries, queries whose list needed a re-scan
// of their bounds, queries left to the one-pass kernel
constexpr uint32_t kVsCtrSeeds = 0, kVsCtrList = 1, kVsCtrRescan = 2, kVsCtrOverflow = 3, kVsCtrWords = 4;

// statistics spread over kVsSpread 128-byte lines (a query adds to line q % kVsSpread) and
// summed by one workgroup at the end of the pass
constexpr uint32_t kVsSpread = 64, kVsSpreadWords = 16;
constexpr uint32_t kVsStSeeds = 0, kVsStList = 1, kVsStRescan = 2, kVsStDropped = 3, kVsStRefined = 4,
                   kVsStSeeded = 5;

struct VsArgs {
    uint32_t *seed_pos;       // [nq][seed_cap]
    float2 *seed_rd, *seed_aux;
    uint32_t *list_pos;       // [nq][list_cap]
    float2 *list_rd, *list_aux;
    uint32_t seed_cap, list_cap;
    VsQuery *qs;              // [nq]
    uint4 *out;               // [nq][out_cap] records to publish, written by the merge
    uint32_t out_cap;
    unsigned long long *spread;  // [kVsSpread][kVsSpreadWords], zeroed before the pass
    unsigned long long *ctr;  // [kVsCtrWords], zeroed before the pass
    uint32_t *overflow;       // [nq] queries left to the one-pass kernel (count in ctr)
    uint32_t seeds;           // seed cut's rank among the sub-stream minima (>= topk, <= 512)
};

// the staged pass: P of 64..1024 with a compiled refinement kernel
bool vanguard_staged_supported(uint32_t W);
// refine_ms: optional events around the two refinement launches (timing)
void launch_vanguard_staged(const ScanParams &p, const VanguardArgs &va, const VsArgs &vs, uint32_t W, uint32_t nq,
                            hipEvent_t ev_r0, hipEvent_t ev_r1, hipEvent_t ev_r2, hipEvent_t ev_r3, hipStream_t s);

// ---- launchers (each defined in the translation unit holding its kernel) ----
void launch_repack(const uint32_t *ref_words, const float *ref_factors, const ClusterMeta *meta,
                   uint32_t nlist, uint32_t W, uint8_t *tiles, uint32_t tile_bytes,
                   hipStream_t s);
// Refinement records from the host's packed ex-codes and ex-factors (rows [g0, g0 + n)),
// then the sign codes of every vector from the tiles.
void launch_ex_record_fill(const uint8_t *codes, const float *factors, uint64_t g0, uint32_t n, uint32_t P,
                           uint8_t *rec, hipStream_t s);
void launch_ex_record_sign(const ClusterMeta *meta, uint32_t nlist, const uint8_t *tiles, uint32_t tile_bytes,
                           uint32_t W, uint8_t *rec, hipStream_t s);
// message returned by cora_tool_last_error() (tools.hip; thread-local)
void set_tool_error(const char *msg);
void launch_rotate(const float *q, const float *R, float *out, uint32_t nq, uint32_t dim,
                   uint32_t P, hipStream_t s);
void launch_query_prep(const float *qrot, uint32_t nq, uint32_t P, uint32_t ex_bits, float *k1,
                       float *kb, float *qnorm, float *qwidth, float *qwidth2, uint32_t *qplanes,
                       int8_t *qbytes, hipStream_t s);
// FP16 nibble tables of the reference's Lut4Bit estimator (query_kernels.cuh:199-221):
// lut[q][g][m] = half(sum over the set bits of m, top bit first, of qrot[q][4g..4g+3]),
// summed in FP32 in dimension order and rounded to nearest even.
void launch_lut_build(const float *qrot, uint32_t nq, uint32_t P, uint16_t *lut, hipStream_t s);
void launch_row_norms(const float *x, uint32_t rows, uint32_t P, float *out, hipStream_t s);
// split-FP16 operand rows: hl = [2][rows][P] (hi rows, then lo rows), scale [rows]
void launch_split_f16(const float *x, uint32_t rows, uint32_t P, uint16_t *hl, float *scale,
                      hipStream_t s);
// the same with the hi and lo rows at separate addresses
void launch_split_f16_rows(const float *x, uint32_t rows, uint32_t P, uint16_t *hi, uint16_t *lo, float *scale,
                           hipStream_t s);
// inner dimension K % 32 == 0 and rows * K < 2^31 for both operands
bool dist_gemm_f16x3_supported(uint32_t K, uint64_t rows_a, uint64_t rows_b);
// Q' [nq][P] = X [nq][dim] . R from split-FP16 X and R^T [P][dim]
void launch_rotate_f16x3(const uint16_t *xhl, const float *xscale, const uint16_t *rthl,
                         const float *rtscale, uint32_t nq, uint32_t dim, uint32_t P, float *out,
                         hipStream_t s);
void launch_rotate_f16x3_rows(const uint16_t *xhi, const uint16_t *xlo, const float *xscale, const uint16_t *rthl,
                              const float *rtscale, uint32_t rows, uint32_t dim, uint32_t P, float *out,
                              hipStream_t s);
void launch_dist_gemm_f16x3(const uint16_t *qhl, const float *qscale, const float *qnorm,
                            const uint16_t *chl, const float *cscale, const float *cnorm, uint32_t nq,
                            uint32_t nl, uint32_t P, float *dist, hipStream_t s);
// Fused coarse-probe select (fused_probe_supported: nl >= 8,192, nl <= kFusedProbeMaxList, and
// nprobe <= 64, or up to 1,024 while a 128-cluster tile holds at most ~4.5 probes on average):
// the split-FP16 distance GEMM keeps fused_probe_slots(nprobe) (8 or 16) candidate keys per
// query and 128-cluster tile in scratch (the distance matrix's memory: at least
// fused_probe_scratch_bytes, and nq x nl floats for the fallback);
// the select part merges them into the top-nprobe idx, and the queries the candidates cannot
// settle (fb: 1 + nq words, [0] their count, then their rows) are selected again from their
// distance rows, computed again into the same scratch.
constexpr uint32_t kFusedProbeMaxList = 65536;
bool fused_probe_supported(uint32_t nl, uint32_t nprobe);
uint32_t fused_probe_slots(uint32_t nprobe);
size_t fused_probe_scratch_bytes(uint32_t nq, uint32_t nl, uint32_t nprobe);
void launch_fused_probe_gemm(const uint16_t *qhl, const float *qscale, const float *qnorm, const uint16_t *chl,
                             const float *cscale, const float *cnorm, uint32_t nq, uint32_t nl, uint32_t P,
                             uint32_t nprobe, void *scratch, uint32_t *fb, hipStream_t s);
// the GEMM part for query rows [r0, r0 + rows) of qhi / qlo ([nq][P] each); fb is not touched
void launch_fused_probe_gemm_rows(const uint16_t *qhi, const uint16_t *qlo, const float *qscale, const float *qnorm,
                                  const uint16_t *chl, const float *cscale, const float *cnorm, uint32_t r0,
                                  uint32_t rows, uint32_t nq, uint32_t nl, uint32_t P, uint32_t nprobe,
                                  void *scratch, hipStream_t s);
// Per query, delta >= |LUT4 estimate - Bitwise estimate| for every code: the Bq=8 quantisation
// error's largest subset sum, the FP16 tables' and the FP32 sums' rounding (an upper bound,
// rounded up).
void launch_lut_margin(const float *qrot, const uint32_t *planes, const float *width, uint32_t nq, uint32_t P,
                       float *margin, hipStream_t s);
void launch_fused_probe_select(const uint16_t *qhl, const float *qscale, const float *qnorm, const uint16_t *chl,
                               const float *cscale, const float *cnorm, uint32_t nq, uint32_t nl, uint32_t P,
                               uint32_t nprobe, void *scratch, uint32_t *fb, int32_t *idx, hipStream_t s);
void launch_dist_gemm(const float *q, const float *qnorm, const float *c, const float *cnorm,
                      uint32_t nq, uint32_t nl, uint32_t P, float *dist, hipStream_t s);
// nprobe <= kSelectMaxProbe (selection held in LDS)
void launch_select(const float *dist, uint32_t nq, uint32_t nl, uint32_t nprobe, int32_t *idx,
                   hipStream_t s);
// any nprobe <= nl (up to 65,536): selection in scratch [nq][2][nprobe] u64
void launch_select_big(const float *dist, uint32_t nq, uint32_t nl, uint32_t nprobe,
                       unsigned long long *scratch, int32_t *idx, hipStream_t s);
// g_error of the selected probes is written as err_scale * ||q' - c'||: the lower bound's
// error term f_error * g_error scaled at one place for every pass that forms a bound.
void launch_probe_refine(const float *qrot, const float *cent, const int32_t *idx, uint32_t nq,
                         uint32_t nprobe, uint32_t P, int metric, float *gadd, float *gerr,
                         float err_scale, hipStream_t s);
// max_units: capacity of units (nq * nprobe * unit_splits(largest cluster)); van_batch:
// pairs per vanguard unit (1, or kMfmaBatchQ for the vanguard lows pass)
void launch_build_pairs(const int32_t *probe_idx, const ClusterMeta *meta, uint32_t nq,
                        uint32_t nprobe, uint32_t nlist, uint32_t vanguard, uint32_t batch_q,
                        uint32_t van_batch, uint32_t bytes_per_vector, uint32_t *bucket_count,
                        uint32_t *bucket_cursor,
                        uint32_t *bucket_offset, uint32_t *unit_offset, Pair *pairs, Unit *units,
                        uint64_t max_units, uint32_t *num_units /*[2]: vanguard, far*/,
                        unsigned long long *scan_stats /*[0..2], [9], [10]*/,
                        unsigned long long *block_tot /*[bucket_scan_words(nlist)] scratch*/,
                        bool counts_zero /*bucket_count is all zero (the last call's scan cleared it)*/,
                        hipStream_t s);
// u64 words of the bucket scan's per-block totals
size_t bucket_scan_words(uint32_t nlist);
void launch_fill_u32(uint32_t *p, uint32_t value, size_t n, hipStream_t s);
void launch_fill_u64(unsigned long long *p, unsigned long long value, size_t n, hipStream_t s);
void launch_queue_reset(QueueDev q, hipStream_t s);
void launch_cursor_init(uint32_t *cursor, const uint32_t *num_units, uint32_t set, hipStream_t s);
// kind: 0 = far pairs (publish below cutoff), 1 = vanguard recovery, 2 = dense debug.
// The grid is the number of resident waves the kernel's occupancy allows (persistent).
int launch_scan(const ScanParams &p, uint32_t W, uint32_t batch_q, int kind, hipStream_t s);
// dense debug pass over one unit set (0 = vanguard units, 1 = far units)
int launch_scan_set(const ScanParams &p, uint32_t W, int kind, uint32_t set, hipStream_t s);
int launch_vanguard_seed(const ScanParams &p, uint32_t W, hipStream_t s);
// Per query: the topk-th smallest refined seed distance, raised by the largest rounding
// bound and above the lower bounds of the seeds at or below it, lowers the query's
// threshold (see scan.hip). count = vanguard * keep seed slots per query.
void launch_seed_thresholds(const float *seed_dist, const float *seed_low, const float *seed_err,
                            const uint4 *seed_rec, uint32_t nq, uint32_t count, uint32_t topk,
                            float *thresholds, unsigned long long *seeded, QueueDev q,
                            hipStream_t s);
// LDS bytes of the fused vanguard pass besides q' and the lower bounds
size_t vanguard_static_lds();
// order[0..nq) = queries sorted by their nearest probed cluster; false (nothing launched)
// when nlist is above the kernel's LDS histogram
bool launch_order_queries(const int32_t *probe_idx, uint32_t nq, uint32_t nprobe, uint32_t nlist,
                          uint32_t *order, hipStream_t s);
void launch_vanguard_query(const ScanParams &p, const VanguardArgs &va, uint32_t W, uint32_t nq,
                           hipStream_t s);
// queries per pass of the LUT4 scan (its tables take the LDS of the q-planes)
constexpr uint32_t kLutMaxBatchQ = 4;
// far-pair scan on the matrix cores (scan_mfma.hip): units of up to kMfmaBatchQ pairs
constexpr uint32_t kMfmaBatchQ = 16;
bool far_mfma_supported(uint32_t W);
// the LUT4 estimator on the matrix-core kernels (the wide kernel: P = 512, 768, 1024)
bool far_mfma_lut_supported(uint32_t W);
void launch_far_mfma(const ScanParams &p, uint32_t W, bool dense, hipStream_t s);
// The vanguard units (units of up to kMfmaBatchQ pairs, set 0) on the matrix cores: the lower
// bound of every (vector, pair) to p.van_lows[(query * p.vanguard + probe) * p.van_stride + v]
// (van_stride a multiple of 256).
void launch_vanguard_lows(const ScanParams &p, uint32_t W, hipStream_t s);
// mode: 0 = far units, publish; 1 = far units, dense debug output; 2 = vanguard lows
void launch_mfma_units(const ScanParams &p, uint32_t W, int mode, hipStream_t s);
// dev[0..n) = the host-coherent thresholds, read with system scope (the per-pass copy the
// scan kernels read, so no unit waits on a host-memory round trip)
void launch_snapshot_thresholds(const float *host, float *dev, uint32_t n, hipStream_t s);
// *dst = *src in stream order (per-pass snapshots of the ring position counter)
void launch_copy_u64(const unsigned long long *src, unsigned long long *dst, hipStream_t s);
// max_ticks: drain wait limit in ticks of the device wall clock (wall_clock64)
void launch_finish(QueueDev q, unsigned long long max_ticks, hipStream_t s);
// GPU-final top-k (final.hip) from the first min(*d_n, cap) records of recs: per query the
// topk smallest (refined distance, cluster-order index), ascending; FLT_MAX / 0xFFFFFFFF pad.
// counts/cursor [nq], offsets [nq + 1], keys [cap].
void launch_final_topk(const SpillRecord *recs, const unsigned long long *d_n, unsigned long long cap, uint32_t nq,
                       uint32_t topk, uint32_t *counts, uint32_t *offsets, uint32_t *cursor, unsigned long long *keys,
                       float *out_dist, uint32_t *out_idx, hipStream_t s);

}  // namespace cora
