// RaBitQ 1-bit scan, shared-threshold filtering and the device side of the GPU->CPU
// candidate ring (gfx950, wave64).
//
// Estimator (reference Bitwise producer, filter_kernels.cuh:79-114):
//     ip_int   = sum_{j<7} 2^j popc(x & q_j) - 2^7 popc(x & q_7)     (x: sign code words,
//                q_j: bit plane j of the Bq=8 two's-complement query; = sum_i b_i*qint_i)
//     exact_ip = width * ip_int
//     low      = f_add + g_add + f_rescale * (exact_ip + k1) - f_error * g_error
// A vector of a (query, probe) pair becomes a candidate when low < threshold[query]
// (filter_kernels.cuh:116, 696, 754). Unlike the reference Bitwise producer there is
// no 2*topk cap per pair and no fixed-size shared output array.
//
// The <q',b> a candidate carries to CPU refinement is refined beyond Bq=8: survivors
// get a second popcount against the quantised residual planes, and
//     exact_ip = width * ip_int + width2 * ip_res     (about 16-bit precision)
// which is what keeps the refined distances as accurate as the reference's default
// FP16-LUT producer (filter_kernels.cuh:655-708) rather than its Bq=8 Bitwise one; the
// filter decision itself uses the Bq=8 lower bound above, bit-exact with Bitwise.
//
// Work decomposition: one wave per workgroup; the waves pull scan units (one cluster
// pass serving up to batch_q pairs) from eight per-XCD cursors over eight contiguous
// unit ranges (workgroup i runs on XCD i % 8), stealing from the next range once
// their own is exhausted, so the passes over one cluster stay on one XCD's L2. Each
// lane evaluates one vector of a 64-vector tile: 128-bit code loads, factor loads from
// the tile's SoA block, q-planes read through uniform (scalar) loads or LDS; the next
// tile's loads are issued before the current tile is evaluated.
//
// Publication (ring_queue.cuh:45-115): survivors are compacted with a ballot and a lane
// rank (mbcnt) into a per-wave LDS stage (record, code words, threshold). A full stage,
// and the last one, is flushed 64 records at a time: each record gets its residual inner
// product (and, with the HBM ex-codes, an optional refined-distance check against its
// threshold), the kept records of the round take one 64-bit atomicAdd on the HBM
// position counter, and each goes to the host-coherent ring with one write-through
// 16-byte store when its position is below the cached write limit (released +
// capacity), or to the HBM spill buffer, which the drain kernel publishes once the CPU
// has released that slot.
#include <float.h>

#include <map>
#include <mutex>
#include <utility>

#include "device_common.h"

namespace cora {
namespace {

enum ScanKind { kFar = 0, kRecovery = 1, kDense = 2 };

// LUT4 tables staged per query in LDS: 64 u32 words (8 nibble groups of 16 FP16 values)
// per code word.
constexpr int kLutWordsPerCodeWord = 64;

// Publish the n staged survivors of this wave (n wave-uniform, 0 < n <= kCap), 64 at a
// time. Must be called by all 64 lanes; the workgroup is this one wave. Staged records
// carry ip_int in their exact_ip word; it is replaced by the two-stage estimate. With
// the refined pre-filter (p.prefilter) a record whose refined distance exceeds its
// unit's threshold by more than the rounding bound is dropped: every published threshold
// is backed by at least topk candidates the CPU consumer will refine, so such a record
// can never enter the top-k and the consumer would discard it. Kept records of each
// round take one reservation on the ring position counter.
template <int W, int EST>
__device__ __forceinline__ void flush_stage(const ScanParams &p, const QueueDev &q, uint32_t n,
                                            const uint4 *s_rec, const uint32_t *s_code,
                                            const float *s_cut, unsigned long long &limit,
                                            uint32_t lane) {
    constexpr int K = Words<W>::kMax;
    constexpr int CAP = Stage<W>::kCap;
    const uint32_t nw = W > 0 ? (uint32_t)W : p.P / 32;
    __syncthreads();  // staged LDS writes of every lane are visible
    for (uint32_t i0 = 0; i0 < n; i0 += 64) {
        const uint32_t i = i0 + lane;
        bool keep = false;
        uint4 rec = make_uint4(0u, 0u, 0u, 0u);
        if (i < n) {
            rec = s_rec[i];
            const uint32_t query = rec.x & 0xFFFFu;
            float ex;
            if constexpr (EST == kEstLut4) {
                ex = __uint_as_float(rec.z);  // the LUT estimate is the exact_ip handed on
            } else {
                uint32_t x[K];
#pragma unroll
                for (int w = 0; w < K; ++w)
                    x[w] = (uint32_t)w < nw ? s_code[w * CAP + i] : 0u;
                const uint32_t *res = p.qplanes + ((size_t)query * 2 + 1) * kBq * nw;
                const int ip_res = popc_ip<W>(x, res, nw);
                ex = two_stage_ip(p.qwidth[query], (int)rec.z, p.qwidth2[query], ip_res);
            }
            rec.z = __float_as_uint(ex);
            keep = true;
            if (p.prefilter) {
                float err;
                const float dist = refine_one(p, query, rec.x >> 16, rec.y, ex, err);
                keep = dist <= s_cut[i] + err;
                if (q.final_mode)
                    rec.z = __float_as_uint(dist);
            }
        }
        const unsigned long long m = __ballot(keep);
        if (p.prefilter && lane == 0) {
            const uint32_t in_round = min(64u, n - i0);
            const uint32_t dropped = in_round - (uint32_t)__popcll(m);
            if (dropped)
                atomicAdd(p.dropped, (unsigned long long)dropped);
        }
        if (m == 0)
            continue;
        const uint32_t cnt = (uint32_t)__popcll(m);
        unsigned long long base = 0;
        if (lane == 0)
            base = atomicAdd(q.produced, (unsigned long long)cnt);
        base = shfl0_u64(base);
        if (base + cnt > limit) {
            unsigned long long fresh = 0;
            if (lane == 0)
                fresh = refresh_limit(q.cached_limit, q.refresh_flag, &q.progress->released, q.capacity,
                                      base + cnt);
            limit = shfl0_u64(fresh);
        }
        if (keep)
            place_record(q, base + lane_rank(m), limit, rec);
    }
    __syncthreads();  // the stage may be refilled
}

__device__ __forceinline__ float read_threshold(const float *thresholds, uint32_t query) {
    return thresholds[query];
}

// Next unit index in [0, U) for this wave, or U when every range is exhausted.
__device__ __forceinline__ uint32_t next_unit(uint32_t *cursor, uint32_t U, uint32_t &range,
                                              uint32_t &tries, uint32_t lane_id) {
    const uint32_t per = (U + kNumXcd - 1) / kNumXcd;
    while (tries < kNumXcd) {
        uint32_t u = 0;
        if (lane_id == 0)
            u = atomicAdd(&cursor[range], 1u);
        u = uniform(u);
        const uint32_t end = min(U, (range + 1) * per);
        if (u < end)
            return u;
        range = (range + 1) % kNumXcd;
        ++tries;
    }
    return U;
}

// q-planes of the unit's queries: held in SGPRs (readfirstlane of a broadcast load) when
// one query with P <= 128 is evaluated per pass, otherwise staged in LDS and read with
// wave-uniform addresses.
template <int W, int QMAX>
struct PlaneStore {
    static constexpr bool kRegs = W > 0 && W <= 4 && QMAX == 1;
};

template <int W, int QMAX, int KIND, int EST>
__global__ __launch_bounds__(64) void scan_kernel(const ScanParams p, uint32_t unit_set) {
    constexpr int K = Words<W>::kMax;
    constexpr int CAP = Stage<W>::kCap;
    constexpr bool kLut = EST == kEstLut4;
    constexpr bool kRegs = !kLut && PlaneStore<W, QMAX>::kRegs;
    constexpr bool kStaged = KIND != kDense;
    // q-planes of the unit's queries (Bitwise), or their LUT4 tables
    __shared__ uint32_t s_planes[kRegs ? 1 : QMAX * (kLut ? kLutWordsPerCodeWord : kBq) * K];
    __shared__ uint4 s_rec[kStaged ? CAP : 1];
    __shared__ uint32_t s_code[kStaged ? CAP * K : 1];
    __shared__ float s_cut[kStaged ? CAP : 1];
    const uint32_t lane = threadIdx.x;
    const uint32_t rw = p.P / 32;
    const uint32_t nw = W > 0 ? (uint32_t)W : rw;
    const uint8_t *__restrict__ tiles = p.tiles;
    const ClusterMeta *__restrict__ meta = p.meta;
    const uint32_t *__restrict__ qplanes = p.qplanes;
    const float *__restrict__ qwidth = p.qwidth;
    const float *__restrict__ qk1 = p.k1;
    const float *__restrict__ pgadd = p.pgadd;
    const float *__restrict__ pgerr = p.pgerr;
    const Pair *__restrict__ pairs = p.pairs;
    const Unit *__restrict__ units = p.units;
    const float *thresholds = p.thresholds;
    const uint32_t nprobe = p.nprobe, tile_bytes = p.tile_bytes;
    const uint32_t *seed_bits = p.seed_bits;
    const uint32_t seed_words = p.seed_words, vanguard = p.vanguard;
    const QueueDev q = p.queue;
    const uint32_t U = p.num_units[unit_set];
    const uint32_t ubase = unit_set ? p.num_units[0] : 0u;
    uint32_t range = blockIdx.x % kNumXcd, tries = 0;
    uint32_t staged = 0;
    unsigned long long limit =
        KIND == kDense ? 0ull
                       : __hip_atomic_load(q.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        const uint32_t u = next_unit(p.unit_cursor, U, range, tries, lane);
        if (u >= U)
            break;
        const Unit un = units[ubase + u];
        const uint32_t cluster = uniform(un.cluster);
        const uint32_t count = uniform(un.count);
        const uint32_t pair_begin = uniform(un.pair_begin);
        const ClusterMeta cm = meta[cluster];
        const uint32_t n = uniform(cm.n), start = uniform(cm.start), tbase = uniform(cm.tile_base);
        const uint32_t t_begin = uniform(un.tiles) >> 8, t_end = t_begin + (uniform(un.tiles) & 255u);
        if (n == 0 || t_begin >= t_end)
            continue;  // an empty cluster owns no tile (its tile_base may be one past the end)

        uint32_t word0[QMAX];
        float width[QMAX], k1[QMAX], gadd[QMAX], gerr[QMAX], cutoff[QMAX];
        uint32_t query0 = 0, probe0 = 0;
#pragma unroll
        for (int j = 0; j < QMAX; ++j) {
            const uint32_t jj = (uint32_t)j < count ? (uint32_t)j : 0u;
            const uint32_t w0 = uniform(pairs[pair_begin + jj].word0);
            const uint32_t query = w0 & 0xFFFFu, probe = w0 >> 16;
            if (j == 0) {
                query0 = query;
                probe0 = probe;
            }
            word0[j] = w0;
            cutoff[j] = KIND == kDense ? FLT_MAX : uniformf(read_threshold(thresholds, query));
            width[j] = uniformf(qwidth[query]);
            k1[j] = uniformf(qk1[query]);
            const size_t pi = (size_t)query * nprobe + probe;
            gadd[j] = uniformf(pgadd[pi]);
            gerr[j] = uniformf(pgerr[pi]);
        }
        uint32_t preg[kRegs ? kBq * (W > 0 ? W : 1) : 1];
        if constexpr (kRegs) {
            const uint32_t *src = qplanes + (size_t)query0 * 2 * kBq * W;
#pragma unroll
            for (int i = 0; i < kBq * W; ++i)
                preg[i] = uniform(src[i]);
        } else {
            __syncthreads();
            const uint32_t per = (kLut ? kLutWordsPerCodeWord : kBq) * nw;
            for (uint32_t i = lane; i < QMAX * per; i += 64) {
                const uint32_t j = i / per, r = i % per;
                uint32_t wj = word0[0];
#pragma unroll
                for (int jj = 1; jj < QMAX; ++jj)
                    if ((uint32_t)jj == j)
                        wj = word0[jj];
                const size_t qj = wj & 0xFFFFu;
                s_planes[i] = j >= count ? 0u : kLut ? p.lut[qj * per + r] : qplanes[qj * 2 * kBq * nw + r];
            }
            __syncthreads();
        }
        const uint32_t *seeds = nullptr;
        if (KIND == kRecovery)
            seeds = seed_bits + ((size_t)query0 * vanguard + probe0) * seed_words;
        if constexpr (KIND == kRecovery) {
            // lower bounds stored by the seed pass; code words are loaded only for the tiles
            // holding a survivor (a non-seed below the current threshold)
            const float *lows = p.van_lows + ((size_t)query0 * vanguard + probe0) * p.van_stride;
            constexpr uint32_t kAhead = 4;  // tiles whose lower bounds are loaded together
            float lb[kAhead];
            for (uint32_t t = t_begin; t < t_end; ++t) {
                const uint32_t r = (t - t_begin) % kAhead;
                if (r == 0) {
#pragma unroll
                    for (uint32_t i = 0; i < kAhead; ++i) {
                        const uint32_t li = (t + i) * kTileVectors + lane;
                        lb[i] = t + i < t_end && li < n ? lows[li] : 0.0f;
                    }
                }
                const uint32_t local = t * kTileVectors + lane;
                const bool valid = local < n;
                float low = lb[0];
#pragma unroll
                for (uint32_t i = 1; i < kAhead; ++i)
                    low = r == i ? lb[i] : low;
                const bool survive =
                    valid && low < cutoff[0] && !((seeds[local >> 5] >> (local & 31)) & 1u);
                const unsigned long long mask = __ballot(survive);
                if (mask == 0)
                    continue;
                uint32_t xr[K];
                load_codes<W>(tiles + (size_t)(tbase + t) * tile_bytes, lane, rw, xr);
                uint32_t zbits;  // ip_int (Bitwise) or the LUT4 estimate's bits
                if constexpr (kLut)
                    zbits = __float_as_uint(lut4_ip<W>(xr, s_planes, rw));
                else if constexpr (kRegs)
                    zbits = (uint32_t)popc_ip<W>(xr, preg, rw);
                else
                    zbits = (uint32_t)popc_ip<W>(xr, s_planes, rw);
                const uint32_t cnt = (uint32_t)__popcll(mask);
                if (staged + cnt > (uint32_t)CAP) {
                    flush_stage<W, EST>(p, q, staged, s_rec, s_code, s_cut, limit, lane);
                    staged = 0;
                }
                if (survive) {
                    const uint32_t k = staged + lane_rank(mask);
                    s_rec[k] = make_uint4(word0[0], start + local, zbits, __float_as_uint(low));
                    s_cut[k] = cutoff[0];
#pragma unroll
                    for (int w = 0; w < K; ++w)
                        if ((uint32_t)w < nw)
                            s_code[w * CAP + k] = xr[w];
                }
                staged += cnt;
            }
            continue;
        }
        // tile t is evaluated while tile t+1 (or t again at the end) is being loaded
        uint32_t x[K], xn[K];
        float fa, fr, fe, fan, frn, fen;
        {
            const uint8_t *tile = tiles + (size_t)(tbase + t_begin) * tile_bytes;
            load_codes<W>(tile, lane, rw, x);
            const float *fac = reinterpret_cast<const float *>(tile + 256u * nw);
            fa = fac[lane];
            fr = fac[64 + lane];
            fe = fac[128 + lane];
        }
        for (uint32_t t = t_begin; t < t_end; ++t) {
            {
                const uint32_t tn = t + 1 < t_end ? t + 1 : t;
                const uint8_t *tile = tiles + (size_t)(tbase + tn) * tile_bytes;
                load_codes<W>(tile, lane, rw, xn);
                const float *fac = reinterpret_cast<const float *>(tile + 256u * nw);
                fan = fac[lane];
                frn = fac[64 + lane];
                fen = fac[128 + lane];
            }
            const uint32_t local = t * kTileVectors + lane;
            const bool valid = local < n;
            bool not_seed = true;
            if (KIND == kRecovery)
                not_seed = !valid || !((seeds[local >> 5] >> (local & 31)) & 1u);
#pragma unroll
            for (int j = 0; j < QMAX; ++j) {
                if ((uint32_t)j >= count)
                    break;
                int ip = 0;
                float ex;
                if constexpr (kLut) {
                    ex = lut4_ip<W>(x, s_planes + j * kLutWordsPerCodeWord * nw, rw);
                } else {
                    if constexpr (kRegs)
                        ip = popc_ip<W>(x, preg, rw);
                    else
                        ip = popc_ip<W>(x, s_planes + j * kBq * nw, rw);
                    ex = width[j] * (float)ip;
                }
                const uint32_t zbits = kLut ? __float_as_uint(ex) : (uint32_t)ip;
                const float low = fa + gadd[j] + fr * (ex + k1[j]) - fe * gerr[j];
                if constexpr (KIND == kDense) {
                    if (valid) {
                        const uint32_t query = word0[j] & 0xFFFFu, probe = word0[j] >> 16;
                        const uint32_t *res = qplanes + ((size_t)query * 2 + 1) * kBq * nw;
                        const size_t o = ((size_t)query * nprobe + probe) * p.dbg_stride + local;
                        p.dbg_ip[o] = (int32_t)zbits;
                        p.dbg_ip2[o] = kLut ? 0 : popc_ip<W>(x, res, rw);
                        p.dbg_low[o] = low;
                    }
                } else {
                    const bool survive = valid && not_seed && low < cutoff[j];
                    const unsigned long long mask = __ballot(survive);
                    if (mask != 0) {
                        const uint32_t cnt = (uint32_t)__popcll(mask);
                        if (staged + cnt > (uint32_t)CAP) {
                            flush_stage<W, EST>(p, q, staged, s_rec, s_code, s_cut, limit, lane);
                            staged = 0;
                        }
                        if (survive) {
                            const uint32_t k = staged + lane_rank(mask);
                            s_rec[k] = make_uint4(word0[j], start + local, zbits, __float_as_uint(low));
                            s_cut[k] = cutoff[j];
#pragma unroll
                            for (int w = 0; w < K; ++w)
                                if ((uint32_t)w < nw)
                                    s_code[w * CAP + k] = x[w];
                        }
                        staged += cnt;
                    }
                }
            }
#pragma unroll
            for (int w = 0; w < K; ++w)
                x[w] = xn[w];
            fa = fan;
            fr = frn;
            fe = fen;
        }
    }
    if constexpr (kStaged) {
        if (staged)
            flush_stage<W, EST>(p, q, staged, s_rec, s_code, s_cut, limit, lane);
    }
}

// ---------------------------------------------------------------------------------
// Vanguard seed pass (reference computeInnerProducts1BitLutProducerVanguard,
// filter_kernels.cuh:308-468): for each vanguard pair (probe rank < vanguard) publish the
// `keep` vectors with the smallest lower bounds below the query's threshold and mark
// them in the pair's seed bitmask; the recovery pass later publishes the remaining
// vectors against the thresholds the CPU has tightened meanwhile. Selection: radix
// select of the keep-th smallest key, all smaller keys plus the lowest-index ties.
// ---------------------------------------------------------------------------------
// Ascending bitonic sort of buf[0, cap) (cap a power of two) by the 64 lanes of a
// one-wave workgroup; the barrier makes each step's LDS writes visible to all lanes.
__device__ void wave_sort(unsigned long long *buf, uint32_t cap, uint32_t lane) {
    for (uint32_t size = 2; size <= cap; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = lane; i < cap / 2; i += 64) {
                const uint32_t a = (i / stride) * 2 * stride + (i % stride), b = a + stride;
                const bool asc = (a & size) == 0;
                const unsigned long long x = buf[a], y = buf[b];
                if ((x > y) == asc) {
                    buf[a] = y;
                    buf[b] = x;
                }
            }
            __syncthreads();
        }
    }
}

// Vanguard seed pass (reference computeInnerProducts1BitLutProducerVanguard,
// filter_kernels.cuh:308-468): for each vanguard pair (probe rank < vanguard) publish the
// `keep` vectors with the smallest lower bounds below the query's threshold (ties to
// the lower index) and mark them in the pair's seed bitmask; the recovery pass later
// publishes the remaining vectors against the thresholds tightened meanwhile.
//
// One wave per pair, streaming the cluster's tiles: candidates enter an LDS buffer as
// keys order_key(low) << 32 | index while below the key of the current keep-th entry;
// a full buffer is sorted (wave bitonic sort) and cut back to keep entries. Every lower
// bound also goes to the pair's slice of the HBM lows buffer, which the recovery pass
// reads instead of recomputing the estimator. With the HBM ex-codes, the seeds are then
// refined on the GPU (16 lanes per seed) for the seed thresholds.
template <int W, int EST>
__global__ __launch_bounds__(64) void seed_kernel(const ScanParams p) {
    constexpr bool kLut = EST == kEstLut4;
    extern __shared__ unsigned long long s_buf[];  // [cap] keys, then [cap] f32 exact_ip
    __shared__ uint32_t s_lut[kLut ? kLutWordsPerCodeWord * Words<W>::kMax : 1];  // the pair's LUT4 table
    const uint32_t cap = p.seed_buf;
    float *s_exk = reinterpret_cast<float *>(s_buf + cap);
    const uint32_t lane = threadIdx.x;
    const uint32_t rw = p.P / 32;
    const uint32_t keep = p.keep;
    const uint32_t U = p.num_units[0];
    const QueueDev q = p.queue;
    uint32_t range = blockIdx.x % kNumXcd, tries = 0;
    unsigned long long limit =
        __hip_atomic_load(q.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        const uint32_t u = next_unit(p.unit_cursor, U, range, tries, lane);
        if (u >= U)
            break;
        const Unit un = p.units[u];
        if ((uniform(un.tiles) >> 8) != 0)
            continue;  // a pair's seeds need its whole cluster: only its first unit seeds
        const ClusterMeta cm = p.meta[uniform(un.cluster)];
        const uint32_t n = uniform(cm.n), start = uniform(cm.start), tbase = uniform(cm.tile_base);
        if (n == 0 || keep == 0)
            continue;
        const uint32_t w0 = uniform(p.pairs[uniform(un.pair_begin)].word0);
        const uint32_t query = w0 & 0xFFFFu, probe = w0 >> 16;
        const float width = uniformf(p.qwidth[query]), k1 = uniformf(p.k1[query]);
        const size_t pi = (size_t)query * p.nprobe + probe;
        const float gadd = uniformf(p.pgadd[pi]), gerr = uniformf(p.pgerr[pi]);
        const float cutoff = uniformf(read_threshold(p.thresholds, query));
        const uint32_t *planes = p.qplanes + (size_t)query * 2 * kBq * rw;
        if constexpr (kLut) {
            __syncthreads();
            for (uint32_t i = lane; i < kLutWordsPerCodeWord * rw; i += 64)
                s_lut[i] = p.lut[(size_t)query * kLutWordsPerCodeWord * rw + i];
            __syncthreads();
        }
        float *lows_out = p.van_lows ? p.van_lows + ((size_t)query * p.vanguard + probe) * p.van_stride
                                     : nullptr;
        const uint32_t ntiles = (n + kTileVectors - 1) / kTileVectors;
        uint32_t count = 0;
        unsigned long long bound = ~0ull;
        // tile t is evaluated while tile t+1 (or t again at the end) is being loaded
        uint32_t x[Words<W>::kMax], xn[Words<W>::kMax];
        float fa, fr, fe, fan, frn, fen;
        {
            const uint8_t *tile = p.tiles + (size_t)tbase * p.tile_bytes;
            load_codes<W>(tile, lane, rw, x);
            const float *fac = reinterpret_cast<const float *>(tile + 256u * rw);
            fa = fac[lane];
            fr = fac[64 + lane];
            fe = fac[128 + lane];
        }
        for (uint32_t t = 0; t < ntiles; ++t) {
            {
                const uint8_t *tile = p.tiles + (size_t)(tbase + (t + 1 < ntiles ? t + 1 : t)) * p.tile_bytes;
                load_codes<W>(tile, lane, rw, xn);
                const float *fac = reinterpret_cast<const float *>(tile + 256u * rw);
                fan = fac[lane];
                frn = fac[64 + lane];
                fen = fac[128 + lane];
            }
            const uint32_t local = t * kTileVectors + lane;
            const bool valid = local < n;
            const float ex = kLut ? lut4_ip<W>(x, s_lut, rw) : width * (float)popc_ip<W>(x, planes, rw);
            const float low = fa + gadd + fr * (ex + k1) - fe * gerr;
#pragma unroll
            for (int w = 0; w < Words<W>::kMax; ++w)
                x[w] = xn[w];
            fa = fan;
            fr = frn;
            fe = fen;
            if (lows_out && valid)
                lows_out[local] = low;
            const unsigned long long key = ((unsigned long long)order_key(low) << 32) | local;
            bool cand = valid && low < cutoff && key < bound;
            unsigned long long m = __ballot(cand);
            uint32_t c = (uint32_t)__popcll(m);
            if (count + c > cap) {
                // cut the buffer back to its keep smallest keys
                for (uint32_t i = count + lane; i < cap; i += 64)
                    s_buf[i] = ~0ull;
                __syncthreads();
                wave_sort(s_buf, cap, lane);
                count = min(count, keep);
                bound = count == keep ? s_buf[keep - 1] : ~0ull;
                cand = cand && key < bound;
                m = __ballot(cand);
                c = (uint32_t)__popcll(m);
            }
            if (cand)
                s_buf[count + lane_rank(m)] = key;
            count += c;
        }
        if (count == 0)
            continue;
        for (uint32_t i = count + lane; i < cap; i += 64)
            s_buf[i] = ~0ull;
        __syncthreads();
        wave_sort(s_buf, cap, lane);
        const uint32_t take = min(count, keep);
        // Seeds refined on the GPU are published later by the seed threshold kernel (only
        // those that can still reach the top-k); otherwise they are published now, with one
        // reservation for the pair (the reference's early publication of vanguard seeds).
        const bool defer = p.seed_dist != nullptr;
        unsigned long long base = 0;
        if (!defer) {
            if (lane == 0)
                base = atomicAdd(q.produced, (unsigned long long)take);
            base = shfl0_u64(base);
            if (base + take > limit) {
                unsigned long long fresh = 0;
                if (lane == 0)
                    fresh = refresh_limit(q.cached_limit, q.refresh_flag, &q.progress->released,
                                          q.capacity, base + take);
                limit = shfl0_u64(fresh);
            }
        }
        uint32_t *seed = p.seed_bits + ((size_t)query * p.vanguard + probe) * p.seed_words;
        const float width2 = uniformf(p.qwidth2[query]);
        for (uint32_t sidx = lane; sidx < take; sidx += 64) {
            const unsigned long long key = s_buf[sidx];
            const uint32_t local = (uint32_t)key;
            const uint8_t *tile = p.tiles + (size_t)(tbase + local / kTileVectors) * p.tile_bytes;
            uint32_t x[Words<W>::kMax];
            load_codes<W>(tile, local % kTileVectors, rw, x);
            const float ex = kLut ? lut4_ip<W>(x, s_lut, rw)
                                  : two_stage_ip(width, popc_ip<W>(x, planes, rw), width2,
                                                 popc_ip<W>(x, planes + kBq * rw, rw));
            s_exk[sidx] = ex;
            atomicOr(&seed[local >> 5], 1u << (local & 31));
            const uint4 rec = make_uint4(w0, start + local, __float_as_uint(ex),
                                         __float_as_uint(key_to_float((uint32_t)(key >> 32))));
            if (defer)
                p.seed_rec[((size_t)query * p.vanguard + probe) * keep + sidx] = rec;
            else
                place_record(q, base + sidx, limit, rec);
        }
        if (p.seed_dist) {
            // Refined distance of every seed, 16 lanes per seed (cpu_refinement.cpp:183-192):
            // f_add_ex + g_add + f_rescale_ex * (2^7 * exact_ip + <q', ex_code> + kbxSumq),
            // with a bound on its rounding difference from the CPU's evaluation.
            __syncthreads();
            const uint32_t sub = lane & 15, chunks = p.P / 8;
            const float *qv = p.qrot + (size_t)query * p.P;
            const float kbq = uniformf(p.kb[query]);
            for (uint32_t sidx = lane >> 4; sidx < take; sidx += 4) {
                const unsigned long long key = s_buf[sidx];
                const uint32_t local = (uint32_t)key;
                const size_t gid = (size_t)start + local;
                const uint8_t *code = p.ex_rec + gid * p.ex_stride;
                float ip = 0.0f, l1 = 0.0f;
                for (uint32_t c = sub; c < chunks; c += 16)
                    ip += excode_chunk_ip(code, p.P, qv, c, &l1);
#pragma unroll
                for (int o = 8; o > 0; o >>= 1) {
                    ip += __shfl_xor(ip, o, 16);
                    l1 += __shfl_xor(l1, o, 16);
                }
                if (sub == 0) {
                    const float2 f = *reinterpret_cast<const float2 *>(code + ex_record_factor_offset(p.P));
                    const float fa = f.x, fr = f.y;
                    const float ex = s_exk[sidx];
                    const float dist = fa + gadd + fr * (128.0f * ex + ip + kbq);
                    const float mag = fabsf(fa) + fabsf(gadd) +
                                      fabsf(fr) * (128.0f * fabsf(ex) + 127.0f * l1 + fabsf(kbq));
                    const size_t o = ((size_t)query * p.vanguard + probe) * keep + sidx;
                    p.seed_dist[o] = dist;
                    p.seed_low[o] = key_to_float((uint32_t)(key >> 32));
                    p.seed_err[o] = p.refine_err * mag;
                }
            }
        }
        __syncthreads();  // the buffer is refilled by the next pair
    }
}

// Per query (one workgroup): the topk-th smallest refined seed distance d_k becomes the
// threshold max(d_k + e, l) + 1 ulp, where e is the largest rounding bound and l the
// largest lower bound among the seeds with distance <= d_k. Those seeds are published
// here, so the CPU consumer, evaluating them, finds at least topk of them strictly below
// the threshold and passing its secondary filter: the threshold is one the CPU would
// publish itself once it has refined them, set before the far and recovery passes read
// it. Written only when lower than the current value; a racing CPU store is harmless,
// every value written is at least the final topk-th distance. The other seeds are
// published only when their refined distance is within their rounding bound of the
// threshold.
constexpr int kThrThreads = 256;

__global__ __launch_bounds__(kThrThreads) void seed_threshold_kernel(
    const float *__restrict__ seed_dist, const float *__restrict__ seed_low,
    const float *__restrict__ seed_err, const uint4 *__restrict__ seed_rec, uint32_t count,
    uint32_t topk, float *thresholds, unsigned long long *seeded, const QueueDev q) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_prefix, s_remaining, s_finite, s_ekey, s_lkey;
    __shared__ uint32_t s_wave[kThrThreads / 64];
    __shared__ float s_thr;
    __shared__ unsigned long long s_base, s_limit;
    const uint32_t qi = blockIdx.x, t = threadIdx.x;
    const size_t base = (size_t)qi * count;
    const float *d = seed_dist + base;
    if (t == 0) {
        s_finite = 0;
        s_remaining = topk;
        s_ekey = 0;
        s_lkey = 0;
    }
    __syncthreads();
    uint32_t nf = 0;
    for (uint32_t i = t; i < count; i += kThrThreads)
        nf += isfinite(d[i]) ? 1u : 0u;
    atomicAdd(&s_finite, nf);
    if (t == 0) {
        s_thr = FLT_MAX;  // fewer refined seeds than topk: no threshold, every seed published
        s_limit = __hip_atomic_load(q.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_finite >= topk) {
    // radix select of the topk-th smallest distance (non-finite keys sort last)
    uint32_t prefix = 0, pmask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[t] = 0;
        __syncthreads();
        for (uint32_t i = t; i < count; i += kThrThreads) {
            const uint32_t key = order_key(d[i]);
            if ((key & pmask) == prefix)
                atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (t == 0) {
            uint32_t rem = s_remaining, cum = 0, dg = 0;
            for (; dg < 255; ++dg) {
                if (cum + hist[dg] >= rem)
                    break;
                cum += hist[dg];
            }
            s_remaining = rem - cum;
            s_prefix = prefix | (dg << shift);
        }
        __syncthreads();
        prefix = s_prefix;
        pmask |= 255u << shift;
    }
    const uint32_t kth = prefix;
    // largest rounding bound (>= 0, so its bits order like the value) and largest lower
    // bound among the seeds at or below the topk-th distance
    uint32_t ekey = 0, lkey = 0;
    for (uint32_t i = t; i < count; i += kThrThreads) {
        if (order_key(d[i]) <= kth) {
            ekey = max(ekey, __float_as_uint(seed_err[base + i]));
            lkey = max(lkey, order_key(seed_low[base + i]));
        }
    }
    atomicMax(&s_ekey, ekey);
    atomicMax(&s_lkey, lkey);
    __syncthreads();
    if (t == 0) {
        const float thr = nextafterf(fmaxf(key_to_float(kth) + __uint_as_float(s_ekey),
                                           key_to_float(s_lkey)),
                                     FLT_MAX);
        // atomic minimum: the CPU consumer may lower the same slot concurrently, and a
        // threshold only ever falls
        uint32_t *slot = reinterpret_cast<uint32_t *>(thresholds) + qi;
        uint32_t cur = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        while (thr < __uint_as_float(cur)) {
            if (__hip_atomic_compare_exchange_strong(slot, &cur, __float_as_uint(thr), __ATOMIC_RELAXED,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM))
                break;
        }
        s_thr = thr;
        atomicAdd(seeded, 1ull);
    }
    __syncthreads();
    }
    // Publish the seeds that can still reach the top-k: refined distance within the
    // rounding bound of the threshold (the refined pre-filter's rule); the topk seeds the
    // threshold rests on always qualify. One reservation per round of 256 slots.
    const float thr = s_thr;
    const uint32_t lane = t & 63, wave = t >> 6;
    for (uint32_t r0 = 0; r0 < count; r0 += kThrThreads) {
        const uint32_t i = r0 + t;
        const bool pub = i < count && isfinite(d[i]) && d[i] <= thr + seed_err[base + i];
        const unsigned long long m = __ballot(pub);
        if (lane == 0)
            s_wave[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t before = 0, total = 0;
#pragma unroll
        for (uint32_t w = 0; w < kThrThreads / 64; ++w) {
            before += w < wave ? s_wave[w] : 0u;
            total += s_wave[w];
        }
        if (total != 0) {
            if (t == 0) {
                const unsigned long long b = atomicAdd(q.produced, (unsigned long long)total);
                unsigned long long lim = s_limit;
                if (b + total > lim)
                    lim = refresh_limit(q.cached_limit, q.refresh_flag, &q.progress->released,
                                        q.capacity, b + total);
                s_base = b;
                s_limit = lim;
            }
            __syncthreads();
            if (pub)
                place_record(q, s_base + before + lane_rank(m), s_limit, seed_rec[base + i]);
        }
        __syncthreads();  // s_wave / s_base reused by the next round
    }
}

__global__ void copy_u64_kernel(const unsigned long long *src, unsigned long long *dst) { *dst = *src; }

__global__ void snapshot_thresholds_kernel(const float *host, float *dev, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        dev[i] = __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t *>(host) + i,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM));
}

__global__ void queue_reset_kernel(QueueDev q) {
    *q.produced = 0;
    *q.spill_count = 0;
    *q.spill_overflow = 0;
    *q.cached_limit = q.capacity;
    *q.refresh_flag = 0;
    *q.stalled = 0;
}

__global__ void cursor_init_kernel(uint32_t *cursor, const uint32_t *num_units, uint32_t set) {
    const uint32_t U = num_units[set];
    const uint32_t per = (U + kNumXcd - 1) / kNumXcd;
    const uint32_t x = threadIdx.x;
    if (x < kNumXcd)
        cursor[x] = x * per;
}

// Queue completion (reference finish_queue, ring_queue.cuh:125-170): publish produced
// and spilled counts, drain spilled records into the ring as the CPU releases space,
// then set Progress::done with a system-scope release. The wait is bounded in time
// (max_ticks of the constant-rate wall clock, whatever a drain pass costs) and honours
// the host abort flag, so the kernel always ends.
__global__ __launch_bounds__(256) void finish_kernel(QueueDev q, unsigned long long max_ticks) {
    __shared__ unsigned long long s_limit;
    __shared__ uint32_t s_remaining;
    __shared__ int s_abort, s_expired;
    const unsigned long long t_start = wall_clock64();
    const uint32_t t = threadIdx.x;
    const unsigned long long produced = *q.produced;
    const unsigned long long spill_total = *q.spill_count;
    const unsigned long long spilled = spill_total < q.spill_capacity ? spill_total : q.spill_capacity;
    const int overflow = *q.spill_overflow;
    if (t == 0) {
        __hip_atomic_store(&q.progress->produced, produced, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(&q.progress->spilled, spill_total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
    bool stalled = false;
    if (!overflow) {
        for (;;) {
            if (t == 0) {
                s_limit = __hip_atomic_load(&q.progress->released, __ATOMIC_ACQUIRE,
                                            __HIP_MEMORY_SCOPE_SYSTEM) +
                          q.capacity;
                s_remaining = 0;
                s_abort = __hip_atomic_load(q.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                s_expired = wall_clock64() - t_start > max_ticks;
            }
            __syncthreads();
            if (s_abort) {
                stalled = true;
                break;
            }
            uint32_t rem = 0;
            const unsigned long long lim = s_limit;
            for (unsigned long long i = t; i < spilled; i += blockDim.x) {
                const unsigned long long pos = q.spill[i].position;
                if (pos == ~0ull)
                    continue;
                if (pos < lim) {
                    store_ring(&q.items[pos & q.mask], q.spill[i].item);
                    q.spill[i].position = ~0ull;
                } else {
                    ++rem;
                }
            }
            if (rem)
                atomicAdd(&s_remaining, rem);
            __syncthreads();
            if (s_remaining == 0)
                break;
            if (s_expired) {
                stalled = true;
                break;
            }
            __builtin_amdgcn_s_sleep(127);
            __syncthreads();
        }
    }
    __syncthreads();
    if (t == 0) {
        if (stalled)
            *q.stalled = 1;
        __threadfence_system();
        if (overflow || stalled)
            __hip_atomic_store(&q.progress->overflow, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(&q.progress->done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Persistent grid = workgroups of this kernel resident on the whole device at once.
template <class F>
uint32_t resident_grid(F kernel, int block, size_t dyn_lds = 0) {
    static std::mutex mu;
    static std::map<std::pair<const void *, size_t>, uint32_t> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    const std::pair<const void *, size_t> key(reinterpret_cast<const void *>(kernel), dyn_lds);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end())
        return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, dyn_lds) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        per_cu <= 0 || cus <= 0) {
        per_cu = 8;
        cus = 256;
    }
    const uint32_t grid = (uint32_t)(per_cu * cus);
    cache.emplace(key, grid);
    return grid;
}

template <int W, int Q, int KIND, int EST = kEstBitwise>
void launch_one(const ScanParams &p, uint32_t set, hipStream_t s) {
    auto *k = scan_kernel<W, Q, KIND, EST>;
    k<<<resident_grid(k, 64), 64, 0, s>>>(p, set);
}

// LUT4 estimator: the generic-width kernels only (an A/B mode), up to kLutMaxBatchQ
// queries per pass
int launch_scan_lut(const ScanParams &p, uint32_t batch_q, int kind, uint32_t set, hipStream_t s) {
    if (kind == kFar) {
        if (batch_q <= 1)
            launch_one<0, 1, kFar, kEstLut4>(p, set, s);
        else
            launch_one<0, kLutMaxBatchQ, kFar, kEstLut4>(p, set, s);
    } else if (kind == kRecovery) {
        launch_one<0, 1, kRecovery, kEstLut4>(p, set, s);
    } else {
        launch_one<0, kLutMaxBatchQ, kDense, kEstLut4>(p, set, s);
    }
    return 0;
}

template <int W>
int launch_scan_w(const ScanParams &p, uint32_t batch_q, int kind, uint32_t set, hipStream_t s) {
    if (p.lut)
        return launch_scan_lut(p, batch_q, kind, set, s);
    if (kind == kFar) {
        if (batch_q <= 1)
            launch_one<W, 1, kFar>(p, set, s);
        else
            launch_one<W, kMaxBatchQ, kFar>(p, set, s);
    } else if (kind == kRecovery) {
        launch_one<W, 1, kRecovery>(p, set, s);
    } else {
        launch_one<W, kMaxBatchQ, kDense>(p, set, s);
    }
    return 0;
}

template <int W, int EST = kEstBitwise>
void launch_seed_w(const ScanParams &p, hipStream_t s) {
    auto *k = seed_kernel<W, EST>;
    const size_t lds = (size_t)p.seed_buf * (sizeof(unsigned long long) + sizeof(float));
    k<<<resident_grid(k, 64, lds), 64, lds, s>>>(p);
}

}  // namespace

int launch_scan(const ScanParams &p, uint32_t W, uint32_t batch_q, int kind, hipStream_t s) {
    // unit set: vanguard units for the recovery pass, far units otherwise
    const uint32_t set = kind == kRecovery ? 0u : 1u;
    switch (W) {
    case 2: return launch_scan_w<2>(p, batch_q, kind, set, s);
    case 4: return launch_scan_w<4>(p, batch_q, kind, set, s);
    case 6: return launch_scan_w<6>(p, batch_q, kind, set, s);
    case 8: return launch_scan_w<8>(p, batch_q, kind, set, s);
    case 12: return launch_scan_w<12>(p, batch_q, kind, set, s);
    case 16: return launch_scan_w<16>(p, batch_q, kind, set, s);
    case 24: return launch_scan_w<24>(p, batch_q, kind, set, s);
    case 32: return launch_scan_w<32>(p, batch_q, kind, set, s);
    default: return launch_scan_w<0>(p, batch_q, kind, set, s);
    }
}

int launch_scan_set(const ScanParams &p, uint32_t W, int kind, uint32_t set, hipStream_t s) {
    switch (W) {
    case 2: return launch_scan_w<2>(p, 8, kind, set, s);
    case 4: return launch_scan_w<4>(p, 8, kind, set, s);
    case 6: return launch_scan_w<6>(p, 8, kind, set, s);
    case 8: return launch_scan_w<8>(p, 8, kind, set, s);
    case 12: return launch_scan_w<12>(p, 8, kind, set, s);
    case 16: return launch_scan_w<16>(p, 8, kind, set, s);
    case 24: return launch_scan_w<24>(p, 8, kind, set, s);
    case 32: return launch_scan_w<32>(p, 8, kind, set, s);
    default: return launch_scan_w<0>(p, 8, kind, set, s);
    }
}

int launch_vanguard_seed(const ScanParams &p, uint32_t W, hipStream_t s) {
    if (p.lut) {
        launch_seed_w<0, kEstLut4>(p, s);
        return 0;
    }
    switch (W) {
    case 2: launch_seed_w<2>(p, s); break;
    case 4: launch_seed_w<4>(p, s); break;
    case 8: launch_seed_w<8>(p, s); break;
    case 24: launch_seed_w<24>(p, s); break;
    default: launch_seed_w<0>(p, s); break;
    }
    return 0;
}

void launch_seed_thresholds(const float *seed_dist, const float *seed_low, const float *seed_err,
                            const uint4 *seed_rec, uint32_t nq, uint32_t count, uint32_t topk,
                            float *thresholds, unsigned long long *seeded, QueueDev q,
                            hipStream_t s) {
    seed_threshold_kernel<<<nq, kThrThreads, 0, s>>>(seed_dist, seed_low, seed_err, seed_rec, count,
                                                     topk, thresholds, seeded, q);
}

void launch_snapshot_thresholds(const float *host, float *dev, uint32_t n, hipStream_t s) {
    if (n)
        snapshot_thresholds_kernel<<<(n + 255) / 256, 256, 0, s>>>(host, dev, n);
}

void launch_copy_u64(const unsigned long long *src, unsigned long long *dst, hipStream_t s) {
    copy_u64_kernel<<<1, 1, 0, s>>>(src, dst);
}

void launch_queue_reset(QueueDev q, hipStream_t s) { queue_reset_kernel<<<1, 1, 0, s>>>(q); }

void launch_cursor_init(uint32_t *cursor, const uint32_t *num_units, uint32_t set, hipStream_t s) {
    cursor_init_kernel<<<1, 64, 0, s>>>(cursor, num_units, set);
}

void launch_finish(QueueDev q, unsigned long long max_ticks, hipStream_t s) {
    finish_kernel<<<1, 256, 0, s>>>(q, max_ticks);
}

}  // namespace cora
