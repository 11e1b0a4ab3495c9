// Far-pair scan on the matrix cores (gfx950 v_mfma_i32_16x16x64_i8, and 16x16x32 for
// P = 64 and 192).
//
// The Bitwise estimator's integer inner product (filter_kernels.cuh:79-114)
//     ip_int = sum_i b_i * qint_i        (b_i the sign bit of dimension i, qint_i in [-128, 127])
// is a product of a 0/1 matrix with an int8 matrix, exact in int32. A scan unit serves up
// to 16 same-cluster pairs, so a 64-vector tile against the unit's queries is a
// [64 x P] x [P x 16] integer product: four 16x16 output blocks, P/64 (P/32) K-steps each.
// The residual product against qres for the two-stage exact_ip is formed by popcount for
// the survivors only (and, at P = 64 and 192, as a second MFMA product). The code bits are
// widened to int8 through a 256-entry table in LDS (one 8-byte read per code byte); the
// queries' int8 values come from the query preparation. ip_int and ip_res are therefore
// bit-identical to the popcount kernel's (scan.hip), and the lower bound uses the same
// expression, so the candidate set is the same.
//
// MFMA lane layout (16x16x32 i8): lane l supplies A[l%16][8(l/16)+e] and B[8(l/16)+e][l%16]
// (byte e of a 64-bit operand) and holds D[4(l/16)+r][l%16], r = 0..3. Here rows are
// vectors (16 m + ...) and columns are the unit's pair slots, so lane l evaluates pair slot
// l % 16 for vectors 16 m + 4 (l / 16) + r.
//
// The same kernels also evaluate the vanguard pairs cluster-major (MfmaMode::kLows): every
// (vector, pair) lower bound of the vanguard units is written to the per-pair lows array,
// which the per-query vanguard pass (vanguard.hip) then streams instead of re-reading each
// query's clusters on its own.
//
// Work distribution, thresholds, staging and publication follow the popcount far scan:
// one wave per workgroup, persistent grid, per-XCD unit cursors, per-pass threshold
// snapshot, survivors staged in LDS and flushed 64 at a time (refined pre-filter with the
// HBM ex-codes, one reservation per round, write-through ring stores).
#include <float.h>

#include <map>
#include <mutex>
#include <utility>

#include "device_common.h"

namespace cora {
namespace {

typedef int32_t v4i32 __attribute__((ext_vector_type(4)));
constexpr int kStage = 256;  // staged survivor records per wave

// What a unit's lower bounds are used for: published below the cutoff (far pairs),
// written with ip_int and ip_res to the debug arrays, or written to the vanguard lows.
// kPublishLut / kLowsLut: the same with the LUT4 estimator (the wide kernel only): the Bitwise
// bounds lowered by lut_slack, and the survivors' LUT4 bounds evaluated exactly.
enum MfmaMode : int { kPublish = 0, kDenseDbg = 1, kLows = 2, kPublishLut = 3, kLowsLut = 4, kDenseLut = 5 };

// The smallest of the lower bounds of vectors o .. o + 3 of a cluster of n vectors (+inf for
// vectors past its end): the group minima of the vanguard lows pass (ScanParams::van_mins).
__device__ __forceinline__ float group_min4(const float (&lw)[4], uint32_t o, uint32_t n) {
    float mn = __int_as_float(0x7F800000);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        mn = o + r < n ? fminf(mn, lw[r]) : mn;
    return mn;
}

// The lows pass stages a tile's lower bounds (64 vectors x the unit's 16 pair slots) in LDS
// and writes them pair by pair: the MFMA result gives a lane 4 consecutive vectors of one
// pair, so direct stores would write each pair's 256 bytes as sixteen 16-byte pieces from
// four instructions; staged, a store instruction writes 4 whole pair rows of 256 bytes.
constexpr uint32_t kLowPitch = 68;  // floats per staged pair row (64 + 4, staggering the banks)

// lower bounds lw of vectors o .. o + 3 of pair slot col
__device__ __forceinline__ void lows_put(float *s_low, uint32_t col, uint32_t o, const float (&lw)[4]) {
    *reinterpret_cast<float4 *>(s_low + col * kLowPitch + o) = make_float4(lw[0], lw[1], lw[2], lw[3]);
}

// Writes the staged bounds of tile t to van_lows (and their group minima to van_mins). w0 is
// the lane's pair word (lanes 0..15 hold slots 0..15), count the unit's pairs, n the cluster
// size. One-wave workgroups: the barriers order the LDS writes, these reads and the next
// tile's writes.
__device__ __forceinline__ void lows_flush(const ScanParams &p, const float *s_low, uint32_t lane, uint32_t w0,
                                           uint32_t count, uint32_t t, uint32_t n) {
    __syncthreads();
    const uint32_t c = lane & 15u, sub = lane >> 4;
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t pr = 4 * i + sub;
        const uint32_t w = __shfl(w0, (int)pr);
        if (pr < count) {
            const float4 v = *reinterpret_cast<const float4 *>(s_low + pr * kLowPitch + 4 * c);
            const size_t row = (size_t)(w & 0xFFFFu) * p.vanguard + (w >> 16);
            const uint32_t o = t * kTileVectors + 4 * c;
            *reinterpret_cast<float4 *>(p.van_lows + row * p.van_stride + o) = v;
            if (p.van_mins) {
                const float lw[4] = {v.x, v.y, v.z, v.w};
                p.van_mins[row * (p.van_stride / 4) + o / 4] = group_min4(lw, o, n);
            }
        }
    }
    __syncthreads();
}

// Bits 0..7 of b as eight int8 0/1 values (bit e in byte e), the 64-bit MFMA operand.
__device__ __forceinline__ long spread_byte(uint32_t b) {
    const uint32_t lo = ((b & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t hi = (((b >> 4) & 15u) * 0x00204081u) & 0x01010101u;
    return (long)(((unsigned long long)hi << 32) | lo);
}

__device__ __forceinline__ uint32_t next_far_unit(uint32_t *cursor, uint32_t U, uint32_t &range,
                                                  uint32_t &tries, uint32_t lane) {
    const uint32_t per = (U + kNumXcd - 1) / kNumXcd;
    while (tries < kNumXcd) {
        uint32_t u = 0;
        if (lane == 0)
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

// Publish n staged records (n wave-uniform, 0 < n <= kStage), 64 at a time; records carry
// their final exact_ip. With the refined pre-filter a record whose refined distance
// exceeds its cutoff by more than the rounding bound is dropped.
__device__ void flush_records(const ScanParams &p, const QueueDev &q, uint32_t n, const uint4 *s_rec,
                              const float *s_cut, unsigned long long &limit, uint32_t lane) {
    __syncthreads();
    for (uint32_t i0 = 0; i0 < n; i0 += 64) {
        const uint32_t i = i0 + lane;
        bool keep = false;
        uint4 rec = make_uint4(0u, 0u, 0u, 0u);
        if (i < n) {
            rec = s_rec[i];
            keep = rec.x != ~0u;  // ~0: dropped by finalize_records (LUT4 bound)
            if (keep && p.prefilter) {
                float err;
                const float dist = refine_one(p, rec.x & 0xFFFFu, rec.x >> 16, rec.y,
                                              __uint_as_float(rec.z), err);
                keep = dist <= s_cut[i] + err;
                if (q.final_mode)
                    rec.z = __float_as_uint(dist);
            }
        }
        const unsigned long long m = __ballot(keep);
        const unsigned long long live = __ballot(i < n && rec.x != ~0u);
        if (p.prefilter && lane == 0) {
            const uint32_t dropped = (uint32_t)__popcll(live) - (uint32_t)__popcll(m);
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
    __syncthreads();
}

// W = P / 32 words per vector, W = 2 or 6 (P = 64, 192; the other widths run the wide
// kernel below): the unit's query operands stay in VGPRs, one v_mfma_i32_16x16x32_i8 per
// code word and row block.
// kDenseDbg: write ip_int, ip_res and the lower bound of every (vector, pair) to the debug
// arrays instead of publishing (the estimator parity test of the kernel the search runs).
// kLows: the vanguard units; every lower bound goes to van_lows, ip_res is not formed.
template <int W, int kMode>
__global__ __launch_bounds__(64) void far_mfma_kernel(const ScanParams p) {
    constexpr bool kDense = kMode != kPublish;
    static_assert(W % 2 == 0 && W >= 2 && W <= 8, "query operands in registers");
    constexpr int G = (W + 3) / 4;  // code word groups of a tile
    __shared__ uint4 s_rec[kDense ? 1 : kStage];
    __shared__ float s_cut[kDense ? 1 : kStage];
    __shared__ __align__(16) float s_low[kMode == kLows ? 16 * kLowPitch : 4];
    // bits 0..7 of a byte b as eight int8 0/1 values (the MFMA operand): s_spread[b]
    __shared__ long s_spread[256];
    const uint32_t lane = threadIdx.x, col = lane & 15, quad = lane >> 4;
    const uint32_t P = 32u * W;
    for (uint32_t b = lane; b < 256; b += 64)
        s_spread[b] = spread_byte(b);
    __syncthreads();
    const QueueDev q = p.queue;
    // kLows runs over the vanguard unit set, kPublish over the far units, the dense debug
    // output over either
    const uint32_t set = kMode == kLows ? 0u : kMode == kPublish ? 1u : p.dbg_set;
    const uint32_t U = p.num_units[set];
    const uint32_t ubase = set ? p.num_units[0] : 0u;
    uint32_t range = blockIdx.x % kNumXcd, tries = 0;
    uint32_t staged = 0;
    unsigned long long limit =
        kDense ? 0ull : __hip_atomic_load(q.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        const uint32_t u = next_far_unit(p.unit_cursor, U, range, tries, lane);
        if (u >= U)
            break;
        const Unit un = p.units[ubase + u];
        const uint32_t cluster = uniform(un.cluster), count = uniform(un.count);
        const ClusterMeta cm = p.meta[cluster];
        const uint32_t n = uniform(cm.n), start = uniform(cm.start), tbase = uniform(cm.tile_base);
        const uint32_t t_begin = uniform(un.tiles) >> 8, t_end = t_begin + (uniform(un.tiles) & 255u);
        if (n == 0 || t_begin >= t_end)
            continue;
        // this lane's pair slot
        const bool slot = col < count;
        const uint32_t w0 = slot ? p.pairs[uniform(un.pair_begin) + col].word0 : 0u;
        const uint32_t query = w0 & 0xFFFFu, probe = w0 >> 16;
        float width = 0.0f, width2 = 0.0f, k1 = 0.0f, gadd = 0.0f, gerr = 0.0f, cutoff = -FLT_MAX;
        long bq[W], br[W];
        if (slot) {
            width = p.qwidth[query];
            width2 = p.qwidth2[query];
            k1 = p.k1[query];
            const size_t pi = (size_t)query * p.nprobe + probe;
            gadd = p.pgadd[pi];
            gerr = p.pgerr[pi];
            cutoff = kDense ? FLT_MAX : p.thresholds[query];
            const int8_t *qb = p.qbytes + (size_t)query * 2 * P + 8 * quad;
#pragma unroll
            for (int kc = 0; kc < W; ++kc) {
                bq[kc] = *reinterpret_cast<const long *>(qb + 32 * kc);
                br[kc] = kMode == kLows ? 0 : *reinterpret_cast<const long *>(qb + P + 32 * kc);
            }
        } else {
#pragma unroll
            for (int kc = 0; kc < W; ++kc)
                bq[kc] = br[kc] = 0;
        }
        for (uint32_t t = t_begin; t < t_end; ++t) {
            const uint8_t *tile = p.tiles + (size_t)(tbase + t) * p.tile_bytes;
            const float *fac = reinterpret_cast<const float *>(tile + 256u * W);
            // words of vector 16 m + col for the four row blocks, and the factors of
            // vectors 16 m + 4 quad + r
            uint32_t xw[4][W];
            float4 fa[4], fr[4], fe[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t v = 16 * m + col;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (4 * g + 4 <= W) {
                        const uint4 c = *reinterpret_cast<const uint4 *>(tile + (size_t)g * 1024 + v * 16);
                        xw[m][4 * g] = c.x;
                        xw[m][4 * g + 1] = c.y;
                        xw[m][4 * g + 2] = c.z;
                        xw[m][4 * g + 3] = c.w;
                    } else {
                        const uint2 c = *reinterpret_cast<const uint2 *>(tile + (size_t)g * 1024 + v * 8);
                        xw[m][4 * g] = c.x;
                        xw[m][4 * g + 1] = c.y;
                    }
                }
                const uint32_t o = 16 * m + 4 * quad;
                fa[m] = *reinterpret_cast<const float4 *>(fac + o);
                fr[m] = *reinterpret_cast<const float4 *>(fac + 64 + o);
                fe[m] = *reinterpret_cast<const float4 *>(fac + 128 + o);
            }
            v4i32 acc[4], accr[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acc[m] = v4i32{0, 0, 0, 0};
                accr[m] = v4i32{0, 0, 0, 0};
#pragma unroll
                for (int kc = 0; kc < W; ++kc) {
                    const long a = s_spread[(xw[m][kc] >> (8 * quad)) & 0xFFu];
                    acc[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq[kc], acc[m], 0, 0, 0);
                    if constexpr (kMode != kLows)
                        accr[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, br[kc], accr[m], 0, 0, 0);
                }
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float fav[4] = {fa[m].x, fa[m].y, fa[m].z, fa[m].w};
                const float frv[4] = {fr[m].x, fr[m].y, fr[m].z, fr[m].w};
                const float fev[4] = {fe[m].x, fe[m].y, fe[m].z, fe[m].w};
                if constexpr (kMode == kLows) {
                    // rows 16 m + 4 quad + r of the pair's tile-padded slice (lanes past the
                    // cluster's end stage values nobody reads)
                    if (slot) {
                        float lw[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            lw[r] = fav[r] + gadd + frv[r] * (width * (float)acc[m][r] + k1) - fev[r] * gerr;
                        lows_put(s_low, col, 16 * m + 4 * quad, lw);
                    }
                    continue;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t local = t * kTileVectors + 16 * m + 4 * quad + r;
                    const bool valid = slot && local < n;
                    const int ip = acc[m][r];
                    const float ex = width * (float)ip;
                    const float low = fav[r] + gadd + frv[r] * (ex + k1) - fev[r] * gerr;
                    if constexpr (kDense) {
                        if (valid) {
                            const size_t o = ((size_t)query * p.nprobe + probe) * p.dbg_stride + local;
                            p.dbg_ip[o] = ip;
                            p.dbg_ip2[o] = accr[m][r];
                            p.dbg_low[o] = low;
                        }
                    } else {
                        const bool survive = valid && low < cutoff;
                        const unsigned long long mask = __ballot(survive);
                        if (mask == 0)
                            continue;
                        const uint32_t cnt = (uint32_t)__popcll(mask);
                        if (staged + cnt > (uint32_t)kStage) {
                            flush_records(p, q, staged, s_rec, s_cut, limit, lane);
                            staged = 0;
                        }
                        if (survive) {
                            const uint32_t k = staged + lane_rank(mask);
                            const float exact = two_stage_ip(width, ip, width2, accr[m][r]);
                            s_rec[k] = make_uint4(w0, start + local, __float_as_uint(exact), __float_as_uint(low));
                            s_cut[k] = cutoff;
                        }
                        staged += cnt;
                    }
                }
            }
            if constexpr (kMode == kLows)
                lows_flush(p, s_low, lane, w0, count, t, n);
        }
    }
    if constexpr (!kDense) {
        if (staged)
            flush_records(p, q, staged, s_rec, s_cut, limit, lane);
    }
}

// Residual inner product <b, qres> of vector v (0..63) of a tile, by popcount over the
// query's residual planes: the wide kernel evaluates it for survivors only (and in the
// dense debug mode), since the lower bound needs ip_int alone.
template <int W>
__device__ __forceinline__ int tile_ip_res(const uint8_t *__restrict__ tile, uint32_t v,
                                           const uint32_t *__restrict__ rplanes) {
    uint32_t x[W];
#pragma unroll
    for (int g = 0; g < W / 4; ++g) {
        const uint4 c = *reinterpret_cast<const uint4 *>(tile + (size_t)g * 1024 + v * 16);
        x[4 * g] = c.x;
        x[4 * g + 1] = c.y;
        x[4 * g + 2] = c.z;
        x[4 * g + 3] = c.w;
    }
    return popc_ip<W>(x, rplanes, W);
}

// Survivors staged with their ip_int and tile position get their two-stage exact_ip. With
// LUT4 they get the LUT4 estimate (filter_kernels.cuh:655-708, one lane per record, in the
// reference's order) and its lower bound, and those whose bound is not below their cutoff are
// marked dropped (x = ~0).
template <int W, bool kLut>
__device__ void finalize_records(const ScanParams &p, uint32_t n, uint4 *s_rec, const uint32_t *s_loc,
                                 const float *s_cut, uint32_t lane) {
    __syncthreads();
    for (uint32_t i = lane; i < n; i += 64) {
        uint4 rec = s_rec[i];
        const uint32_t query = rec.x & 0xFFFFu, loc = s_loc[i];
        const uint8_t *tile = p.tiles + (size_t)(loc >> 6) * p.tile_bytes;
        const uint32_t v = loc & 63u;
        if constexpr (kLut) {
            uint32_t x[W];
#pragma unroll
            for (int g = 0; g < W / 4; ++g) {
                const uint4 c = *reinterpret_cast<const uint4 *>(tile + (size_t)g * 1024 + v * 16);
                x[4 * g] = c.x;
                x[4 * g + 1] = c.y;
                x[4 * g + 2] = c.z;
                x[4 * g + 3] = c.w;
            }
            const float ex = lut4_ip<W>(x, p.lut + (size_t)query * 2 * p.P, W);
            const float *fac = reinterpret_cast<const float *>(tile + 256u * W);
            const size_t pi = (size_t)query * p.nprobe + (rec.x >> 16);
            const float low = fac[v] + p.pgadd[pi] + fac[64 + v] * (ex + p.k1[query]) - fac[128 + v] * p.pgerr[pi];
            rec.z = __float_as_uint(ex);
            rec.w = __float_as_uint(low);
            if (!(low < s_cut[i]))
                rec.x = ~0u;
        } else {
            const int ipr = tile_ip_res<W>(tile, v, p.qplanes + ((size_t)query * 16 + 8) * W);
            rec.z = __float_as_uint(two_stage_ip(p.qwidth[query], (int)rec.z, p.qwidth2[query], ipr));
        }
        s_rec[i] = rec;
    }
}

// Finalize and publish the wide kernel's staged survivors; out of line, so the unrolled
// scan loop carries one call instead of the refinement and publication code.
template <int W, bool kLut>
__device__ __noinline__ void flush_wide(const ScanParams &p, uint32_t n, uint4 *s_rec, const float *s_cut,
                                        const uint32_t *s_loc, unsigned long long &limit, uint32_t lane) {
    finalize_records<W, kLut>(p, n, s_rec, s_loc, s_cut, lane);
    flush_records(p, p.queue, n, s_rec, s_cut, limit, lane);
}

constexpr int kStageWide = 384;  // wide kernel: flushed when a row block could overflow it

// The Bitwise lower bound of a (vector, pair) from its ip_int (the popcount kernels'
// expression, filter_kernels.cuh:96-112), in one place so that the publication test and
// the staged record see the same value.
__device__ __forceinline__ float lower_bound_of(float fa, float fr, float fe, float gadd, float gerr, float width,
                                                float k1, int ip) {
    const float ex = width * (float)ip;
    return fa + gadd + fr * (ex + k1) - fe * gerr;
}

// ip_int of a row block: at W <= 8 one accumulator chain through the K-steps (the four row
// blocks are independent chains), above that two chains (low and high halves of the words).
template <int WQ, class Spread>
__device__ __forceinline__ v4i32 tile_ip_int(const uint32_t (&xw)[WQ], const v4i32 *bq, const Spread &spread16) {
    v4i32 acc = v4i32{0, 0, 0, 0};
    if constexpr (WQ <= 2) {
#pragma unroll
        for (int j = 0; j < WQ; ++j) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(spread16(xw[j] & 0xFFFFu), bq[2 * j], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(spread16(xw[j] >> 16), bq[2 * j + 1], acc, 0, 0, 0);
        }
    } else {
        v4i32 acc1 = v4i32{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < WQ; ++j) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(spread16(xw[j] & 0xFFFFu), bq[2 * j], acc, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(spread16(xw[j] >> 16), bq[2 * j + 1], acc1, 0, 0, 0);
        }
        acc += acc1;
    }
    return acc;
}

// A tile's operands for the wide kernel's lane (col, quad): code words [WQ quad, WQ quad +
// WQ) of vectors 16 m + col, and the factors of vectors 16 m + 4 quad + r, m = 0..3.
template <int WQ>
struct TileRegs {
    uint32_t xt[4][WQ];
    float4 fa[4], fr[4], fe[4];
};

template <int W>
__device__ __forceinline__ void load_tile(const uint8_t *tile, uint32_t col, uint32_t quad, TileRegs<W / 4> &r) {
    constexpr int WQ = W / 4;
    const float *fac = reinterpret_cast<const float *>(tile + 256u * W);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t v = 16 * m + col;
        r.fa[m] = gload<float4>(fac + 16 * m + 4 * quad);
        r.fr[m] = gload<float4>(fac + 64 + 16 * m + 4 * quad);
        r.fe[m] = gload<float4>(fac + 128 + 16 * m + 4 * quad);
        if constexpr (WQ == 1) {
            r.xt[m][0] = gload<uint32_t>(tile + v * 16 + quad * 4);
        } else {
#pragma unroll
            for (int j = 0; j < WQ; j += 2) {
                const uint32_t w = WQ * quad + j;  // even: the pair lies in one 4-word group
                const uint2 c = gload<uint2>(tile + (size_t)(w >> 2) * 1024 + v * 16 + (w & 3u) * 4);
                r.xt[m][j] = c.x;
                r.xt[m][j + 1] = c.y;
            }
        }
    }
}

// Codes of W = 4, 8, 16, 24, 32 words (P = 128, 256, 512, 768, 1024) on
// v_mfma_i32_16x16x64_i8. Lane-group g = lane / 16 owns code words [g W/4, (g+1) W/4) of
// every vector: K-step s (64 dimensions) takes the 16-bit half s % 2 of word g W/4 + s / 2,
// i.e. dimensions 8 W g + 16 s + e, e = 0..15, and the query operand the same 16 bytes of
// qint, so each lane loads W/8 aligned 8-byte pairs (one word at W = 4) per row block and
// the unit's qint operands (W/2 x 16 bytes) stay in VGPRs. Only the dimension pairing between the two operands
// matters to the sum, so ip_int is exact. The lower bound uses the popcount kernels'
// expression; ip_res is evaluated for survivors when they are published.
// The sixteen code bits of an operand become sixteen int8 0/1 bytes through a 256-entry
// table in LDS (two 8-byte reads per operand): widening them arithmetically took 16 VALU
// instructions per operand and bounded the kernel (10-13% faster at P = 768).
template <int W, int kModeT>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void far_mfma_wide_kernel(const ScanParams p) {
    constexpr bool kLut = kModeT == kPublishLut || kModeT == kLowsLut || kModeT == kDenseLut;
    constexpr int kMode = kModeT == kPublishLut ? kPublish
                          : kModeT == kLowsLut  ? kLows
                          : kModeT == kDenseLut ? kDenseDbg
                                                : kModeT;
    constexpr bool kDense = kMode != kPublish;
    static_assert(W == 4 || W == 8 || (W % 8 == 0 && W >= 16 && W <= 32), "whole words per lane-group");
    static_assert(!kLut || W >= 16, "LUT4 modes for P >= 512");
    constexpr int WQ = W / 4;  // code words per lane-group
    constexpr int S = W / 2;   // K-steps of 64 dimensions
    constexpr uint32_t P = 32u * W;
    constexpr bool kPrefetch = W == 4 || (kMode == kLows && W <= 24);
    // publication test without per-element validity or pair-slot terms: the cutoff of an
    // empty pair slot is -inf and the rows past the cluster's end are masked per tile in
    // SGPRs, so each (vector, pair) costs its bound and one compare
    // (measured: far scan 2.38 -> 2.13 ms at P = 128, config 5; 1.37 -> 1.31 ms at P = 768,
    // config 4)
    constexpr bool kFastPub = kMode == kPublish && !kLut;
    __shared__ uint4 s_rec[kDense ? 1 : kStageWide];
    __shared__ float s_cut[kDense ? 1 : kStageWide];
    __shared__ uint32_t s_loc[kDense ? 1 : kStageWide];
    __shared__ __align__(16) float s_low[kMode == kLows ? 16 * kLowPitch : 4];
    // bits 0..7 of a byte b as eight int8 0/1 values: s_spread[b]
    __shared__ uint2 s_spread[256];
    const uint32_t lane = threadIdx.x, col = lane & 15, quad = lane >> 4;
    for (uint32_t b = lane; b < 256; b += 64) {
        const long v = spread_byte(b);
        s_spread[b] = make_uint2((uint32_t)v, (uint32_t)((unsigned long long)v >> 32));
    }
    __syncthreads();
    const auto spread16_lds = [&](uint32_t h) -> v4i32 {
        const uint2 a = s_spread[h & 255u], b = s_spread[(h >> 8) & 255u];
        return v4i32{(int)a.x, (int)a.y, (int)b.x, (int)b.y};
    };
    const QueueDev q = p.queue;
    // read once: p's address escapes to the out-of-line flush, so p lives in scratch and a
    // read of it inside the tile loop is a scratch load, whose wait also waits for every tile
    // load in flight
    const uint8_t *const tiles = p.tiles;
    const size_t tile_bytes = p.tile_bytes;
    // kLows runs over the vanguard unit set, kPublish over the far units, the dense debug
    // output over either
    const uint32_t set = kMode == kLows ? 0u : kMode == kPublish ? 1u : p.dbg_set;
    const uint32_t U = p.num_units[set];
    const uint32_t ubase = set ? p.num_units[0] : 0u;
    uint32_t range = blockIdx.x % kNumXcd, tries = 0;
    uint32_t staged = 0;
    unsigned long long limit =
        kDense ? 0ull : __hip_atomic_load(q.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
        const uint32_t u = next_far_unit(p.unit_cursor, U, range, tries, lane);
        if (u >= U)
            break;
        // every load of the kernel body through global pointers: p escapes to flush_wide, so
        // pointers read from it are generic, and flat loads would make each LDS wait of the
        // widening also wait for the tile loads in flight
        const uint4 un = gload<uint4>(p.units + ubase + u);  // Unit: cluster, pair_begin, count, tiles
        const uint32_t cluster = uniform(un.x), count = uniform(un.z);
        const uint4 cm = gload<uint4>(p.meta + cluster);  // ClusterMeta: start, n, tile_base
        const uint32_t n = uniform(cm.y), start = uniform(cm.x), tbase = uniform(cm.z);
        const uint32_t t_begin = uniform(un.w) >> 8, t_end = t_begin + (uniform(un.w) & 255u);
        if (n == 0 || t_begin >= t_end)
            continue;
        const bool slot = col < count;
        const uint32_t w0 = slot ? gload<uint32_t>(&p.pairs[uniform(un.y) + col].word0) : 0u;
        const uint32_t query = w0 & 0xFFFFu, probe = w0 >> 16;
        float width = 0.0f, k1 = 0.0f, gadd = 0.0f, gerr = 0.0f, cutoff = -FLT_MAX, delta = 0.0f;
        v4i32 bq[S];
        if (slot) {
            width = gload<float>(p.qwidth + query);
            k1 = gload<float>(p.k1 + query);
            if constexpr (kLut)
                delta = gload<float>(p.lut_margin + query);
            const size_t pi = (size_t)query * p.nprobe + probe;
            gadd = gload<float>(p.pgadd + pi);
            gerr = gload<float>(p.pgerr + pi);
            cutoff = kDense ? FLT_MAX : gload<float>(p.thresholds + query);
            const v4i32 *qb = reinterpret_cast<const v4i32 *>(p.qbytes + (size_t)query * 2 * P + 8 * W * quad);
#pragma unroll
            for (int s = 0; s < S; ++s)
                bq[s] = gload<v4i32>(qb + s);
        } else {
#pragma unroll
            for (int s = 0; s < S; ++s)
                bq[s] = v4i32{0, 0, 0, 0};
        }
        // the tile's code words and factors for all four row blocks go out first (one
        // memory round trip per tile; at P >= 512 two waves per SIMD hold them in 251 VGPRs
        // without spilling, measured 22% faster than three waves loading per row block); then
        // one row block of 16 vectors at a time: its K-steps and its lower bounds. For
        // P = 128 (W = 4, 52 VGPRs a tile), and in the lows pass up to P = 768 (whose bounds
        // need no survivor staging: 250 VGPRs at P = 768, 0.78 -> 0.73 ms at config 4), the
        // next tile's loads are issued before the current tile's MFMAs, so each wave keeps a
        // tile's loads in flight while it computes.
        // The tile loop's body, for tile t: its code words and factors come from cur when
        // they were prefetched, else it loads them.
        const auto tile_pass = [&](const uint32_t t, const TileRegs<WQ> &cur) __attribute__((always_inline)) {
            const uint8_t *tile = tiles + (size_t)(tbase + t) * tile_bytes;
            // (at P >= 512 the loads are written out here: through the TileRegs helper the
            // compiler schedules the wide tiles' code differently, measured 11% slower)
            uint32_t xt[4][WQ];
            float4 fat[4], frt[4], fet[4];
            if constexpr (kPrefetch) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    fat[m] = cur.fa[m];
                    frt[m] = cur.fr[m];
                    fet[m] = cur.fe[m];
#pragma unroll
                    for (int j = 0; j < WQ; ++j)
                        xt[m][j] = cur.xt[m][j];
                }
            } else {
                const float *fac = reinterpret_cast<const float *>(tile + 256u * W);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t v = 16 * m + col;
                    fat[m] = gload<float4>(fac + 16 * m + 4 * quad);
                    frt[m] = gload<float4>(fac + 64 + 16 * m + 4 * quad);
                    fet[m] = gload<float4>(fac + 128 + 16 * m + 4 * quad);
#pragma unroll
                    for (int j = 0; j < WQ; j += 2) {
                        const uint32_t w = WQ * quad + j;  // even: the pair lies in one 4-word group
                        const uint2 c = gload<uint2>(tile + (size_t)(w >> 2) * 1024 + v * 16 + (w & 3u) * 4);
                        xt[m][j] = c.x;
                        xt[m][j + 1] = c.y;
                    }
                }
            }
            if constexpr (kFastPub) {
                const float cut_eff = slot ? cutoff : -__builtin_inff();
                // rows of the tile past the cluster's end: lane-group quad holds rows
                // 16 m + 4 quad + r, valid while that is below n - 64 t
                const uint32_t n_rem = n - t * kTileVectors;  // >= 1
                v4i32 accs[4];
                unsigned long long masks[4][4], any = 0;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    accs[m] = tile_ip_int<WQ>(xt[m], bq, spread16_lds);
                    const float4 fa = fat[m], fr = frt[m], fe = fet[m];
                    const float fav[4] = {fa.x, fa.y, fa.z, fa.w};
                    const float frv[4] = {fr.x, fr.y, fr.z, fr.w};
                    const float fev[4] = {fe.x, fe.y, fe.z, fe.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float low = lower_bound_of(fav[r], frv[r], fev[r], gadd, gerr, width, k1, accs[m][r]);
                        unsigned long long mk = __ballot(low < cut_eff);
                        if (n_rem < kTileVectors) {
                            const int rows = (int)n_rem - 16 * m - r;  // valid lane-groups: 4 quad < rows
                            const int groups = rows <= 0 ? 0 : min(4, (rows + 3) >> 2);
                            mk &= groups >= 4 ? ~0ull : (1ull << (16 * groups)) - 1ull;
                        }
                        masks[m][r] = mk;
                        any |= mk;
                    }
                }
                if (any) {
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const uint32_t o = 16 * m + 4 * quad;
                        const float4 fa = fat[m], fr = frt[m], fe = fet[m];
                        const float fav[4] = {fa.x, fa.y, fa.z, fa.w};
                        const float frv[4] = {fr.x, fr.y, fr.z, fr.w};
                        const float fev[4] = {fe.x, fe.y, fe.z, fe.w};
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const unsigned long long mk = masks[m][r];
                            if (mk == 0)
                                continue;
                            if (staged + 64 > (uint32_t)kStageWide) {
                                flush_wide<W, kLut>(p, staged, s_rec, s_cut, s_loc, limit, lane);
                                staged = 0;
                            }
                            if ((mk >> lane) & 1ull) {
                                const int ip = accs[m][r];
                                const float low = lower_bound_of(fav[r], frv[r], fev[r], gadd, gerr, width, k1, ip);
                                const uint32_t k = staged + lane_rank(mk);
                                s_rec[k] = make_uint4(w0, start + t * kTileVectors + o + r, (uint32_t)ip,
                                                      __float_as_uint(low));
                                s_cut[k] = cutoff;
                                s_loc[k] = (tbase + t) * kTileVectors + o + r;
                            }
                            staged += (uint32_t)__popcll(mk);
                        }
                    }
                }
                return;
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t (&xw)[WQ] = xt[m];
                // two accumulator chains (low and high halves of the words)
                v4i32 acc = v4i32{0, 0, 0, 0}, acc1 = v4i32{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < WQ; ++j) {
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(spread16_lds(xw[j] & 0xFFFFu), bq[2 * j], acc, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(spread16_lds(xw[j] >> 16), bq[2 * j + 1], acc1, 0, 0, 0);
                }
                acc += acc1;
                const uint32_t o = 16 * m + 4 * quad;
                const float4 fa = fat[m], fr = frt[m], fe = fet[m];
                const float fav[4] = {fa.x, fa.y, fa.z, fa.w};
                const float frv[4] = {fr.x, fr.y, fr.z, fr.w};
                const float fev[4] = {fe.x, fe.y, fe.z, fe.w};
                if constexpr (kMode == kLows) {
                    // rows o + r of the pair's tile-padded slice (lanes past the cluster's
                    // end stage values nobody reads)
                    if (slot) {
                        float lw[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float ex = width * (float)acc[r];
                            lw[r] = fav[r] + gadd + frv[r] * (ex + k1) - fev[r] * gerr;
                            // LUT4: a lower bound of the LUT4 bound
                            if constexpr (kLut)
                                lw[r] -= lut_slack(delta, fav[r], frv[r], fev[r], gadd, gerr, ex, k1);
                        }
                        lows_put(s_low, col, o, lw);
                    }
                    continue;
                }
                if constexpr (!kDense) {
                    // a row block stages at most 4 x 64 records
                    if (staged + 4 * 64 > (uint32_t)kStageWide) {
                        flush_wide<W, kLut>(p, staged, s_rec, s_cut, s_loc, limit, lane);
                        staged = 0;
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t local = t * kTileVectors + o + r;
                    const bool valid = slot && local < n;
                    const int ip = acc[r];
                    const float ex = width * (float)ip;
                    const float low = fav[r] + gadd + frv[r] * (ex + k1) - fev[r] * gerr;
                    if constexpr (kDense) {
                        if (valid) {
                            const size_t od = ((size_t)query * p.nprobe + probe) * p.dbg_stride + local;
                            if constexpr (kLut) {
                                // the LUT4 estimate (its FP32 bits) and bound, as finalize_records
                                // evaluates them for survivors
                                uint32_t x[W];
#pragma unroll
                                for (int g = 0; g < W / 4; ++g) {
                                    const uint4 c =
                                        *reinterpret_cast<const uint4 *>(tile + (size_t)g * 1024 + (o + r) * 16);
                                    x[4 * g] = c.x;
                                    x[4 * g + 1] = c.y;
                                    x[4 * g + 2] = c.z;
                                    x[4 * g + 3] = c.w;
                                }
                                const float exl = lut4_ip<W>(x, p.lut + (size_t)query * 2 * P, W);
                                p.dbg_ip[od] = (int32_t)__float_as_uint(exl);
                                p.dbg_ip2[od] = 0;
                                p.dbg_low[od] = fav[r] + gadd + frv[r] * (exl + k1) - fev[r] * gerr;
                            } else {
                                p.dbg_ip[od] = ip;
                                p.dbg_ip2[od] = tile_ip_res<W>(tile, o + r, p.qplanes + ((size_t)query * 16 + 8) * W);
                                p.dbg_low[od] = low;
                            }
                        }
                    } else {
                        // LUT4: every vector whose LUT4 bound can lie below the cutoff;
                        // finalize_records evaluates that bound and drops the others
                        const bool survive =
                            valid && (kLut ? low - lut_slack(delta, fav[r], frv[r], fev[r], gadd, gerr, ex, k1)
                                            : low) < cutoff;
                        const unsigned long long mask = __ballot(survive);
                        if (mask == 0)
                            continue;
                        const uint32_t cnt = (uint32_t)__popcll(mask);
                        if (survive) {
                            const uint32_t k = staged + lane_rank(mask);
                            s_rec[k] = make_uint4(w0, start + local, (uint32_t)ip, __float_as_uint(low));
                            s_cut[k] = cutoff;
                            s_loc[k] = (tbase + t) * kTileVectors + o + r;
                        }
                        staged += cnt;
                    }
                }
            }
            if constexpr (kMode == kLows)
                lows_flush(p, s_low, lane, w0, count, t, n);
        };
        const auto tile_at = [&](uint32_t t) { return tiles + (size_t)(tbase + t) * tile_bytes; };
        if constexpr (kPrefetch && W <= 16) {
            // two register sets in turn, so the loads of the tile after next are issued before
            // the wait for the next tile's: while a wave waits, two tiles' loads are in flight
            // (copying one prefetched set into the other made it wait for all of them first)
            TileRegs<WQ> ra, rb;
            load_tile<W>(tile_at(t_begin), col, quad, ra);
            for (uint32_t t = t_begin; t < t_end; t += 2) {
                // past the last tile its successor is that tile again (a cached reload, no
                // branch); the scheduling barriers keep the loads ahead of the other set's waits
                load_tile<W>(tile_at(t + 1 < t_end ? t + 1 : t), col, quad, rb);
                __builtin_amdgcn_sched_barrier(0);
                tile_pass(t, ra);
                if (t + 1 == t_end)
                    break;
                load_tile<W>(tile_at(t + 2 < t_end ? t + 2 : t + 1), col, quad, ra);
                __builtin_amdgcn_sched_barrier(0);
                tile_pass(t + 1, rb);
            }
        } else if constexpr (kPrefetch) {
            // P = 768 (the lows pass): two sets in turn would spill; the next tile's set is
            // copied into the current one instead
            TileRegs<WQ> cur, nxt;
            load_tile<W>(tile_at(t_begin), col, quad, cur);
            for (uint32_t t = t_begin; t < t_end; ++t) {
                load_tile<W>(tile_at(t + 1 < t_end ? t + 1 : t), col, quad, nxt);
                tile_pass(t, cur);
                cur = nxt;
            }
        } else {
            const TileRegs<WQ> none{};
            for (uint32_t t = t_begin; t < t_end; ++t)
                tile_pass(t, none);
        }
    }
    if constexpr (!kDense) {
        if (staged)
            flush_wide<W, kLut>(p, staged, s_rec, s_cut, s_loc, limit, lane);
    }
}

template <class F>
uint32_t resident_grid_mfma(F kernel) {
    static std::mutex mu;
    static std::map<const void *, uint32_t> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(reinterpret_cast<const void *>(kernel));
    if (it != cache.end())
        return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 ||
        cus <= 0) {
        per_cu = 8;
        cus = 256;
    }
    const uint32_t grid = (uint32_t)(per_cu * cus);
    cache.emplace(reinterpret_cast<const void *>(kernel), grid);
    return grid;
}

template <int W, int kMode>
void launch_w(const ScanParams &p, hipStream_t s) {
    if constexpr (W == 2 || W == 6) {
        static_assert(kMode != kPublishLut && kMode != kLowsLut && kMode != kDenseLut, "LUT4 on the wide kernel only");
        auto *k = far_mfma_kernel<W, kMode>;
        k<<<resident_grid_mfma(k), 64, 0, s>>>(p);
    } else {
        auto *k = far_mfma_wide_kernel<W, kMode>;
        k<<<resident_grid_mfma(k), 64, 0, s>>>(p);
    }
}

template <int W>
void launch_mode(const ScanParams &p, int mode, hipStream_t s) {
    if constexpr (W >= 16) {
        if (mode == kLowsLut)
            return launch_w<W, kLowsLut>(p, s);
        if (mode == kPublishLut)
            return launch_w<W, kPublishLut>(p, s);
        if (mode == kDenseLut)
            return launch_w<W, kDenseLut>(p, s);
    }
    if (mode == kLows)
        launch_w<W, kLows>(p, s);
    else if (mode == kDenseDbg)
        launch_w<W, kDenseDbg>(p, s);
    else
        launch_w<W, kPublish>(p, s);
}

}  // namespace

bool far_mfma_supported(uint32_t W) {
    return W == 2 || W == 4 || W == 6 || W == 8 || W == 16 || W == 24 || W == 32;
}

bool far_mfma_lut_supported(uint32_t W) { return W == 16 || W == 24 || W == 32; }

void launch_far_mfma(const ScanParams &p, uint32_t W, bool dense, hipStream_t s) {
    launch_mfma_units(p, W, dense ? (p.lut ? kDenseLut : kDenseDbg) : p.lut ? kPublishLut : kPublish, s);
}

void launch_vanguard_lows(const ScanParams &p, uint32_t W, hipStream_t s) {
    launch_mfma_units(p, W, p.lut ? kLowsLut : kLows, s);
}

void launch_mfma_units(const ScanParams &p, uint32_t W, int mode, hipStream_t s) {
    switch (W) {
    case 2: launch_mode<2>(p, mode, s); break;
    case 4: launch_mode<4>(p, mode, s); break;
    case 6: launch_mode<6>(p, mode, s); break;
    case 8: launch_mode<8>(p, mode, s); break;
    case 16: launch_mode<16>(p, mode, s); break;
    case 24: launch_mode<24>(p, mode, s); break;
    case 32: launch_mode<32>(p, mode, s); break;
    default: break;
    }
}

}  // namespace cora
