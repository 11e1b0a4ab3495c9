// Staged vanguard pass: the work of the fused per-query pass (vanguard.hip) split so that
// the refinement gathers, nearly all of its bytes, are issued from a grid-wide kernel with
// many records in flight per CU instead of a few queries' latency chains.
//
// The reference runs the vanguard pairs as a seed kernel that publishes the best
// max(topk, 20) lower bounds of each pair (filter_kernels.cuh:308-468) and a recovery kernel
// that later publishes the pair's other vectors with low < threshold
// (filter_kernels.cuh:470-582), the threshold falling meanwhile as the CPU consumer refines.
// Here, with every vanguard lower bound already written by the matrix-core lows pass
// (ScanParams::van_lows, [query][pair][van_stride]):
//
//   1. seed select (one workgroup per query): the lows pass also wrote the minimum of every
//      group of 4 consecutive bounds (ScanParams::van_mins). One read of the query's group
//      minima gives 512 sub-stream minima (two per thread); the `seeds`-th smallest of them is
//      the cut, and the bounds of the groups whose minimum lies at or below it (one more read)
//      that are themselves at or below it are the seeds. At least `seeds` bounds lie at or
//      below the cut, one per sub-stream, and with the groups spread over the sub-streams by
//      position, not by value, not many more;
//   2. refinement (grid-wide): each seed's refinement record (ex-code, sign code,
//      ex-factors) is read and its refined distance evaluated with the CPU consumer's formula
//      (cpu_refinement.cpp:183-192), with a bound on the rounding difference to the CPU's own
//      evaluation;
//   3. threshold and list (per query): the seeds' topk best refined distances back the
//      threshold max(d_k + e, l) + 1 ulp (d_k the k-th distance, e the largest rounding
//      bound and l the largest lower bound among those k; lowered only); every other vector
//      whose bound is below it joins the list (the groups whose minimum lies below it, then
//      their bounds);
//   4. refinement of the list (as 2);
//   5. merge and publication (per query): the topk best of all refined vectors lower the
//      threshold again by the same rule; every refined vector whose distance is within its
//      rounding bound of that threshold is published (the refined pre-filter rule), the
//      others are counted as dropped, and the query's threshold is lowered (atomic minimum)
//      for the far pass and the CPU consumer.
//
// Every vector whose bound is below the final threshold is refined (it lies below the
// threshold of stage 3, which only falls), and what is published and the final threshold
// follow the fused pass's rules, so the guarantees of that pass carry over. A query whose
// seeds or list do not fit their region is marked and left to the fused per-query kernel,
// which runs afterwards over exactly those queries.
#include <float.h>

#include <algorithm>
#include <map>
#include <mutex>

#include "device_common.h"

namespace cora {
namespace {

constexpr int kVsThreads = 256;
constexpr int kVsWaves = kVsThreads / 64;
constexpr int kVsRegs = 32;                            // bounds per thread per chunk
constexpr uint32_t kVsChunk = kVsRegs * kVsThreads;    // 8,192
constexpr uint32_t kVsCand = 2048;    // candidate keys the threshold and merge stages hold in LDS
constexpr uint32_t kVsRankMax = 512;  // up to this many candidates: ranks by counting, else radix

// Inclusive prefix sum over the workgroup (thread order); red holds kVsWaves words.
__device__ __forceinline__ uint32_t vs_block_scan(uint32_t v, uint32_t *red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(v, o);
        if (lane >= (uint32_t)o)
            v += y;
    }
    if (lane == 63)
        red[wave] = v;
    __syncthreads();
    uint32_t add = 0;
    for (uint32_t w = 0; w < wave; ++w)
        add += red[w];
    __syncthreads();
    return v + add;
}

// Workgroup maximum / sum of a 32-bit word (red: kVsWaves words); every thread gets it.
__device__ __forceinline__ uint32_t vs_block_max(uint32_t v, uint32_t *red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v = max(v, (uint32_t)__shfl_xor(v, o));
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    uint32_t m = 0;
#pragma unroll
    for (int w = 0; w < kVsWaves; ++w)
        m = max(m, red[w]);
    __syncthreads();
    return m;
}

__device__ __forceinline__ uint32_t vs_block_sum(uint32_t v, uint32_t *red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o);
    if (lane == 0)
        red[wave] = v;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kVsWaves; ++w)
        t += red[w];
    __syncthreads();
    return t;
}

// The k-th smallest (1 <= k <= n) of n distinct 64-bit keys key_at(i), i < n, 8 bits at a
// time from the top; hist holds 256 words.
template <class F>
__device__ unsigned long long block_kth_u64(F key_at, uint32_t n, uint32_t k, uint32_t *hist, uint32_t *red,
                                            uint32_t *sc) {
    const uint32_t tid = threadIdx.x;
    unsigned long long prefix = 0, pmask = 0;
    for (int shift = 56; shift >= 0; shift -= 8) {
        hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kVsThreads) {
            const unsigned long long v = key_at(i);
            if ((v & pmask) == prefix)
                atomicAdd(&hist[(uint32_t)(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        const uint32_t h = hist[tid];
        const uint32_t incl = vs_block_scan(h, red);
        if (incl >= k && incl - h < k) {
            sc[0] = tid;
            sc[1] = k - (incl - h);
        }
        __syncthreads();
        prefix |= (unsigned long long)sc[0] << shift;
        pmask |= 255ull << shift;
        k = sc[1];
        __syncthreads();
    }
    return prefix;
}

// Wave-aggregated slot in a block-local counter: the lanes with take get consecutive slots.
__device__ __forceinline__ uint32_t wave_slot(bool take, uint32_t *counter) {
    const unsigned long long m = __ballot(take);
    uint32_t base = 0;
    if (m && (threadIdx.x & 63) == 0)
        base = atomicAdd(counter, (uint32_t)__popcll(m));
    base = __builtin_amdgcn_readfirstlane(base);
    return base + lane_rank(m);
}

// Mark a query for the one-pass kernel (thread 0).
__device__ void overflow_query(const VsArgs &vs, uint32_t q) {
    const unsigned long long o = atomicAdd(&vs.ctr[kVsCtrOverflow], 1ull);
    vs.overflow[o] = q;
    vs.qs[q].flags = kVsOverflow;
}

// ---- a query's vanguard lower bounds ----
// Concatenated over its pairs (pair j's n_j bounds from row j of van_lows), and likewise the
// minima of its groups of 4 consecutive vectors (pair j's ceil(n_j / 4) from row j of
// van_mins). Either is read in chunks of kVsChunk elements: thread t holds element
// c * kVsChunk + r * 256 + t of chunk c as an order key (0xFFFFFFFF for a value at or above
// thr_in and for padding).
struct QueryRows {
    const float *rows;      // the query's rows
    const uint32_t *s_off;  // LDS: first element of each pair, s_off[V] = total
    uint32_t stride, total;
};

// Slot j * stride + i - s_off[j] of element i (i < total) for a thread walking its elements
// in increasing order: the pair j and its element range [lo, hi) stay in registers, and the
// LDS is read only when the walk enters the next pair.
struct PairWalk {
    uint32_t j, lo, hi;
    __device__ explicit PairWalk(const QueryRows &qr) : j(0), lo(0), hi(qr.s_off[1]) {}
    __device__ __forceinline__ uint32_t slot(const QueryRows &qr, uint32_t i) {
        while (i >= hi) {
            ++j;
            lo = hi;
            hi = qr.s_off[j + 1];
        }
        return j * qr.stride + (i - lo);
    }
};

// The thread's keys of chunk c: every load is issued (global loads, counted by vmcnt only, so
// the LDS reads of the pair walk do not wait for them) before the first is used.
__device__ __forceinline__ void load_keys(const QueryRows &qr, uint32_t c, float thr_in, uint32_t (&key)[kVsRegs]) {
    float l[kVsRegs];
    PairWalk w(qr);
#pragma unroll
    for (int r = 0; r < kVsRegs; ++r) {
        const uint32_t i = c * kVsChunk + r * kVsThreads + threadIdx.x;
        const uint32_t slot = i < qr.total ? w.slot(qr, i) : 0u;  // slot 0 is in bounds
        l[r] = gload<float>(qr.rows + slot);
    }
#pragma unroll
    for (int r = 0; r < kVsRegs; ++r) {
        const bool ok = c * kVsChunk + r * kVsThreads + threadIdx.x < qr.total && l[r] < thr_in;
        key[r] = ok ? order_key(l[r]) : 0xFFFFFFFFu;
    }
}

__device__ __forceinline__ uint32_t num_chunks(const QueryRows &qr) {
    return max(1u, (qr.total + kVsChunk - 1) / kVsChunk);
}

// Pair sizes of query q into s_n, and the running offsets of its elements into s_off and of
// its groups of 4 into s_goff (s_off[V], s_goff[V]: the totals).
__device__ void load_pairs(const ScanParams &p, const VanguardArgs &va, uint32_t q, uint32_t *s_n, uint32_t *s_off,
                           uint32_t *s_goff) {
    const uint32_t V = va.depth, tid = threadIdx.x;
    if (tid < V)
        s_n[tid] = p.meta[va.probe_idx[(size_t)q * p.nprobe + tid]].n;
    __syncthreads();
    if (tid == 0) {
        uint32_t o = 0, g = 0;
        for (uint32_t j = 0; j < V; ++j) {
            s_off[j] = o;
            s_goff[j] = g;
            o += s_n[j];
            g += (s_n[j] + 3) / 4;
        }
        s_off[V] = o;
        s_goff[V] = g;
    }
    __syncthreads();
}

// Exclusive prefix of per-thread counts over the workgroup, and their total (red: kVsWaves
// words; ends with a barrier, so red may be reused at once).
__device__ __forceinline__ uint32_t block_offset(uint32_t cnt, uint32_t *red, uint32_t &total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t v = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(v, o);
        if (lane >= (uint32_t)o)
            v += y;
    }
    if (lane == 63)
        red[wave] = v;
    __syncthreads();
    uint32_t before = 0, t = 0;
#pragma unroll
    for (uint32_t w = 0; w < (uint32_t)kVsWaves; ++w) {
        before += w < wave ? red[w] : 0u;
        t += red[w];
    }
    __syncthreads();
    total = t;
    return before + v - cnt;
}

// Every bound below thr_in of the groups whose minimum's key satisfies pick. The groups are
// listed in s_sel first (up to kVsSel), then their bounds are read (one round trip per eight
// groups a thread) and handed to f in rounds of kVsRegs per thread: f(key[], slot[]) with
// slot = j * van_stride + v and key 0xFFFFFFFF for a bound at or above thr_in, past its
// cluster's end or padding. With more than kVsSel groups, every bound of the query is handed
// over instead. Every thread of the workgroup calls it and sees the same number of rounds, so
// f may compact by workgroup.
constexpr uint32_t kVsSel = 2048;
constexpr int kVsSelRegs = kVsRegs / 4;  // groups per thread and round

template <class Pick, class F>
__device__ __forceinline__ void for_bounds_of_groups(const QueryRows &qg, const QueryRows &qb, const uint32_t *s_n, float thr_in,
                                     Pick pick, F f, uint32_t *s_sel, uint32_t *red) {
    const uint32_t tid = threadIdx.x;
    uint32_t key[kVsRegs], slot[kVsRegs];
    const uint32_t chunks = num_chunks(qg);
    uint32_t nsel = 0;
    for (uint32_t c = 0; c < chunks; ++c) {
        load_keys(qg, c, thr_in, key);
        uint32_t cnt = 0;
#pragma unroll
        for (int r = 0; r < kVsRegs; ++r)
            cnt += key[r] != 0xFFFFFFFFu && pick(key[r]) ? 1u : 0u;
        uint32_t total = 0;
        uint32_t o = nsel + block_offset(cnt, red, total);
        PairWalk w(qg);
#pragma unroll
        for (int r = 0; r < kVsRegs; ++r) {
            const uint32_t i = c * kVsChunk + r * kVsThreads + tid;
            if (key[r] != 0xFFFFFFFFu && pick(key[r])) {
                const uint32_t gs = w.slot(qg, i);
                if (o < kVsSel)
                    s_sel[o] = gs;
                ++o;
            }
        }
        nsel += total;
    }
    __syncthreads();
    if (nsel <= kVsSel) {
        for (uint32_t k0 = 0; k0 < nsel; k0 += kVsSelRegs * kVsThreads) {
            // the selected groups' bounds, all loads issued first
            float4 b[kVsSelRegs];
            uint32_t gs[kVsSelRegs];
#pragma unroll
            for (int k = 0; k < kVsSelRegs; ++k) {
                const uint32_t i = k0 + k * kVsThreads + tid;
                gs[k] = i < nsel ? s_sel[i] : 0u;
                b[k] = gload<float4>(qb.rows + 4 * (size_t)gs[k]);
            }
#pragma unroll
            for (int k = 0; k < kVsSelRegs; ++k) {
                const uint32_t i = k0 + k * kVsThreads + tid;
                const uint32_t j = gs[k] / qg.stride, v0 = 4 * (gs[k] - j * qg.stride);
                const float lv[4] = {b[k].x, b[k].y, b[k].z, b[k].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = i < nsel && v0 + e < s_n[j] && lv[e] < thr_in;
                    key[4 * k + e] = ok ? order_key(lv[e]) : 0xFFFFFFFFu;
                    slot[4 * k + e] = 4 * gs[k] + e;
                }
            }
            f(key, slot);
        }
    } else {
        // too many groups: every bound
        const uint32_t bchunks = num_chunks(qb);
        for (uint32_t c = 0; c < bchunks; ++c) {
            load_keys(qb, c, thr_in, key);
            PairWalk w(qb);
#pragma unroll
            for (int r = 0; r < kVsRegs; ++r) {
                const uint32_t i = c * kVsChunk + r * kVsThreads + tid;
                slot[r] = key[r] != 0xFFFFFFFFu ? w.slot(qb, i) : 0u;
            }
            f(key, slot);
        }
    }
}

// A visitor of for_bounds_of_groups that appends the slots whose key satisfies take to
// out[0, cap) (workgroup compaction, no atomics); *n counts them all, also beyond cap.
template <class Take>
struct Compactor {
    Take take;
    uint32_t *out, cap, *red, *n;
    __device__ __forceinline__ void operator()(const uint32_t (&key)[kVsRegs], const uint32_t (&slot)[kVsRegs]) const {
        uint32_t cnt = 0;
#pragma unroll
        for (int r = 0; r < kVsRegs; ++r)
            cnt += take(key[r]) ? 1u : 0u;
        uint32_t total = 0;
        uint32_t o = *n + block_offset(cnt, red, total);
#pragma unroll
        for (int r = 0; r < kVsRegs; ++r) {
            if (take(key[r])) {
                if (o < cap)
                    out[o] = slot[r];
                ++o;
            }
        }
        *n += total;
    }
};

// Sub-stream minima a thread keeps in the seed select (kVsSub x 256 in all).
constexpr int kVsSub = 16;

// The k-th smallest (1 <= k <= kVsSub x 256) of the workgroup's keys (kVsSub per thread), bit by
// bit from the top: bit b of the answer is 0 when at least k keys lie at or below the answer's
// higher bits followed by b ones. Each step counts by wave ballots and adds the four waves'
// counts through red2 (2 x kVsWaves words, alternating, so one barrier a step suffices).
__device__ __forceinline__ uint32_t block_kth_sub(const uint32_t (&keys)[kVsSub], uint32_t k, uint32_t *red2) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t res = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t t = res | ((1u << bit) - 1u);
        uint32_t n = 0;
#pragma unroll
        for (int i = 0; i < kVsSub; ++i)
            n += (uint32_t)__popcll(__ballot(keys[i] <= t));
        uint32_t *r = red2 + (bit & 1) * kVsWaves;
        if (lane == 0)
            r[wave] = n;
        __syncthreads();
        uint32_t all = 0;
#pragma unroll
        for (int w = 0; w < kVsWaves; ++w)
            all += r[w];
        if (all < k)
            res |= 1u << bit;
    }
    __syncthreads();
    return res;
}

// ---- 1. seed select ----
// The seeds are the bounds below thr_in in the groups of 4 whose minimum's key is at most
// cut1, the `seeds`-th smallest (at most 2,048) of 4,096 sub-stream minima of the query's
// group minima (kVsSub per thread: its elements r * 256 + t with r = s mod kVsSub, s = 0 ..
// kVsSub - 1; with at most 4,096 groups each sub-stream holds one, and cut1 is the exact
// seeds-th smallest group minimum). At least `seeds` bounds lie at or below cut1, one per
// sub-stream, and with the groups spread over the sub-streams by position, not by value, not
// many more. With fewer sub-streams holding a bound below thr_in, every bound below thr_in is a
// seed.
__global__ __launch_bounds__(kVsThreads) void vs_seed_kernel(const ScanParams p, const VanguardArgs va,
                                                             const VsArgs vs) {
    __shared__ uint32_t s_n[kVanguardMaxPairs], s_off[kVanguardMaxPairs + 1], s_goff[kVanguardMaxPairs + 1];
    __shared__ uint32_t s_sel[kVsSel];
    __shared__ uint32_t red[kVsWaves], s_red2[2 * kVsWaves];
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    if (q >= va.nq)
        return;
    load_pairs(p, va, q, s_n, s_off, s_goff);
    const float thr_in = p.thresholds[q];
    const uint32_t V = va.depth, gstride = p.van_stride / 4;
    const QueryRows qb{p.van_lows + (size_t)q * V * p.van_stride, s_off, p.van_stride, s_off[V]};
    const QueryRows qg{p.van_mins + (size_t)q * V * gstride, s_goff, gstride, s_goff[V]};
    uint32_t key[kVsRegs], mn[kVsSub];
#pragma unroll
    for (int i = 0; i < kVsSub; ++i)
        mn[i] = 0xFFFFFFFFu;
    const uint32_t chunks = num_chunks(qg);
    for (uint32_t c = 0; c < chunks; ++c) {
        load_keys(qg, c, thr_in, key);
#pragma unroll
        for (int r = 0; r < kVsRegs; ++r)
            mn[r % kVsSub] = min(mn[r % kVsSub], key[r]);
    }
    // 0xFFFFFFFF (fewer valid minima than `seeds`) becomes 0xFFFFFFFE: every bound below
    // thr_in, the invalid keys left out
    const uint32_t want = min(vs.seeds, (uint32_t)kVsSub * kVsThreads);
    const uint32_t cut1 = min(block_kth_sub(mn, want, s_red2), 0xFFFFFFFEu);
    uint32_t nseed = 0;
    uint32_t *seed_pos = vs.seed_pos + (size_t)q * vs.seed_cap;
    auto is_seed = [cut1](uint32_t k) { return k <= cut1; };
    for_bounds_of_groups(qg, qb, s_n, thr_in, is_seed,
                         Compactor<decltype(is_seed)>{is_seed, seed_pos, vs.seed_cap, red, &nseed}, s_sel, red);
    if (tid == 0) {
        if (nseed > vs.seed_cap) {
            overflow_query(vs, q);
        } else {
            VsQuery st{};
            st.seed_n = nseed;
            st.cut1 = cut1;
            st.thr_in = thr_in;
            st.thr = thr_in;
            st.dk_key = 0xFFFFFFFFu;
            vs.qs[q] = st;
            atomicAdd(&vs.spread[(q % kVsSpread) * kVsSpreadWords + kVsStSeeds], (unsigned long long)nseed);
        }
    }
}

// ---- 2. and 4. refinement ----
// L lanes per entry (L = min(4, G), G = W / 2 groups of 64 dimensions): lane sub reads the
// sign-code words [sub W/L, (sub + 1) W/L) and the ex-code groups sub, sub + L, ... of the
// entry's refinement record (8-byte loads), all before any arithmetic; q' and the Bq=8 and
// residual planes are read from LDS. A chunk of 256 / L entries is one round of the
// workgroup.
template <int W>
struct VsShape {
    static constexpr int kGroups = W / 2;  // 64-dimension groups
    static constexpr int kLanes = kGroups >= 4 ? 4 : kGroups;
    static constexpr int kGrp = kGroups / kLanes;  // groups per lane
    static constexpr uint32_t kChunk = kVsThreads / kLanes;
    static_assert(kGroups % kLanes == 0, "lane split");
};

template <int W, bool kLut>
__global__ __launch_bounds__(kVsThreads) __attribute__((amdgpu_waves_per_eu(W >= 32 ? 3 : 4))) void vs_refine_kernel(const ScanParams p, const VanguardArgs va,
                                                               const VsArgs vs, uint32_t stage) {
    using S = VsShape<W>;
    constexpr int L = S::kLanes, kG = S::kGrp, kW = 2 * S::kGrp;  // groups and sign-code words per lane
    constexpr uint32_t P = 32 * W, E = S::kChunk;
    __shared__ __align__(16) float s_q[P];
    __shared__ uint32_t s_planes[2 * kBq * W];
    __shared__ uint32_t s_lut[kLut ? 2 * P : 1];  // LUT4: the query's FP16 nibble table
    __shared__ uint32_t s_start[kVanguardMaxPairs], s_tbase[kVanguardMaxPairs];
    __shared__ float s_gadd[kVanguardMaxPairs], s_gerr[kVanguardMaxPairs];
    __shared__ uint32_t s_red[kVsWaves];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t sub = tid % L, el = tid / L;
    constexpr bool lut = kLut;
    const uint32_t cap = stage ? vs.list_cap : vs.seed_cap;
    const uint32_t *pos_r = stage ? vs.list_pos : vs.seed_pos;
    float2 *rd_r = stage ? vs.list_rd : vs.seed_rd;
    float2 *aux_r = stage ? vs.list_aux : vs.seed_aux;
    const uint32_t V = va.depth, stride = p.van_stride;
    // a contiguous range of (query, chunk) slots per workgroup, cpq chunk slots per query, the
    // queries taken in the order of their nearest cluster (va.order); workgroup b runs on XCD
    // b % 8, and each XCD takes an eighth of that order, so an XCD's workgroups refine vectors
    // of nearby clusters at the same time
    const uint32_t cpq = (cap + E - 1) / E;
    const uint64_t nslots = (uint64_t)va.nq * cpq;
    const uint64_t per = (nslots + gridDim.x - 1) / gridDim.x;
    const uint32_t range =
        gridDim.x % kNumXcd == 0 ? (blockIdx.x % kNumXcd) * (gridDim.x / kNumXcd) + blockIdx.x / kNumXcd : blockIdx.x;
    const uint64_t v_begin = (uint64_t)range * per, v_end = min(nslots, v_begin + per);
    for (uint64_t v = v_begin; v < v_end;) {
        const uint32_t qs = (uint32_t)(v / cpq), c0 = (uint32_t)(v % cpq);
        const uint32_t q = va.order ? va.order[qs] : qs;
        const uint64_t q_end = (uint64_t)(qs + 1) * cpq;
        const VsQuery st = vs.qs[q];
        const uint32_t n = (st.flags & kVsOverflow) ? 0u : stage ? st.list_n : st.seed_n;
        const uint32_t c1 = (uint32_t)min<uint64_t>((n + E - 1) / E, min(q_end, v_end) - (uint64_t)qs * cpq);
        v = q_end;
        if (c0 >= c1)
            continue;  // nothing of this query in the range (every thread reads the same)
        // the query's q', Bq=8 and residual planes, pair constants and scalars, once every
        // wave is done with the previous query's
        __syncthreads();
        float l1p = 0.0f;
        for (uint32_t i = tid; i < P; i += kVsThreads) {
            const float x = p.qrot[(size_t)q * P + i];
            s_q[i] = x;
            l1p += fabsf(x);
        }
        if constexpr (lut)
            for (uint32_t i = tid; i < 2 * P; i += kVsThreads)
                s_lut[i] = p.lut[(size_t)q * 2 * P + i];
        else
            for (uint32_t i = tid; i < 2 * kBq * W; i += kVsThreads)
                s_planes[i] = p.qplanes[(size_t)q * 2 * kBq * W + i];
        if (tid < V) {
            const size_t pi = (size_t)q * p.nprobe + tid;
            const ClusterMeta cm = p.meta[va.probe_idx[pi]];
            s_start[tid] = cm.start;
            s_tbase[tid] = cm.tile_base;
            s_gadd[tid] = p.pgadd[pi];
            s_gerr[tid] = p.pgerr[pi];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            l1p += __shfl_xor(l1p, o);
        if (lane == 0)
            s_red[wave] = __float_as_uint(l1p);
        __syncthreads();
        float l1q = 0.0f;
#pragma unroll
        for (int w = 0; w < kVsWaves; ++w)
            l1q += __uint_as_float(s_red[w]);
        const float width = p.qwidth[q], width2 = p.qwidth2[q], kbq = p.kb[q], k1 = p.k1[q];
        for (uint32_t c = c0; c < c1; ++c) {
            const uint32_t idx = c * E + el;
            const bool have = idx < n;
            const size_t e = (size_t)q * cap + idx;
            uint2 grp[kG][7];
            uint32_t xw[kW];
            float fa = 0.0f, fr = 0.0f, low = 0.0f, sfa = 0.0f, sfr = 0.0f, sfe = 0.0f;
            uint32_t j = 0;
            if (have) {
                const uint32_t pos = pos_r[e];
                j = pos / stride;
                const size_t gid = (size_t)s_start[j] + (pos - j * stride);
                const uint8_t *rec = p.ex_rec + gid * p.ex_stride;
                // sign-code words sub kW .. sub kW + kW - 1, then the groups' ex-code words
                const uint2 *wp = reinterpret_cast<const uint2 *>(rec + ex_record_sign_word(P, sub * kW));
#pragma unroll
                for (int i = 0; i < kW / 2; ++i) {
                    const uint2 x = gload<uint2>(wp + i);
                    xw[2 * i] = x.x;
                    xw[2 * i + 1] = x.y;
                }
#pragma unroll
                for (int gi = 0; gi < kG; ++gi) {
                    const uint2 *gp = reinterpret_cast<const uint2 *>(rec + ex_record_group_word(P, sub + L * gi, 0));
#pragma unroll
                    for (int k = 0; k < 7; ++k)
                        grp[gi][k] = gload<uint2>(gp + k);
                }
                if (sub == 0) {
                    const uint2 f = gload<uint2>(rec + P);
                    fa = __uint_as_float(f.x);
                    fr = __uint_as_float(f.y);
                    if constexpr (lut) {
                        // LUT4: the vector's own lower bound is evaluated below (the lows are
                        // lowered Bitwise bounds), from its short factors in the tile
                        const uint32_t lv = pos - j * stride;
                        const float *fac = reinterpret_cast<const float *>(
                            p.tiles + (size_t)(s_tbase[j] + lv / kTileVectors) * p.tile_bytes + 256u * W);
                        sfa = gload<float>(fac + lv % kTileVectors);
                        sfr = gload<float>(fac + 64 + lv % kTileVectors);
                        sfe = gload<float>(fac + 128 + lv % kTileVectors);
                    } else {
                        low = gload<float>(p.van_lows + (size_t)q * V * stride + pos);
                    }
                }
            }
            // the plane and q' reads stay behind the record loads (hoisted above them, the
            // query's planes alone would take many registers and halve the waves that keep
            // records in flight)
            asm volatile("" ::: "memory");
            int ipa = 0, ipb = 0;
            float ipx = 0.0f, a0 = 0.0f, a1 = 0.0f;
            if (lut && have) {
                // LUT4 estimate of the lane's sign-code words (nibble j = 8 w + i of word w,
                // even j into a0, odd into a1, filter_kernels.cuh:655-708); the lanes' partial
                // sums are added below
                const uint16_t *h = reinterpret_cast<const uint16_t *>(s_lut);
#pragma unroll
                for (int i = 0; i < kW; ++i) {
                    const uint32_t c = __builtin_bitreverse32(xw[i]);
                    const uint16_t *t = h + (size_t)(sub * kW + i) * 128;
#pragma unroll
                    for (int n = 0; n < 8; n += 2) {
                        a0 += (float)__builtin_bit_cast(_Float16, t[n * 16 + ((c >> (28 - 4 * n)) & 15u)]);
                        a1 += (float)__builtin_bit_cast(_Float16, t[(n + 1) * 16 + ((c >> (24 - 4 * n)) & 15u)]);
                    }
                }
            }
            if (have) {
                uint32_t pz = 0;
                asm volatile("" : "+s"(pz));
                const uint32_t *planes = s_planes + pz + sub * kW;
                const float *qv = s_q + pz;
                // plane by plane (Bq=8 planes 0..7, residual planes 8..15), so only one
                // plane's words of the lane are in registers at a time
#pragma unroll 2
                for (int b = 0; b < (lut ? 0 : 2 * kBq); ++b) {
                    int cnt = 0;
#pragma unroll
                    for (int i = 0; i < kW; ++i)
                        cnt += __popc(xw[i] & planes[b * W + i]);
                    const int bb = b & (kBq - 1);
                    const int term = bb < kBq - 1 ? cnt << bb : -(cnt << (kBq - 1));
                    if (b < kBq)
                        ipa += term;
                    else
                        ipb += term;
                }
#pragma unroll
                for (int gi = 0; gi < kG; ++gi)
                    ipx += excode_group_ip(grp[gi], qv + 64 * (sub + L * gi));
            }
#pragma unroll
            for (int o = 1; o < L; o <<= 1) {
                ipa += __shfl_xor(ipa, o, L);
                ipb += __shfl_xor(ipb, o, L);
                ipx += __shfl_xor(ipx, o, L);
                a0 += __shfl_xor(a0, o, L);
                a1 += __shfl_xor(a1, o, L);
            }
            if (have && sub == 0) {
                const float ex = lut ? a0 + a1 : two_stage_ip(width, ipa, width2, ipb);
                const float gadd = s_gadd[j];
                if (lut)
                    low = sfa + gadd + sfr * (ex + k1) - sfe * s_gerr[j];
                const float rd = fa + gadd + fr * (128.0f * ex + ipx + kbq);
                const float err =
                    refine_err_scale(P) * (fabsf(fa) + fabsf(gadd) + fabsf(fr) * (128.0f * fabsf(ex) + 127.0f * l1q + fabsf(kbq)));
                rd_r[e] = make_float2(rd, err);
                aux_r[e] = make_float2(ex, low);
            }
        }
    }
}

// ---- selection of a query's topk best refined entries ----
// A query's refined entries: its seeds, then its list.
struct Entries {
    const uint32_t *seed_pos, *list_pos;
    const float2 *seed_rd, *list_rd, *seed_aux, *list_aux;
    uint32_t seed_n, n;
    __device__ Entries(const VsArgs &vs, uint32_t q, uint32_t sn, uint32_t total)
        : seed_pos(vs.seed_pos + (size_t)q * vs.seed_cap), list_pos(vs.list_pos + (size_t)q * vs.list_cap),
          seed_rd(vs.seed_rd + (size_t)q * vs.seed_cap), list_rd(vs.list_rd + (size_t)q * vs.list_cap),
          seed_aux(vs.seed_aux + (size_t)q * vs.seed_cap), list_aux(vs.list_aux + (size_t)q * vs.list_cap),
          seed_n(sn), n(total) {}
    __device__ float2 rd(uint32_t i) const { return i < seed_n ? seed_rd[i] : list_rd[i - seed_n]; }
    __device__ float2 aux(uint32_t i) const { return i < seed_n ? seed_aux[i] : list_aux[i - seed_n]; }
    __device__ uint32_t pos(uint32_t i) const { return i < seed_n ? seed_pos[i] : list_pos[i - seed_n]; }
    __device__ unsigned long long key(uint32_t i) const {
        return ((unsigned long long)order_key(rd(i).x) << 32) | pos(i);
    }
};

// The k-th smallest key (distance key << 32 | position) among the entries whose distance key
// is at most dk (all when dk is ~0u; there are at least k of them), and the threshold the k
// best back: max(d_k + e, l) + 1 ulp, e the largest rounding bound and l the largest lower
// bound among them. Candidates are held in LDS (s_key, s_ent: kVsCand) when they fit.
__device__ float topk_threshold(const Entries &en, uint32_t dk, uint32_t k, unsigned long long *s_key,
                                uint32_t *s_ent, uint32_t *hist, uint32_t *red, uint32_t *sc,
                                unsigned long long *s_kth, unsigned long long &kth_out) {
    const uint32_t tid = threadIdx.x;
    if (tid == 0)
        sc[3] = 0;
    __syncthreads();
    // candidates into LDS (every entry's distance is read before any is used)
    constexpr int kR = 8;
    for (uint32_t r0 = 0; r0 < en.n; r0 += kR * kVsThreads) {
        float d[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const uint32_t i = r0 + r * kVsThreads + tid;
            d[r] = i < en.n ? en.rd(i).x : __uint_as_float(0x7FC00000u);
        }
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const uint32_t i = r0 + r * kVsThreads + tid;
            const bool take = i < en.n && order_key(d[r]) <= dk;
            const uint32_t slot = wave_slot(take, &sc[3]);
            if (take && slot < kVsCand) {
                s_key[slot] = ((unsigned long long)order_key(d[r]) << 32) | en.pos(i);
                s_ent[slot] = i;
            }
        }
    }
    __syncthreads();
    const uint32_t nc = sc[3];
    __syncthreads();
    unsigned long long kth;
    uint32_t ekey = 0, lkey = 0;
    if (nc <= kVsCand) {
        if (nc <= kVsRankMax) {
            // rank of each key = keys below it (every thread reads the keys in the same order)
            for (uint32_t i = tid; i < nc; i += kVsThreads) {
                const unsigned long long v = s_key[i];
                uint32_t rank = 0;
                for (uint32_t m = 0; m < nc; ++m)
                    rank += s_key[m] < v ? 1u : 0u;
                if (rank == k - 1)
                    *s_kth = v;
            }
            __syncthreads();
            kth = *s_kth;
        } else {
            kth = block_kth_u64([&](uint32_t i) { return s_key[i]; }, nc, k, hist, red, sc);
        }
        for (uint32_t i = tid; i < nc; i += kVsThreads) {
            if (s_key[i] <= kth) {
                ekey = max(ekey, __float_as_uint(en.rd(s_ent[i]).y));  // >= 0: bits order like values
                lkey = max(lkey, order_key(en.aux(s_ent[i]).y));
            }
        }
    } else {
        // more candidates than the LDS holds: the select reads the regions directly
        auto key_at = [&](uint32_t i) { return order_key(en.rd(i).x) <= dk ? en.key(i) : ~0ull; };
        kth = block_kth_u64(key_at, en.n, k, hist, red, sc);
        for (uint32_t i = tid; i < en.n; i += kVsThreads) {
            if (key_at(i) <= kth) {
                ekey = max(ekey, __float_as_uint(en.rd(i).y));
                lkey = max(lkey, order_key(en.aux(i).y));
            }
        }
    }
    ekey = vs_block_max(ekey, red);
    lkey = vs_block_max(lkey, red);
    kth_out = kth;
    const float dkv = key_to_float((uint32_t)(kth >> 32));
    return nextafterf(fmaxf(dkv + __uint_as_float(ekey), key_to_float(lkey)), FLT_MAX);
}

// ---- 3. threshold from the seeds, and the list of the other vectors below it ----
__global__ __launch_bounds__(kVsThreads) void vs_list_kernel(const ScanParams p, const VanguardArgs va,
                                                             const VsArgs vs) {
    __shared__ unsigned long long s_key[kVsCand];
    __shared__ uint32_t s_ent[kVsCand];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_n[kVanguardMaxPairs], s_off[kVanguardMaxPairs + 1], s_goff[kVanguardMaxPairs + 1];
    __shared__ uint32_t red[kVsWaves];
    __shared__ uint32_t sc[2];
    __shared__ unsigned long long s_kth;
    // the group list of the list stage reuses the candidate keys' memory
    static_assert(kVsSel * 4 <= kVsCand * 8, "group list within the candidate keys");
    uint32_t *s_sel = reinterpret_cast<uint32_t *>(s_key);
    const uint32_t q = blockIdx.x, tid = threadIdx.x;
    if (q >= va.nq)
        return;
    VsQuery st = vs.qs[q];
    if (st.flags & kVsOverflow)
        return;
    float thr = st.thr_in;
    if (st.seed_n >= va.topk) {
        unsigned long long kth = 0;
        const float t = topk_threshold(Entries(vs, q, st.seed_n, st.seed_n), 0xFFFFFFFFu, va.topk, s_key, s_ent,
                                       hist, red, sc, &s_kth, kth);
        st.dk_key = (uint32_t)(kth >> 32);
        if (t < thr)
            thr = t;
    }
    // every other vector with low < thr: key below thr's and above the seeds' cut, from the
    // groups whose minimum lies below thr
    const uint32_t kthr = order_key(thr), cut1 = st.cut1;
    uint32_t *list = vs.list_pos + (size_t)q * vs.list_cap;
    load_pairs(p, va, q, s_n, s_off, s_goff);
    const uint32_t V = va.depth, gstride = p.van_stride / 4;
    const QueryRows qb{p.van_lows + (size_t)q * V * p.van_stride, s_off, p.van_stride, s_off[V]};
    const QueryRows qg{p.van_mins + (size_t)q * V * gstride, s_goff, gstride, s_goff[V]};
    uint32_t nlist = 0;
    auto listed = [kthr, cut1](uint32_t k) { return k < kthr && k > cut1; };
    for_bounds_of_groups(
        qg, qb, s_n, st.thr_in, [kthr](uint32_t k) { return k < kthr; },
        Compactor<decltype(listed)>{listed, list, vs.list_cap, red, &nlist}, s_sel, red);
    if (tid == 0) {
        const uint32_t n = nlist;
        if (n > vs.list_cap) {
            overflow_query(vs, q);
        } else {
            st.list_n = n;
            st.thr = thr;
            vs.qs[q] = st;
            atomicAdd(&vs.spread[(q % kVsSpread) * kVsSpreadWords + kVsStList], (unsigned long long)n);
        }
    }
}

// ---- 5. merge and publication ----
__global__ __launch_bounds__(kVsThreads) void vs_merge_kernel(const ScanParams p, const VanguardArgs va,
                                                              const VsArgs vs) {
    __shared__ unsigned long long s_key[kVsCand];
    __shared__ uint32_t s_ent[kVsCand];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_start[kVanguardMaxPairs];
    __shared__ uint32_t red[kVsWaves];
    __shared__ uint32_t sc[4];
    __shared__ unsigned long long s_base, s_limit, s_kth;
    const uint32_t q = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (q >= va.nq)
        return;
    const VsQuery st = vs.qs[q];
    if (st.flags & kVsOverflow)
        return;
    const uint32_t V = va.depth, stride = p.van_stride;
    const QueueDev qd = p.queue;
    if (tid < V)
        s_start[tid] = p.meta[va.probe_idx[(size_t)q * p.nprobe + tid]].start;
    if (tid == 0)
        s_limit = __hip_atomic_load(qd.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const Entries en(vs, q, st.seed_n, st.seed_n + st.list_n);
    float thr = st.thr;
    bool backed = false;
    if (st.dk_key != 0xFFFFFFFFu) {
        // the topk best lie among the entries whose distance key is at most the seeds' k-th
        unsigned long long kth = 0;
        const float t = topk_threshold(en, st.dk_key, va.topk, s_key, s_ent, hist, red, sc, &s_kth, kth);
        if (t < thr)
            thr = t;
        backed = true;
    }
    // publication: refined distance within its rounding bound of the threshold. The records go
    // to the query's out region, which vs_publish_kernel copies to the ring with one
    // reservation per batch of queries; a query with more than out_cap of them publishes them
    // itself (one ring reservation per round of 256).
    uint32_t npub = 0;
    for (uint32_t i = tid; i < en.n; i += kVsThreads) {
        const float2 rde = en.rd(i);
        npub += rde.x <= thr + rde.y ? 1u : 0u;
    }
    npub = vs_block_sum(npub, red);
    const bool direct = npub > vs.out_cap;
    uint4 *out = vs.out + (size_t)q * vs.out_cap;
    uint32_t dropped = 0;
    if (tid == 0)
        sc[2] = 0;
    __syncthreads();
    for (uint32_t r0 = 0; r0 < en.n; r0 += kVsThreads) {
        const uint32_t i = r0 + tid;
        bool pub = false;
        float2 rde = make_float2(0.0f, 0.0f);
        if (i < en.n) {
            rde = en.rd(i);
            pub = rde.x <= thr + rde.y;
            dropped += (!pub && !isnan(rde.x)) ? 1u : 0u;
        }
        uint4 rec = make_uint4(0u, 0u, 0u, 0u);
        if (pub) {
            const uint32_t pos = en.pos(i);
            const uint32_t j = pos / stride;
            const uint32_t gid = s_start[j] + (pos - j * stride);
            const float2 ax = en.aux(i);
            rec = make_uint4((j << 16) | q, gid, __float_as_uint(qd.final_mode ? rde.x : ax.x), __float_as_uint(ax.y));
        }
        if (!direct) {
            const uint32_t slot = wave_slot(pub, &sc[2]);
            if (pub)
                out[slot] = rec;
            continue;
        }
        const unsigned long long m = __ballot(pub);
        if (lane == 0)
            red[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t before = 0, cnt = 0;
#pragma unroll
        for (uint32_t w = 0; w < (uint32_t)kVsWaves; ++w) {
            before += w < wave ? red[w] : 0u;
            cnt += red[w];
        }
        if (cnt != 0) {
            if (tid == 0) {
                const unsigned long long b = atomicAdd(qd.produced, (unsigned long long)cnt);
                unsigned long long lim = s_limit;
                if (b + cnt > lim)
                    lim = refresh_limit(qd.cached_limit, qd.refresh_flag, &qd.progress->released, qd.capacity,
                                        b + cnt);
                s_base = b;
                s_limit = lim;
            }
            __syncthreads();
            if (pub)
                place_record(qd, s_base + before + lane_rank(m), s_limit, rec);
        }
        __syncthreads();  // red, s_base reused by the next round
    }
    dropped = vs_block_sum(dropped, red);
    if (tid == 0) {
        vs.qs[q].pub_n = direct ? 0u : npub;
        unsigned long long *sp = &vs.spread[(q % kVsSpread) * kVsSpreadWords];
        if (dropped)
            atomicAdd(&sp[kVsStDropped], (unsigned long long)dropped);
        if (en.n)
            atomicAdd(&sp[kVsStRefined], (unsigned long long)en.n);
        if (backed && thr < st.thr_in) {
            uint32_t *slot = reinterpret_cast<uint32_t *>(va.thr_out) + q;
            if (direct) {
                // its records are in the ring already: the CPU consumer may have lowered the
                // threshold meanwhile, so only an atomic minimum
                uint32_t cur = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                while (thr < __uint_as_float(cur)) {
                    if (__hip_atomic_compare_exchange_strong(slot, &cur, __float_as_uint(thr), __ATOMIC_RELAXED,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM))
                        break;
                }
            } else {
                // none of the query's records has been published in this search yet (its vanguard
                // records go out after this kernel, its far records after this pass), so no
                // consumer has changed its threshold since the snapshot thr_in was taken: a
                // store (through to host memory) lowers it without a round trip
                __hip_atomic_store(slot, __float_as_uint(thr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            atomicAdd(&sp[kVsStSeeded], 1ull);
        }
    }
}

// ---- publication of the merged records and the pass's statistics ----
constexpr uint32_t kVsPubGrid = 256;

// Workgroup b copies the out regions of queries [b * per, (b + 1) * per) to the ring with one
// reservation (records in query order); overflowed and directly published queries have none.
__global__ __launch_bounds__(kVsThreads) void vs_publish_kernel(const ScanParams p, const VanguardArgs va,
                                                                const VsArgs vs) {
    __shared__ uint32_t s_cnt[kVsThreads];
    __shared__ uint32_t red[kVsWaves];
    __shared__ unsigned long long s_base, s_limit;
    const uint32_t tid = threadIdx.x;
    const QueueDev qd = p.queue;
    const uint32_t per = (va.nq + gridDim.x - 1) / gridDim.x;
    const uint32_t q0 = blockIdx.x * per, q1 = min(va.nq, q0 + per);
    for (uint32_t b0 = q0; b0 < q1; b0 += kVsThreads) {
        // the counts of up to 256 queries, their offsets within the batch
        const uint32_t q = b0 + tid;
        uint32_t n = 0;
        if (q < q1) {
            const VsQuery st = vs.qs[q];
            n = (st.flags & kVsOverflow) ? 0u : st.pub_n;
        }
        const uint32_t incl = vs_block_scan(n, red);
        s_cnt[tid] = incl - n;
        const uint32_t total = vs_block_max(incl, red);  // the last thread's inclusive sum
        if (total == 0)
            continue;
        if (tid == 0) {
            const unsigned long long b = atomicAdd(qd.produced, (unsigned long long)total);
            unsigned long long lim = __hip_atomic_load(qd.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (b + total > lim)
                lim = refresh_limit(qd.cached_limit, qd.refresh_flag, &qd.progress->released, qd.capacity,
                                    b + total);
            s_base = b;
            s_limit = lim;
        }
        __syncthreads();
        // one wave per query, its records in order
        const uint32_t lane = tid & 63, wave = tid >> 6;
        for (uint32_t k = wave; k < kVsThreads && b0 + k < q1; k += kVsWaves) {
            const uint32_t qq = b0 + k;
            const uint32_t off = s_cnt[k];
            const uint32_t nn = (k + 1 < kVsThreads && b0 + k + 1 < q1 ? s_cnt[k + 1] : total) - off;
            const uint4 *out = vs.out + (size_t)qq * vs.out_cap;
            for (uint32_t r = lane; r < nn; r += 64)
                place_record(qd, s_base + off + r, s_limit, out[r]);
        }
        __syncthreads();  // s_cnt, s_base reused by the next batch
    }
}

// One workgroup: the spread statistics summed into the engine's counters.
__global__ __launch_bounds__(64) void vs_stats_kernel(const ScanParams p, const VanguardArgs va, const VsArgs vs) {
    const uint32_t t = threadIdx.x;
    unsigned long long v[6] = {0, 0, 0, 0, 0, 0};
    for (uint32_t line = t; line < kVsSpread; line += 64)
#pragma unroll
        for (int f = 0; f < 6; ++f)
            v[f] += vs.spread[line * kVsSpreadWords + f];
#pragma unroll
    for (int f = 0; f < 6; ++f)
        for (int o = 32; o > 0; o >>= 1)
            v[f] += __shfl_xor(v[f], o);
    if (t == 0) {
        vs.ctr[kVsCtrSeeds] = v[kVsStSeeds];
        vs.ctr[kVsCtrList] = v[kVsStList];
        vs.ctr[kVsCtrRescan] = v[kVsStRescan];
        if (v[kVsStDropped])
            atomicAdd(p.dropped, v[kVsStDropped]);
        if (v[kVsStRefined])
            atomicAdd(va.refined, v[kVsStRefined]);
        if (v[kVsStSeeded])
            atomicAdd(va.seeded, v[kVsStSeeded]);
    }
}

// Grid = workgroups of the kernel resident on the whole device at once.
template <class F>
uint32_t vs_resident_grid(F kernel) {
    static std::mutex mu;
    static std::map<const void *, uint32_t> cache;
    const void *key = reinterpret_cast<const void *>(kernel);
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end())
        return it->second;
    int dev = 0, per_cu = 0, cus = 0;
    (void)hipGetDevice(&dev);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kVsThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 ||
        cus <= 0) {
        per_cu = 4;
        cus = 256;
    }
    const uint32_t grid = (uint32_t)(per_cu * cus);
    cache.emplace(key, grid);
    return grid;
}

template <int W>
void launch_vs_w(const ScanParams &p, const VanguardArgs &va, const VsArgs &vs, uint32_t nq, hipEvent_t ev_r0,
                 hipEvent_t ev_r1, hipEvent_t ev_r2, hipEvent_t ev_r3, hipStream_t s) {
    auto *rk = p.lut ? vs_refine_kernel<W, true> : vs_refine_kernel<W, false>;
    const uint32_t grid = vs_resident_grid(rk);
    vs_seed_kernel<<<nq, kVsThreads, 0, s>>>(p, va, vs);
    if (ev_r0)
        (void)hipEventRecord(ev_r0, s);
    rk<<<grid, kVsThreads, 0, s>>>(p, va, vs, 0u);
    if (ev_r1)
        (void)hipEventRecord(ev_r1, s);
    vs_list_kernel<<<nq, kVsThreads, 0, s>>>(p, va, vs);
    if (ev_r2)
        (void)hipEventRecord(ev_r2, s);
    rk<<<grid, kVsThreads, 0, s>>>(p, va, vs, 1u);
    if (ev_r3)
        (void)hipEventRecord(ev_r3, s);
    vs_merge_kernel<<<nq, kVsThreads, 0, s>>>(p, va, vs);
    vs_publish_kernel<<<std::min<uint32_t>(kVsPubGrid, nq), kVsThreads, 0, s>>>(p, va, vs);
    vs_stats_kernel<<<1, 64, 0, s>>>(p, va, vs);
    // the queries whose seeds or list did not fit: the fused per-query kernel (with LUT4 it
    // refines them with the two-stage Bitwise estimate, and selects and publishes on the
    // lowered bounds)
    // (above the one-pass kernel's top-k the regions hold every vanguard vector: no query
    // overflows)
    if (va.topk > kVanguardMaxTopk)
        return;
    VanguardArgs fb = va;
    fb.list = vs.overflow;
    fb.list_count = &vs.ctr[kVsCtrOverflow];
    launch_vanguard_query(p, fb, W, nq, s);
}

}  // namespace

bool vanguard_staged_supported(uint32_t W) {
    return W == 2 || W == 4 || W == 8 || W == 16 || W == 24 || W == 32;
}

void launch_vanguard_staged(const ScanParams &p, const VanguardArgs &va, const VsArgs &vs, uint32_t W, uint32_t nq,
                            hipEvent_t ev_r0, hipEvent_t ev_r1, hipEvent_t ev_r2, hipEvent_t ev_r3, hipStream_t s) {
    if (nq == 0 || va.depth == 0)
        return;
    switch (W) {
    case 2: launch_vs_w<2>(p, va, vs, nq, ev_r0, ev_r1, ev_r2, ev_r3, s); break;
    case 4: launch_vs_w<4>(p, va, vs, nq, ev_r0, ev_r1, ev_r2, ev_r3, s); break;
    case 8: launch_vs_w<8>(p, va, vs, nq, ev_r0, ev_r1, ev_r2, ev_r3, s); break;
    case 16: launch_vs_w<16>(p, va, vs, nq, ev_r0, ev_r1, ev_r2, ev_r3, s); break;
    case 24: launch_vs_w<24>(p, va, vs, nq, ev_r0, ev_r1, ev_r2, ev_r3, s); break;
    case 32: launch_vs_w<32>(p, va, vs, nq, ev_r0, ev_r1, ev_r2, ev_r3, s); break;
    default: break;
    }
}

}  // namespace cora
