// Fused vanguard pass: one workgroup per query over all of its vanguard pairs (probe rank
// < vanguard), replacing the per-pair seed pass, the seed threshold kernel and the
// per-pair recovery pass when the ex-codes are resident in HBM.
//
// The reference runs the vanguard pairs as a seed kernel that publishes the best
// max(topk, 20) lower bounds of each pair (filter_kernels.cuh:308-468), and a recovery
// kernel that later publishes the pair's other vectors with low < threshold
// (filter_kernels.cuh:470-582), the threshold being lowered meanwhile by the CPU
// consumer from the refined distances. Here the whole query is handled in one place:
//
//   1. the four waves stream the tiles of the query's vanguard clusters (nearest first)
//      and evaluate the Bitwise lower bound of the scan kernels (same expression) — or,
//      when the matrix-core pass has already written every vanguard lower bound
//      cluster-major (launch_vanguard_lows: each cluster read once per unit of up to 16
//      pairs instead of once per query), stream those 4-byte bounds; a vector whose bound
//      is below the query's current threshold joins an LDS candidate list (lower bound,
//      position), compacted per wave with a ballot;
//   2. every 8 tiles per wave, once the list holds 1,024 entries (and at the end), the
//      list is refined: while fewer than topk vectors are refined, the 128 smallest
//      bounds first (radix select), then every remaining bound below the threshold, in
//      chunks of 128 vectors (two lanes each) with the CPU's formula
//      (cpu_refinement.cpp:183-192) on the HBM ex-codes and a bound on the rounding
//      difference to the CPU's own evaluation; each chunk is merged into the query's
//      top-k of refined distances, which lowers the threshold to max(d_k + e, l) + 1 ulp
//      (d_k the k-th distance, e the largest rounding bound and l the largest lower bound
//      among those k); a vector whose bound is at or above the threshold is skipped;
//   3. every refined vector whose distance is within its rounding bound of the final
//      threshold is published to the ring (the refined pre-filter rule), and the
//      threshold is lowered (atomic minimum) for the far pass and the CPU consumer.
//
// Only bounds below a threshold backed by refined distances are ever dropped, and the
// threshold only falls, so every vector whose bound is below the final threshold is
// refined. Safety is that of the refined pre-filter: the k vectors behind the threshold
// are published, the CPU evaluates each below the threshold (distance and lower bound),
// so the CPU's final k-th distance is at most the threshold, and a vector dropped here
// has a CPU-evaluated distance above the threshold, which the CPU consumer itself would
// reject.
#include <float.h>

#include <map>
#include <mutex>
#include <utility>

#include "device_common.h"

namespace cora {
namespace {

constexpr int kVqThreads = 256;
constexpr int kVqWaves = kVqThreads / 64;
constexpr uint32_t kVqWin = 512;     // window capacity (sorted u64 keys in LDS)
constexpr uint32_t kVqChunk = 128;   // refinements between threshold updates
constexpr uint32_t kVqHeld = 256;    // refined vectors held before publication
constexpr uint32_t kVqMaxW = 32;     // P <= 1024
constexpr uint32_t kVqSegTiles = 8;  // tiles per wave between list checks
constexpr uint32_t kVqHigh = 1024;   // list entries that trigger a refinement round
constexpr uint32_t kVqList = kVqHigh + kVqWaves * kVqSegTiles * kTileVectors;  // list capacity
// precomputed bounds: chunks of 256 (one 16-byte load per lane), two per wave per segment
// (the same 512 list entries per wave and segment as kVqSegTiles tiles), the next
// segment's two in flight meanwhile
constexpr uint32_t kPreChunk = 256;
constexpr uint32_t kPreSegChunks = 2;
static_assert(kPreSegChunks * kPreChunk == kVqSegTiles * kTileVectors, "list capacity per segment");
static_assert(kVqChunk * 2 == kVqThreads, "one chunk vector per two lanes");

__device__ __forceinline__ float processed_mark() { return __uint_as_float(0x7FC00000u); }

// Inclusive prefix sum over the workgroup (thread order); s_red holds kVqWaves words.
__device__ __forceinline__ uint32_t block_incl_scan(uint32_t v, uint32_t *s_red) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(v, o);
        if (lane >= (uint32_t)o)
            v += y;
    }
    if (lane == 63)
        s_red[wave] = v;
    __syncthreads();
    uint32_t add = 0;
    for (uint32_t w = 0; w < wave; ++w)
        add += s_red[w];
    __syncthreads();
    return v + add;
}

// The k-th smallest (k >= 1) order key among lows(i) < thr, i < n (4 radix passes of 8
// bits; the caller guarantees at least k such entries).
template <class L>
__device__ uint32_t block_select(L lows, uint32_t n, float thr, uint32_t k, uint32_t *s_hist,
                                 uint32_t *s_red, uint32_t *s_sc) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, pmask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        s_hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += kVqThreads) {
            const float l = lows(i);
            if (l < thr) {
                const uint32_t key = order_key(l);
                if ((key & pmask) == prefix)
                    atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
            }
        }
        __syncthreads();
        const uint32_t h = s_hist[tid];
        const uint32_t incl = block_incl_scan(h, s_red);
        if (incl >= k && incl - h < k) {
            s_sc[0] = tid;
            s_sc[1] = k - (incl - h);
        }
        __syncthreads();
        prefix |= s_sc[0] << shift;
        pmask |= 255u << shift;
        k = s_sc[1];
        __syncthreads();
    }
    return prefix;
}

struct VqShared {
    uint32_t planes[2 * kBq * kVqMaxW];
    uint32_t start[kVanguardMaxPairs], n[kVanguardMaxPairs], tbase[kVanguardMaxPairs];
    uint32_t off[kVanguardMaxPairs + 1], toff[kVanguardMaxPairs + 1];
    float gadd[kVanguardMaxPairs], gerr[kVanguardMaxPairs];
    uint32_t win[kVqWin];
    uint32_t hist[256];
    uint32_t red[kVqWaves];
    uint32_t sc[4];
    uint32_t cnt[kVqChunk / 64][2];
    // refined vectors awaiting publication
    uint32_t h_word0[kVqHeld], h_gid[kVqHeld];
    float h_ex[kVqHeld], h_low[kVqHeld], h_rd[kVqHeld], h_err[kVqHeld];
    // the query's current top-k (double buffered): order_key(rd) << 32 | position
    unsigned long long t_key[2][kVanguardMaxTopk];
    float t_err[2][kVanguardMaxTopk], t_low[2][kVanguardMaxTopk];
    // results of the current chunk (~0 key: not refined)
    unsigned long long c_key[kVqChunk];
    float c_err[kVqChunk], c_low[kVqChunk];
    // the chunk's vectors entering the top-k
    unsigned long long e_key[kVqChunk];
    float e_err[kVqChunk], e_low[kVqChunk];
    float l1;  // sum |q'| of the query
    // candidate list: lower bound and position of vectors below the threshold
    float l_low[kVqList];
    uint32_t l_pos[kVqList];
    float thr;
    uint32_t nheld, kc, tb, nlist;
    uint32_t ndropped, nrefined;  // statistics of the query
    unsigned long long base, limit;
};

// Append list index i to the window when take (wave-level compaction, one LDS atomic
// per wave); entries beyond the window capacity are left for a later window.
__device__ __forceinline__ void append_window(VqShared &S, uint32_t i, bool take) {
    const uint32_t lane = threadIdx.x & 63;
    const unsigned long long m = __ballot(take);
    if (m == 0)
        return;
    uint32_t base = 0;
    if (lane == 0)
        base = atomicAdd(&S.sc[2], (uint32_t)__popcll(m));
    base = __builtin_amdgcn_readfirstlane(base);
    const uint32_t slot = base + lane_rank(m);
    if (take && slot < kVqWin)
        S.win[slot] = i;
}

// Publish the held refined vectors whose distance is within their rounding bound of the
// current threshold (one ring reservation per round of 256), count the others as dropped
// (S.ndropped). last: the query's final publication, after which the workgroup only ends,
// so no barrier follows the last round's stores (a barrier waits for their write-through
// to host memory), and the dropped ones are counted straight into last_dropped.
__device__ void publish_held(VqShared &S, const QueueDev &q, bool last = false,
                             unsigned long long *last_dropped = nullptr) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float thr = S.thr;
    const uint32_t nheld = S.nheld;
    for (uint32_t r0 = 0; r0 < nheld; r0 += kVqThreads) {
        const uint32_t i = r0 + tid;
        bool pub = false, drop = false;
        if (i < nheld) {
            const float rd = S.h_rd[i];
            pub = rd <= thr + S.h_err[i];
            drop = !pub && !isnan(rd);
        }
        const unsigned long long m = __ballot(pub), dm = __ballot(drop);
        if (lane == 0) {
            S.red[wave] = (uint32_t)__popcll(m);
            if (dm) {
                if (last)
                    atomicAdd(last_dropped, (unsigned long long)__popcll(dm));
                else
                    atomicAdd(&S.ndropped, (uint32_t)__popcll(dm));
            }
        }
        __syncthreads();
        uint32_t before = 0, total = 0;
#pragma unroll
        for (uint32_t w = 0; w < (uint32_t)kVqWaves; ++w) {
            before += w < wave ? S.red[w] : 0u;
            total += S.red[w];
        }
        if (total != 0) {
            if (tid == 0) {
                const unsigned long long b = atomicAdd(q.produced, (unsigned long long)total);
                unsigned long long lim = S.limit;
                if (b + total > lim)
                    lim = refresh_limit(q.cached_limit, q.refresh_flag, &q.progress->released,
                                        q.capacity, b + total);
                S.base = b;
                S.limit = lim;
            }
            __syncthreads();
            if (pub)
                place_record(q, S.base + before + lane_rank(m), S.limit,
                             make_uint4(S.h_word0[i], S.h_gid[i],
                                        __float_as_uint(q.final_mode ? S.h_rd[i] : S.h_ex[i]),
                                        __float_as_uint(S.h_low[i])));
        }
        if (last && r0 + kVqThreads >= nheld)
            return;
        __syncthreads();  // S.red / S.base reused by the next round
    }
    if (last)
        return;
    if (tid == 0)
        S.nheld = 0;
    __syncthreads();
}

// Make room among the held refined vectors without publishing: those whose distance is
// beyond their rounding bound of the current threshold can never be published (the
// threshold only falls), so they are counted as dropped and the others are compacted in
// order. Publication then happens with the final threshold, as in the staged pass, instead
// of with the threshold of the moment the buffer filled (config 5, top-100: 146 -> ~103
// records a query to the CPU). kVqHeld = kVqThreads: one held vector per thread.
__device__ void compact_held(VqShared &S) {
    static_assert(kVqHeld == kVqThreads, "one held vector per thread");
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float thr = S.thr;
    const uint32_t nheld = S.nheld;
    bool keep = false, drop = false;
    uint32_t w0 = 0, gid = 0;
    float ex = 0.0f, low = 0.0f, rd = 0.0f, err = 0.0f;
    if (tid < nheld) {
        w0 = S.h_word0[tid];
        gid = S.h_gid[tid];
        ex = S.h_ex[tid];
        low = S.h_low[tid];
        rd = S.h_rd[tid];
        err = S.h_err[tid];
        keep = rd <= thr + err;
        drop = !keep && !isnan(rd);
    }
    const unsigned long long m = __ballot(keep), dm = __ballot(drop);
    if (lane == 0) {
        S.red[wave] = (uint32_t)__popcll(m);
        if (dm)
            atomicAdd(&S.ndropped, (uint32_t)__popcll(dm));
    }
    __syncthreads();  // every held vector is in registers before any is overwritten
    uint32_t before = 0, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < (uint32_t)kVqWaves; ++w) {
        before += w < wave ? S.red[w] : 0u;
        total += S.red[w];
    }
    if (keep) {
        const uint32_t k = before + lane_rank(m);
        S.h_word0[k] = w0;
        S.h_gid[k] = gid;
        S.h_ex[k] = ex;
        S.h_low[k] = low;
        S.h_rd[k] = rd;
        S.h_err[k] = err;
    }
    __syncthreads();  // S.red is read above before anyone reuses it
    if (tid == 0)
        S.nheld = total;
    __syncthreads();
}

// The query's Bq=8 planes [kBq][W] in the constant address space: wave-uniform reads
// become scalar loads whose words feed the AND as scalar operands.
typedef __attribute__((address_space(4))) const uint32_t *ConstWords;

// ip_int of one vector (words x) for W >= 16: the planes are read one 4-word group at a
// time (8 x 4 scalar words), so they never occupy vector registers; the opaque per-group
// base also keeps the loads in the caller's loop instead of hoisted out of it.
template <int W>
__device__ __forceinline__ int popc_ip_scalar(const uint32_t (&x)[Words<W>::kMax], ConstWords planes) {
    int a[kBq];
#pragma unroll
    for (int j = 0; j < kBq; ++j)
        a[j] = 0;
#pragma unroll
    for (int g = 0; g < W / 4; ++g) {
        // an opaque base per group: its 8 x 4 words load as their own scalar loads, not
        // merged with the neighbouring groups' (which would hold ~80 scalar registers)
        ConstWords pg = planes + 4 * g;
        asm volatile("" : "+s"(pg));
#pragma unroll
        for (int j = 0; j < kBq; ++j) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                a[j] += __popc(x[4 * g + k] & pg[j * W + k]);
        }
    }
    int ip = -(a[kBq - 1] << (kBq - 1));
#pragma unroll
    for (int j = 0; j < kBq - 1; ++j)
        ip += a[j] << j;
    return ip;
}

// P <= 128 and P >= 512: at most 168 VGPRs so three workgroups (12 waves) share a CU,
// which the LDS footprint also allows. kPre: the lower bounds come from p.van_lows.
template <int W, bool kPre>
__global__ __launch_bounds__(kVqThreads, kPre && W >= 16 ? 2 : (W > 0 && W <= 4) || W >= 16 || kPre ? 3 : 1) void vanguard_query_kernel(
    const ScanParams p, const VanguardArgs va) {
    extern __shared__ __align__(16) float s_dyn[];  // q' [P]
    __shared__ VqShared S;
    constexpr int K = Words<W>::kMax;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // workgroup b runs on XCD b % 8 and takes the (b / 8)-th query of that XCD's slice of
    // the queries ordered by nearest cluster, so each XCD's L2 serves about an eighth of
    // the clusters
    uint32_t qi;
    if (va.list) {
        // list mode: workgroup b takes entry b of a device-side list of queries (the staged
        // pass's overflow), the grid sized for the longest list; the others return at once
        if (blockIdx.x >= *va.list_count)
            return;
        qi = va.list[blockIdx.x];
    } else {
        const uint32_t per_xcd = (va.nq + kNumXcd - 1) / kNumXcd;
        const uint32_t slot = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
        if (slot >= va.nq)
            return;
        qi = va.order ? va.order[slot] : slot;
    }
    const uint32_t V = va.depth, topk = va.topk;
    const uint32_t P = p.P, nw = W > 0 ? (uint32_t)W : P / 32;
    const QueueDev q = p.queue;
    float *s_q = s_dyn;
    // vectors per streamed unit: a tile of codes, or a chunk of 256 precomputed bounds
    constexpr uint32_t kStreamVectors = kPre ? kPreChunk : (uint32_t)kTileVectors;

    // ---- set-up: pair metadata, q-planes and q' in LDS ----
    if (tid < V) {
        const size_t pi = (size_t)qi * p.nprobe + tid;
        const ClusterMeta cm = p.meta[va.probe_idx[pi]];
        S.start[tid] = cm.start;
        S.n[tid] = cm.n;
        S.tbase[tid] = cm.tile_base;
        S.gadd[tid] = p.pgadd[pi];
        S.gerr[tid] = p.pgerr[pi];
    }
    for (uint32_t i = tid; i < 2 * kBq * nw; i += kVqThreads)
        S.planes[i] = p.qplanes[(size_t)qi * 2 * kBq * nw + i];
    float l1p = 0.0f;
    for (uint32_t i = tid; i < P; i += kVqThreads) {
        const float v = p.qrot[(size_t)qi * P + i];
        s_q[i] = v;
        l1p += fabsf(v);
    }
    if (tid == 0) {
        S.thr = p.thresholds[qi];
        S.nheld = 0;
        S.kc = 0;
        S.tb = 0;
        S.nlist = 0;
        S.ndropped = 0;
        S.nrefined = 0;
        S.limit = __hip_atomic_load(q.cached_limit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t o = 0, to = 0;
        for (uint32_t j = 0; j < V; ++j) {
            S.off[j] = o;
            S.toff[j] = to;
            o += S.n[j];
            to += (S.n[j] + kStreamVectors - 1) / kStreamVectors;
        }
        S.off[V] = o;
        S.toff[V] = to;
    }
    __syncthreads();
    const uint32_t T = S.toff[V];
    const float thr_in = S.thr;
    bool early_pub = false;  // held records went out before the final threshold
    // sum |q'| for the rounding bound (the same for every vector of the query)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        l1p += __shfl_xor(l1p, o);
    if (lane == 0)
        S.red[wave] = __float_as_uint(l1p);
    __syncthreads();
    float l1q = 0.0f;
#pragma unroll
    for (int w = 0; w < kVqWaves; ++w)
        l1q += __uint_as_float(S.red[w]);
    __syncthreads();
    const float width = p.qwidth[qi], width2 = p.qwidth2[qi], k1 = p.k1[qi], kbq = p.kb[qi];

    // ---- lower bounds streamed into the candidate list, refined when it fills ----
    // W <= 4: the Bq=8 planes held in VGPRs during the tile stream (the same value in every
    // lane; as SGPRs they would be spilled and re-read per tile), reloaded from LDS for
    // every segment so they are not live across the list refinement
    uint32_t preg[W > 0 && W <= 4 ? kBq * W : 1];
    const ConstWords cplanes = (ConstWords)(p.qplanes + (size_t)qi * 2 * kBq * nw);
    auto process_list = [&]() {
        const uint32_t nl = S.nlist;
        for (;;) {
            const float thr0 = S.thr;
            const bool seeding = S.kc < topk;
            // window: the remaining bounds below the threshold, up to kVqWin of them; while
            // fewer than topk vectors are refined, only the kVqChunk smallest (all keys up
            // to the selected one), which then set the first threshold
            if (tid == 0)
                S.sc[2] = 0;
            __syncthreads();
            for (uint32_t i0 = 0; i0 < nl; i0 += kVqThreads) {
                const uint32_t i = i0 + tid;
                append_window(S, i, i < nl && S.l_low[i] < thr0);
            }
            __syncthreads();
            const uint32_t cnt = S.sc[2];
            if (cnt == 0)
                break;
            if (seeding && cnt > kVqChunk) {
                const uint32_t kth = block_select([&](uint32_t i) -> float { return S.l_low[i]; }, nl,
                                                  thr0, kVqChunk, S.hist, S.red, S.sc);
                if (tid == 0)
                    S.sc[2] = 0;
                __syncthreads();
                for (uint32_t i0 = 0; i0 < nl; i0 += kVqThreads) {
                    const uint32_t i = i0 + tid;
                    const float l = i < nl ? S.l_low[i] : processed_mark();
                    append_window(S, i, l < thr0 && order_key(l) <= kth);
                }
                __syncthreads();
            }
            const uint32_t nwin = min(S.sc[2], kVqWin);
            for (uint32_t c0 = 0; c0 < nwin; c0 += kVqChunk) {
                const float thr = S.thr;
                if (S.nheld + kVqChunk > kVqHeld)
                    compact_held(S);
                if (S.nheld + kVqChunk > kVqHeld) {
                    publish_held(S, q);
                    early_pub = true;
                }
                const uint32_t cn = min(kVqChunk, nwin - c0);
                const uint32_t held0 = S.nheld;
                // the refined distance of chunk vector e (lane sub == 0 of its group) into the
                // chunk results and the held records
                auto emit = [&](uint32_t e, bool have, uint32_t j, uint32_t pos, size_t gid, float low,
                                int ipa, int ipb, float ipx, float fa, float fr) {
                    if (!have) {
                        S.c_key[e] = ~0ull;
                        if (e < cn)
                            S.h_rd[held0 + e] = processed_mark();
                        return;
                    }
                    const float ex = two_stage_ip(width, ipa, width2, ipb);
                    const float gadd = S.gadd[j];
                    const float rd = fa + gadd + fr * (128.0f * ex + ipx + kbq);
                    const float err = p.refine_err * (fabsf(fa) + fabsf(gadd) +
                                               fabsf(fr) * (128.0f * fabsf(ex) + 127.0f * l1q + fabsf(kbq)));
                    S.c_key[e] = ((unsigned long long)order_key(rd) << 32) | pos;
                    S.c_err[e] = err;
                    S.c_low[e] = low;
                    const uint32_t h = held0 + e;
                    S.h_word0[h] = (j << 16) | qi;
                    S.h_gid[h] = (uint32_t)gid;
                    S.h_ex[h] = ex;
                    S.h_low[h] = low;
                    S.h_rd[h] = rd;
                    S.h_err[h] = err;
                };
                if constexpr (W >= 16) {
                    // P >= 512: four lanes per vector, the chunk in two halves of 64 vectors;
                    // each lane issues all of its loads from the vector's refinement record
                    // (W/4 sign-code words, W/8 ex-code groups of 56 bytes, the ex-factors)
                    // before any arithmetic, so a half costs one memory round trip instead of
                    // one per loop iteration
                    constexpr int kWq = W / 4, kG = W / 8;
#pragma unroll 1
                    for (uint32_t half = 0; half < 2; ++half) {
                        const uint32_t e = half * 64 + (tid >> 2), sub = tid & 3;
                        const uint32_t li = e < cn ? S.win[c0 + e] : 0u;
                        const float low = e < cn ? S.l_low[li] : processed_mark();
                        const bool have = low < thr;
                        const uint32_t pos = have ? S.l_pos[li] : 0u;
                        uint32_t j = 0;
                        while (have && pos >= S.off[j + 1])
                            ++j;
                        const size_t gid = (size_t)S.start[j] + (pos - S.off[j]);
                        const uint8_t *rec = p.ex_rec + gid * p.ex_stride;
                        uint32_t pz = 0;  // opaque zero, as below
                        asm volatile("" : "+s"(pz));
                        const uint32_t *planes = S.planes + pz;
                        const float *qv = s_q + pz;
                        uint32_t xw[kWq];
                        uint2 grp[kG][7];
                        float fa = 0.0f, fr = 0.0f;
                        if (have) {
                            // sign-code words sub kWq .. sub kWq + kWq - 1, in 8-byte pairs
                            const uint2 *wp = reinterpret_cast<const uint2 *>(rec + ex_record_sign_word(P, sub * kWq));
#pragma unroll
                            for (int i = 0; i < kWq / 2; ++i) {
                                const uint2 v = wp[i];
                                xw[2 * i] = v.x;
                                xw[2 * i + 1] = v.y;
                            }
#pragma unroll
                            for (int gi = 0; gi < kG; ++gi) {
                                const uint2 *gp =
                                    reinterpret_cast<const uint2 *>(rec + ex_record_group_word(P, sub + 4 * gi, 0));
#pragma unroll
                                for (int k = 0; k < 7; ++k)
                                    grp[gi][k] = gp[k];
                            }
                            if (sub == 0) {
                                const float2 f = *reinterpret_cast<const float2 *>(rec + P);
                                fa = f.x;
                                fr = f.y;
                            }
                        }
                        int ipa = 0, ipb = 0;
                        float ipx = 0.0f;
                        if (have) {
#pragma unroll
                            for (int i = 0; i < kWq; ++i) {
                                const uint32_t w = sub * kWq + i;
#pragma unroll
                                for (int b = 0; b < kBq - 1; ++b) {
                                    ipa += __popc(xw[i] & planes[b * W + w]) << b;
                                    ipb += __popc(xw[i] & planes[(kBq + b) * W + w]) << b;
                                }
                                ipa -= __popc(xw[i] & planes[(kBq - 1) * W + w]) << (kBq - 1);
                                ipb -= __popc(xw[i] & planes[(2 * kBq - 1) * W + w]) << (kBq - 1);
                            }
#pragma unroll
                            for (int gi = 0; gi < kG; ++gi)
                                ipx += excode_group_ip(grp[gi], qv + 64 * (sub + 4 * gi));
                        }
#pragma unroll
                        for (int o = 1; o < 4; o <<= 1) {
                            ipa += __shfl_xor(ipa, o, 4);
                            ipb += __shfl_xor(ipb, o, 4);
                            ipx += __shfl_xor(ipx, o, 4);
                        }
                        if (sub == 0)
                            emit(e, have, j, pos, gid, low, ipa, ipb, ipx, fa, fr);
                    }
                } else {
                {
                    // vector e of the chunk on lanes 2e, 2e+1; each lane takes every other code
                    // word and every other 8-dimension ex-code chunk, so all loads of the chunk
                    // are in flight together
                    const uint32_t e = tid >> 1, sub = tid & 1;
                    const uint32_t li = e < cn ? S.win[c0 + e] : 0u;
                    const float low = e < cn ? S.l_low[li] : processed_mark();
                    const bool have = low < thr;
                    const uint32_t pos = have ? S.l_pos[li] : 0u;
                    uint32_t j = 0;
                    while (have && pos >= S.off[j + 1])
                        ++j;
                    const size_t gid = (size_t)S.start[j] + (pos - S.off[j]);
                    const uint8_t *code = p.ex_rec + gid * p.ex_stride;
                    int ipa = 0, ipb = 0;
                    float ipx = 0.0f, fa = 0.0f, fr = 0.0f;
                    // an opaque zero: plane and q' reads indexed with it stay in the chunk
                    // instead of being hoisted into registers (half of q' alone would take
                    // 384 per lane at P = 768)
                    uint32_t pz = 0;
                    asm volatile("" : "+s"(pz));
                    const uint32_t *planes = S.planes + pz;
                    const float *qv = s_q + pz;
                    if (have) {
                        if (sub == 0) {
                            const float2 f = *reinterpret_cast<const float2 *>(code + P);
                            fa = f.x;
                            fr = f.y;
                        }
                        constexpr int kWl = W > 0 ? (W + 1) / 2 : kVqMaxW / 2;
                        // lane sub takes the sign-code words sub nw/2 .. (sub + 1) nw/2 - 1 (nw is
                        // even: P % 64 == 0); two words per iteration: unrolled fully, the 16
                        // plane reads per word would all be scheduled ahead (192 registers at
                        // P = 768)
                        const uint32_t half_w = nw / 2;
#pragma unroll 2
                        for (int i = 0; i < kWl; ++i) {
                            if ((uint32_t)i < half_w) {
                                const uint32_t w = sub * half_w + i;
                                const uint32_t xw = *reinterpret_cast<const uint32_t *>(code + ex_record_sign_word(P, w));
#pragma unroll
                                for (int b = 0; b < kBq - 1; ++b) {
                                    ipa += __popc(xw & planes[b * nw + w]) << b;
                                    ipb += __popc(xw & planes[(kBq + b) * nw + w]) << b;
                                }
                                ipa -= __popc(xw & planes[(kBq - 1) * nw + w]) << (kBq - 1);
                                ipb -= __popc(xw & planes[(2 * kBq - 1) * nw + w]) << (kBq - 1);
                            }
                        }
                        constexpr int kCl = W > 0 ? 2 * W : 2 * kVqMaxW;  // P/8 chunks over 2 lanes
#pragma unroll 4
                        for (int i = 0; i < kCl; ++i) {
                            const uint32_t c = sub + 2 * i;
                            if (c < P / 8)
                                ipx += excode_chunk_ip<false>(code, P, qv, c);
                        }
                    }
                    ipa += __shfl_xor(ipa, 1, 2);
                    ipb += __shfl_xor(ipb, 1, 2);
                    ipx += __shfl_xor(ipx, 1, 2);
                    if (sub == 0 && e < kVqChunk)
                        emit(e, have, j, pos, gid, low, ipa, ipb, ipx, fa, fr);
                }
                }
                __syncthreads();
                // merge the chunk's entering vectors (refined, below the current k-th key) into
                // the top-k: rank = entries with a smaller key
                const uint32_t kc = S.kc, tb = S.tb;
                const unsigned long long worst = kc == topk ? S.t_key[tb][topk - 1] : ~0ull;
                unsigned long long ckey = ~0ull, em = 0;
                if (wave < kVqChunk / 64) {
                    ckey = S.c_key[tid];
                    const unsigned long long vm = __ballot(ckey != ~0ull);
                    em = __ballot(ckey != ~0ull && ckey < worst);
                    if (lane == 0) {
                        S.cnt[wave][0] = (uint32_t)__popcll(vm);
                        S.cnt[wave][1] = (uint32_t)__popcll(em);
                    }
                }
                __syncthreads();
                uint32_t valid = 0, enter = 0, before = 0;
#pragma unroll
                for (uint32_t w = 0; w < kVqChunk / 64; ++w) {
                    valid += S.cnt[w][0];
                    enter += S.cnt[w][1];
                    before += w < wave ? S.cnt[w][1] : 0u;
                }
                if (tid == 0)
                    S.nrefined += valid;
                if (enter) {
                    if (wave < kVqChunk / 64 && ((em >> lane) & 1ull)) {
                        const uint32_t o = before + lane_rank(em);
                        S.e_key[o] = ckey;
                        S.e_err[o] = S.c_err[tid];
                        S.e_low[o] = S.c_low[tid];
                    }
                    __syncthreads();
                    for (uint32_t i = tid; i < kc + enter; i += kVqThreads) {
                        unsigned long long key;
                        float err, low;
                        uint32_t rank = 0;
                        if (i < kc) {
                            key = S.t_key[tb][i];
                            err = S.t_err[tb][i];
                            low = S.t_low[tb][i];
                            rank = i;
                        } else {
                            const uint32_t e = i - kc;
                            key = S.e_key[e];
                            err = S.e_err[e];
                            low = S.e_low[e];
                            uint32_t lo = 0, hi = kc;  // top-k keys below key (sorted)
                            while (lo < hi) {
                                const uint32_t mid = (lo + hi) >> 1;
                                if (S.t_key[tb][mid] < key)
                                    lo = mid + 1;
                                else
                                    hi = mid;
                            }
                            rank = lo;
                        }
                        for (uint32_t e = 0; e < enter; ++e)
                            rank += S.e_key[e] < key ? 1u : 0u;
                        if (rank < topk) {
                            S.t_key[tb ^ 1][rank] = key;
                            S.t_err[tb ^ 1][rank] = err;
                            S.t_low[tb ^ 1][rank] = low;
                        }
                    }
                    __syncthreads();
                    const uint32_t kn = min(topk, kc + enter);
                    if (kn == topk && wave == 0) {
                        // threshold backed by the k best: max(d_k + e, l) + 1 ulp (one wave: topk
                        // <= 128, two entries a lane)
                        uint32_t ekey = 0, lkey = 0;
                        for (uint32_t i = lane; i < topk; i += 64) {
                            ekey = max(ekey, __float_as_uint(S.t_err[tb ^ 1][i]));  // >= 0: bits order like values
                            lkey = max(lkey, order_key(S.t_low[tb ^ 1][i]));
                        }
#pragma unroll
                        for (int o = 32; o > 0; o >>= 1) {
                            ekey = max(ekey, (uint32_t)__shfl_xor(ekey, o));
                            lkey = max(lkey, (uint32_t)__shfl_xor(lkey, o));
                        }
                        if (lane == 0) {
                            const float dk = key_to_float((uint32_t)(S.t_key[tb ^ 1][topk - 1] >> 32));
                            const float t =
                                nextafterf(fmaxf(dk + __uint_as_float(ekey), key_to_float(lkey)), FLT_MAX);
                            if (t < S.thr)
                                S.thr = t;
                        }
                    }
                    if (tid == 0) {
                        S.kc = kn;
                        S.tb = tb ^ 1;
                    }
                }
                if (tid == 0)
                    S.nheld = held0 + cn;
                __syncthreads();
            }
            // every window entry is done: refined, or at/above the threshold
            for (uint32_t i = tid; i < nwin; i += kVqThreads)
                S.l_low[S.win[i]] = processed_mark();
            __syncthreads();
        }

    };
    if constexpr (kPre) {
        // ---- precomputed bounds: wave w takes chunks w, w + 4, ... of the query (pairs in
        // probe order); four chunk buffers per wave, the current segment's two and the next
        // segment's two, which stay in flight (or in registers) across a refinement of the
        // list (six VGPRs per chunk) ----
        struct Chunk {
            float4 v;                // bounds of vectors 4 lane .. 4 lane + 3 of the chunk
            uint32_t lim, posbase;   // wave-uniform: valid vectors, list position of vector 0
        };
        // pair cursor, advanced by fetches in increasing chunk order
        uint32_t jf = 0, f_next = uniform(S.toff[1]), f_toff = 0, f_n = uniform(S.n[0]), f_off = 0;
        auto fetch = [&](uint32_t gg, Chunk &c) {
            while (gg >= f_next) {
                ++jf;
                f_toff = f_next;
                f_next = uniform(S.toff[jf + 1]);
                f_n = uniform(S.n[jf]);
                f_off = uniform(S.off[jf]);
            }
            const uint32_t lc = gg - f_toff;
            // the pair's slice is padded to whole chunks: lanes past the cluster read values
            // that lim masks
            c.v = *reinterpret_cast<const float4 *>(p.van_lows + ((size_t)qi * V + jf) * p.van_stride +
                                                    lc * kPreChunk + 4 * lane);
            c.lim = f_n - lc * kPreChunk;
            c.posbase = f_off + lc * kPreChunk;
        };
        auto scan = [&](const Chunk &c, float cut) {
            const float lv[4] = {c.v.x, c.v.y, c.v.z, c.v.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t i = 4 * lane + (uint32_t)r;
                const bool pass = i < c.lim && lv[r] < cut;
                const unsigned long long m = __ballot(pass);
                if (m) {
                    uint32_t base = 0;
                    if (lane == 0)
                        base = atomicAdd(&S.nlist, (uint32_t)__popcll(m));
                    base = uniform(base);
                    if (pass) {
                        const uint32_t k = base + lane_rank(m);
                        S.l_low[k] = lv[r];
                        S.l_pos[k] = c.posbase + i;
                    }
                }
            }
        };
        const uint32_t per_seg = kPreSegChunks * kVqWaves;
        const uint32_t nseg = (T + per_seg - 1) / per_seg;
        Chunk c0{}, c1{}, c2{}, c3{};
        if (wave < T)
            fetch(wave, c0);
        if (wave + kVqWaves < T)
            fetch(wave + kVqWaves, c1);
        if (wave + per_seg < T)
            fetch(wave + per_seg, c2);
        if (wave + per_seg + kVqWaves < T)
            fetch(wave + per_seg + kVqWaves, c3);
        // segment seg scans a, b (chunks g0, g0 + 4 of this wave); na, nb hold segment seg + 1;
        // a, b are refilled with segment seg + 2
        auto segment = [&](uint32_t seg, Chunk &a, Chunk &b, Chunk &na, Chunk &nb) {
            const float cut = S.thr;
            const uint32_t g0 = seg * per_seg + wave;
            if (g0 < T)
                scan(a, cut);
            if (g0 + kVqWaves < T)
                scan(b, cut);
            __syncthreads();
            const uint32_t g1 = g0 + per_seg, g2 = g1 + per_seg;
            if (S.nlist >= kVqHigh || seg + 1 == nseg) {
                process_list();
                if (tid == 0)
                    S.nlist = 0;
                __syncthreads();
            }
            if (g2 < T)
                fetch(g2, a);
            if (g2 + kVqWaves < T)
                fetch(g2 + kVqWaves, b);
        };
        // one call site (the refinement code is inlined once); the buffers rotate by value
        for (uint32_t seg = 0; seg < nseg; ++seg) {
            segment(seg, c0, c1, c2, c3);
            const Chunk t0 = c0, t1 = c1;
            c0 = c2;
            c1 = c3;
            c2 = t0;
            c3 = t1;
        }
    } else {
        // kBufs tile buffers per wave in turn: tile t is evaluated from one while tiles
        // t + 4, ..., t + 4 (kBufs - 1) are in flight into the others, then t + 4 kBufs is
        // fetched into the first; every kVqSegTiles tiles per wave the list is refined once
        // it holds kVqHigh entries
        constexpr int kBufs = W > 0 && W <= 8 ? 4 : 2;
        struct TileRegs {
            uint32_t x[K];
            float fa, fr, fe;
            // wave-uniform: the pair's g_add / g_error, the valid lanes of the tile and the
            // list position of its lane 0
            float gadd, gerr;
            uint32_t lim, posbase;
        };
        TileRegs bufs[kBufs];
        // pair of the fetch cursor and its constants, wave-uniform (scalar registers); the
        // fetches are in increasing tile order
        uint32_t jf = 0, f_next = uniform(S.toff[1]), f_toff = 0, f_tbase = uniform(S.tbase[0]);
        uint32_t f_n = uniform(S.n[0]), f_off = 0;
        float f_gadd = uniformf(S.gadd[0]), f_gerr = uniformf(S.gerr[0]);
        auto fetch = [&](uint32_t tt, TileRegs &r) {
            while (tt >= f_next) {
                ++jf;
                f_toff = f_next;
                f_next = uniform(S.toff[jf + 1]);
                f_tbase = uniform(S.tbase[jf]);
                f_n = uniform(S.n[jf]);
                f_off = uniform(S.off[jf]);
                f_gadd = uniformf(S.gadd[jf]);
                f_gerr = uniformf(S.gerr[jf]);
            }
            const uint32_t lt = tt - f_toff;
            const uint8_t *tile = p.tiles + (size_t)(f_tbase + lt) * p.tile_bytes;
            load_codes<W>(tile, lane, nw, r.x);
            const float *fac = reinterpret_cast<const float *>(tile + 256u * nw);
            r.fa = fac[lane];
            r.fr = fac[64 + lane];
            r.fe = fac[128 + lane];
            r.gadd = f_gadd;
            r.gerr = f_gerr;
            r.lim = f_n - lt * kTileVectors;
            r.posbase = f_off + lt * kTileVectors;
        };
        uint32_t t = wave;
    #pragma unroll
        for (int b = 0; b < kBufs; ++b)
            if (t + b * kVqWaves < T)
                fetch(t + b * kVqWaves, bufs[b]);
        auto step = [&](TileRegs &cur, float cut) {
            int ip;
            if constexpr (W > 0 && W <= 4) {
                ip = popc_ip<W>(cur.x, preg, nw);
            } else if constexpr (W >= 16) {
                ip = popc_ip_scalar<W>(cur.x, cplanes);
            } else {
                ip = popc_ip<W>(cur.x, S.planes, nw);
            }
            const float ex = width * (float)ip;
            const float low = cur.fa + cur.gadd + cur.fr * (ex + k1) - cur.fe * cur.gerr;
            const bool pass = lane < cur.lim && low < cut;
            const unsigned long long m = __ballot(pass);
            if (m) {
                uint32_t base = 0;
                if (lane == 0)
                    base = atomicAdd(&S.nlist, (uint32_t)__popcll(m));
                base = uniform(base);
                if (pass) {
                    const uint32_t k = base + lane_rank(m);
                    S.l_low[k] = low;
                    S.l_pos[k] = cur.posbase + lane;
                }
            }
            if (t + kBufs * kVqWaves < T)
                fetch(t + kBufs * kVqWaves, cur);
            t += kVqWaves;
        };
        // a segment is kVqSegTiles (a multiple of kBufs) tiles per wave, so every segment
        // starts on buffer 0 and the buffer of each step is a constant
        static_assert(kVqSegTiles % kBufs == 0, "segments start on the first buffer");
        const uint32_t nseg = (T + kVqWaves * kVqSegTiles - 1) / (kVqWaves * kVqSegTiles);
        for (uint32_t seg = 0; seg < nseg; ++seg) {
            const float cut = S.thr;
            const uint32_t seg_end = min(T, (seg + 1) * kVqWaves * kVqSegTiles);
            if constexpr (W > 0 && W <= 4) {
    #pragma unroll
                for (int i = 0; i < kBq * W; ++i)
                    preg[i] = S.planes[i];
            }
            for (uint32_t r = 0; r < kVqSegTiles / kBufs; ++r) {
    #pragma unroll
                for (int b = 0; b < kBufs; ++b)
                    if (t < seg_end)
                        step(bufs[b], cut);
            }
            __syncthreads();
            if (S.nlist >= kVqHigh || seg + 1 == nseg) {
                process_list();
                if (tid == 0)
                    S.nlist = 0;
                __syncthreads();
                if constexpr (W >= 16) {
                    // P >= 512: the tiles prefetched before the refinement are fetched again
                    // after it (the cursor restarts at the first pair), so they hold no
                    // registers across it; 2 tiles per wave and refinement, ~6% of the
                    // query's tile bytes
                    jf = 0;
                    f_toff = 0;
                    f_next = uniform(S.toff[1]);
                    f_tbase = uniform(S.tbase[0]);
                    f_n = uniform(S.n[0]);
                    f_off = 0;
                    f_gadd = uniformf(S.gadd[0]);
                    f_gerr = uniformf(S.gerr[0]);
    #pragma unroll
                    for (int b = 0; b < kBufs; ++b) {
                        if (t + b * kVqWaves < T)
                            fetch(t + b * kVqWaves, bufs[b]);
                        else
                            bufs[b] = TileRegs{};
                    }
                }
            }
        }
    }

    // ---- 3. the query's threshold and publication ----
    if (tid == 0) {
        if (S.ndropped)
            atomicAdd(p.dropped, (unsigned long long)S.ndropped);
        if (S.nrefined)
            atomicAdd(va.refined, (unsigned long long)S.nrefined);
        const float thr = S.thr;
        if (S.kc == topk && thr < thr_in) {
            uint32_t *slot = reinterpret_cast<uint32_t *>(va.thr_out) + qi;
            if (!early_pub) {
                // none of the query's records has been published in this search yet (the far
                // pass runs after this kernel), so no consumer has changed its threshold since
                // the snapshot thr_in: a store lowers it without a host round trip
                __hip_atomic_store(slot, __float_as_uint(thr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            } else {
                uint32_t cur = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                while (thr < __uint_as_float(cur)) {
                    if (__hip_atomic_compare_exchange_strong(slot, &cur, __float_as_uint(thr),
                                                             __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_SYSTEM))
                        break;
                }
            }
            atomicAdd(va.seeded, 1ull);
        }
    }
    publish_held(S, q, true, p.dropped);
}

template <int W>
void launch_vq_w(const ScanParams &p, const VanguardArgs &va, uint32_t nq, hipStream_t s) {
    const size_t dyn = (size_t)p.P * sizeof(float);
    const uint32_t grid = (nq + kNumXcd - 1) / kNumXcd * kNumXcd;
    if (va.lows_ready)
        vanguard_query_kernel<W, true><<<grid, kVqThreads, dyn, s>>>(p, va);
    else
        vanguard_query_kernel<W, false><<<grid, kVqThreads, dyn, s>>>(p, va);
}

// Queries ordered by nearest probed cluster (counting sort in one workgroup; the order
// inside a cluster is not fixed). nlist <= kOrderBins.
constexpr uint32_t kOrderBins = 16384;
constexpr uint32_t kOrderThreads = 1024;

__global__ __launch_bounds__(kOrderThreads) void order_queries_kernel(const int32_t *__restrict__ probe_idx,
                                                                      uint32_t nq, uint32_t nprobe,
                                                                      uint32_t nlist,
                                                                      uint32_t *__restrict__ order) {
    extern __shared__ uint32_t h[];
    __shared__ uint32_t s_red[kOrderThreads / 64];
    const uint32_t t = threadIdx.x;
    for (uint32_t c = t; c < nlist; c += kOrderThreads)
        h[c] = 0;
    __syncthreads();
    for (uint32_t q = t; q < nq; q += kOrderThreads)
        atomicAdd(&h[probe_idx[(size_t)q * nprobe]], 1u);
    __syncthreads();
    // exclusive scan: thread t owns bins [t * per, (t + 1) * per)
    const uint32_t per = (nlist + kOrderThreads - 1) / kOrderThreads;
    const uint32_t c0 = min(nlist, t * per), c1 = min(nlist, c0 + per);
    uint32_t sum = 0;
    for (uint32_t c = c0; c < c1; ++c)
        sum += h[c];
    const uint32_t lane = t & 63, wave = t >> 6;
    uint32_t v = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(v, o);
        if (lane >= (uint32_t)o)
            v += y;
    }
    if (lane == 63)
        s_red[wave] = v;
    __syncthreads();
    uint32_t base = v - sum;
    for (uint32_t w = 0; w < wave; ++w)
        base += s_red[w];
    for (uint32_t c = c0; c < c1; ++c) {
        const uint32_t n = h[c];
        h[c] = base;
        base += n;
    }
    __syncthreads();
    for (uint32_t q = t; q < nq; q += kOrderThreads)
        order[atomicAdd(&h[probe_idx[(size_t)q * nprobe]], 1u)] = q;
}

}  // namespace

size_t vanguard_static_lds() { return sizeof(VqShared); }

bool launch_order_queries(const int32_t *probe_idx, uint32_t nq, uint32_t nprobe, uint32_t nlist,
                          uint32_t *order, hipStream_t s) {
    if (nlist > kOrderBins || nq == 0)
        return false;
    order_queries_kernel<<<1, kOrderThreads, (size_t)nlist * sizeof(uint32_t), s>>>(probe_idx, nq, nprobe,
                                                                                  nlist, order);
    return true;
}

void launch_vanguard_query(const ScanParams &p, const VanguardArgs &va, uint32_t W, uint32_t nq,
                           hipStream_t s) {
    if (nq == 0 || va.depth == 0)
        return;
    switch (W) {
    case 2: launch_vq_w<2>(p, va, nq, s); break;
    case 4: launch_vq_w<4>(p, va, nq, s); break;
    case 8: launch_vq_w<8>(p, va, nq, s); break;
    case 24: launch_vq_w<24>(p, va, nq, s); break;
    default: launch_vq_w<0>(p, va, nq, s); break;
    }
}

}  // namespace cora
