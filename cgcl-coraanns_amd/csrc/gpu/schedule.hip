// Pair scheduling: the reference flattens (cluster, query, probe) pairs and sorts them
// with PairSortCompare — vanguard pairs (probe < vanguard) first, then by cluster
// (query_kernels.cuh:105-113, kernel_types.cuh:34-60, hybrid.cu:504-508). Here the
// same grouping is a counting sort into 2*nlist buckets (bucket = cluster for vanguard
// pairs, nlist + cluster for the rest) followed by cutting every bucket into scan
// units of at most batch_q pairs (van_batch for vanguard buckets: 1 for the per-pair
// passes, the matrix-core unit size for the vanguard lows pass), each split further into
// ranges of at most kUnitTiles tiles of the cluster. Pair order inside a bucket is not
// fixed; every pair's results are independent of it.
#include "engine_internal.h"

namespace cora {
namespace {

__global__ void fill_u32_kernel(uint32_t *p, uint32_t v, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void fill_u64_kernel(unsigned long long *p, unsigned long long v, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// Bucket of pair i: cluster for vanguard pairs (probe rank < vanguard), nlist + cluster
// for the rest.
__device__ __forceinline__ uint32_t pair_bucket(const int32_t *__restrict__ probe_idx, size_t i,
                                                uint32_t nprobe, uint32_t nlist, uint32_t vanguard) {
    const uint32_t p = (uint32_t)(i % nprobe);
    return (p >= vanguard ? nlist : 0u) + (uint32_t)probe_idx[i];
}

// Counting with a per-block LDS histogram over contiguous pair ranges, so a bucket takes
// one global atomic per block instead of one per pair (popular clusters otherwise
// serialise thousands of same-address atomics). Needs 2 * nlist <= kLdsBuckets (128 KB of
// LDS at the maximum, beyond the default 64 KB dynamic limit).
constexpr uint32_t kLdsBuckets = 32768;
constexpr uint32_t kHistThreads = 1024;
constexpr uint32_t kHistPairs = 4096;  // pairs per block

__global__ __launch_bounds__(kHistThreads) void count_pairs_lds_kernel(
    const int32_t *__restrict__ probe_idx, size_t np, uint32_t nprobe, uint32_t nlist,
    uint32_t vanguard, uint32_t *__restrict__ count) {
    extern __shared__ uint32_t h[];
    const uint32_t nb = 2 * nlist, t = threadIdx.x;
    for (uint32_t b = t; b < nb; b += kHistThreads)
        h[b] = 0;
    __syncthreads();
    const size_t b0 = (size_t)blockIdx.x * kHistPairs, b1 = min(np, b0 + kHistPairs);
    for (size_t i = b0 + t; i < b1; i += kHistThreads)
        atomicAdd(&h[pair_bucket(probe_idx, i, nprobe, nlist, vanguard)], 1u);
    __syncthreads();
    for (uint32_t b = t; b < nb; b += kHistThreads)
        if (h[b])
            atomicAdd(&count[b], h[b]);
}

// Each block reserves one range per bucket it touches, then places its pairs in it.
__global__ __launch_bounds__(kHistThreads) void scatter_pairs_lds_kernel(
    const int32_t *__restrict__ probe_idx, size_t np, uint32_t nprobe, uint32_t nlist,
    uint32_t vanguard, const uint32_t *__restrict__ bucket_offset, uint32_t *__restrict__ cursor,
    Pair *__restrict__ pairs) {
    extern __shared__ uint32_t h[];
    const uint32_t nb = 2 * nlist, t = threadIdx.x;
    for (uint32_t b = t; b < nb; b += kHistThreads)
        h[b] = 0;
    __syncthreads();
    const size_t b0 = (size_t)blockIdx.x * kHistPairs, b1 = min(np, b0 + kHistPairs);
    for (size_t i = b0 + t; i < b1; i += kHistThreads)
        atomicAdd(&h[pair_bucket(probe_idx, i, nprobe, nlist, vanguard)], 1u);
    __syncthreads();
    for (uint32_t b = t; b < nb; b += kHistThreads)
        if (h[b])
            h[b] = bucket_offset[b] + atomicAdd(&cursor[b], h[b]);
    __syncthreads();
    for (size_t i = b0 + t; i < b1; i += kHistThreads) {
        const uint32_t q = (uint32_t)(i / nprobe), p = (uint32_t)(i % nprobe);
        const uint32_t pos = atomicAdd(&h[pair_bucket(probe_idx, i, nprobe, nlist, vanguard)], 1u);
        pairs[pos] = Pair{(p << 16) | q, (uint32_t)probe_idx[i]};
    }
}

__global__ void count_pairs_kernel(const int32_t *__restrict__ probe_idx, uint32_t nq,
                                   uint32_t nprobe, uint32_t nlist, uint32_t vanguard,
                                   uint32_t *__restrict__ count) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= (size_t)nq * nprobe)
        return;
    const uint32_t p = (uint32_t)(i % nprobe);
    const uint32_t c = (uint32_t)probe_idx[i];
    atomicAdd(&count[(p >= vanguard ? nlist : 0u) + c], 1u);
}

// Bucket scan over many workgroups, kScanBlock buckets each (one a thread): the first
// kernel writes every block's totals of the eight sums, the second scans its buckets on
// top of the totals of the blocks before it, and its last block writes the grand totals.
// The second also clears each bucket's scatter cursor and, once it has read it, its count,
// so the next search's counting starts from zero without a fill.
constexpr uint32_t kScanBlock = 1024;
constexpr int kScanWaves = kScanBlock / 64;
constexpr int kScanSums = 8;

// The eight per-bucket terms: pairs, units, vanguard units, far-scan bytes, far units, far
// pair-vectors, vanguard-scan bytes, vanguard pair-vectors. Buckets past the end add nothing.
__device__ __forceinline__ void bucket_terms(uint32_t b, uint32_t nb, const uint32_t *count,
                                             const ClusterMeta *__restrict__ meta, uint32_t nlist,
                                             uint32_t batch_q, uint32_t van_batch, uint32_t bpv,
                                             unsigned long long v[kScanSums]) {
    const uint32_t m = b < nb ? count[b] : 0u;
    const uint32_t n = b < nb ? meta[b < nlist ? b : b - nlist].n : 0u;
    const bool van = b < nlist;
    const uint32_t u = (m + (van ? van_batch : batch_q) - 1) / (van ? van_batch : batch_q);
    const unsigned long long scan = (unsigned long long)u * n * bpv, pv = (unsigned long long)m * n;
    v[0] = m;
    v[1] = (unsigned long long)u * unit_splits(n);
    v[2] = van ? v[1] : 0ull;
    v[3] = van ? 0ull : scan;
    v[4] = van ? 0ull : u;
    v[5] = van ? 0ull : pv;
    v[6] = van ? scan : 0ull;
    v[7] = van ? pv : 0ull;
}

__global__ __launch_bounds__(kScanBlock) void bucket_totals_kernel(
    const uint32_t *__restrict__ count, const ClusterMeta *__restrict__ meta, uint32_t nlist,
    uint32_t batch_q, uint32_t van_batch, uint32_t bpv, unsigned long long *__restrict__ block_tot) {
    __shared__ unsigned long long s_w[kScanSums][kScanWaves];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    unsigned long long v[kScanSums];
    bucket_terms(blockIdx.x * kScanBlock + t, 2 * nlist, count, meta, nlist, batch_q, van_batch, bpv, v);
#pragma unroll
    for (int a = 0; a < kScanSums; ++a) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
            v[a] += __shfl_xor(v[a], o);
        if (lane == 0)
            s_w[a][wave] = v[a];
    }
    __syncthreads();
    if (t < (uint32_t)kScanSums) {
        unsigned long long x = 0;
        for (int w = 0; w < kScanWaves; ++w)
            x += s_w[t][w];
        block_tot[(size_t)t * gridDim.x + blockIdx.x] = x;
    }
}

__global__ __launch_bounds__(kScanBlock) void bucket_scan_kernel(
    uint32_t *count /*cleared after it is read*/, const ClusterMeta *__restrict__ meta, uint32_t nlist,
    uint32_t batch_q, uint32_t van_batch, uint32_t bpv, const unsigned long long *__restrict__ block_tot,
    uint32_t *__restrict__ cursor, uint32_t *__restrict__ bucket_offset, uint32_t *__restrict__ unit_offset, uint32_t *__restrict__ num_units,
    unsigned long long *__restrict__ stats) {
    __shared__ uint32_t s_w[2][kScanWaves];
    __shared__ unsigned long long s_pre[2];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6, nb = 2 * nlist;
    const uint32_t b = blockIdx.x * kScanBlock + t;
    const uint32_t nblk = gridDim.x;
    // offsets of this block's first bucket: the totals of the blocks before it
    if (t < 2) {
        unsigned long long x = 0;
        for (uint32_t w = 0; w < blockIdx.x; ++w)
            x += block_tot[(size_t)t * nblk + w];
        s_pre[t] = x;
    }
    // the last block also writes the grand totals
    if (blockIdx.x == nblk - 1 && t >= 64 && t < 64 + (uint32_t)kScanSums) {
        const uint32_t a = t - 64;
        unsigned long long x = 0;
        for (uint32_t w = 0; w < nblk; ++w)
            x += block_tot[(size_t)a * nblk + w];
        switch (a) {
        case 0: bucket_offset[nb] = (uint32_t)x; break;
        case 1: unit_offset[nb] = (uint32_t)x; break;
        case 2: {
            unsigned long long all = 0;
            for (uint32_t w = 0; w < nblk; ++w)
                all += block_tot[(size_t)1 * nblk + w];
            num_units[0] = (uint32_t)x;
            num_units[1] = (uint32_t)(all - x);
            break;
        }
        case 3: stats[0] = x; break;
        case 4: stats[1] = x; break;
        case 5: stats[2] = x; break;
        case 6: stats[9] = x; break;
        default: stats[10] = x; break;
        }
    }
    unsigned long long v[kScanSums];
    bucket_terms(b, nb, count, meta, nlist, batch_q, van_batch, bpv, v);
    // inclusive scans of pairs and units within the wave, then the waves before
    uint32_t inc[2] = {(uint32_t)v[0], (uint32_t)v[1]};
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(inc[a], o);
            if (lane >= (uint32_t)o)
                inc[a] += y;
        }
        if (lane == 63)
            s_w[a][wave] = inc[a];
    }
    __syncthreads();
    if (b >= nb)
        return;
    uint32_t off[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        uint32_t x = (uint32_t)s_pre[a] + inc[a] - (uint32_t)v[a];
        for (uint32_t w = 0; w < wave; ++w)
            x += s_w[a][w];
        off[a] = x;
    }
    bucket_offset[b] = off[0];
    unit_offset[b] = off[1];
    cursor[b] = 0u;
    count[b] = 0u;  // read above (bucket_terms) and by the totals kernel before
}

__global__ void scatter_pairs_kernel(const int32_t *__restrict__ probe_idx, uint32_t nq,
                                     uint32_t nprobe, uint32_t nlist, uint32_t vanguard,
                                     const uint32_t *__restrict__ bucket_offset,
                                     uint32_t *__restrict__ cursor, Pair *__restrict__ pairs) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= (size_t)nq * nprobe)
        return;
    const uint32_t q = (uint32_t)(i / nprobe), p = (uint32_t)(i % nprobe);
    const uint32_t c = (uint32_t)probe_idx[i];
    const uint32_t b = (p >= vanguard ? nlist : 0u) + c;
    const uint32_t pos = bucket_offset[b] + atomicAdd(&cursor[b], 1u);
    pairs[pos] = Pair{(p << 16) | q, c};
}

__global__ void build_units_kernel(const uint32_t *__restrict__ bucket_offset,
                                   const uint32_t *__restrict__ unit_offset,
                                   const uint32_t *__restrict__ num_units,
                                   const ClusterMeta *__restrict__ meta, uint32_t nlist,
                                   uint32_t batch_q, uint32_t van_batch, uint64_t max_units,
                                   Unit *__restrict__ units) {
    const uint64_t u64 = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
    if (u64 >= max_units || u64 >= (uint64_t)num_units[0] + num_units[1])
        return;
    const uint32_t u = (uint32_t)u64;
    // last bucket b with unit_offset[b] <= u (empty buckets share offsets)
    uint32_t lo = 0, hi = 2 * nlist;  // unit_offset[2*nlist] = total > u
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (unit_offset[mid] <= u)
            lo = mid;
        else
            hi = mid;
    }
    const uint32_t b = lo, c = b % nlist;
    const uint32_t q = b < nlist ? van_batch : batch_q;
    const uint32_t n = meta[c].n, sp = unit_splits(n), ntiles = (n + kTileVectors - 1) / kTileVectors;
    const uint32_t local = u - unit_offset[b];
    const uint32_t group = local / sp, split = local % sp;
    const uint32_t m = bucket_offset[b + 1] - bucket_offset[b];
    const uint32_t t0 = split * kUnitTiles, tc = min(kUnitTiles, ntiles - min(ntiles, t0));
    units[u] = Unit{c, bucket_offset[b] + group * q, min(q, m - group * q), (t0 << 8) | tc};
}

}  // namespace

size_t bucket_scan_words(uint32_t nlist) {
    return (size_t)kScanSums * ((2 * (size_t)nlist + kScanBlock - 1) / kScanBlock);
}

void launch_fill_u32(uint32_t *p, uint32_t value, size_t n, hipStream_t s) {
    if (!n)
        return;
    const uint32_t grid = (uint32_t)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    fill_u32_kernel<<<grid, 256, 0, s>>>(p, value, n);
}

void launch_fill_u64(unsigned long long *p, unsigned long long value, size_t n, hipStream_t s) {
    if (!n)
        return;
    const uint32_t grid = (uint32_t)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    fill_u64_kernel<<<grid, 256, 0, s>>>(p, value, n);
}

void launch_build_pairs(const int32_t *probe_idx, const ClusterMeta *meta, uint32_t nq,
                        uint32_t nprobe, uint32_t nlist, uint32_t vanguard, uint32_t batch_q,
                        uint32_t van_batch, uint32_t bytes_per_vector, uint32_t *bucket_count,
                        uint32_t *bucket_cursor,
                        uint32_t *bucket_offset, uint32_t *unit_offset, Pair *pairs, Unit *units,
                        uint64_t max_units, uint32_t *num_units, unsigned long long *scan_stats,
                        unsigned long long *block_tot, bool counts_zero, hipStream_t s) {
    const size_t np = (size_t)nq * nprobe;
    if (!counts_zero)
        launch_fill_u32(bucket_count, 0, 2 * (size_t)nlist, s);
    const uint32_t grid = (uint32_t)((np + 255) / 256);
    const bool lds = 2 * (size_t)nlist <= kLdsBuckets;
    const uint32_t hgrid = (uint32_t)((np + kHistPairs - 1) / kHistPairs);
    const size_t hbytes = 2 * (size_t)nlist * sizeof(uint32_t);
    static bool raised = false;  // dynamic LDS above 64 KB must be allowed explicitly
    if (lds && hbytes > 65536 && !raised) {
        for (const void *f : {reinterpret_cast<const void *>(&count_pairs_lds_kernel),
                              reinterpret_cast<const void *>(&scatter_pairs_lds_kernel)})
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)(kLdsBuckets * sizeof(uint32_t))) != hipSuccess)
                (void)hipGetLastError();  // leave no sticky error; the launch then reports it
        raised = true;
    }
    if (lds)
        count_pairs_lds_kernel<<<hgrid, kHistThreads, hbytes, s>>>(probe_idx, np, nprobe, nlist, vanguard,
                                                                  bucket_count);
    else
        count_pairs_kernel<<<grid, 256, 0, s>>>(probe_idx, nq, nprobe, nlist, vanguard, bucket_count);
    const uint32_t sgrid = (2 * nlist + kScanBlock - 1) / kScanBlock;
    bucket_totals_kernel<<<sgrid, kScanBlock, 0, s>>>(bucket_count, meta, nlist, batch_q, van_batch,
                                                      bytes_per_vector, block_tot);
    bucket_scan_kernel<<<sgrid, kScanBlock, 0, s>>>(bucket_count, meta, nlist, batch_q, van_batch,
                                                    bytes_per_vector, block_tot, bucket_cursor,
                                                    bucket_offset, unit_offset,
                                                    num_units, scan_stats);
    if (lds)
        scatter_pairs_lds_kernel<<<hgrid, kHistThreads, hbytes, s>>>(probe_idx, np, nprobe, nlist, vanguard,
                                                                    bucket_offset, bucket_cursor, pairs);
    else
        scatter_pairs_kernel<<<grid, 256, 0, s>>>(probe_idx, nq, nprobe, nlist, vanguard,
                                                  bucket_offset, bucket_cursor, pairs);
    build_units_kernel<<<(uint32_t)((max_units + 255) / 256), 256, 0, s>>>(
        bucket_offset, unit_offset, num_units, meta, nlist, batch_q, van_batch, max_units, units);
}

}  // namespace cora
