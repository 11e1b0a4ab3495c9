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

constexpr int kScanThreads = 1024;

// Single block: exclusive scans of bucket sizes and unit counts, unit totals and the
// algorithmic traffic of the far-pair scan.
__global__ __launch_bounds__(kScanThreads) void scan_buckets_kernel(
    const uint32_t *__restrict__ count, const ClusterMeta *__restrict__ meta, uint32_t nlist,
    uint32_t batch_q, uint32_t van_batch, uint32_t bpv, uint32_t *__restrict__ bucket_offset,
    uint32_t *__restrict__ unit_offset, uint32_t *__restrict__ num_units,
    unsigned long long *__restrict__ stats) {
    constexpr int kWaves = kScanThreads / 64;
    // per-wave totals of the eight sums (inclusive scans run within each wave by shuffles)
    __shared__ unsigned long long s_tot[8][kWaves];
    const uint32_t nb = 2 * nlist;
    const int t = threadIdx.x;
    const uint32_t chunk = (nb + kScanThreads - 1) / kScanThreads;
    const uint32_t b0 = min(nb, t * chunk), b1 = min(nb, b0 + chunk);
    uint32_t pairs = 0, units = 0, van_units = 0;
    unsigned long long bytes = 0, fu = 0, vec = 0, vbytes = 0, vvec = 0;
    // the thread's buckets 16 at a time: their loads issued together (one round trip per
    // 16 buckets instead of one per bucket; this single workgroup is latency-bound)
    constexpr uint32_t kBatch = 16;
    uint32_t mv[kBatch], nv[kBatch];
    auto fetch = [&](uint32_t bb) {
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t b = bb + j;
            mv[j] = b < b1 ? count[b] : 0u;
            nv[j] = b < b1 ? meta[b < nlist ? b : b - nlist].n : 0u;
        }
    };
    for (uint32_t bb = b0; bb < b1; bb += kBatch) {
        fetch(bb);
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t b = bb + j;  // past b1: m = 0 and n = 0, which add nothing
            const uint32_t m = mv[j];
            pairs += m;
            const uint32_t n = nv[j], sp = unit_splits(n);
            if (b < nlist) {
                const uint32_t u = (m + van_batch - 1) / van_batch;
                units += u * sp;
                van_units += u * sp;
                vbytes += (unsigned long long)u * n * bpv;  // one pass per vanguard unit
                vvec += (unsigned long long)m * n;
            } else {
                const uint32_t u = (m + batch_q - 1) / batch_q;
                units += u * sp;
                bytes += (unsigned long long)u * n * bpv;
                fu += u;
                vec += (unsigned long long)m * n;
            }
        }
    }
    // inclusive scans over the block: within each wave by shuffles, then the totals of the
    // waves before (one barrier)
    const int lane = t & 63, wave = t >> 6;
    unsigned long long v[8] = {pairs, units, van_units, bytes, fu, vec, vbytes, vvec};
#pragma unroll
    for (int a = 0; a < 8; ++a) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned long long y = __shfl_up(v[a], o);
            if (lane >= o)
                v[a] += y;
        }
        if (lane == 63)
            s_tot[a][wave] = v[a];
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 8; ++a)
        for (int w = 0; w < wave; ++w)
            v[a] += s_tot[a][w];
    uint32_t po = (uint32_t)v[0] - pairs, uo = (uint32_t)v[1] - units;
    for (uint32_t bb = b0; bb < b1; bb += kBatch) {
        fetch(bb);
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t b = bb + j;
            const uint32_t m = mv[j];
            if (b < b1) {
                bucket_offset[b] = po;
                unit_offset[b] = uo;
            }
            po += m;
            const uint32_t sp = unit_splits(nv[j]);
            uo += (b < nlist ? (m + van_batch - 1) / van_batch : (m + batch_q - 1) / batch_q) * sp;
        }
    }
    if (t == kScanThreads - 1) {
        bucket_offset[nb] = (uint32_t)v[0];
        unit_offset[nb] = (uint32_t)v[1];
        num_units[0] = (uint32_t)v[2];
        num_units[1] = (uint32_t)(v[1] - v[2]);
        stats[0] = v[3];
        stats[1] = v[4];
        stats[2] = v[5];
        stats[9] = v[6];
        stats[10] = v[7];
    }
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
                        hipStream_t s) {
    const size_t np = (size_t)nq * nprobe;
    launch_fill_u32(bucket_count, 0, 2 * (size_t)nlist, s);
    launch_fill_u32(bucket_cursor, 0, 2 * (size_t)nlist, s);
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
    scan_buckets_kernel<<<1, kScanThreads, 0, s>>>(bucket_count, meta, nlist, batch_q, van_batch,
                                                   bytes_per_vector, bucket_offset, unit_offset,
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
