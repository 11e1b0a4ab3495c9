// GPU-final top-k (CORA_FLAG_GPU_FINAL): the final per-query top-k formed on the GPU from
// the records the scan passes publish, for searches where the CPU refinement would bound the
// step (the idea of the reference's GPU baseline engine, src/baselines/gpu.cu:630-700).
//
// In this mode every publication site stores its record in the HBM spill array at the
// record's position (place_record) with the refined distance, which the fused vanguard pass
// and the refined pre-filter have already evaluated with the CPU consumer's formula
// (cpu_refinement.cpp:183-192), in place of exact_ip. Then:
//   1. count the records of each query;
//   2. exclusive scan of the counts (one workgroup);
//   3. scatter (refined distance key << 32 | cluster-order index) per query;
//   4. per query, the topk smallest keys in ascending order (ties by cluster-order index):
//      a bitonic sort in LDS for up to kFinalLds records, else a radix select of the
//      topk-th key over the query's records in HBM (eight 8-bit passes on the unique 64-bit
//      keys) and a sort of the topk selected.
// Unfilled slots get FLT_MAX and index 0xFFFFFFFF (the host maps indexes to ids).
#include <float.h>

#include "device_common.h"

namespace cora {
namespace {

constexpr int kFinalThreads = 256;
constexpr uint32_t kFinalLds = 4096;  // records sorted in LDS (32 KB)

__global__ void final_count_kernel(const SpillRecord *__restrict__ recs, const unsigned long long *__restrict__ n_ptr,
                                   unsigned long long cap, uint32_t *__restrict__ counts) {
    const unsigned long long n = min(*n_ptr, cap);
    for (unsigned long long i = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x; i < n;
         i += (unsigned long long)gridDim.x * blockDim.x)
        atomicAdd(&counts[recs[i].item.x & 0xFFFFu], 1u);
}

// offsets[0..nq] = exclusive prefix of counts; cursor[q] = 0
__global__ __launch_bounds__(1024) void final_scan_kernel(const uint32_t *__restrict__ counts, uint32_t nq,
                                                          uint32_t *__restrict__ offsets,
                                                          uint32_t *__restrict__ cursor) {
    __shared__ uint32_t s_w[16];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t per = (nq + 1023) / 1024;
    const uint32_t q0 = min(nq, t * per), q1 = min(nq, q0 + per);
    uint32_t sum = 0;
    for (uint32_t q = q0; q < q1; ++q)
        sum += counts[q];
    uint32_t x = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o);
        if (lane >= (uint32_t)o)
            x += y;
    }
    if (lane == 63)
        s_w[wave] = x;
    __syncthreads();
    uint32_t run = x - sum;
    for (uint32_t w = 0; w < wave; ++w)
        run += s_w[w];
    for (uint32_t q = q0; q < q1; ++q) {
        offsets[q] = run;
        cursor[q] = 0;
        run += counts[q];
    }
    if (t == 1023)
        offsets[nq] = run;
}

__global__ void final_scatter_kernel(const SpillRecord *__restrict__ recs, const unsigned long long *__restrict__ n_ptr,
                                     unsigned long long cap, const uint32_t *__restrict__ offsets,
                                     uint32_t *__restrict__ cursor, unsigned long long *__restrict__ keys) {
    const unsigned long long n = min(*n_ptr, cap);
    for (unsigned long long i = blockIdx.x * (unsigned long long)blockDim.x + threadIdx.x; i < n;
         i += (unsigned long long)gridDim.x * blockDim.x) {
        const uint4 r = recs[i].item;
        const uint32_t q = r.x & 0xFFFFu;
        const uint32_t slot = offsets[q] + atomicAdd(&cursor[q], 1u);
        keys[slot] = ((unsigned long long)order_key(__uint_as_float(r.z)) << 32) | r.y;
    }
}

__device__ __forceinline__ void bitonic_lds(unsigned long long *s, uint32_t n) {
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = threadIdx.x; i < n / 2; i += kFinalThreads) {
                const uint32_t lo = 2 * i - (i & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool up = (lo & size) == 0;
                const unsigned long long a = s[lo], b = s[hi];
                if ((a > b) == up) {
                    s[lo] = b;
                    s[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(kFinalThreads) void final_select_kernel(const unsigned long long *__restrict__ keys,
                                                                     const uint32_t *__restrict__ offsets,
                                                                     uint32_t topk, float *__restrict__ out_dist,
                                                                     uint32_t *__restrict__ out_idx) {
    __shared__ unsigned long long s[kFinalLds];
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_sel[2];
    __shared__ uint32_t s_n;
    const uint32_t q = blockIdx.x, t = threadIdx.x;
    const uint32_t b = offsets[q], n = offsets[q + 1] - b;
    const unsigned long long *k = keys + b;
    uint32_t m = n;  // sorted entries in s
    if (n <= kFinalLds) {
        uint32_t pw = 1;
        while (pw < n)
            pw <<= 1;
        for (uint32_t i = t; i < pw; i += kFinalThreads)
            s[i] = i < n ? k[i] : ~0ull;
        __syncthreads();
        bitonic_lds(s, pw);
    } else {
        // radix select of the topk-th smallest (unique) key, 8 bits at a time from the top
        unsigned long long prefix = 0, pmask = 0;
        uint32_t need = topk;
        for (int shift = 56; shift >= 0; shift -= 8) {
            for (uint32_t i = t; i < 256; i += kFinalThreads)
                s_hist[i] = 0;
            __syncthreads();
            for (uint32_t i = t; i < n; i += kFinalThreads) {
                const unsigned long long v = k[i];
                if ((v & pmask) == prefix)
                    atomicAdd(&s_hist[(uint32_t)(v >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (t == 0) {
                uint32_t acc = 0, d = 0;
                while (acc + s_hist[d] < need)
                    acc += s_hist[d++];
                s_sel[0] = d;
                s_sel[1] = need - acc;
            }
            __syncthreads();
            prefix |= (unsigned long long)s_sel[0] << shift;
            pmask |= 255ull << shift;
            need = s_sel[1];
            __syncthreads();
        }
        // the topk keys at or below it (unique keys: exactly topk), then sorted
        if (t == 0)
            s_n = 0;
        __syncthreads();
        for (uint32_t i = t; i < n; i += kFinalThreads) {
            const unsigned long long v = k[i];
            if (v <= prefix) {
                // keys are unique per query, so at most topk land here; a duplicate record
                // would add more, which the bound keeps inside the array
                const uint32_t pos = atomicAdd(&s_n, 1u);
                if (pos < kFinalLds)
                    s[pos] = v;
            }
        }
        __syncthreads();
        uint32_t pw = 1;
        while (pw < topk)
            pw <<= 1;
        for (uint32_t i = topk + t; i < pw; i += kFinalThreads)
            s[i] = ~0ull;
        __syncthreads();
        bitonic_lds(s, pw);
        m = topk;
    }
    for (uint32_t r = t; r < topk; r += kFinalThreads) {
        const bool have = r < m;
        const unsigned long long v = have ? s[r] : ~0ull;
        out_dist[(size_t)q * topk + r] = have ? key_to_float((uint32_t)(v >> 32)) : FLT_MAX;
        out_idx[(size_t)q * topk + r] = have ? (uint32_t)(v & 0xFFFFFFFFull) : 0xFFFFFFFFu;
    }
}

}  // namespace

void launch_final_topk(const SpillRecord *recs, const unsigned long long *d_n, unsigned long long cap, uint32_t nq,
                       uint32_t topk, uint32_t *counts, uint32_t *offsets, uint32_t *cursor, unsigned long long *keys,
                       float *out_dist, uint32_t *out_idx, hipStream_t s) {
    launch_fill_u32(counts, 0u, nq, s);
    final_count_kernel<<<1024, 256, 0, s>>>(recs, d_n, cap, counts);
    final_scan_kernel<<<1, 1024, 0, s>>>(counts, nq, offsets, cursor);
    final_scatter_kernel<<<1024, 256, 0, s>>>(recs, d_n, cap, offsets, cursor, keys);
    final_select_kernel<<<nq, kFinalThreads, 0, s>>>(keys, offsets, topk, out_dist, out_idx);
}

}  // namespace cora
