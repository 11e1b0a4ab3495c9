// Index-build and evaluation tools on the GPU (C-ABI in include/cora_gpu.h, cora_tool_*):
// rotation of a row block, Lloyd k-means, nearest-centroid assignment and exhaustive
// top-k (ground truth). They reuse the engine's FP32 GEMM, row-norm and top-k select
// kernels; host arrays in, host arrays out, device memory allocated per call.
#include <float.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <random>
#include <string>
#include <vector>

#include "../../../include/cora_gpu.h"
#include "engine_internal.h"

using namespace cora;

namespace {

thread_local std::string g_tool_error;

// argmin over each row of dist [rows][k]; ties -> lower index.
__global__ __launch_bounds__(64) void row_argmin_kernel(const float *__restrict__ dist, uint32_t k,
                                                        uint32_t *__restrict__ out) {
    const float *row = dist + (size_t)blockIdx.x * k;
    float best = FLT_MAX;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t j = threadIdx.x; j < k; j += 64) {
        const float v = row[j];
        if (v < best || (v == best && j < bi)) {
            best = v;
            bi = j;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (ov < best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    if (threadIdx.x == 0)
        out[blockIdx.x] = bi == 0xFFFFFFFFu ? 0u : bi;
}

// grid-stride over rows (a dispatch counts its work-items in 32 bits)
__global__ void accumulate_kernel(const float *__restrict__ x, const uint32_t *__restrict__ assign,
                                  uint32_t rows, uint32_t dim, float *__restrict__ sums,
                                  uint32_t *__restrict__ counts) {
    for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const uint32_t c = assign[r];
        for (uint32_t d = threadIdx.x; d < dim; d += blockDim.x)
            atomicAdd(&sums[(size_t)c * dim + d], x[(size_t)r * dim + d]);
        if (threadIdx.x == 0)
            atomicAdd(&counts[c], 1u);
    }
}

__global__ void update_kernel(float *__restrict__ cent, const float *__restrict__ sums,
                              const uint32_t *__restrict__ counts, uint32_t k, uint32_t dim) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= (size_t)k * dim)
        return;
    const uint32_t c = (uint32_t)(i / dim);
    if (counts[c])
        cent[i] = sums[i] / (float)counts[c];
}

// The k selected of one base block, as (distance, global id) candidates:
// cd/ci[row][slot0 + t] for t < k, from the block's distances [rows][len].
__global__ void gather_block_topk_kernel(const float *__restrict__ dist, uint32_t len,
                                         const int32_t *__restrict__ idx, uint32_t rows, uint32_t k,
                                         uint32_t base0, uint32_t stride, uint32_t slot0,
                                         float *__restrict__ cd, uint32_t *__restrict__ ci) {
    const size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (t >= (size_t)rows * k)
        return;
    const size_t r = t / k, j = t % k;
    const uint32_t i = (uint32_t)idx[t];
    cd[r * stride + slot0 + j] = dist[r * len + i];
    ci[r * stride + slot0 + j] = base0 + i;
}

struct DevBuf {
    void *p = nullptr;
    ~DevBuf() {
        if (p)
            (void)hipFree(p);
    }
};

#define TCHK(call)                                                                  \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            g_tool_error = std::string(#call) + ": " + hipGetErrorString(e_);       \
            return CORA_ERR_RUNTIME;                                                \
        }                                                                           \
    } while (0)

template <class T>
int dev(DevBuf &b, size_t n) {
    TCHK(hipMalloc(&b.p, std::max<size_t>(1, n) * sizeof(T)));
    return CORA_OK;
}

// Assign rows [0, n) of device matrix x to the nearest of k device centroids.
int assign_rows(const float *d_x, size_t n, uint32_t dim, const float *d_c, const float *d_cn,
                uint32_t k, uint32_t *d_assign, float *d_xn, float *d_dist, size_t chunk,
                hipStream_t s) {
    for (size_t b = 0; b < n; b += chunk) {
        const uint32_t rows = (uint32_t)std::min(chunk, n - b);
        launch_row_norms(d_x + b * dim, rows, dim, d_xn, s);
        launch_dist_gemm(d_x + b * dim, d_xn, d_c, d_cn, rows, k, dim, d_dist, s);
        row_argmin_kernel<<<rows, 64, 0, s>>>(d_dist, k, d_assign + b);
    }
    TCHK(hipGetLastError());
    return CORA_OK;
}

// ---- scratch of the allocation-free assignment (cora_tool_assign_noalloc) ----
// Centroid norms, row norms and one block of distances live in this static device array;
// every GPU the library runs on holds its own copy until the process ends. Its host-side
// name is not a device address: host code uses the per-device address that
// hipGetSymbolAddress returns (scratch_address) for kernel arguments.
constexpr size_t kScratchFloats = size_t{4} << 20;  // 16 MiB
static_assert(CORA_NOALLOC_MAX_CENTROIDS * 3 + 192 <= kScratchFloats,
              "the scratch holds the centroid norms and at least one row of distances");
static __device__ __align__(256) float scratch[kScratchFloats];

std::mutex g_scratch_mu;
std::map<int, float *> g_scratch_addr;  // device ordinal -> address of its scratch
// one allocation-free call at a time per device: a call holds its device's lock from the
// scratch address until its kernels have finished
std::mutex g_scratch_use_mu;
std::map<int, std::mutex> g_scratch_use;  // device ordinal -> lock of its scratch

std::mutex &scratch_lock(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_use_mu);
    return g_scratch_use[device];  // std::map never moves its elements
}

// The calling device's scratch address, resolved once per device (the device is current).
int scratch_address(int device, float **out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_addr.find(device);
    if (it == g_scratch_addr.end()) {
        float *ptr = nullptr;
        TCHK(hipGetSymbolAddress(reinterpret_cast<void **>(&ptr), HIP_SYMBOL(scratch)));
        if (!ptr) {
            g_tool_error = "hipGetSymbolAddress returned no address for the scratch array";
            return CORA_ERR_RUNTIME;
        }
        it = g_scratch_addr.emplace(device, ptr).first;
    }
    *out = it->second;
    return CORA_OK;
}

constexpr size_t round_floats(size_t n) { return (n + 63) / 64 * 64; }  // 256-byte slots

}  // namespace

void cora::set_tool_error(const char *msg) { g_tool_error = msg; }

extern "C" {

const char *cora_tool_last_error(void) { return g_tool_error.c_str(); }

int cora_tool_rotate(const float *h_x, uint64_t n, uint64_t dim, const float *h_R, uint64_t P,
                     float *h_out, int device) {
    if (!h_x || !h_R || !h_out || !n || !dim || P < dim)
        return CORA_ERR_INVALID_ARGUMENT;
    TCHK(hipSetDevice(device));
    DevBuf x, r, o;
    const size_t chunk = 1u << 20;
    if (dev<float>(x, std::min<size_t>(n, chunk) * dim) || dev<float>(r, dim * P) ||
        dev<float>(o, std::min<size_t>(n, chunk) * P))
        return CORA_ERR_RUNTIME;
    TCHK(hipMemcpy(r.p, h_R, dim * P * 4, hipMemcpyHostToDevice));
    for (size_t b = 0; b < n; b += chunk) {
        const size_t rows = std::min<size_t>(chunk, n - b);
        TCHK(hipMemcpy(x.p, h_x + b * dim, rows * dim * 4, hipMemcpyHostToDevice));
        launch_rotate((float *)x.p, (float *)r.p, (float *)o.p, (uint32_t)rows, (uint32_t)dim,
                      (uint32_t)P, nullptr);
        TCHK(hipGetLastError());
        TCHK(hipMemcpy(h_out + b * P, o.p, rows * P * 4, hipMemcpyDeviceToHost));
    }
    return CORA_OK;
}

}  // extern "C"

namespace {

// Re-seed every empty cluster by splitting a populated one, as Faiss's Lloyd k-means does
// after each update (the k-means the reference's index recipe trains with): cluster j is
// chosen with probability proportional to (size_j - 1), its centroid is copied, the two
// copies are pushed apart by a relative 1/1024 in alternating directions per dimension,
// and the size is assumed to split evenly. Without it a centroid left empty stays where it
// was; on well-separated data such centroids drift towards the origin and end up closer
// to every query than any populated cluster, so probe lists fill with empty clusters.
// Returns the number of clusters re-seeded; cent [k][dim] and counts are host copies.
uint32_t split_empty_clusters(std::vector<float> &cent, std::vector<uint32_t> &counts, uint32_t dim,
                              std::mt19937_64 &gen) {
    const uint32_t k = (uint32_t)counts.size();
    constexpr float kEps = 1.0f / 1024.0f;
    uint32_t split = 0;
    for (uint32_t ci = 0; ci < k; ++ci) {
        if (counts[ci])
            continue;
        uint64_t total = 0;
        for (uint32_t j = 0; j < k; ++j)
            total += counts[j] > 1 ? counts[j] - 1 : 0;
        if (!total)
            break;  // nothing left to split
        uint64_t r = std::uniform_int_distribution<uint64_t>(0, total - 1)(gen);
        uint32_t cj = 0;
        for (; cj < k; ++cj) {
            const uint64_t w = counts[cj] > 1 ? counts[cj] - 1 : 0;
            if (r < w)
                break;
            r -= w;
        }
        float *a = &cent[(size_t)ci * dim], *b = &cent[(size_t)cj * dim];
        for (uint32_t d = 0; d < dim; ++d) {
            const float v = b[d];
            a[d] = v * (d % 2 == 0 ? 1 + kEps : 1 - kEps);
            b[d] = v * (d % 2 == 0 ? 1 - kEps : 1 + kEps);
        }
        counts[ci] = counts[cj] / 2;
        counts[cj] -= counts[ci];
        ++split;
    }
    return split;
}

}  // namespace

extern "C" {

// Lloyd k-means on n rows (FP32 squared L2), initial centroids = k distinct rows chosen
// with a seeded generator; after each update, empty clusters are re-seeded by splitting
// populated ones (split_empty_clusters).
int cora_tool_kmeans(const float *h_x, uint64_t n, uint64_t dim, uint64_t k, uint32_t iters,
                     uint64_t seed, float *h_centroids, int device) {
    if (!h_x || !h_centroids || !n || !dim || !k || k > n || k > 0x7FFFFFFF)
        return CORA_ERR_INVALID_ARGUMENT;
    TCHK(hipSetDevice(device));
    std::vector<uint64_t> pick(n);
    for (uint64_t i = 0; i < n; ++i)
        pick[i] = i;
    std::mt19937_64 gen(seed);
    for (uint64_t i = 0; i < k; ++i) {
        std::uniform_int_distribution<uint64_t> u(i, n - 1);
        std::swap(pick[i], pick[u(gen)]);
    }
    std::vector<float> init(k * dim);
    for (uint64_t i = 0; i < k; ++i)
        memcpy(&init[i * dim], h_x + pick[i] * dim, dim * 4);
    const size_t chunk = std::max<size_t>(1, std::min<size_t>(n, (size_t)(1u << 30) / (k * 4)));
    DevBuf x, c, cn, xn, dist, asg, sums, cnt;
    if (dev<float>(x, n * dim) || dev<float>(c, k * dim) || dev<float>(cn, k) ||
        dev<float>(xn, chunk) || dev<float>(dist, chunk * k) || dev<uint32_t>(asg, n) ||
        dev<float>(sums, k * dim) || dev<uint32_t>(cnt, k))
        return CORA_ERR_RUNTIME;
    TCHK(hipMemcpy(x.p, h_x, n * dim * 4, hipMemcpyHostToDevice));
    TCHK(hipMemcpy(c.p, init.data(), k * dim * 4, hipMemcpyHostToDevice));
    std::vector<uint32_t> counts(k);
    std::mt19937_64 split_gen(seed ^ 0x9E3779B97F4A7C15ull);
    for (uint32_t it = 0; it < iters; ++it) {
        launch_row_norms((float *)c.p, (uint32_t)k, (uint32_t)dim, (float *)cn.p, nullptr);
        if (int rc = assign_rows((float *)x.p, n, (uint32_t)dim, (float *)c.p, (float *)cn.p,
                                 (uint32_t)k, (uint32_t *)asg.p, (float *)xn.p, (float *)dist.p,
                                 chunk, nullptr))
            return rc;
        TCHK(hipMemset(sums.p, 0, k * dim * 4));
        TCHK(hipMemset(cnt.p, 0, k * 4));
        accumulate_kernel<<<(uint32_t)std::min<uint64_t>(n, 1u << 20), 64>>>((float *)x.p, (uint32_t *)asg.p, (uint32_t)n,
                                                (uint32_t)dim, (float *)sums.p, (uint32_t *)cnt.p);
        update_kernel<<<(uint32_t)((k * dim + 255) / 256), 256>>>((float *)c.p, (float *)sums.p,
                                                                   (uint32_t *)cnt.p, (uint32_t)k,
                                                                   (uint32_t)dim);
        TCHK(hipGetLastError());
        TCHK(hipMemcpy(counts.data(), cnt.p, k * 4, hipMemcpyDeviceToHost));
        if (std::find(counts.begin(), counts.end(), 0u) != counts.end()) {
            TCHK(hipMemcpy(init.data(), c.p, k * dim * 4, hipMemcpyDeviceToHost));
            if (split_empty_clusters(init, counts, (uint32_t)dim, split_gen))
                TCHK(hipMemcpy(c.p, init.data(), k * dim * 4, hipMemcpyHostToDevice));
        }
    }
    TCHK(hipDeviceSynchronize());
    TCHK(hipMemcpy(h_centroids, c.p, k * dim * 4, hipMemcpyDeviceToHost));
    return CORA_OK;
}

int cora_tool_assign(const float *h_x, uint64_t n, uint64_t dim, const float *h_centroids,
                     uint64_t k, uint32_t *h_assign, int device) {
    if (!h_x || !h_centroids || !h_assign || !n || !dim || !k)
        return CORA_ERR_INVALID_ARGUMENT;
    TCHK(hipSetDevice(device));
    const size_t rows_dev = std::min<size_t>(n, 1u << 22);
    const size_t chunk = std::max<size_t>(1, std::min<size_t>(rows_dev, (size_t)(1u << 30) / (k * 4)));
    DevBuf x, c, cn, xn, dist, asg;
    if (dev<float>(x, rows_dev * dim) || dev<float>(c, k * dim) || dev<float>(cn, k) ||
        dev<float>(xn, chunk) || dev<float>(dist, chunk * k) || dev<uint32_t>(asg, rows_dev))
        return CORA_ERR_RUNTIME;
    TCHK(hipMemcpy(c.p, h_centroids, k * dim * 4, hipMemcpyHostToDevice));
    launch_row_norms((float *)c.p, (uint32_t)k, (uint32_t)dim, (float *)cn.p, nullptr);
    for (size_t b = 0; b < n; b += rows_dev) {
        const size_t rows = std::min(rows_dev, n - b);
        TCHK(hipMemcpy(x.p, h_x + b * dim, rows * dim * 4, hipMemcpyHostToDevice));
        if (int rc = assign_rows((float *)x.p, rows, (uint32_t)dim, (float *)c.p, (float *)cn.p,
                                 (uint32_t)k, (uint32_t *)asg.p, (float *)xn.p, (float *)dist.p,
                                 chunk, nullptr))
            return rc;
        TCHK(hipMemcpy(h_assign + b, asg.p, rows * 4, hipMemcpyDeviceToHost));
    }
    return CORA_OK;
}

// The same assignment on device arrays the caller owns, with no allocation: centroid norms,
// row norms and distance blocks in the static scratch array (nothing in it has to start at
// zero: every value is written before it is read). Calls on one GPU from several host threads
// take turns (a per-device lock held until the call's kernels have finished), so they never
// share the array at the same time.
int cora_tool_assign_noalloc(const float *d_x, uint64_t n, uint64_t dim, const float *d_centroids,
                             uint64_t k, uint32_t *d_assign, int device) {
    if (!d_x || !d_centroids || !d_assign || !n || !dim || !k) {
        g_tool_error = "assign_noalloc: null array or zero size";
        return CORA_ERR_INVALID_ARGUMENT;
    }
    if (k > CORA_NOALLOC_MAX_CENTROIDS || dim > CORA_NOALLOC_MAX_DIM || n > 0xFFFFFFFFull) {
        g_tool_error = "assign_noalloc: at most " + std::to_string(CORA_NOALLOC_MAX_CENTROIDS) +
                       " centroids, dimension " + std::to_string(CORA_NOALLOC_MAX_DIM) +
                       " and 2^32 - 1 rows (the scratch holds " + std::to_string(kScratchFloats * 4 >> 20) + " MiB)";
        return CORA_ERR_INVALID_ARGUMENT;
    }
    TCHK(hipSetDevice(device));
    std::lock_guard<std::mutex> use(scratch_lock(device));
    float *base = nullptr;
    if (int rc = scratch_address(device, &base))
        return rc;
    // layout: centroid norms [k], then per block row norms [chunk] and distances [chunk][k]
    const size_t cn_slot = round_floats(k);
    // rows per block: what the scratch holds, and row offsets of a block within 2^31 elements
    const size_t chunk = std::min<size_t>({n, (kScratchFloats - cn_slot - 64) / (k + 1), ((1ull << 31) - 1) / dim});
    float *cn = base, *xn = base + cn_slot, *dist = xn + round_floats(chunk);
    if (chunk == 0 || (size_t)(dist - base) + chunk * k > kScratchFloats) {
        g_tool_error = "assign_noalloc: the scratch cannot hold one row of distances";
        return CORA_ERR_INVALID_ARGUMENT;
    }
    launch_row_norms(d_centroids, (uint32_t)k, (uint32_t)dim, cn, nullptr);
    if (int rc = assign_rows(d_x, n, (uint32_t)dim, d_centroids, cn, (uint32_t)k, d_assign, xn, dist, chunk,
                             nullptr))
        return rc;
    TCHK(hipStreamSynchronize(nullptr));
    return CORA_OK;
}

// Exhaustive top-k of nq queries over nb base rows by FP32 distance (L2: ||q-x||^2 through
// the norm expansion; IP: -<q,x>), ascending, ties by base index. Callers that need the
// exact order re-rank a few extra candidates in FP64.
int cora_tool_topk(const float *h_base, uint64_t nb, const float *h_q, uint64_t nq, uint64_t dim,
                   uint64_t k, int metric, uint32_t *h_ids, int device) {
    if (!h_base || !h_q || !h_ids || !nb || !nq || !dim || !k || k > nb ||
        k > (uint64_t)kSelectMaxProbe || nb > 0x7FFFFFFF)
        return CORA_ERR_INVALID_ARGUMENT;
    TCHK(hipSetDevice(device));
    // Two levels: the base is cut into nblk blocks of <= 2^20 rows; each (query chunk, block)
    // distance tile is selected to its k best, and the nblk * k candidates of a query are
    // merged on the host by (distance, id), the select's own tie order.
    const size_t nblk = (nb + (1u << 20) - 1) >> 20, blk = (nb + nblk - 1) / nblk;
    const size_t qchunk = std::max<size_t>(1, std::min<size_t>(nq, (size_t)(1ull << 30) / blk));
    const size_t stride = nblk * k;
    DevBuf b, bn, q, qn, dist, ids, cd, ci;
    if (dev<float>(b, nb * dim) || dev<float>(bn, nb) || dev<float>(q, qchunk * dim) ||
        dev<float>(qn, qchunk) || dev<float>(dist, qchunk * blk) || dev<int32_t>(ids, qchunk * k) ||
        dev<float>(cd, qchunk * stride) || dev<uint32_t>(ci, qchunk * stride))
        return CORA_ERR_RUNTIME;
    TCHK(hipMemcpy(b.p, h_base, nb * dim * 4, hipMemcpyHostToDevice));
    if (metric == 0)
        launch_row_norms((float *)b.p, (uint32_t)nb, (uint32_t)dim, (float *)bn.p, nullptr);
    else
        TCHK(hipMemset(bn.p, 0, nb * 4));
    std::vector<float> hd(qchunk * stride);
    std::vector<uint32_t> hi(qchunk * stride), order(stride);
    for (size_t s = 0; s < nq; s += qchunk) {
        const size_t rows = std::min(qchunk, nq - s);
        TCHK(hipMemcpy(q.p, h_q + s * dim, rows * dim * 4, hipMemcpyHostToDevice));
        if (metric == 0)
            launch_row_norms((float *)q.p, (uint32_t)rows, (uint32_t)dim, (float *)qn.p, nullptr);
        else  // an[m] + bn[n] - 2 * ip with zero norms = -2 ip: same order as -ip
            TCHK(hipMemset(qn.p, 0, rows * 4));
        for (size_t j = 0; j < nblk; ++j) {
            const size_t b0 = j * blk, len = std::min(blk, nb - b0);
            launch_dist_gemm((float *)q.p, (float *)qn.p, (float *)b.p + b0 * dim, (float *)bn.p + b0,
                             (uint32_t)rows, (uint32_t)len, (uint32_t)dim, (float *)dist.p, nullptr);
            launch_select((float *)dist.p, (uint32_t)rows, (uint32_t)len, (uint32_t)k, (int32_t *)ids.p,
                          nullptr);
            const size_t n = rows * k;
            gather_block_topk_kernel<<<(unsigned)((n + 255) / 256), 256>>>(
                (float *)dist.p, (uint32_t)len, (int32_t *)ids.p, (uint32_t)rows, (uint32_t)k, (uint32_t)b0,
                (uint32_t)stride, (uint32_t)(j * k), (float *)cd.p, (uint32_t *)ci.p);
        }
        TCHK(hipGetLastError());
        TCHK(hipMemcpy(hd.data(), cd.p, rows * stride * 4, hipMemcpyDeviceToHost));
        TCHK(hipMemcpy(hi.data(), ci.p, rows * stride * 4, hipMemcpyDeviceToHost));
        for (size_t r = 0; r < rows; ++r) {
            const float *d = hd.data() + r * stride;
            const uint32_t *id = hi.data() + r * stride;
            for (size_t t = 0; t < stride; ++t)
                order[t] = (uint32_t)t;
            std::partial_sort(order.begin(), order.begin() + k, order.end(), [&](uint32_t a, uint32_t c) {
                return d[a] < d[c] || (d[a] == d[c] && id[a] < id[c]);
            });
            for (size_t t = 0; t < k; ++t)
                h_ids[(s + r) * k + t] = id[order[t]];
        }
    }
    return CORA_OK;
}

}  // extern "C"
