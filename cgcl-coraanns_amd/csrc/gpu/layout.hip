// Index layout builder ("src/index" GPU-native layout). Converts the reference's
// SearchData arrays (search_data.cpp:45-82: per-cluster word-major u32 codes with
// dimension 32w+l at bit 31-l, AoS float3 factors) into the engine's tile layout
// (engine_internal.h): bit-reversed words, 64-vector tiles, 128-bit lane groups,
// SoA factors. One wave per cluster walks the cluster's tiles; lanes past the end of
// the cluster get zero codes and zero factors.
#include <algorithm>

#include "engine_internal.h"

namespace cora {
namespace {

__global__ __launch_bounds__(64) void repack_kernel(const uint32_t *__restrict__ ref_words,
                                                     const float *__restrict__ ref_factors,
                                                     const ClusterMeta *__restrict__ meta,
                                                     uint32_t W, uint8_t *__restrict__ tiles,
                                                     uint32_t tile_bytes) {
    const ClusterMeta cm = meta[blockIdx.x];
    const uint32_t lane = threadIdx.x;
    const uint32_t ntiles = (cm.n + kTileVectors - 1) / kTileVectors;
    const uint32_t full_groups = W / 4;
    for (uint32_t t = 0; t < ntiles; ++t) {
        uint8_t *tile = tiles + (size_t)(cm.tile_base + t) * tile_bytes;
        const uint32_t local = t * kTileVectors + lane;
        const bool valid = local < cm.n;
        for (uint32_t w = 0; w < W; ++w) {
            const uint32_t v =
                valid ? __brev(ref_words[(size_t)cm.start * W + (size_t)w * cm.n + local]) : 0u;
            const uint32_t g = w / 4, c = w % 4;
            uint32_t *dst;
            if (g < full_groups)
                dst = reinterpret_cast<uint32_t *>(tile + (size_t)(g * 64 + lane) * 16) + c;
            else
                dst = reinterpret_cast<uint32_t *>(tile + (size_t)full_groups * 1024 + lane * 8) + c;
            *dst = v;
        }
        float *fac = reinterpret_cast<float *>(tile + 256u * W);
        const size_t gi = (size_t)cm.start + local;
        fac[lane] = valid ? ref_factors[gi * 3 + 0] : 0.0f;
        fac[64 + lane] = valid ? ref_factors[gi * 3 + 1] : 0.0f;
        fac[128 + lane] = valid ? ref_factors[gi * 3 + 2] : 0.0f;
    }
}

// Refinement records (engine_internal.h), first part: rows [g0, g0 + n) of the packed
// ex-codes (P*7/8 bytes each) and ex-factors (two floats each) into their records, one
// 8-byte word per thread.
__global__ __launch_bounds__(256) void ex_record_fill_kernel(const uint8_t *__restrict__ codes,
                                                             const float *__restrict__ factors, uint64_t g0,
                                                             uint32_t n, uint32_t P, uint8_t *__restrict__ rec) {
    const uint32_t words = P * 7 / 64;  // 8-byte words of an ex-code (P % 64 == 0)
    const uint32_t stride = ex_record_bytes(P);
    const uint64_t total = (uint64_t)n * (words + 1);
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t r = i / (words + 1);
        const uint32_t k = (uint32_t)(i % (words + 1));
        uint8_t *dst = rec + (g0 + r) * stride;
        if (k < words)
            *reinterpret_cast<uint2 *>(dst + ex_record_group_word(P, k / 7, k % 7)) =
                reinterpret_cast<const uint2 *>(codes + r * words * 8)[k];
        else
            *reinterpret_cast<float2 *>(dst + ex_record_factor_offset(P)) =
                make_float2(factors[2 * r], factors[2 * r + 1]);
    }
}

// Second part: each vector's sign-code words, copied from the tiles (one wave per cluster).
__global__ __launch_bounds__(64) void ex_record_sign_kernel(const ClusterMeta *__restrict__ meta,
                                                            const uint8_t *__restrict__ tiles,
                                                            uint32_t tile_bytes, uint32_t W,
                                                            uint8_t *__restrict__ rec) {
    const ClusterMeta cm = meta[blockIdx.x];
    const uint32_t P = 32 * W, stride = ex_record_bytes(P), full_groups = W / 4;
    for (uint32_t local = threadIdx.x; local < cm.n; local += kTileVectors) {
        const uint8_t *tile = tiles + (size_t)(cm.tile_base + local / kTileVectors) * tile_bytes;
        const uint32_t vl = local % kTileVectors;
        uint8_t *dst = rec + ((size_t)cm.start + local) * stride;
        for (uint32_t w = 0; w < W; ++w) {
            const uint32_t g = w / 4, c = w % 4;
            const uint32_t *src =
                g < full_groups ? reinterpret_cast<const uint32_t *>(tile + (size_t)(g * 64 + vl) * 16) + c
                                : reinterpret_cast<const uint32_t *>(tile + (size_t)full_groups * 1024 + vl * 8) + c;
            *reinterpret_cast<uint32_t *>(dst + ex_record_sign_word(P, w)) = *src;
        }
    }
}

}  // namespace

void launch_ex_record_fill(const uint8_t *codes, const float *factors, uint64_t g0, uint32_t n, uint32_t P,
                           uint8_t *rec, hipStream_t s) {
    if (!n)
        return;
    const uint64_t total = (uint64_t)n * (P * 7 / 64 + 1);
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, 65536);
    ex_record_fill_kernel<<<blocks, 256, 0, s>>>(codes, factors, g0, n, P, rec);
}

void launch_ex_record_sign(const ClusterMeta *meta, uint32_t nlist, const uint8_t *tiles, uint32_t tile_bytes,
                           uint32_t W, uint8_t *rec, hipStream_t s) {
    ex_record_sign_kernel<<<nlist, 64, 0, s>>>(meta, tiles, tile_bytes, W, rec);
}

void launch_repack(const uint32_t *ref_words, const float *ref_factors, const ClusterMeta *meta,
                   uint32_t nlist, uint32_t W, uint8_t *tiles, uint32_t tile_bytes,
                   hipStream_t s) {
    repack_kernel<<<nlist, 64, 0, s>>>(ref_words, ref_factors, meta, W, tiles, tile_bytes);
}

}  // namespace cora
