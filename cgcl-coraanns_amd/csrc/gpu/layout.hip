// Index layout builder ("src/index" GPU-native layout). Converts the reference's
// SearchData arrays (search_data.cpp:45-82: per-cluster word-major u32 codes with
// dimension 32w+l at bit 31-l, AoS float3 factors) into the engine's tile layout
// (engine_internal.h): bit-reversed words, 64-vector tiles, 128-bit lane groups,
// SoA factors. One wave per cluster walks the cluster's tiles; lanes past the end of
// the cluster get zero codes and zero factors.
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

}  // namespace

void launch_repack(const uint32_t *ref_words, const float *ref_factors, const ClusterMeta *meta,
                   uint32_t nlist, uint32_t W, uint8_t *tiles, uint32_t tile_bytes,
                   hipStream_t s) {
    repack_kernel<<<nlist, 64, 0, s>>>(ref_words, ref_factors, meta, W, tiles, tile_bytes);
}

}  // namespace cora
