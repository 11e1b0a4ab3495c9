// IVF-RaBitQ index construction into the reference on-disk format. Restates the
// reference quantizer (third_party/rabitq/.../quantization/rabitq_impl.hpp:76-137
// one_bit_code_with_factor, 276-333 best_rescale_factor, 336-360 quantize_ex,
// 405-500 ex_bits_code_with_factor), the 7-bit ex-code packing (pack_excode.hpp:216-265)
// and FastScan code packing (fastscan.hpp:69-106). Inputs are already rotated (the
// caller applies R, so rotation can run on the GPU); cluster assignment is the caller's.
#pragma once

#include <cstddef>
#include <cstdint>

#include "coraanns/index/ivf_file.hpp"

namespace coraanns::index {

struct BuildInput {
    const float *rotated_data = nullptr;       // [n][padded_dim]
    const float *rotated_centroids = nullptr;  // [nlist][padded_dim]
    const uint32_t *assignments = nullptr;     // [n] cluster of each vector
    const float *rotator = nullptr;            // [dim][padded_dim]
    std::size_t n = 0, dim = 0, padded_dim = 0, nlist = 0, ex_bits = 7;
    int metric = 0;  // 0 = L2, 1 = IP
};

IvfFile build_ivf(const BuildInput &in, int threads = 0);

// The same index from raw rows, rotated and quantised on GPU `device` (cora_tool_quantize,
// bit-identical to build_ivf on the GPU-rotated rows); the host packs the codes.
struct GpuBuildInput {
    const float *data = nullptr;               // [n][dim] raw rows
    const float *rotated_centroids = nullptr;  // [nlist][padded_dim]
    const uint32_t *assignments = nullptr;     // [n]
    const float *rotator = nullptr;            // [dim][padded_dim]
    std::size_t n = 0, dim = 0, padded_dim = 0, nlist = 0, ex_bits = 7;
    int metric = 0;
};

IvfFile build_ivf_gpu(const GpuBuildInput &in, int device = 0, int threads = 0);

// bits: u8 {0,1} [P]; factors: f_add, f_rescale, f_error.
void quantize_one_bit(const float *x, const float *c, std::size_t P, uint8_t *bits,
                      float *factors, int metric);
// code: u8 [P] ex-codes (values < 2^ex_bits); factors: f_add_ex, f_rescale_ex.
void quantize_ex_bits(const float *x, const float *c, std::size_t P, std::size_t ex_bits,
                      uint8_t *code, float *factors, int metric);
// 7-bit packing, P % 64 == 0: out has P*7/8 bytes.
void pack_excode7(const uint8_t *code, std::size_t P, uint8_t *out);
// FastScan packing of n sign codes (compact big-endian bytes [n][P/8]) into
// ceil(n/32) blocks of P*4 bytes.
void fastscan_pack(const uint8_t *compact, std::size_t n, std::size_t P, uint8_t *blocks);

}  // namespace coraanns::index
