// The reference's on-disk IVF-RaBitQ index (third_party/rabitq/.../ivf/ivf.hpp:403-539):
//   size_t num, dim, nlist, ex_bits; u8 rotator type; u8 metric;
//   size_t cluster_sizes[nlist];
//   MatrixRotator: f32 [dim][padded_dim] (rotator.hpp:89-94), q' = q . R;
//   flat initializer: rotated centroids f32 [nlist][padded_dim] (initializer.hpp:147-169);
//   batch data: per cluster ceil(n/32) blocks of (padded_dim*4 B FastScan sign codes,
//     32 f_add, 32 f_rescale, 32 f_error) (data_layout.hpp:57-83);
//   ex data: per vector padded_dim*ex_bits/8 B packed ex-code + f_add_ex + f_rescale_ex
//     (data_layout.hpp:158-178);
//   u32 ids[num] in cluster order.
// padded_dim = round_up(dim, 64) (ivf.hpp:242). Indexes whose centroids live in an HNSW
// sidecar (nlist >= 20000, initializer.hpp:23-27) are rejected by load().
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace coraanns::index {

struct IvfFile {
    uint64_t num = 0, dim = 0, padded_dim = 0, nlist = 0, ex_bits = 0;
    uint8_t rotator_type = 0;  // 0 = MatrixRotator
    uint8_t metric = 0;        // 0 = L2, 1 = IP
    std::vector<uint64_t> cluster_sizes;
    std::vector<float> rotator;    // [dim][padded_dim]
    std::vector<float> centroids;  // [nlist][padded_dim]
    std::vector<uint8_t> batch_data;
    std::vector<uint8_t> ex_data;  // [num][ex_stride()]
    std::vector<uint32_t> ids;

    std::size_t batch_block_bytes() const { return padded_dim * 4 + 32 * 12; }
    std::size_t ex_code_bytes() const { return (padded_dim * ex_bits + 7) / 8; }
    std::size_t ex_stride() const { return ex_bits ? padded_dim * ex_bits / 8 + 8 : 0; }

    static IvfFile load(const std::string &path);  // throws std::runtime_error
    void save(const std::string &path) const;      // throws std::runtime_error
};

}  // namespace coraanns::index
