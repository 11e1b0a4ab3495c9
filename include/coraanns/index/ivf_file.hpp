// The reference's on-disk IVF-RaBitQ index (third_party/rabitq/.../ivf/ivf.hpp:403-539):
//   size_t num, dim, nlist, ex_bits; u8 rotator type; u8 metric;
//   size_t cluster_sizes[nlist];
//   MatrixRotator: f32 [dim][padded_dim] (rotator.hpp:89-94), q' = q . R;
//   centroids, one of (detected by the bytes left after the rotator, ivf.hpp:487-520):
//     embedded: rotated centroids f32 [nlist][padded_dim] (initializer.hpp:147-169);
//     HNSW sidecar: nothing here; the centroids are the vectors of the hnswlib graph saved
//       as "<index>.hnsw" (initializer.hpp:255-279, hnswalg.h:685-713), the vector of
//       label c being centroid c;
//   batch data: per cluster ceil(n/32) blocks of (padded_dim*4 B FastScan sign codes,
//     32 f_add, 32 f_rescale, 32 f_error) (data_layout.hpp:57-83);
//   ex data: per vector padded_dim*ex_bits/8 B packed ex-code + f_add_ex + f_rescale_ex
//     (data_layout.hpp:158-178);
//   u32 ids[num] in cluster order.
// padded_dim = round_up(dim, 64) (ivf.hpp:242). The reference writes the sidecar form when
// nlist >= 20000 (initializer.hpp:23); save() here always embeds the centroids, which the
// reference's load() accepts at any nlist.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace coraanns::index {

enum class CentroidStorage : uint8_t { Embedded = 0, HnswSidecar = 1 };

struct IvfHeader {
    uint64_t num = 0, dim = 0, padded_dim = 0, nlist = 0, ex_bits = 0;
    uint8_t rotator_type = 0;  // 0 = MatrixRotator
    uint8_t metric = 0;        // 0 = L2, 1 = IP
    CentroidStorage centroid_storage = CentroidStorage::Embedded;
    std::vector<uint64_t> cluster_sizes;

    std::size_t batch_block_bytes() const { return padded_dim * 4 + 32 * 12; }
    std::size_t ex_code_bytes() const { return (padded_dim * ex_bits + 7) / 8; }
    std::size_t ex_stride() const { return ex_bits ? padded_dim * ex_bits / 8 + 8 : 0; }
};

struct IvfFile : IvfHeader {
    std::vector<float> rotator;    // [dim][padded_dim]
    std::vector<float> centroids;  // [nlist][padded_dim]
    std::vector<uint8_t> batch_data;
    std::vector<uint8_t> ex_data;  // [num][ex_stride()]
    std::vector<uint32_t> ids;

    static IvfFile load(const std::string &path);  // whole file in memory; throws std::runtime_error
    void save(const std::string &path) const;      // embedded centroids; throws std::runtime_error
};

// Sectioned reader of an index file: the constructor reads the header, cluster sizes and
// rotator and detects the centroid storage like IVF::load (ivf.hpp:447-520); the payload
// sections are then read piecewise (positioned reads), so a caller can stream them.
class IvfReader {
  public:
    explicit IvfReader(const std::string &path);
    ~IvfReader();
    IvfReader(const IvfReader &) = delete;
    IvfReader &operator=(const IvfReader &) = delete;

    const IvfHeader &header() const { return h_; }
    std::vector<float> read_rotator() const;
    std::vector<float> read_centroids() const;  // embedded, or from "<path>.hnsw"
    // blocks [first, first+count) of the batch data (batch_block_bytes() each)
    void read_batch_blocks(uint64_t first, uint64_t count, uint8_t *dst) const;
    // ex-data records [first, first+count) (ex_stride() bytes each)
    void read_ex_records(uint64_t first, uint64_t count, uint8_t *dst) const;
    void read_ids(uint32_t *dst) const;  // [num]

  private:
    void read_at(uint64_t offset, uint64_t bytes, void *dst, const char *what) const;
    std::string path_;
    int fd_ = -1;
    IvfHeader h_;
    uint64_t rotator_off_ = 0, centroid_off_ = 0, batch_off_ = 0, ex_off_ = 0, ids_off_ = 0;
};

// Centroids [nlist][padded_dim] from an hnswlib index file: the level-0 element of each
// internal id holds its vector at offsetData_ and its label at label_offset_ (hnswalg.h:
// 685-713); the vector of label c becomes row c (initializer.hpp:181-198). Rejects files
// hnswlib's loadIndex rejects (hnswalg.h:716-770), a count other than nlist, labels out of
// range or repeated, and vectors whose size is not padded_dim floats.
std::vector<float> read_hnsw_centroids(const std::string &sidecar, uint64_t nlist, uint64_t padded_dim);

}  // namespace coraanns::index
