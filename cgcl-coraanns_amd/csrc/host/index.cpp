// IVF file I/O, SearchData adaptation and index construction (host side of the
// "src/index" layer). See include/coraanns/index/*.hpp for the formats.
#include <fcntl.h>
#include <omp.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <future>
#include <limits>
#include <numeric>
#include <queue>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "cora_gpu.h"
#include "coraanns/index/ivf_builder.hpp"
#include "coraanns/index/ivf_file.hpp"
#include "coraanns/index/search_data.hpp"

namespace coraanns::index {
namespace {

// FastScan interleave of 16 vectors in a 32-vector block (fastscan.hpp:40-42).
constexpr int kPerm0[16] = {0, 8, 1, 9, 2, 10, 3, 11, 4, 12, 5, 13, 6, 14, 7, 15};

// Streaming loads read the batch and ex sections in chunks of about this size
// (CORA_IVF_CHUNK_BYTES in the environment overrides it; a chunk always holds at least one
// cluster or record).
constexpr uint64_t kStreamChunkBytes = uint64_t{64} << 20;

uint64_t stream_chunk_bytes() {
    if (const char *e = std::getenv("CORA_IVF_CHUNK_BYTES")) {
        char *end = nullptr;
        const unsigned long long v = std::strtoull(e, &end, 10);
        if (end != e && *end == '\0' && v > 0)
            return v;
    }
    return kStreamChunkBytes;
}

template <class T>
void write_all(std::ofstream &out, const T *src, std::size_t count) {
    out.write(reinterpret_cast<const char *>(src), static_cast<std::streamsize>(count * sizeof(T)));
}

std::size_t round_up(std::size_t v, std::size_t m) { return (v + m - 1) / m * m; }

// Exactly `bytes` from `offset` (EINTR and short reads retried).
void pread_exact(int fd, uint64_t offset, uint64_t bytes, void *dst, const std::string &file, const char *what) {
    char *p = static_cast<char *>(dst);
    while (bytes) {
        const std::size_t want = static_cast<std::size_t>(std::min<uint64_t>(bytes, uint64_t{1} << 30));
        const ssize_t got = ::pread(fd, p, want, static_cast<off_t>(offset));
        if (got < 0 && errno == EINTR)
            continue;
        if (got < 0)
            throw std::runtime_error(std::string("read error (") + std::strerror(errno) + ") in " + file +
                                     " while reading " + what);
        if (got == 0)
            throw std::runtime_error("truncated file " + file + " while reading " + what);
        p += got;
        offset += static_cast<uint64_t>(got);
        bytes -= static_cast<uint64_t>(got);
    }
}

uint64_t file_size(int fd, const std::string &file) {
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size < 0)
        throw std::runtime_error("cannot stat " + file);
    return static_cast<uint64_t>(st.st_size);
}

struct FdGuard {
    int fd;
    ~FdGuard() {
        if (fd >= 0)
            ::close(fd);
    }
};

uint64_t batch_blocks(const IvfHeader &h) {
    uint64_t b = 0;
    for (uint64_t s : h.cluster_sizes)
        b += (s + 31) / 32;
    return b;
}

// Words and factors of one cluster's FastScan blocks into the SearchData arrays (cluster
// starts at global vector s; words are word-major within the cluster, search_data.cpp:45-82).
void unpack_cluster(const uint8_t *blocks, std::size_t n, std::size_t s, std::size_t P, uint32_t *short_data,
                    float *short_factors, std::vector<uint32_t> &words) {
    const std::size_t W = P / 32, block_bytes = P * 4 + 32 * 12;
    words.resize(32 * W);
    for (std::size_t i = 0; i < n; i += 32) {
        const uint8_t *blk = blocks + (i / 32) * block_bytes;
        const std::size_t len = std::min<std::size_t>(32, n - i);
        unpack_fastscan_block(blk, P, len, words.data());
        const float *fl = reinterpret_cast<const float *>(blk + P * 4);
        for (std::size_t v = 0; v < len; ++v) {
            for (std::size_t w = 0; w < W; ++w)
                short_data[s * W + w * n + i + v] = words[v * W + w];
            short_factors[(s + i + v) * 3 + 0] = fl[v];
            short_factors[(s + i + v) * 3 + 1] = fl[32 + v];
            short_factors[(s + i + v) * 3 + 2] = fl[64 + v];
        }
    }
}

}  // namespace

// ------------------------------------------------------------------------------------
// Reading (IVF::load, ivf.hpp:447-539; HNSWInitializer::load, initializer.hpp:255-279)
// ------------------------------------------------------------------------------------
IvfReader::IvfReader(const std::string &path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0)
        throw std::runtime_error("Cannot open IVF index: " + path);
    try {
        const uint64_t size = file_size(fd_, path);
        uint64_t hdr[4];
        read_at(0, sizeof(hdr), hdr, "header");
        h_.num = hdr[0];
        h_.dim = hdr[1];
        h_.nlist = hdr[2];
        h_.ex_bits = hdr[3];
        uint8_t tm[2];
        read_at(32, 2, tm, "rotator type and metric");
        h_.rotator_type = tm[0];
        h_.metric = tm[1];
        if (h_.rotator_type != 0)
            throw std::runtime_error("only MatrixRotator indexes are supported");
        // the reference's ids are u32 (defines.hpp PID); the dimension bound keeps every
        // byte count below 2^64
        if (h_.metric > 1 || h_.ex_bits > 8 || h_.dim == 0 || h_.dim > (uint64_t{1} << 20) || h_.nlist == 0 ||
            h_.num == 0 || h_.num > (uint64_t{1} << 32))
            throw std::runtime_error("invalid IVF header");
        h_.padded_dim = round_up(h_.dim, 64);
        if (h_.nlist > (size - 34) / 8)
            throw std::runtime_error("truncated IVF index while reading cluster sizes");
        h_.cluster_sizes.resize(h_.nlist);
        read_at(34, 8 * h_.nlist, h_.cluster_sizes.data(), "cluster sizes");
        uint64_t total = 0;
        for (uint64_t s : h_.cluster_sizes) {
            if (s > h_.num - total)
                throw std::runtime_error("The sum of cluster num != total number of points");
            total += s;
        }
        if (total != h_.num)
            throw std::runtime_error("The sum of cluster num != total number of points");
        rotator_off_ = 34 + 8 * h_.nlist;
        const uint64_t rot_bytes = 4 * h_.dim * h_.padded_dim;
        if (rot_bytes > size - rotator_off_)
            throw std::runtime_error("truncated IVF index while reading rotator");
        // the stored representation of the centroids follows from the bytes left
        // (ivf.hpp:487-520)
        const uint64_t here = rotator_off_ + rot_bytes, remaining = size - here;
        const uint64_t batch_bytes = batch_blocks(h_) * h_.batch_block_bytes();
        const uint64_t payload = batch_bytes + h_.ex_stride() * h_.num + 4 * h_.num;
        const uint64_t cent_bytes = 4 * h_.padded_dim * h_.nlist;
        if (remaining == payload + cent_bytes) {
            h_.centroid_storage = CentroidStorage::Embedded;
            centroid_off_ = here;
            batch_off_ = here + cent_bytes;
        } else if (remaining == payload) {
            h_.centroid_storage = CentroidStorage::HnswSidecar;
            batch_off_ = here;
        } else {
            throw std::runtime_error("IVF index size does not match a supported centroid layout");
        }
        ex_off_ = batch_off_ + batch_bytes;
        ids_off_ = ex_off_ + h_.ex_stride() * h_.num;
    } catch (...) {
        ::close(fd_);
        fd_ = -1;
        throw;
    }
}

IvfReader::~IvfReader() {
    if (fd_ >= 0)
        ::close(fd_);
}

void IvfReader::read_at(uint64_t offset, uint64_t bytes, void *dst, const char *what) const {
    pread_exact(fd_, offset, bytes, dst, path_, what);
}

std::vector<float> IvfReader::read_rotator() const {
    std::vector<float> r(h_.dim * h_.padded_dim);
    read_at(rotator_off_, 4 * r.size(), r.data(), "rotator");
    return r;
}

std::vector<float> IvfReader::read_centroids() const {
    if (h_.centroid_storage == CentroidStorage::HnswSidecar)
        return read_hnsw_centroids(path_ + ".hnsw", h_.nlist, h_.padded_dim);
    std::vector<float> c(h_.nlist * h_.padded_dim);
    read_at(centroid_off_, 4 * c.size(), c.data(), "centroids");
    return c;
}

void IvfReader::read_batch_blocks(uint64_t first, uint64_t count, uint8_t *dst) const {
    read_at(batch_off_ + first * h_.batch_block_bytes(), count * h_.batch_block_bytes(), dst, "batch data");
}

void IvfReader::read_ex_records(uint64_t first, uint64_t count, uint8_t *dst) const {
    read_at(ex_off_ + first * h_.ex_stride(), count * h_.ex_stride(), dst, "ex data");
}

void IvfReader::read_ids(uint32_t *dst) const { read_at(ids_off_, 4 * h_.num, dst, "ids"); }

std::vector<float> read_hnsw_centroids(const std::string &sidecar, uint64_t nlist, uint64_t padded_dim) {
    FdGuard g{::open(sidecar.c_str(), O_RDONLY | O_CLOEXEC)};
    if (g.fd < 0)
        throw std::runtime_error("Cannot open HNSW centroid sidecar: " + sidecar);
    const uint64_t size = file_size(g.fd, sidecar);
    // saveIndex header (hnswalg.h:689-702): six size_t, int maxlevel_, u32 enterpoint_node_,
    // size_t maxM_, maxM0_, M_, double mult_, size_t ef_construction_
    constexpr uint64_t kHeader = 6 * 8 + 4 + 4 + 3 * 8 + 8 + 8;
    unsigned char hb[kHeader];
    if (size < kHeader)
        throw std::runtime_error("Index seems to be corrupted or unsupported: " + sidecar);
    pread_exact(g.fd, 0, kHeader, hb, sidecar, "HNSW header");
    uint64_t count, per_element, label_off, data_off;
    std::memcpy(&count, hb + 16, 8);
    std::memcpy(&per_element, hb + 24, 8);
    std::memcpy(&label_off, hb + 32, 8);
    std::memcpy(&data_off, hb + 40, 8);
    if (count != nlist)
        throw std::runtime_error("HNSW centroid count does not match the IVF cluster count");
    const uint64_t vec_bytes = 4 * padded_dim;
    if (per_element == 0 || label_off > per_element || per_element - label_off < 8 || data_off > label_off ||
        label_off - data_off != vec_bytes)
        throw std::runtime_error("HNSW centroid sidecar does not hold vectors of padded_dim floats: " + sidecar);
    if (count > (size - kHeader) / per_element)
        throw std::runtime_error("Index seems to be corrupted or unsupported: " + sidecar);
    // upper-level link lists: a u32 size and that many bytes per element, ending exactly at
    // the end of the file (the check of hnswalg.h:754-770)
    const uint64_t links_off = kHeader + count * per_element;
    {
        std::vector<unsigned char> links(size - links_off);
        if (!links.empty())
            pread_exact(g.fd, links_off, links.size(), links.data(), sidecar, "HNSW link lists");
        uint64_t pos = 0;
        for (uint64_t i = 0; i < count; ++i) {
            if (pos >= links.size() || links.size() - pos < 4)
                throw std::runtime_error("Index seems to be corrupted or unsupported: " + sidecar);
            uint32_t len;
            std::memcpy(&len, links.data() + pos, 4);
            pos += 4 + static_cast<uint64_t>(len);
        }
        if (pos != links.size())
            throw std::runtime_error("Index seems to be corrupted or unsupported: " + sidecar);
    }
    std::vector<float> cent(nlist * padded_dim);
    std::vector<uint8_t> seen(nlist, 0);
    const uint64_t per_chunk = std::max<uint64_t>(1, stream_chunk_bytes() / per_element);
    std::vector<unsigned char> buf;
    for (uint64_t e0 = 0; e0 < count; e0 += per_chunk) {
        const uint64_t m = std::min(per_chunk, count - e0);
        buf.resize(m * per_element);
        pread_exact(g.fd, kHeader + e0 * per_element, buf.size(), buf.data(), sidecar, "HNSW level-0 elements");
        for (uint64_t e = 0; e < m; ++e) {
            const unsigned char *el = buf.data() + e * per_element;
            uint64_t label;
            std::memcpy(&label, el + label_off, 8);
            if (label >= nlist || seen[label])
                throw std::runtime_error("Invalid or duplicate HNSW centroid label");
            seen[label] = 1;
            std::memcpy(cent.data() + label * padded_dim, el + data_off, vec_bytes);
        }
    }
    return cent;
}

IvfFile IvfFile::load(const std::string &path) {
    const IvfReader rd(path);
    IvfFile f;
    static_cast<IvfHeader &>(f) = rd.header();
    f.rotator = rd.read_rotator();
    f.centroids = rd.read_centroids();
    uint64_t blocks = batch_blocks(f);
    f.batch_data.resize(blocks * f.batch_block_bytes());
    rd.read_batch_blocks(0, blocks, f.batch_data.data());
    f.ex_data.resize(f.ex_stride() * f.num);
    rd.read_ex_records(0, f.ex_stride() ? f.num : 0, f.ex_data.data());
    f.ids.resize(f.num);
    rd.read_ids(f.ids.data());
    return f;
}

void IvfFile::save(const std::string &path) const {
    std::ofstream out(path, std::ios::binary);
    if (!out)
        throw std::runtime_error("Cannot write IVF index: " + path);
    const uint64_t hdr[4] = {num, dim, nlist, ex_bits};
    write_all(out, hdr, 4);
    write_all(out, &rotator_type, 1);
    write_all(out, &metric, 1);
    write_all(out, cluster_sizes.data(), cluster_sizes.size());
    write_all(out, rotator.data(), rotator.size());
    write_all(out, centroids.data(), centroids.size());
    write_all(out, batch_data.data(), batch_data.size());
    write_all(out, ex_data.data(), ex_data.size());
    write_all(out, ids.data(), ids.size());
    if (!out)
        throw std::runtime_error("failed writing IVF index: " + path);
}

void unpack_fastscan_block(const uint8_t *codes, std::size_t P, std::size_t batch_len,
                           uint32_t *out_words) {
    int inv[16];
    for (int j = 0; j < 16; ++j)
        inv[kPerm0[j]] = j;
    const std::size_t W = P / 32;
    for (std::size_t v = 0; v < batch_len; ++v) {
        const int slot = inv[v % 16];
        const bool high = v >= 16;
        for (std::size_t w = 0; w < W; ++w) {
            uint32_t word = 0;
            for (int l = 0; l < 32; ++l) {
                const std::size_t d = w * 32 + l;
                const std::size_t in_group = d % 8;
                const uint8_t byte = codes[(d / 8) * 32 + (in_group < 4 ? 0 : 16) + slot];
                const uint8_t nib = high ? (byte >> 4) : (byte & 0x0F);
                word |= static_cast<uint32_t>((nib >> (3 - in_group % 4)) & 1u) << (31 - l);
            }
            out_words[v * W + w] = word;
        }
    }
}

SearchData::SearchData(IvfFile &src, bool include_extended, int cpu_threads) {
    const std::size_t P = src.padded_dim, W = P / 32, N = src.num;
    h_centroids = src.centroids;
    host_rotator = src.rotator;
    cluster_sizes.assign(src.cluster_sizes.begin(), src.cluster_sizes.end());
    for (std::size_t s : cluster_sizes)
        max_cluster_size = std::max(max_cluster_size, s);
    host_short_data.assign(N * W, 0u);
    host_short_factors.assign(N * 3, 0.0f);
    // block offsets per cluster so clusters can be unpacked in parallel
    std::vector<std::size_t> start(src.nlist), block0(src.nlist);
    std::size_t g = 0, b = 0;
    for (std::size_t c = 0; c < src.nlist; ++c) {
        start[c] = g;
        block0[c] = b;
        g += cluster_sizes[c];
        b += (cluster_sizes[c] + 31) / 32;
    }
    const std::size_t block_bytes = src.batch_block_bytes();
    const int threads = cpu_threads > 0 ? cpu_threads : omp_get_max_threads();
#pragma omp parallel num_threads(threads)
    {
        std::vector<uint32_t> words;
#pragma omp for schedule(dynamic, 16)
        for (long long cl = 0; cl < static_cast<long long>(src.nlist); ++cl) {
            const std::size_t c = static_cast<std::size_t>(cl);
            unpack_cluster(src.batch_data.data() + block0[c] * block_bytes, cluster_sizes[c], start[c], P,
                           host_short_data.data(), host_short_factors.data(), words);
        }
    }
    if (include_extended && src.ex_bits > 0) {
        const std::size_t lc = src.ex_code_bytes(), stride = src.ex_stride();
        host_ex_factors.assign(N * 2, 0.0f);
        extended_storage_ = std::move(src.ex_data);
        uint8_t *ex = extended_storage_.data();
        for (std::size_t i = 0; i < N; ++i) {
            const uint8_t *rec = ex + i * stride;
            float f[2];
            std::memcpy(f, rec + lc, sizeof(f));
            host_ex_factors[2 * i] = f[0];
            host_ex_factors[2 * i + 1] = f[1];
            std::memmove(ex + i * lc, rec, lc);  // destination never passes the source
        }
        // the storage keeps its ex-data capacity (no shrinking copy of a multi-GB array)
        extended_storage_.resize(N * lc);
        host_long_codes = extended_storage_.data();
    }
}

std::unique_ptr<SearchData> SearchData::load(const std::string &path, bool include_extended, int cpu_threads,
                                             IvfHeader *header, HugeVector<uint32_t> *ids) {
    const IvfReader rd(path);
    const IvfHeader &h = rd.header();
    const std::size_t P = h.padded_dim, W = P / 32, N = h.num, nl = h.nlist;
    const int threads = cpu_threads > 0 ? cpu_threads : omp_get_max_threads();
    std::unique_ptr<SearchData> sd(new SearchData());
    sd->host_rotator = rd.read_rotator();
    sd->h_centroids = rd.read_centroids();
    sd->cluster_sizes.assign(h.cluster_sizes.begin(), h.cluster_sizes.end());
    for (std::size_t s : sd->cluster_sizes)
        sd->max_cluster_size = std::max(sd->max_cluster_size, s);
    sd->host_short_data.assign(N * W, 0u);
    sd->host_short_factors.assign(N * 3, 0.0f);

    // Chunked pipeline: chunk k+1 is read by a reader thread while chunk k is unpacked.
    // `plan` gives the item ranges, `read` fills a buffer, `work` consumes it.
    auto pipeline = [](const std::vector<std::pair<uint64_t, uint64_t>> &plan, auto read, auto work) {
        std::vector<uint8_t> buf[2];
        std::future<void> pending;
        if (!plan.empty())
            pending = std::async(std::launch::async, [&] { read(plan[0], buf[0]); });
        for (std::size_t k = 0; k < plan.size(); ++k) {
            pending.get();
            if (k + 1 < plan.size())
                pending = std::async(std::launch::async, [&, k] { read(plan[k + 1], buf[(k + 1) & 1]); });
            try {
                work(plan[k], buf[k & 1]);
            } catch (...) {
                if (pending.valid())
                    pending.wait();
                throw;
            }
        }
    };

    // batch data: whole clusters per chunk (a chunk holds at least one cluster)
    std::vector<uint64_t> start(nl + 1, 0), block0(nl + 1, 0);
    for (std::size_t c = 0; c < nl; ++c) {
        start[c + 1] = start[c] + h.cluster_sizes[c];
        block0[c + 1] = block0[c] + (h.cluster_sizes[c] + 31) / 32;
    }
    const uint64_t block_bytes = h.batch_block_bytes(), chunk = stream_chunk_bytes();
    std::vector<std::pair<uint64_t, uint64_t>> cplan;  // cluster ranges [c0, c1)
    for (uint64_t c0 = 0; c0 < nl;) {
        uint64_t c1 = c0 + 1;
        while (c1 < nl && (block0[c1 + 1] - block0[c0]) * block_bytes <= chunk)
            ++c1;
        cplan.emplace_back(c0, c1);
        c0 = c1;
    }
    pipeline(
        cplan,
        [&](std::pair<uint64_t, uint64_t> r, std::vector<uint8_t> &buf) {
            const uint64_t nb = block0[r.second] - block0[r.first];
            buf.resize(nb * block_bytes);
            rd.read_batch_blocks(block0[r.first], nb, buf.data());
        },
        [&](std::pair<uint64_t, uint64_t> r, std::vector<uint8_t> &buf) {
#pragma omp parallel num_threads(threads)
            {
                std::vector<uint32_t> words;
#pragma omp for schedule(dynamic, 16)
                for (long long cl = static_cast<long long>(r.first); cl < static_cast<long long>(r.second); ++cl) {
                    const std::size_t c = static_cast<std::size_t>(cl);
                    unpack_cluster(buf.data() + (block0[c] - block0[r.first]) * block_bytes, h.cluster_sizes[c],
                                   start[c], P, sd->host_short_data.data(), sd->host_short_factors.data(), words);
                }
            }
        });

    // ex data: records split into the dense code array and the factor pairs
    // (search_data.cpp:84-123 compacts the same split in place)
    if (include_extended && h.ex_bits > 0) {
        const std::size_t lc = h.ex_code_bytes(), stride = h.ex_stride();
        sd->host_ex_factors.assign(N * 2, 0.0f);
        sd->extended_huge_.resize(N * lc);
        const uint64_t per = std::max<uint64_t>(1, chunk / stride);
        std::vector<std::pair<uint64_t, uint64_t>> vplan;
        for (uint64_t v0 = 0; v0 < N; v0 += per)
            vplan.emplace_back(v0, std::min<uint64_t>(N, v0 + per));
        uint8_t *codes = sd->extended_huge_.data();
        float *fac = sd->host_ex_factors.data();
        pipeline(
            vplan,
            [&](std::pair<uint64_t, uint64_t> r, std::vector<uint8_t> &buf) {
                buf.resize((r.second - r.first) * stride);
                rd.read_ex_records(r.first, r.second - r.first, buf.data());
            },
            [&](std::pair<uint64_t, uint64_t> r, std::vector<uint8_t> &buf) {
                const long long n = static_cast<long long>(r.second - r.first);
#pragma omp parallel for schedule(static) num_threads(threads)
                for (long long i = 0; i < n; ++i) {
                    const uint8_t *rec = buf.data() + static_cast<std::size_t>(i) * stride;
                    const std::size_t v = r.first + static_cast<std::size_t>(i);
                    std::memcpy(codes + v * lc, rec, lc);
                    std::memcpy(fac + 2 * v, rec + lc, 2 * sizeof(float));
                }
            });
        sd->host_long_codes = codes;
    }
    if (ids) {
        ids->resize(N);
        rd.read_ids(ids->data());
    }
    if (header)
        *header = h;
    return sd;
}

// ------------------------------------------------------------------------------------
// Quantizer (rabitq_impl.hpp). Float reductions accumulate in double and round once.
// ------------------------------------------------------------------------------------
namespace {
constexpr float kConstEpsilon = 1.9f;                          // rabitq_impl.hpp:18
constexpr double kTightStart[9] = {0, 0.15, 0.20, 0.52, 0.59, 0.71, 0.75, 0.77, 0.81};  // :263-273

// best_rescale_factor (rabitq_impl.hpp:276-333): sweep t upward through the points where
// some coordinate's code increments and keep the t maximising <code + 1/2, |o|> / ||code + 1/2||.
// The reference pops these events from a priority queue of (t, coordinate) pairs; the
// events it pops are fixed in advance (per coordinate: its first increment, then each next
// one while the code is below 2^ex - 1 and t < t_end), so the same sequence is produced
// here by a bucket sort of all events on t, ties in coordinate order, in O(events), and
// swept with the same double-precision updates in the same order.
double best_rescale_factor(const float *o_abs, std::size_t dim, std::size_t ex_bits) {
    constexpr double kEps = 1e-5;
    constexpr int kNEnum = 10;
    const int cap = (1 << ex_bits) - 1;
    const double max_o = *std::max_element(o_abs, o_abs + dim);
    const double t_end = static_cast<double>(cap + kNEnum) / max_o;
    const double t_start = t_end * kTightStart[ex_bits];
    struct Event {
        double t;
        uint32_t dim;
    };
    thread_local std::vector<Event> ev, sorted;
    thread_local std::vector<uint32_t> bucket;
    ev.clear();
    double sqr_den = static_cast<double>(dim) * 0.25;
    double num = 0;
    for (std::size_t i = 0; i < dim; ++i) {
        const int c = static_cast<int>(std::fma(t_start, static_cast<double>(o_abs[i]), kEps));
        sqr_den += c * c + c;
        num += (c + 0.5) * o_abs[i];
        const double oi = o_abs[i];
        ev.push_back({static_cast<double>(c + 1) / oi, static_cast<uint32_t>(i)});
        for (int v = c + 1; v < cap; ++v) {  // code after the previous pop is v
            const double tn = static_cast<double>(v + 1) / oi;
            if (!(tn < t_end))
                break;
            ev.push_back({tn, static_cast<uint32_t>(i)});
        }
    }
    // Events below t_end are bucket-sorted over [lo, t_end) (bucket index monotone in t;
    // stable, so coordinate order within a bucket, then insertion-sorted on (t, coordinate)).
    // The few events at or above t_end (first increments of near-zero coordinates, +inf for a
    // zero one) all come after them and are sorted on their own.
    double lo = t_end;
    std::size_t n_main = 0;
    for (const Event &e : ev)
        if (e.t < t_end) {
            lo = std::min(lo, e.t);
            ++n_main;
        }
    // one bucket per event; the bucket of each event is computed once
    const std::size_t nb = n_main + 1;
    const double scale = t_end > lo ? static_cast<double>(nb - 1) / (t_end - lo) : 0.0;
    thread_local std::vector<uint32_t> bid;
    bid.resize(ev.size());
    bucket.assign(nb + 1, 0);
    for (std::size_t k = 0; k < ev.size(); ++k) {
        const double t = ev[k].t;
        const uint32_t b = t < t_end ? static_cast<uint32_t>(std::min<double>((t - lo) * scale, nb - 1))
                                     : static_cast<uint32_t>(nb);
        bid[k] = b;
        if (b < nb)
            ++bucket[b + 1];
    }
    for (std::size_t b = 0; b < nb; ++b)
        bucket[b + 1] += bucket[b];
    sorted.resize(ev.size());
    std::size_t n_over = 0;
    for (std::size_t k = 0; k < ev.size(); ++k) {
        if (bid[k] < nb)
            sorted[bucket[bid[k]]++] = ev[k];
        else
            sorted[n_main + n_over++] = ev[k];
    }
    auto before = [](const Event &a, const Event &b) { return a.t < b.t || (a.t == b.t && a.dim < b.dim); };
    for (std::size_t b = 0, s0 = 0; b < nb; ++b) {
        const std::size_t s1 = bucket[b];
        for (std::size_t i = s0 + 1; i < s1; ++i) {
            const Event x = sorted[i];
            std::size_t j = i;
            while (j > s0 && before(x, sorted[j - 1])) {
                sorted[j] = sorted[j - 1];
                --j;
            }
            sorted[j] = x;
        }
        s0 = s1;
    }
    std::sort(sorted.begin() + n_main, sorted.end(), before);
    thread_local std::vector<int> cur;
    cur.resize(dim);
    for (std::size_t i = 0; i < dim; ++i)
        cur[i] = static_cast<int>(std::fma(t_start, static_cast<double>(o_abs[i]), kEps));
    double best_ip = 0, best_t = 0;
    for (const Event &e : sorted) {
        const int v = ++cur[e.dim];
        sqr_den += 2 * v;
        num += o_abs[e.dim];
        const double ip = num / std::sqrt(sqr_den);
        if (ip > best_ip) {
            best_ip = ip;
            best_t = e.t;
        }
    }
    return best_t;
}

double dot(const float *a, const float *b, std::size_t n) {
    double s = 0;
    for (std::size_t i = 0; i < n; ++i)
        s += static_cast<double>(a[i]) * b[i];
    return s;
}
}  // namespace

void quantize_one_bit(const float *x, const float *c, std::size_t P, uint8_t *bits, float *f,
                      int metric) {
    std::vector<float> o(P), xu(P);
    for (std::size_t i = 0; i < P; ++i) {
        o[i] = x[i] - c[i];
        bits[i] = o[i] > 0 ? 1 : 0;
        xu[i] = static_cast<float>(bits[i]) - 0.5f;
    }
    const float l2_sqr = static_cast<float>(dot(o.data(), o.data(), P));
    const float l2 = std::sqrt(l2_sqr);
    float ip_resi = static_cast<float>(dot(o.data(), xu.data(), P));
    const float ip_cent = static_cast<float>(dot(c, xu.data(), P));
    if (ip_resi == 0)
        ip_resi = std::numeric_limits<float>::infinity();
    const float xu_sqr = static_cast<float>(dot(xu.data(), xu.data(), P));
    const float err = l2 * kConstEpsilon *
                      std::sqrt((((l2_sqr * xu_sqr) / (ip_resi * ip_resi)) - 1) /
                                static_cast<float>(P - 1));
    if (metric == 0) {
        f[0] = l2_sqr + (2 * l2_sqr * ip_cent / ip_resi);
        f[1] = -2 * l2_sqr / ip_resi;
        f[2] = 2 * err;
    } else {
        f[0] = 1 - static_cast<float>(dot(o.data(), c, P)) + (l2_sqr * ip_cent / ip_resi);
        f[1] = -l2_sqr / ip_resi;
        f[2] = err;
    }
}

void quantize_ex_bits(const float *x, const float *c, std::size_t P, std::size_t ex_bits,
                      uint8_t *code, float *f, int metric) {
    std::vector<float> o(P), o_abs(P);
    for (std::size_t i = 0; i < P; ++i)
        o[i] = x[i] - c[i];
    const float norm = std::sqrt(static_cast<float>(dot(o.data(), o.data(), P)));
    for (std::size_t i = 0; i < P; ++i)
        o_abs[i] = std::fabs(o[i] / norm);
    // quantize_ex (rabitq_impl.hpp:336-360)
    constexpr double kEps = 1e-5;
    const double t = best_rescale_factor(o_abs.data(), P, ex_bits);
    const int cap = (1 << ex_bits) - 1;
    double ipnorm = 0;
    for (std::size_t i = 0; i < P; ++i) {
        int v = static_cast<int>(std::fma(t, static_cast<double>(o_abs[i]), kEps));
        v = std::min(v, cap);
        code[i] = static_cast<uint8_t>(v);
        ipnorm += (v + 0.5) * o_abs[i];
    }
    float ipnorm_inv = static_cast<float>(1 / ipnorm);
    if (!std::isnormal(ipnorm_inv))
        ipnorm_inv = 1.0f;
    // negative residual dimensions store the bitwise complement (rabitq_impl.hpp:423-429)
    for (std::size_t i = 0; i < P; ++i)
        if (o[i] < 0)
            code[i] = static_cast<uint8_t>((~code[i]) & cap);
    // factors on total_code = code + (o >= 0) * 2^ex (rabitq_impl.hpp:455-499)
    std::vector<float> xu(P);
    const float cb = -(static_cast<float>(1 << ex_bits) - 0.5f);
    for (std::size_t i = 0; i < P; ++i)
        xu[i] = static_cast<float>(code[i] + ((o[i] >= 0) ? (1 << ex_bits) : 0)) + cb;
    const float l2_sqr = static_cast<float>(dot(o.data(), o.data(), P));
    const float l2 = std::sqrt(l2_sqr);
    float ip_resi = static_cast<float>(dot(o.data(), xu.data(), P));
    const float ip_cent = static_cast<float>(dot(c, xu.data(), P));
    if (ip_resi == 0)
        ip_resi = std::numeric_limits<float>::infinity();
    if (metric == 0) {
        f[0] = l2_sqr + (2 * l2_sqr * ip_cent / ip_resi);
        f[1] = ipnorm_inv * -2 * l2;
    } else {
        f[0] = 1 - static_cast<float>(dot(o.data(), c, P)) + (l2_sqr * ip_cent / ip_resi);
        f[1] = ipnorm_inv * -l2;
    }
}

void pack_excode7(const uint8_t *code, std::size_t P, uint8_t *out) {
    for (std::size_t g = 0; g < P; g += 64) {
        const uint8_t *v = code + g;
        uint8_t *o = out + g / 64 * 56;
        for (int i = 0; i < 16; ++i) {
            const uint8_t hi = v[48 + i];
            o[i] = static_cast<uint8_t>((v[i] & 0x3F) | ((hi << 6) & 0xC0));
            o[16 + i] = static_cast<uint8_t>((v[16 + i] & 0x3F) | ((hi << 4) & 0xC0));
            o[32 + i] = static_cast<uint8_t>((v[32 + i] & 0x3F) | ((hi << 2) & 0xC0));
        }
        uint64_t top = 0;
        for (int d = 0; d < 64; ++d)
            top |= static_cast<uint64_t>((v[d] >> 6) & 1) << (8 * (d % 8) + d / 8);
        std::memcpy(o + 48, &top, 8);
    }
}

void fastscan_pack(const uint8_t *compact, std::size_t n, std::size_t P, uint8_t *blocks) {
    const std::size_t cols = P / 8;
    const std::size_t nb = (n + 31) / 32;
    for (std::size_t b = 0; b < nb; ++b) {
        for (std::size_t col = 0; col < cols; ++col) {
            uint8_t hi[32], lo[32];
            for (int r = 0; r < 32; ++r) {
                const std::size_t row = b * 32 + r;
                const uint8_t v = row < n ? compact[row * cols + col] : 0;
                hi[r] = v >> 4;
                lo[r] = v & 15;
            }
            uint8_t *o = blocks + (b * cols + col) * 32;
            for (int j = 0; j < 16; ++j) {
                o[j] = static_cast<uint8_t>(hi[kPerm0[j]] | (hi[kPerm0[j] + 16] << 4));
                o[j + 16] = static_cast<uint8_t>(lo[kPerm0[j]] | (lo[kPerm0[j] + 16] << 4));
            }
        }
    }
}

namespace {

// Cluster order of the rows and the 32-row block of each cluster's first row.
struct ClusterLayout {
    std::vector<std::size_t> start, block0;
};

// Header, rotator, centroids, cluster sizes and ids (cluster order) of an index over
// `assign`, with zeroed code arrays.
ClusterLayout layout_index(IvfFile &f, const float *rotated_centroids, const float *rotator,
                           const uint32_t *assign, std::size_t n, std::size_t dim, std::size_t P,
                           std::size_t nlist, std::size_t ex_bits, int metric) {
    f.num = n;
    f.dim = dim;
    f.padded_dim = P;
    f.nlist = nlist;
    f.ex_bits = ex_bits;
    f.metric = static_cast<uint8_t>(metric);
    f.rotator.assign(rotator, rotator + dim * P);
    f.centroids.assign(rotated_centroids, rotated_centroids + nlist * P);
    f.cluster_sizes.assign(nlist, 0);
    for (std::size_t i = 0; i < n; ++i) {
        if (assign[i] >= nlist)
            throw std::invalid_argument("build_ivf: bad cluster id");
        ++f.cluster_sizes[assign[i]];
    }
    ClusterLayout L;
    L.start.assign(nlist + 1, 0);
    L.block0.assign(nlist + 1, 0);
    for (std::size_t c = 0; c < nlist; ++c) {
        L.start[c + 1] = L.start[c] + f.cluster_sizes[c];
        L.block0[c + 1] = L.block0[c] + (f.cluster_sizes[c] + 31) / 32;
    }
    f.ids.resize(n);
    std::vector<std::size_t> fill(L.start.begin(), L.start.end() - 1);
    for (std::size_t i = 0; i < n; ++i)
        f.ids[fill[assign[i]]++] = static_cast<uint32_t>(i);
    f.batch_data.assign(L.block0[nlist] * f.batch_block_bytes(), 0);
    f.ex_data.assign(n * f.ex_stride(), 0);
    return L;
}

// Every cluster's 32-row FastScan blocks and every row's ex-code record. quant(c, id,
// compact, f1, code, f2) gives row `id` of cluster c: its sign bits as big-endian bytes
// [P/8], f_add / f_rescale / f_error, its ex-code values [P] and f_add_ex / f_rescale_ex.
template <class Quant>
void fill_index(IvfFile &f, const ClusterLayout &L, int threads, Quant quant) {
    const std::size_t P = f.padded_dim, n_all = f.num;
    const std::size_t block_bytes = f.batch_block_bytes(), stride = f.ex_stride();
    const std::size_t lc = f.ex_code_bytes();
    const int nt = threads > 0 ? threads : omp_get_max_threads();
    // large builds report every tenth of the vectors quantised on stderr
    const std::size_t report = n_all >= (std::size_t{1} << 22) ? n_all / 10 : 0;
    std::atomic<std::size_t> done{0};
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
    for (long long cl = 0; cl < static_cast<long long>(f.nlist); ++cl) {
        const std::size_t c = static_cast<std::size_t>(cl);
        const std::size_t n = f.cluster_sizes[c];
        std::vector<uint8_t> compact(32 * P / 8), code(P);
        for (std::size_t i0 = 0; i0 < n; i0 += 32) {
            const std::size_t len = std::min<std::size_t>(32, n - i0);
            uint8_t *blk = f.batch_data.data() + (L.block0[c] + i0 / 32) * block_bytes;
            float *fl = reinterpret_cast<float *>(blk + P * 4);
            std::fill(compact.begin(), compact.end(), 0);
            for (std::size_t v = 0; v < len; ++v) {
                const std::size_t gi = L.start[c] + i0 + v;
                float f1[3], f2[2];
                quant(c, f.ids[gi], compact.data() + v * (P / 8), f1, code.data(), f2);
                fl[v] = f1[0];
                fl[32 + v] = f1[1];
                fl[64 + v] = f1[2];
                uint8_t *rec = f.ex_data.data() + gi * stride;
                pack_excode7(code.data(), P, rec);
                std::memcpy(rec + lc, f2, sizeof(f2));
            }
            fastscan_pack(compact.data(), len, P, blk);
        }
        if (report) {
            const std::size_t before = done.fetch_add(n, std::memory_order_relaxed);
            if (before / report != (before + n) / report)
                std::fprintf(stderr, "[build_ivf] packed %zu / %zu vectors\n", before + n, n_all);
        }
    }
}

}  // namespace

IvfFile build_ivf(const BuildInput &in, int threads) {
    if (!in.rotated_data || !in.rotated_centroids || !in.assignments || !in.rotator || !in.n ||
        !in.dim || in.padded_dim % 64 || in.padded_dim < in.dim || !in.nlist || in.ex_bits != 7)
        throw std::invalid_argument("build_ivf: invalid input (ex_bits must be 7)");
    const std::size_t P = in.padded_dim;
    IvfFile f;
    const ClusterLayout L = layout_index(f, in.rotated_centroids, in.rotator, in.assignments, in.n, in.dim, P,
                                         in.nlist, in.ex_bits, in.metric);
    fill_index(f, L, threads,
               [&](std::size_t c, uint32_t id, uint8_t *compact, float *f1, uint8_t *code, float *f2) {
                   thread_local std::vector<uint8_t> bits;
                   bits.resize(P);
                   const float *x = in.rotated_data + static_cast<std::size_t>(id) * P;
                   const float *cent = in.rotated_centroids + c * P;
                   quantize_one_bit(x, cent, P, bits.data(), f1, in.metric);
                   for (std::size_t d = 0; d < P; ++d)
                       compact[d / 8] |= static_cast<uint8_t>(bits[d] << (7 - d % 8));
                   quantize_ex_bits(x, cent, P, in.ex_bits, code, f2, in.metric);
               });
    return f;
}

IvfFile build_ivf_gpu(const GpuBuildInput &in, int device, int threads) {
    if (!in.data || !in.rotated_centroids || !in.assignments || !in.rotator || !in.n || !in.dim ||
        in.padded_dim % 64 || in.padded_dim < in.dim || in.padded_dim > 1024 || !in.nlist || in.ex_bits != 7)
        throw std::invalid_argument("build_ivf_gpu: invalid input (ex_bits must be 7, P <= 1024)");
    const std::size_t P = in.padded_dim, n = in.n;
    IvfFile f;
    const ClusterLayout L = layout_index(f, in.rotated_centroids, in.rotator, in.assignments, n, in.dim, P,
                                         in.nlist, in.ex_bits, in.metric);
    std::vector<uint8_t> bits(n * (P / 8)), code(n * P);
    std::vector<float> f1(n * 3), f2(n * 2);
    if (int rc = cora_tool_quantize(in.data, n, in.dim, in.rotator, P, in.rotated_centroids, in.nlist,
                                    in.assignments, in.metric, bits.data(), f1.data(), code.data(), f2.data(),
                                    device))
        throw std::runtime_error(std::string("build_ivf_gpu: ") + cora_tool_last_error() + " (status " +
                                 std::to_string(rc) + ")");
    fill_index(f, L, threads,
               [&](std::size_t, uint32_t id, uint8_t *compact, float *g1, uint8_t *cd, float *g2) {
                   std::memcpy(compact, bits.data() + static_cast<std::size_t>(id) * (P / 8), P / 8);
                   std::memcpy(g1, f1.data() + static_cast<std::size_t>(id) * 3, 12);
                   std::memcpy(cd, code.data() + static_cast<std::size_t>(id) * P, P);
                   std::memcpy(g2, f2.data() + static_cast<std::size_t>(id) * 2, 8);
               });
    return f;
}

}  // namespace coraanns::index
