// Golden-vector dumper for the reference CPU path.
//
// Test infrastructure only. This program is compiled by oracle/Makefile against
// the reference's own headers and sources where they lie under /root/reference
// (rabitqlib + src/index/search_data.cpp) into oracle/_ref/, and is run in the
// build container only, by tests/golden/make_golden.py, to write the fixtures
// committed under tests/golden/. Nothing in the product links or runs it.
//
// Modes
//   ref_dump index <ivf.index> <queries.fbin> <outdir> <topk> <nprobe>...
//       Loads the index with rabitqlib::ivf::IVF::load (ivf.hpp:447-539), adapts it
//       with coraanns::index::SearchData (search_data.cpp:9-127) and dumps every
//       array HybridIndex::load_from_raw_pointers consumes, the rotated queries
//       (MatrixRotator::rotate, rotator.hpp:108-112), the flat-initializer probe
//       distances (initializer.hpp:128-145), FastScan-hacc estimates and the
//       split_distance_boosting ex-distances for each query's first probe
//       (estimator.hpp:25-103), and IVF::search top-k ids (ivf.hpp:670-732).
//   ref_dump quant <rows.f32> <n> <dim> <outdir>
//       Row 0 of the input is the centroid, rows 1..n are data points. Dumps
//       one_bit_code_with_factor and ex_bits_code_with_factor (rabitq_impl.hpp:76-137,
//       435-500) for L2 and IP, packing_7bit_excode (pack_excode.hpp:216-265),
//       ip64_fxu7_avx against the centroid row used as a query (space.hpp:677-761)
//       and fastscan::pack_codes of the sign bits (fastscan.hpp:69-106).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "coraanns/index/search_data.hpp"
#include "rabitqlib/defines.hpp"
#include "rabitqlib/fastscan/fastscan.hpp"
#include "rabitqlib/index/estimator.hpp"
#include "rabitqlib/index/ivf/ivf.hpp"
#include "rabitqlib/index/query.hpp"
#include "rabitqlib/quantization/data_layout.hpp"
#include "rabitqlib/quantization/pack_excode.hpp"
#include "rabitqlib/quantization/rabitq_impl.hpp"
#include "rabitqlib/utils/rotator.hpp"
#include "rabitqlib/utils/space.hpp"

namespace {

struct Manifest {
    std::string dir;
    std::ofstream list;
    explicit Manifest(const std::string &d) : dir(d), list(d + "/manifest.txt") {}
    template <class T>
    void put(const std::string &name, const char *dtype, const T *data, size_t count,
             const std::string &shape) {
        std::ofstream out(dir + "/" + name + ".bin", std::ios::binary);
        out.write(reinterpret_cast<const char *>(data), sizeof(T) * count);
        list << name << ' ' << dtype << ' ' << shape << '\n';
    }
};

std::string shape2(size_t a, size_t b) { return std::to_string(a) + "," + std::to_string(b); }

std::vector<float> read_fbin(const char *path, uint32_t &rows, uint32_t &cols) {
    std::ifstream in(path, std::ios::binary);
    if (!in)
        throw std::runtime_error(std::string("cannot open ") + path);
    in.read(reinterpret_cast<char *>(&rows), 4);
    in.read(reinterpret_cast<char *>(&cols), 4);
    std::vector<float> v(size_t(rows) * cols);
    in.read(reinterpret_cast<char *>(v.data()), v.size() * 4);
    return v;
}

int dump_index(int argc, char **argv) {
    const char *index_path = argv[2];
    const char *query_path = argv[3];
    Manifest m(argv[4]);
    const size_t topk = std::strtoull(argv[5], nullptr, 10);
    std::vector<size_t> nprobes;
    for (int i = 6; i < argc; ++i)
        nprobes.push_back(std::strtoull(argv[i], nullptr, 10));

    rabitqlib::ivf::IVF ivf;
    ivf.load(index_path);
    const size_t n = ivf.num_vectors(), dim = ivf.dim(), P = ivf.padded_dim();
    const size_t nl = ivf.num_clusters(), ex = ivf.ex_bits();

    // Rotator and probe helpers come from the IVF before SearchData takes the ex-codes.
    std::vector<float> rot(dim * P);
    ivf.save_rotator(reinterpret_cast<char *>(rot.data()));
    rabitqlib::rotator_impl::MatrixRotator<float> rotator(dim, P);
    rotator.load(reinterpret_cast<const char *>(rot.data()));

    uint32_t nq = 0, qd = 0;
    std::vector<float> queries = read_fbin(query_path, nq, qd);
    if (qd != dim)
        throw std::runtime_error("query dim mismatch");

    // IVF::search top-k ids for every nprobe (hacc = true, the rabitq_cpu default).
    std::vector<uint32_t> ids(nprobes.size() * nq * topk, 0);
    for (size_t l = 0; l < nprobes.size(); ++l)
        for (size_t q = 0; q < nq; ++q)
            ivf.search(&queries[q * dim], topk, nprobes[l], &ids[(l * nq + q) * topk], true);
    m.put("search_ids", "u32", ids.data(), ids.size(),
          std::to_string(nprobes.size()) + "," + shape2(nq, topk));
    std::vector<uint64_t> np64(nprobes.begin(), nprobes.end());
    m.put("search_nprobes", "u64", np64.data(), np64.size(), std::to_string(np64.size()));

    // Rotated queries, centroid distances (flat initializer formula) and per-cluster estimates.
    std::vector<float> rq(size_t(nq) * P);
    std::vector<float> cdist(size_t(nq) * nl), cip(size_t(nq) * nl);
    for (size_t q = 0; q < nq; ++q) {
        rotator.rotate(&queries[q * dim], &rq[q * P]);
        for (size_t c = 0; c < nl; ++c) {
            cdist[q * nl + c] = std::sqrt(rabitqlib::euclidean_sqr(&rq[q * P], ivf.centroid(c), P));
            cip[q * nl + c] = rabitqlib::dot_product<float>(&rq[q * P], ivf.centroid(c), P);
        }
    }
    m.put("rotated_queries", "f32", rq.data(), rq.size(), shape2(nq, P));
    m.put("centroid_dist", "f32", cdist.data(), cdist.size(), shape2(nq, nl));
    m.put("centroid_ip", "f32", cip.data(), cip.size(), shape2(nq, nl));

    // FastScan-hacc estimate and ex-distance of every vector of cluster (q % nl) for each query.
    std::vector<float> est(size_t(nq) * 0), low, ipx0, exd, kvals;
    std::vector<uint32_t> est_cluster(nq);
    const size_t ex_stride = rabitqlib::ExDataMap<float>::data_bytes(P, ex);
    auto ipf = rabitqlib::select_excode_ipfunc(ex);
    for (size_t q = 0; q < nq; ++q) {
        const size_t c = q % nl;
        est_cluster[q] = c;
        rabitqlib::SplitBatchQuery<float> qo(&rq[q * P], P, ex, ivf.metric_type(), true);
        qo.set_g_add(cdist[q * nl + c], cip[q * nl + c]);
        kvals.push_back(qo.k1xsumq());
        kvals.push_back(qo.kbxsumq());
        kvals.push_back(qo.g_add());
        kvals.push_back(qo.g_error());
        kvals.push_back(qo.delta());
        kvals.push_back(qo.sum_vl_lut());
        const auto &cl = ivf.clusters()[c];
        const char *batch = cl.batch_data();
        const char *exd_ptr = cl.ex_data();
        for (size_t i = 0; i < cl.num(); i += rabitqlib::fastscan::kBatchSize) {
            float e[32], lo[32], x0[32];
            rabitqlib::split_batch_estdist(batch, qo, P, e, lo, x0, true);
            const size_t cnt = std::min<size_t>(32, cl.num() - i);
            for (size_t v = 0; v < cnt; ++v) {
                est.push_back(e[v]);
                low.push_back(lo[v]);
                ipx0.push_back(x0[v]);
                exd.push_back(rabitqlib::split_distance_boosting(exd_ptr, ipf, qo, P, ex, x0[v]));
                exd_ptr += ex_stride;
            }
            batch += rabitqlib::BatchDataMap<float>::data_bytes(P);
        }
    }
    m.put("est_cluster", "u32", est_cluster.data(), nq, std::to_string(nq));
    m.put("est_qvals", "f32", kvals.data(), kvals.size(), shape2(nq, 6));
    m.put("est_dist", "f32", est.data(), est.size(), std::to_string(est.size()));
    m.put("est_low", "f32", low.data(), low.size(), std::to_string(low.size()));
    m.put("est_ipx0", "f32", ipx0.data(), ipx0.size(), std::to_string(ipx0.size()));
    m.put("est_exdist", "f32", exd.data(), exd.size(), std::to_string(exd.size()));

    // Raw IVF payload pieces needed to re-read the file independently.
    std::vector<uint64_t> meta = {n, dim, P, nl, ex, uint64_t(ivf.metric_type())};
    m.put("meta", "u64", meta.data(), meta.size(), "6");
    std::vector<uint32_t> pids(ivf.ids(), ivf.ids() + n);
    m.put("ids", "u32", pids.data(), n, std::to_string(n));

    // SearchData: the exact arrays HybridIndex::load_from_raw_pointers receives.
    coraanns::index::SearchData sd(ivf, true, 1);
    m.put("centroids", "f32", sd.h_centroids.data(), sd.h_centroids.size(), shape2(nl, P));
    m.put("rotator", "f32", sd.host_rotator.data(), sd.host_rotator.size(), shape2(dim, P));
    m.put("short_data", "u32", sd.host_short_data.data(), sd.host_short_data.size(),
          shape2(n, P / 32));
    m.put("short_factors", "f32", sd.host_short_factors.data(), sd.host_short_factors.size(),
          shape2(n, 3));
    const size_t lc = (P * ex + 7) / 8;
    m.put("long_codes", "u8", sd.host_long_codes, n * lc, shape2(n, lc));
    m.put("ex_factors", "f32", sd.host_ex_factors.data(), sd.host_ex_factors.size(), shape2(n, 2));
    std::vector<uint64_t> sizes(sd.cluster_sizes.begin(), sd.cluster_sizes.end());
    m.put("cluster_sizes", "u64", sizes.data(), sizes.size(), std::to_string(nl));
    return 0;
}

int dump_quant(int argc, char **argv) {
    (void)argc;
    const char *path = argv[2];
    const size_t n = std::strtoull(argv[3], nullptr, 10);
    const size_t dim = std::strtoull(argv[4], nullptr, 10);
    Manifest m(argv[5]);
    std::vector<float> rows((n + 1) * dim);
    {
        std::ifstream in(path, std::ios::binary);
        in.read(reinterpret_cast<char *>(rows.data()), rows.size() * 4);
        if (!in)
            throw std::runtime_error("short quant input");
    }
    const float *centroid = rows.data();
    const size_t ex_bits = 7;
    for (int metric = 0; metric < 2; ++metric) {
        const auto mt = metric == 0 ? rabitqlib::METRIC_L2 : rabitqlib::METRIC_IP;
        const std::string tag = metric == 0 ? "l2" : "ip";
        std::vector<int32_t> bits(n * dim);
        std::vector<float> f1(n * 3);
        std::vector<uint8_t> excode(n * dim);
        std::vector<float> f2(n * 3);
        for (size_t i = 0; i < n; ++i) {
            const float *x = rows.data() + (i + 1) * dim;
            rabitqlib::quant::rabitq_impl::one_bit::one_bit_code_with_factor<float>(
                x, centroid, dim, &bits[i * dim], f1[i * 3], f1[i * 3 + 1], f1[i * 3 + 2], mt);
            rabitqlib::quant::rabitq_impl::ex_bits::ex_bits_code_with_factor<float, uint8_t>(
                x, centroid, dim, ex_bits, &excode[i * dim], f2[i * 3], f2[i * 3 + 1], f2[i * 3 + 2],
                mt);
        }
        m.put("bits_" + tag, "i32", bits.data(), bits.size(), shape2(n, dim));
        m.put("f1_" + tag, "f32", f1.data(), f1.size(), shape2(n, 3));
        m.put("excode_" + tag, "u8", excode.data(), excode.size(), shape2(n, dim));
        m.put("f2_" + tag, "f32", f2.data(), f2.size(), shape2(n, 3));
        if (metric == 0) {
            // 7-bit packing, AVX2 ex-code inner product and FastScan packing of the sign bits.
            const size_t lc = dim * ex_bits / 8;
            std::vector<uint8_t> packed(n * lc);
            std::vector<float> ip(n);
            for (size_t i = 0; i < n; ++i) {
                rabitqlib::quant::rabitq_impl::ex_bits::packing_7bit_excode(
                    &excode[i * dim], &packed[i * lc], dim);
                ip[i] = rabitqlib::excode_ipimpl::ip64_fxu7_avx(centroid, &packed[i * lc], dim);
            }
            m.put("packed7", "u8", packed.data(), packed.size(), shape2(n, lc));
            m.put("ip_fxu7", "f32", ip.data(), ip.size(), std::to_string(n));
            std::vector<uint8_t> compact(n * dim / 8);
            for (size_t i = 0; i < n; ++i)
                rabitqlib::pack_binary(&bits[i * dim], &compact[i * dim / 8], dim);
            const size_t nb = (n + 31) / 32;
            std::vector<uint8_t> blocks(nb * 32 * dim / 8);
            rabitqlib::fastscan::pack_codes(dim, compact.data(), n, blocks.data());
            m.put("compact_bits", "u8", compact.data(), compact.size(), shape2(n, dim / 8));
            m.put("fastscan_blocks", "u8", blocks.data(), blocks.size(),
                  std::to_string(blocks.size()));
        }
    }
    return 0;
}

} // namespace

int main(int argc, char **argv) {
    try {
        if (argc >= 6 && std::string(argv[1]) == "index")
            return dump_index(argc, argv);
        if (argc == 6 && std::string(argv[1]) == "quant")
            return dump_quant(argc, argv);
        std::fprintf(stderr, "usage: ref_dump index <ivf> <queries.fbin> <outdir> <topk> <nprobe>...\n"
                             "       ref_dump quant <rows.f32> <n> <dim> <outdir>\n");
        return 2;
    } catch (const std::exception &e) {
        std::fprintf(stderr, "ref_dump: %s\n", e.what());
        return 1;
    }
}
