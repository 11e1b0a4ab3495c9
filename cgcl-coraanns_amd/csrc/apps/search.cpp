// coraanns_search: GPU filter / CPU refine benchmark driver.
//
// Same command line, output lines and final table as the reference driver
// (apps/search.cpp:27-320): options --k v or --k=v (duplicates and unknown keys rejected,
// booleans true/1/yes/on, false/0/no/off; include/coraanns/benchmark/options.hpp:17-92),
// the default nprobe grid (options.hpp:94-132), query chunks of at most 65,535, warmup
// and timed rounds per nprobe with QPS = nq / wall time, recall outside the timer
// (ID recall, or distance-aware with --recall-base; recall.hpp:74-275), and the final
// "nprobe\tQPS\trecall" table. --batch-q accepts 1..64 here (the reference 1..6).
#include <fcntl.h>
#include <omp.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <limits>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "coraanns/benchmark/recall.hpp"
#include "coraanns/index/ivf_file.hpp"
#include "coraanns/index/search_data.hpp"
#include "coraanns/search/hybrid.hpp"

namespace {

void print_usage(const char *program) {
    std::cerr << "Usage: " << program
              << " <index_file> <query_file> <gt_file>"
                 " [--topk 100] [--nprobes 40,50,...] [--rounds 5]"
                 " [--warmup 1] [--batch-q 4] [--query-chunk N] [--threads N]"
                 " [--vanguard-size 5] [--cpu-secondary-filter true]"
                 " [--queue-capacity 67108864] [--queue-spill-capacity 16777216]"
                 " [--cross-query-reuse true] [--candidate-stats false]"
                 " [--gpu-filter-timing false] [--profile false]"
                 " [--exact-base FILE] [--recall-base FILE] [--recall-once false]"
                 " [--lower-bound-scale 1.3]\n";
}

class Options {
  public:
    Options(int argc, char **argv, int begin) {
        for (int i = begin; i < argc; ++i) {
            std::string arg(argv[i]);
            if (arg.rfind("--", 0) != 0)
                throw std::invalid_argument("Unexpected positional argument: " + arg);
            arg.erase(0, 2);
            std::string key, value;
            const auto eq = arg.find('=');
            if (eq != std::string::npos) {
                key = arg.substr(0, eq);
                value = arg.substr(eq + 1);
            } else {
                key = arg;
                if (i + 1 >= argc || std::strncmp(argv[i + 1], "--", 2) == 0)
                    throw std::invalid_argument("Missing value for --" + key);
                value = argv[++i];
            }
            if (key.empty() || kv_.count(key))
                throw std::invalid_argument("Invalid or duplicate option --" + key);
            kv_[key] = value;
        }
    }
    void require_known(const std::vector<std::string> &known) const {
        for (const auto &e : kv_)
            if (std::find(known.begin(), known.end(), e.first) == known.end())
                throw std::invalid_argument("Unknown option --" + e.first);
    }
    std::string get(const std::string &k, const std::string &d) const {
        auto it = kv_.find(k);
        return it == kv_.end() ? d : it->second;
    }
    std::size_t size(const std::string &k, std::size_t d) const {
        const std::string t = get(k, "");
        if (t.empty())
            return d;
        if (t[0] == '-' || t[0] == '+')
            throw std::invalid_argument("Invalid integer for --" + k + ": " + t);
        std::size_t used = 0;
        const unsigned long long v = std::stoull(t, &used);
        if (used != t.size())
            throw std::invalid_argument("Invalid integer for --" + k + ": " + t);
        return static_cast<std::size_t>(v);
    }
    bool flag(const std::string &k, bool d) const {
        const std::string t = get(k, d ? "true" : "false");
        if (t == "true" || t == "1" || t == "yes" || t == "on")
            return true;
        if (t == "false" || t == "0" || t == "no" || t == "off")
            return false;
        throw std::invalid_argument("Invalid boolean for --" + k + ": " + t);
    }

  private:
    std::map<std::string, std::string> kv_;
};

std::vector<std::size_t> parse_nprobes(const std::string &text, std::size_t nlist) {
    std::vector<std::size_t> out;
    if (text.empty()) {
        for (std::size_t v : {40, 50, 60, 75, 95, 128, 180, 255, 400, 535, 775, 1400})
            if (v <= nlist)
                out.push_back(v);
        if (out.empty())
            out.push_back(nlist);
        return out;
    }
    std::size_t begin = 0;
    while (begin <= text.size()) {
        const auto comma = text.find(',', begin);
        const std::string tok = text.substr(begin, comma == std::string::npos ? std::string::npos : comma - begin);
        if (tok.empty() || tok[0] == '-' || tok[0] == '+')
            throw std::invalid_argument("Invalid value in --nprobes: " + tok);
        std::size_t used = 0;
        const unsigned long long v = std::stoull(tok, &used);
        if (used != tok.size() || v == 0 || v > nlist)
            throw std::invalid_argument("Each nprobe must be in [1, nlist]; got: " + tok);
        if (std::find(out.begin(), out.end(), v) != out.end())
            throw std::invalid_argument("Duplicate nprobe value: " + tok);
        out.push_back(v);
        if (comma == std::string::npos)
            break;
        begin = comma + 1;
    }
    return out;
}

// Read-only mapping of an .fvecs/.ivecs or .fbin/.ibin matrix (4-byte elements).
class Matrix {
  public:
    explicit Matrix(const std::string &path) {
        fd_ = open(path.c_str(), O_RDONLY);
        if (fd_ < 0)
            throw std::runtime_error("File " + path + " not exists");
        struct stat st {};
        fstat(fd_, &st);
        size_ = static_cast<std::size_t>(st.st_size);
        map_ = static_cast<const uint8_t *>(mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0));
        if (map_ == MAP_FAILED)
            throw std::runtime_error("cannot map " + path);
        const bool vecs = path.size() > 4 && path.compare(path.size() - 4, 4, "vecs") == 0;
        if (vecs) {
            uint32_t d;
            std::memcpy(&d, map_, 4);
            cols_ = d;
            stride_ = 4 + 4ull * d;
            offset_ = 4;
            rows_ = size_ / stride_;
        } else {
            uint32_t rc[2];
            std::memcpy(rc, map_, 8);
            rows_ = rc[0];
            cols_ = rc[1];
            stride_ = 4ull * cols_;
            offset_ = 8;
            if (8 + rows_ * stride_ > size_)
                throw std::runtime_error("truncated matrix file " + path);
        }
    }
    ~Matrix() {
        if (map_ && map_ != MAP_FAILED)
            munmap(const_cast<uint8_t *>(map_), size_);
        if (fd_ >= 0)
            close(fd_);
    }
    std::size_t rows() const { return rows_; }
    std::size_t cols() const { return cols_; }
    template <class T>
    const T *row(std::size_t i) const {
        return reinterpret_cast<const T *>(map_ + offset_ + i * stride_);
    }
    template <class T>
    std::vector<T> dense() const {
        std::vector<T> out(rows_ * cols_);
        for (std::size_t i = 0; i < rows_; ++i)
            std::memcpy(out.data() + i * cols_, row<T>(i), 4 * cols_);
        return out;
    }
    const uint8_t *mapping() const { return map_; }
    std::size_t stride() const { return stride_; }
    std::size_t offset() const { return offset_; }

  private:
    int fd_ = -1;
    const uint8_t *map_ = nullptr;
    std::size_t size_ = 0, rows_ = 0, cols_ = 0, stride_ = 0, offset_ = 0;
};

// Distance-aware recall needs the base rows; the mapping above provides them.
coraanns::benchmark::MatrixView view_of(const Matrix &m) {
    coraanns::benchmark::MatrixView v;
    v.data = m.mapping();
    v.offset = m.offset();
    v.stride = m.stride();
    v.rows = m.rows();
    v.cols = m.cols();
    return v;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 4) {
        print_usage(argv[0]);
        return 1;
    }
    try {
        Options opt(argc, argv, 4);
        opt.require_known({"topk", "nprobes", "rounds", "warmup", "batch-q", "threads",
                           "query-chunk", "vanguard-size", "cpu-secondary-filter", "profile",
                           "cross-query-reuse", "candidate-stats", "gpu-filter-timing",
                           "exact-base", "recall-once", "queue-capacity", "queue-spill-capacity",
                           "recall-base", "lower-bound-scale"});
        const std::size_t topk = opt.size("topk", 100);
        const std::size_t rounds = opt.size("rounds", 5);
        const std::size_t warmup = opt.size("warmup", 1);
        const bool recall_once = opt.flag("recall-once", false);
        const std::size_t batch_q = opt.size("batch-q", coraanns::default_batch_q);
        if (batch_q < 1 || batch_q > static_cast<std::size_t>(coraanns::max_batch_q))
            throw std::invalid_argument("batch-q must be in [1, 64]");
        const std::size_t threads = opt.size("threads", static_cast<std::size_t>(omp_get_max_threads()));
        if (threads == 0 || threads > static_cast<std::size_t>(std::numeric_limits<int>::max()))
            throw std::invalid_argument("threads must be a positive int");
        omp_set_dynamic(0);
        omp_set_num_threads(static_cast<int>(threads));
        const std::size_t vanguard = opt.size("vanguard-size", coraanns::default_vanguard_size);
        const bool profile = opt.flag("profile", false);
        const bool cand_stats = opt.flag("candidate-stats", false);
        const bool filter_timing = opt.flag("gpu-filter-timing", false);
        const bool reuse = opt.flag("cross-query-reuse", true);
        const bool secondary = opt.flag("cpu-secondary-filter", true);
        const std::size_t qcap = opt.size("queue-capacity", coraanns::queue::default_capacity);
        const std::size_t scap = opt.size("queue-spill-capacity", coraanns::queue::default_spill_capacity);
        if (qcap == 0 || (qcap & (qcap - 1)))
            throw std::invalid_argument("queue-capacity must be a positive power of two");
        const std::string exact_file = opt.get("exact-base", "");
        const std::string recall_base = opt.get("recall-base", "");

        std::cout << "Loading queries and groundtruth..." << std::endl;
        Matrix qm(argv[2]), gt(argv[3]);
        const std::vector<float> query = qm.dense<float>();
        const std::size_t nq = qm.rows(), dim = qm.cols();
        std::cout << "Loaded " << nq << " queries with dimension " << dim << std::endl;
        const std::size_t chunk =
            std::min({opt.size("query-chunk", nq), nq, coraanns::max_query_chunk});
        if (chunk == 0)
            throw std::invalid_argument("query-chunk must be positive");

        std::cout << "Initializing GPU Index..." << std::endl;
        // header first (shape checks before the payload is read), then one streaming pass
        const coraanns::index::IvfHeader ivf = coraanns::index::IvfReader(argv[1]).header();
        const int metric = ivf.metric;
        if (topk == 0 || rounds == 0 || nq == 0 || gt.rows() != nq || dim != ivf.dim || gt.cols() < topk)
            throw std::invalid_argument("query/ground-truth/index shapes do not match");
        std::unique_ptr<Matrix> base_map;
        coraanns::benchmark::MatrixView base_view;
        if (!recall_base.empty()) {
            base_map = std::make_unique<Matrix>(recall_base);
            base_view = view_of(*base_map);
        }
        const std::vector<uint32_t> gt_ids = gt.dense<uint32_t>();
        using Evaluator = coraanns::benchmark::RecallEvaluator;
        auto make_evaluator = [&] {
            auto e = std::make_unique<Evaluator>(query.data(), nq, dim, gt_ids.data(), gt.rows(), gt.cols(), topk,
                                                 base_map ? &base_view : nullptr, metric);
            std::cout << "[Recall] mode=" << (base_map ? "distance-aware" : "id")
                      << " metric=" << (metric == 0 ? "l2" : "ip") << " topk=" << topk << "\n";
            return e;
        };
        std::unique_ptr<Evaluator> evaluator;
        if (!recall_once)
            evaluator = make_evaluator();
        std::unique_ptr<Matrix> exact;
        if (!exact_file.empty()) {
            if (metric != 0) {
                std::cerr << "Exact-refine diagnostic currently supports only L2 indexes.\n";
                return 1;
            }
            exact = std::make_unique<Matrix>(exact_file);
            if (exact->rows() != ivf.num || exact->cols() != ivf.dim) {
                std::cerr << "Exact-refine base shape mismatch\n";
                return 1;
            }
        }
        const auto nprobes = parse_nprobes(opt.get("nprobes", ""), ivf.nlist);
        const std::size_t max_nprobe = *std::max_element(nprobes.begin(), nprobes.end());
        coraanns::validate_search_shape(chunk, topk, max_nprobe, ivf.nlist, ivf.padded_dim);
        coraanns::index::HugeVector<uint32_t> ids;
        const std::unique_ptr<coraanns::index::SearchData> packed_ptr =
            coraanns::index::SearchData::load(argv[1], !exact, static_cast<int>(threads), nullptr, &ids);
        const coraanns::index::SearchData &packed = *packed_ptr;
        if (ivf.centroid_storage == coraanns::index::CentroidStorage::HnswSidecar)
            std::cout << "Centroids: HNSW sidecar " << argv[1] << ".hnsw" << std::endl;
        coraanns::HybridIndex engine;
        engine.set_profiling(profile);
        engine.set_candidate_stats(cand_stats);
        engine.set_gpu_filter_timing(filter_timing);
        engine.set_cross_query_reuse(reuse);
        engine.set_cpu_secondary_filter(secondary);
        engine.set_vanguard_size(vanguard);
        const std::string lbs = opt.get("lower-bound-scale", "");
        if (!lbs.empty()) {
            std::size_t used = 0;
            const float v = std::stof(lbs, &used);
            if (used != lbs.size())
                throw std::invalid_argument("Invalid number for --lower-bound-scale: " + lbs);
            engine.set_lower_bound_scale(v);
        }
        engine.set_metric(metric);
        engine.load_from_raw_pointers(ivf.num, ivf.dim, ivf.padded_dim, ivf.nlist, ivf.ex_bits,
                                      packed.h_centroids.data(), packed.host_rotator.data(),
                                      packed.host_short_data.data(),
                                      packed.host_short_factors.data(), packed.host_long_codes,
                                      packed.host_ex_factors.data(), ids.data(),
                                      packed.cluster_sizes.data());
        if (exact)
            engine.enable_exact_refine(exact->mapping(), exact->rows(), exact->cols(),
                                       exact->stride(), exact->offset());
        std::cout << "Max cluster size: " << packed.max_cluster_size << std::endl;
        engine.set_queue_capacity(qcap);
        engine.set_queue_spill_capacity(scap);
        std::cout << "Allocating GPU workspace...\n";
        engine.prepare_workspace(chunk, topk, max_nprobe);
        std::cout << "Algorithm: CoraANN (GPU filtering + CPU refinement) on MI355X\n"
                  << "topk: " << topk << "\nbatch_q: " << batch_q << "\nquery_chunk: " << chunk
                  << "\ncpu_threads: " << threads << "\nqueue_capacity: " << qcap
                  << "\nqueue_spill_capacity: " << scap << "\nvanguard_size: " << vanguard
                  << "\ncpu_secondary_filter: " << (secondary ? "true" : "false")
                  << "\ncross_query_reuse: " << (reuse ? "true" : "false")
                  << "\nlower_bound_scale: " << engine.get_lower_bound_scale()
                  << "\nrounds: " << rounds << "\nwarmup_rounds: " << warmup << "\n";

        std::vector<float> dists(nq * topk);
        std::vector<uint32_t> result(nq * topk);
        struct Stats {
            uint64_t submitted = 0, refined = 0, spilled = 0, wraps = 0;
            double filter_ms = 0;
        };
        auto run = [&](std::size_t nprobe) {
            Stats s;
            for (std::size_t b = 0; b < nq; b += chunk) {
                const std::size_t n = std::min(chunk, nq - b);
                engine.reset_buffer(query.data() + b * dim, n);
                engine.search(query.data() + b * dim, n, topk, nprobe, dists.data() + b * topk,
                              result.data() + b * topk, static_cast<int>(batch_q));
                s.submitted += engine.get_last_submitted_count();
                s.refined += engine.get_last_refined_count();
                s.spilled += engine.get_last_spilled_count();
                s.filter_ms += engine.get_last_gpu_filter_ms();
                const auto sub = engine.get_last_submitted_count();
                s.wraps += sub == 0 ? 0 : (sub - 1) / qcap;
            }
            return s;
        };
        std::cout << "Starting batch benchmark..." << std::endl;
        std::vector<double> qps(nprobes.size(), 0), rec(nprobes.size(), 0);
        std::vector<std::vector<uint32_t>> saved(recall_once ? nprobes.size() : 0);
        for (std::size_t l = 0; l < nprobes.size(); ++l) {
            const std::size_t np = nprobes[l];
            for (std::size_t w = 0; w < warmup; ++w)
                run(np);
            for (std::size_t r = 0; r < rounds; ++r) {
                const auto t0 = std::chrono::steady_clock::now();
                const Stats s = run(np);
                const double us = std::chrono::duration<double, std::micro>(
                                      std::chrono::steady_clock::now() - t0).count();
                const double v = nq / (us / 1e6);
                qps[l] += v / rounds;
                // recall first (its [RecallEval] line precedes the [Run] line, as in the
                // reference driver, apps/search.cpp:256-271)
                double rr = 0.0;
                if (recall_once) {
                    if (r == 0)
                        saved[l] = result;
                } else {
                    rr = evaluator->evaluate(result.data(), result.size());
                    rec[l] += rr / rounds;
                }
                std::cout << "[Run] round=" << (r + 1) << " nprobe=" << np << " QPS=" << v;
                if (recall_once)
                    std::cout << " recall=deferred\n";
                else
                    std::cout << " recall=" << rr << '\n';
                std::cout.flush();
                std::printf("[QueueStats] round=%zu nprobe=%zu submitted=%llu spilled=%llu wraps=%llu\n",
                            r + 1, np, (unsigned long long)s.submitted, (unsigned long long)s.spilled,
                            (unsigned long long)s.wraps);
                if (cand_stats)
                    std::printf("[CandidateStats] round=%zu nprobe=%zu queries=%zu submitted=%llu "
                                "actual_refined=%llu submitted_per_query=%.6f "
                                "actual_refined_per_query=%.6f\n",
                                r + 1, np, nq, (unsigned long long)s.submitted,
                                (unsigned long long)s.refined, double(s.submitted) / nq,
                                double(s.refined) / nq);
                if (filter_timing)
                    std::printf("[GPUFilter] round=%zu nprobe=%zu queries=%zu total_ms=%.6f "
                                "ms_per_query=%.9f\n",
                                r + 1, np, nq, s.filter_ms, s.filter_ms / nq);
            }
        }
        if (recall_once) {
            evaluator = make_evaluator();
            for (std::size_t l = 0; l < nprobes.size(); ++l) {
                rec[l] = evaluator->evaluate(saved[l].data(), saved[l].size());
                std::cout << "[RecallPoint] nprobe=" << nprobes[l] << " source_round=1 recall="
                          << rec[l] << '\n';
            }
        }
        std::cout << "nprobe\tQPS\trecall\n";
        for (std::size_t l = 0; l < nprobes.size(); ++l)
            std::cout << nprobes[l] << '\t' << qps[l] << '\t' << rec[l] << '\n';
    } catch (const std::exception &e) {
        std::cerr << "coraanns_search failed: " << e.what() << '\n';
        print_usage(argv[0]);
        return 1;
    }
    return 0;
}
