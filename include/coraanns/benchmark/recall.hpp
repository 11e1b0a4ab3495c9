// Recall@k evaluation for the search driver, outside the timed region.
//
// Semantics of the reference evaluator (include/coraanns/benchmark/recall.hpp:74-275):
//   * ID mode: a result counts when its id is in the query's ground-truth top-k.
//   * Distance-aware mode (a base matrix is given): a result outside the ground-truth ids
//     still counts when its exact FP64 distance is within the k-th ground-truth
//     distance (<= for L2, >= for inner product), with no epsilon; NaN and infinity
//     never count.
//   * Only the first topk results are examined; missing results stay in the
//     denominator; negative ids, ids >= 2^32 - 1 and ids past the base matrix are
//     misses; a repeated id counts once.
//   * The constructor rejects a ground truth with fewer than topk columns, a wrong row
//     count, an invalid id (2^32 - 1, or past the base), duplicate ids in a top-k, or a
//     non-finite k-th distance.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <type_traits>
#include <vector>

namespace coraanns::benchmark {

// Read-only view of a row-major FP32 matrix inside a mapping (an .fbin or .fvecs file).
struct MatrixView {
    const std::uint8_t *data = nullptr;  // start of the mapping
    std::size_t offset = 0;              // bytes before row 0
    std::size_t stride = 0;              // bytes between rows
    std::size_t rows = 0, cols = 0;
    const float *row(std::size_t i) const {
        return reinterpret_cast<const float *>(data + offset + i * stride);
    }
};

struct RecallCounts {
    std::size_t total = 0;          // topk per evaluated query
    std::size_t id_hits = 0;        // results whose id is a ground-truth id
    std::size_t distance_hits = 0;  // further results within the k-th ground-truth distance
    std::size_t exact_checks = 0;   // exact distances computed
    std::size_t correct() const { return id_hits + distance_hits; }
    RecallCounts &operator+=(const RecallCounts &o) {
        total += o.total;
        id_hits += o.id_hits;
        distance_hits += o.distance_hits;
        exact_checks += o.exact_checks;
        return *this;
    }
};

class RecallEvaluator {
  public:
    // queries: [nq x dim] FP32, gt: [nq x gt_cols] u32 ids; both must outlive the
    // evaluator. base: nullptr for ID recall. metric: 0 = L2, 1 = inner product.
    RecallEvaluator(const float *queries, std::size_t nq, std::size_t dim, const std::uint32_t *gt,
                    std::size_t gt_rows, std::size_t gt_cols, std::size_t topk, const MatrixView *base,
                    int metric)
        : q_(queries), nq_(nq), dim_(dim), k_(topk), base_(base), metric_(metric) {
        if (!queries || !gt || nq == 0 || dim == 0 || topk == 0 || gt_rows != nq || gt_cols < topk)
            throw std::invalid_argument("Invalid query/GT shape for recall@k");
        if (metric != 0 && metric != 1)
            throw std::invalid_argument("Recall evaluation supports only L2 and IP");
        if (base && base->cols != dim)
            throw std::invalid_argument("Recall base and query dimensions differ");
        truth_.resize(nq * topk);
        radius_.assign(nq, 0.0);
        for (std::size_t i = 0; i < nq; ++i) {
            const std::uint32_t *g = gt + i * gt_cols;
            for (std::size_t k = 0; k < topk; ++k)
                if (g[k] == std::numeric_limits<std::uint32_t>::max() || (base && g[k] >= base->rows))
                    throw std::invalid_argument("Invalid GT ID for recall base");
            if (base) {
                radius_[i] = score(i, g[topk - 1]);  // rank k of the ground truth, not its largest id
                if (!finite(radius_[i]))
                    throw std::invalid_argument("Non-finite query/GT distance");
            }
            std::uint32_t *t = truth_.data() + i * topk;
            std::copy(g, g + topk, t);
            std::sort(t, t + topk);
            if (std::adjacent_find(t, t + topk) != t + topk)
                throw std::invalid_argument("GT top-k contains duplicate IDs");
        }
    }

    bool distance_aware() const { return base_ != nullptr; }

    template <class Id>
    RecallCounts count_query(std::size_t q, const Id *results, std::size_t count) const {
        static_assert(std::is_integral_v<Id>, "result ids must be integers");
        if (q >= nq_)
            throw std::out_of_range("Recall query is out of range");
        RecallCounts c;
        c.total = k_;
        std::vector<std::uint32_t> ids;
        ids.reserve(std::min(count, k_));
        for (std::size_t i = 0; i < std::min(count, k_); ++i) {
            if constexpr (std::is_signed_v<Id>) {
                if (results[i] < 0)
                    continue;
            }
            const auto wide = static_cast<std::uint64_t>(results[i]);
            if (wide >= std::numeric_limits<std::uint32_t>::max() || (base_ && wide >= base_->rows))
                continue;
            ids.push_back(static_cast<std::uint32_t>(wide));
        }
        std::sort(ids.begin(), ids.end());
        ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
        const std::uint32_t *t = truth_.data() + q * k_;
        for (std::uint32_t id : ids) {
            if (std::binary_search(t, t + k_, id)) {
                ++c.id_hits;
            } else if (base_) {
                const double s = score(q, id);
                ++c.exact_checks;
                if (finite(s) && (metric_ == 0 ? s <= radius_[q] : s >= radius_[q]))
                    ++c.distance_hits;
            }
        }
        return c;
    }

    // Recall over all queries of `results` ([nq x topk]); prints the [RecallEval] line.
    template <class Id>
    double evaluate(const Id *results, std::size_t n_results, bool print = true) const {
        if (n_results < nq_ * k_)
            throw std::invalid_argument("Result array is smaller than nq * topk");
        RecallCounts total;
        std::vector<RecallCounts> per(nq_);
#pragma omp parallel for schedule(static) if (base_ && nq_ >= 128)
        for (std::size_t q = 0; q < nq_; ++q)
            per[q] = count_query(q, results + q * k_, k_);
        for (const auto &c : per)
            total += c;
        const double denom = static_cast<double>(total.total);
        if (print)
            std::printf("[RecallEval] id_recall=%g recall=%g distance_hits=%zu exact_checks=%zu\n",
                        total.id_hits / denom, total.correct() / denom, total.distance_hits,
                        total.exact_checks);
        return total.correct() / denom;
    }

  private:
    // exponent test instead of std::isfinite: stays a real test under -Ofast
    static bool finite(double v) {
        std::uint64_t b;
        std::memcpy(&b, &v, sizeof(b));
        return (b & 0x7ff0000000000000ull) != 0x7ff0000000000000ull;
    }
    double score(std::size_t q, std::uint32_t id) const {
        const float *a = q_ + q * dim_;
        const float *x = base_->row(id);
        double s = 0.0;
        if (metric_ == 0) {
            for (std::size_t d = 0; d < dim_; ++d) {
                const double diff = static_cast<double>(a[d]) - x[d];
                s += diff * diff;
            }
        } else {
            for (std::size_t d = 0; d < dim_; ++d)
                s += static_cast<double>(a[d]) * x[d];
        }
        return s;
    }

    const float *q_;
    std::size_t nq_, dim_, k_;
    const MatrixView *base_;
    int metric_;
    std::vector<std::uint32_t> truth_;
    std::vector<double> radius_;
};

}  // namespace coraanns::benchmark
