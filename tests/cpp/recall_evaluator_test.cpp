// RecallEvaluator cases: the behaviour the reference pins for its evaluator in
// tests/recall_evaluator_test.cpp:89-117 (id and distance-aware hits, equal-distance
// non-GT vectors, no epsilon at the radius, duplicate result ids, missing results,
// only the first topk examined, negative / >= 2^32-1 / past-the-base ids, NaN and
// infinite rows, the radius taken from the k-th ground-truth rank rather than the largest
// id, an exact-zero radius, the inner-product direction), plus the constructor's
// rejections. Fixtures are this test's own.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <limits>
#include <stdexcept>
#include <vector>

#include "coraanns/benchmark/recall.hpp"

using coraanns::benchmark::MatrixView;
using coraanns::benchmark::RecallEvaluator;

#define CHECK(c, m)                                \
    do {                                           \
        if (!(c)) {                                \
            std::fprintf(stderr, "FAIL: %s\n", m); \
            return 1;                              \
        }                                          \
    } while (0)

template <class F>
bool throws(F &&f) {
    try {
        f();
    } catch (const std::exception &) {
        return true;
    }
    return false;
}

int main() {
    const float nan = std::numeric_limits<float>::quiet_NaN();
    const float inf = std::numeric_limits<float>::infinity();
    // base rows (dim 2) and their squared distance to q0 = (0, 0)
    std::vector<float> base = {
        0, 0,         // 0: 0
        1, 0,         // 1: 1
        0, 1,         // 2: 1
        1, 0,         // 3: 1 (same coordinates as row 1, a distinct id)
        0, -1,        // 4: 1
        3, 0,         // 5: 9
        1.0001f, 0,   // 6: just outside a radius of 1
        -1, 0,        // 7: 1
        nan, 0,       // 8: NaN
        inf, 0,       // 9: infinity
        0, 1e-3f,     // 10: 1e-6
        2, 1.5f,      // 11: 2.25 from q1 = (2, 0)
        0, 0,         // 12: same coordinates as row 0
    };
    MatrixView bv;
    bv.data = reinterpret_cast<const std::uint8_t *>(base.data());
    bv.offset = 0;
    bv.stride = 2 * sizeof(float);
    bv.rows = base.size() / 2;
    bv.cols = 2;

    const std::vector<float> q = {0, 0, 2, 0};
    // q1's rank-3 ground-truth id is 0 (distance 4); its largest id, 5, lies at distance 1
    const std::vector<std::uint32_t> gt = {0, 1, 2, 5, 1, 0};
    RecallEvaluator ev(q.data(), 2, 2, gt.data(), 2, 3, 3, &bv, 0);
    auto count = [&](std::size_t qi, std::vector<long long> ids) {
        return ev.count_query(qi, ids.data(), ids.size());
    };
    auto c = count(0, {0, 1, 2});
    CHECK(c.id_hits == 3 && c.exact_checks == 0, "all ground-truth ids are id hits without distances");
    c = count(0, {7, 3, 4});
    CHECK(c.id_hits == 0 && c.distance_hits == 3 && c.exact_checks == 3,
          "non-GT vectors at the k-th distance are distance hits");
    c = count(0, {0, 3, 5});
    CHECK(c.id_hits == 1 && c.distance_hits == 1, "one id hit, one distance hit, one miss");
    CHECK(count(0, {6}).correct() == 0, "no epsilon at the radius");
    c = count(0, {0, 0, 3});
    CHECK(c.id_hits == 1 && c.distance_hits == 1 && c.total == 3, "a repeated id counts once");
    CHECK(count(0, {0, 1}).correct() == 2 && count(0, {0, 1}).total == 3,
          "missing results stay in the denominator");
    CHECK(count(0, {0, 1, 5, 2}).correct() == 2, "only the first topk results are examined");
    CHECK(count(0, {-1, 4294967295LL, 4294967297LL}).correct() == 0, "negative and >= 2^32-1 ids are misses");
    CHECK(count(0, {13}).exact_checks == 0 && count(0, {13}).correct() == 0, "ids past the base are misses");
    CHECK(count(0, {8, 9}).correct() == 0 && count(0, {8, 9}).exact_checks == 2, "NaN and infinity never count");
    CHECK(count(1, {11}).distance_hits == 1, "radius from the k-th ground-truth rank, not the largest id");
    CHECK(count(1, {4}).correct() == 0, "outside q1's radius");
    const std::vector<std::uint32_t> short_res = {0};
    CHECK(throws([&] { ev.evaluate(short_res.data(), short_res.size(), false); }),
          "result array shorter than nq * topk is rejected");
    CHECK(throws([&] { count(2, {0}); }), "query index out of range is rejected");
    const std::vector<std::uint32_t> all = {0, 1, 2, 5, 11, 4};
    CHECK(std::fabs(ev.evaluate(all.data(), all.size(), false) - 5.0 / 6.0) < 1e-12, "evaluate sums the queries");

    // ID mode ignores distances
    RecallEvaluator ids_only(q.data(), 2, 2, gt.data(), 2, 3, 3, nullptr, 0);
    const std::uint32_t pred[] = {0, 3, 4};
    c = ids_only.count_query(0, pred, 3);
    CHECK(c.correct() == 1 && c.exact_checks == 0, "id mode counts only id hits");

    // a radius of exactly zero: an identical vector counts, a near one does not
    const std::vector<float> zq = {0, 0};
    const std::vector<std::uint32_t> zgt = {0};
    RecallEvaluator zero(zq.data(), 1, 2, zgt.data(), 1, 1, 1, &bv, 0);
    const std::uint32_t same = 12, near = 10;
    CHECK(zero.count_query(0, &same, 1).correct() == 1, "identical coordinates at radius zero");
    CHECK(zero.count_query(0, &near, 1).correct() == 0, "a near vector at radius zero");

    // inner product: larger is better
    const std::vector<float> iq = {1, 0};
    const std::vector<std::uint32_t> igt = {5, 1};
    RecallEvaluator ip(iq.data(), 1, 2, igt.data(), 1, 2, 2, &bv, 1);
    const std::uint32_t ip_ids[] = {6, 4};
    c = ip.count_query(0, ip_ids, 2);
    CHECK(c.id_hits == 0 && c.distance_hits == 1, "inner product: >= the k-th score counts");

    // constructor rejections
    const std::vector<std::uint32_t> bad_max = {0, 1, 0xFFFFFFFFu};
    const std::vector<std::uint32_t> bad_past = {0, 1, 13};
    const std::vector<std::uint32_t> dup = {0, 1, 1};
    const std::vector<std::uint32_t> to_nan = {0, 1, 8};
    CHECK(throws([&] { RecallEvaluator(q.data(), 1, 2, bad_max.data(), 1, 3, 3, nullptr, 0); }),
          "2^32-1 in the ground truth is rejected");
    CHECK(throws([&] { RecallEvaluator(q.data(), 1, 2, bad_past.data(), 1, 3, 3, &bv, 0); }),
          "a ground-truth id past the base is rejected");
    CHECK(throws([&] { RecallEvaluator(q.data(), 1, 2, dup.data(), 1, 3, 3, nullptr, 0); }),
          "duplicate ground-truth ids are rejected");
    CHECK(throws([&] { RecallEvaluator(q.data(), 1, 2, to_nan.data(), 1, 3, 3, &bv, 0); }),
          "a non-finite k-th distance is rejected");
    CHECK(throws([&] { RecallEvaluator(q.data(), 2, 2, gt.data(), 2, 3, 4, nullptr, 0); }),
          "fewer ground-truth columns than topk are rejected");
    CHECK(throws([&] { RecallEvaluator(q.data(), 2, 2, gt.data(), 1, 3, 3, nullptr, 0); }),
          "a ground-truth row count different from nq is rejected");
    CHECK(throws([&] { RecallEvaluator(q.data(), 2, 2, gt.data(), 2, 3, 3, nullptr, 2); }),
          "metrics other than L2 and IP are rejected");
    MatrixView wide = bv;
    wide.cols = 3;
    CHECK(throws([&] { RecallEvaluator(q.data(), 2, 2, gt.data(), 2, 3, 3, &wide, 0); }),
          "base and query dimensions must agree");
    std::printf("PASS\n");
    return 0;
}
