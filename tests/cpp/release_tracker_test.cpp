// ReleaseTracker cases (the behaviour the reference pins in
// tests/ring_release_tracker_test.cpp:17-75): out-of-order completion releases only a
// contiguous prefix, a slow first consumer keeps its slots, many wraps, 64-bit
// positions, concurrent completion, invalid sizes rejected.
#include <atomic>
#include <cstdio>
#include <stdexcept>
#include <thread>
#include <vector>

#include "coraanns/queue/release_tracker.hpp"

using coraanns::queue::Progress;
using coraanns::queue::ReleaseTracker;

#define CHECK(c, m)                                   \
    do {                                              \
        if (!(c)) {                                   \
            std::fprintf(stderr, "FAIL: %s\n", m);    \
            return 1;                                 \
        }                                             \
    } while (0)

int main() {
    {
        Progress pg;
        ReleaseTracker tr(pg, 16, 4);
        tr.complete(8);
        tr.complete(4);
        CHECK(tr.released() == 0, "prefix released before chunk 0 completed");
        CHECK(!tr.readable_generation(16), "next generation readable too early");
        CHECK(tr.readable_generation(15), "current generation not readable");
        tr.complete(0);
        CHECK(tr.released() == 12, "prefix 0..12 not released");
        tr.complete(12);
        CHECK(tr.released() == 16, "full ring not released");
        for (unsigned long long base = 16; base < 100000; base += 16) {
            tr.complete(base + 4);
            tr.complete(base + 12);
            tr.complete(base + 8);
            CHECK(tr.released() == base, "stale tag of an old generation was accepted");
            tr.complete(base);
            CHECK(tr.released() == base + 16, "wrap prefix lost");
        }
    }
    {
        Progress pg;
        ReleaseTracker tr(pg, 32, 8);
        std::atomic<bool> go{false};
        std::thread slow([&] {
            while (!go.load())
                std::this_thread::yield();
            tr.complete(0);
        });
        std::vector<std::thread> fast;
        for (unsigned long long s : {8ull, 16ull, 24ull})
            fast.emplace_back([&, s] { tr.complete(s); });
        for (auto &t : fast)
            t.join();
        const bool held = tr.released() == 0;
        go.store(true);
        slow.join();
        CHECK(held, "slow consumer lost its slots");
        CHECK(tr.released() == 32, "slow completion did not release the prefix");
    }
    {
        Progress pg;
        pg.released = 1ull << 42;
        ReleaseTracker tr(pg, 8, 2);
        tr.complete((1ull << 42) + 2);
        tr.complete(1ull << 42);
        CHECK(tr.released() == (1ull << 42) + 4, "64-bit positions truncated");
    }
    {
        Progress pg;
        ReleaseTracker tr(pg, 128, 8);
        for (unsigned long long base = 0; base < 128 * 500; base += 128) {
            std::vector<std::thread> ws;
            for (int i = 0; i < 8; ++i)
                ws.emplace_back([&, i, base] {
                    tr.complete(base + (15 - i) * 8);
                    tr.complete(base + i * 8);
                });
            for (auto &w : ws)
                w.join();
            CHECK(tr.released() == base + 128, "concurrent completion lost progress");
        }
    }
    for (auto bad : {std::pair<size_t, size_t>{16, 0}, {12, 4}, {16, 3}, {4, 8}}) {
        bool threw = false;
        try {
            Progress pg;
            ReleaseTracker tr(pg, bad.first, bad.second);
        } catch (const std::invalid_argument &) {
            threw = true;
        }
        CHECK(threw, "invalid capacity/chunk accepted");
    }
    std::printf("PASS: prefix release, slow consumer, wraps, 64-bit positions, concurrency\n");
    return 0;
}
