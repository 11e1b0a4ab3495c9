// HugePageAllocator (include/coraanns/index/search_data.hpp): blocks of 4 MB and more are
// 2 MB aligned and hold their values through vector growth, copies and moves; small blocks
// come from operator new; a huge-page vector behaves as a std::vector.
#include <cstdint>
#include <cstdio>
#include <numeric>
#include <vector>

#include "coraanns/index/search_data.hpp"

using coraanns::index::HugeVector;

static int failures = 0;
#define CHECK(c)                                                   \
    do {                                                           \
        if (!(c)) {                                                \
            std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); \
            ++failures;                                            \
        }                                                          \
    } while (0)

int main() {
    const std::size_t huge = std::size_t{2} << 20;
    // large: aligned, zero-filled by resize, values kept
    HugeVector<uint32_t> a;
    a.resize(3u << 20);  // 12 MB
    CHECK(reinterpret_cast<std::uintptr_t>(a.data()) % huge == 0);
    CHECK(a[0] == 0 && a[a.size() - 1] == 0);
    std::iota(a.begin(), a.end(), 7u);
    CHECK(a[12345] == 12352u);
    // growth reallocates and keeps the values
    a.resize(5u << 20);
    CHECK(reinterpret_cast<std::uintptr_t>(a.data()) % huge == 0);
    CHECK(a[(3u << 20) - 1] == (3u << 20) + 6u && a[(5u << 20) - 1] == 0);
    // copy and move
    HugeVector<uint32_t> b = a;
    CHECK(b == a);
    HugeVector<uint32_t> c = std::move(b);
    CHECK(c.size() == a.size() && c[99] == 106u);
    // assign (the ex-factor arrays' use) and small blocks
    HugeVector<float> f;
    f.assign(2u << 20, 1.5f);  // 8 MB
    CHECK(reinterpret_cast<std::uintptr_t>(f.data()) % huge == 0 && f[f.size() - 1] == 1.5f);
    HugeVector<uint8_t> s(100, 3);
    CHECK(s.size() == 100 && s[99] == 3);
    s.clear();
    s.shrink_to_fit();
    CHECK(s.empty());
    if (failures == 0)
        std::printf("PASS\n");
    return failures == 0 ? 0 : 1;
}
