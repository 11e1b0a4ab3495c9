// validate_search_shape accept/reject boundaries (the reference pins them in
// tests/search_parameters_test.cpp:16-25).
#include <cstdio>
#include <stdexcept>

#include "coraanns/search/parameters.hpp"

static bool rejects(std::size_t q, std::size_t k, std::size_t np, std::size_t c, std::size_t p) {
    try {
        coraanns::validate_search_shape(q, k, np, c, p);
    } catch (const std::invalid_argument &) {
        return true;
    }
    return false;
}

int main() {
    struct Case {
        std::size_t q, k, np, c, p;
        bool reject;
    } cases[] = {
        {10000, 100, 640, 65536, 128, false}, {65535, 10, 8, 8, 128, false},
        {1, 100, 65536, 65536, 128, false},   {65536, 10, 8, 8, 128, true},
        {1, 10, 65537, 65537, 128, true},     {0, 10, 8, 8, 128, true},
        {1, 0, 8, 8, 128, true},              {1, 10, 0, 8, 128, true},
        {1, 10, 9, 8, 128, true},             {65535, 10, 65536, 65536, 128, true},
        {2, 10, 1, 1, 0, true},
    };
    for (const auto &c : cases) {
        if (rejects(c.q, c.k, c.np, c.c, c.p) != c.reject) {
            std::fprintf(stderr, "FAIL: q=%zu k=%zu np=%zu c=%zu p=%zu\n", c.q, c.k, c.np, c.c, c.p);
            return 1;
        }
    }
    std::printf("PASS: search shape limits\n");
    return 0;
}
