// Seeded synthetic Gaussian-mixture rows for the large benchmark configurations.
//
// Every value is a pure function of (seed, row, column): a counter hashed with the
// SplitMix64 finaliser gives the uniforms, Box-Muller turns pairs of them into normals, and
// the row's mixture label comes from its own counter. The output is therefore the same for
// any thread count, and rows are generated in parallel without a shared generator.
#include <omp.h>

#include <cmath>
#include <cstdint>

#include "cora_host.h"

namespace {

inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// uniform in (0, 1], 53 bits
inline double unit(uint64_t h) { return (static_cast<double>(h >> 11) + 1.0) * 0x1.0p-53; }

inline uint64_t counter(uint64_t seed, uint64_t stream, uint64_t i) {
    return mix64(mix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) ^ i);
}

}  // namespace

extern "C" int cora_gaussian_mixture(const float *centers, uint64_t n_centers, uint64_t dim,
                                     const float *sd, uint64_t n, uint64_t seed, int normalize,
                                     int threads, float *out, uint32_t *labels) {
    if (!centers || !sd || !out || !n_centers || !dim || dim % 2)
        return CORA_ERR_INVALID_ARGUMENT;
    const int nt = threads > 0 ? threads : omp_get_max_threads();
    constexpr double kTwoPi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static, 256) num_threads(nt)
    for (long long r = 0; r < static_cast<long long>(n); ++r) {
        const uint64_t row = static_cast<uint64_t>(r);
        const uint64_t lab = counter(seed, 1, row) % n_centers;
        if (labels)
            labels[row] = static_cast<uint32_t>(lab);
        const float *c = centers + lab * dim;
        float *x = out + row * dim;
        double ss = 0.0;
        for (uint64_t j = 0; j < dim; j += 2) {
            const uint64_t k = (row * dim + j) >> 1;
            const double rad = std::sqrt(-2.0 * std::log(unit(counter(seed, 2, k))));
            const double ang = kTwoPi * unit(counter(seed, 3, k));
            const float a = static_cast<float>(c[j] + sd[j] * rad * std::cos(ang));
            const float b = static_cast<float>(c[j + 1] + sd[j + 1] * rad * std::sin(ang));
            x[j] = a;
            x[j + 1] = b;
            ss += static_cast<double>(a) * a + static_cast<double>(b) * b;
        }
        if (normalize && ss > 0.0) {
            const float inv = static_cast<float>(1.0 / std::sqrt(ss));
            for (uint64_t j = 0; j < dim; ++j)
                x[j] *= inv;
        }
    }
    return CORA_OK;
}
