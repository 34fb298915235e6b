// synthetic.cpp -- counter-based SplitMix64 streams for synthetic scenes.
#include <cmath>

#include "msplat_synth.h"

namespace {

inline uint64_t splitmix(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline double unit(uint64_t seed, uint64_t i) {
    return (double)(splitmix(seed, i) >> 11) * (1.0 / 9007199254740992.0);
}

}  // namespace

extern "C" void msplat_synth_uniform(uint64_t seed, uint64_t offset, int64_t n, double lo, double hi, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < n; ++k) out[k] = (float)(lo + (hi - lo) * unit(seed, offset + (uint64_t)k));
}

extern "C" void msplat_synth_normal(uint64_t seed, uint64_t offset, int64_t n, double mean, double std,
                                    float *out) {
    const double two_pi = 6.283185307179586476925286766559;
    const int64_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < pairs; ++j) {
        const double u1 = 1.0 - unit(seed, offset + 2 * (uint64_t)j);
        const double u2 = unit(seed, offset + 2 * (uint64_t)j + 1);
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[2 * j] = (float)(mean + std * r * std::cos(two_pi * u2));
        if (2 * j + 1 < n) out[2 * j + 1] = (float)(mean + std * r * std::sin(two_pi * u2));
    }
}
