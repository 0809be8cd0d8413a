// Reproduces the inputs of the reference's own sampling tests: std::mt19937 seeded with
// `seed`, drawn through std::normal_distribution<float>(mean, sd), exactly as
// tests/test_sampling.cpp:177-180 and :238-242 build their logit rows. The numbers come from
// libstdc++, the same library the reference's tests link against on this image.
//
// TEST INFRASTRUCTURE ONLY (see oracle.h).
#include "oracle.h"

#include <random>

extern "C" void or_gen_mt19937_normal(uint32_t seed, float mean, float sd, size_t n, float* out) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(mean, sd);
    for (size_t i = 0; i < n; ++i) out[i] = nd(rng);
}

// libstdc++'s own draws of speculator.cpp:87-89,105: std::mt19937_64(seed) through
// std::uniform_real_distribution<float>(0, 1), two per seed (out[2i], out[2i+1]).
extern "C" void or_std_rejection_uniforms(const uint64_t* seeds, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) {
        std::mt19937_64 rng(seeds[i]);
        std::uniform_real_distribution<float> udist(0.0f, 1.0f);
        out[2 * i] = udist(rng);
        out[2 * i + 1] = udist(rng);
    }
}

// The 10000th output of a default-constructed std::mt19937_64 (the standard's known answer).
extern "C" uint64_t or_std_mt64_10000th(void) {
    std::mt19937_64 rng;
    rng.discard(9999);
    return rng();
}
