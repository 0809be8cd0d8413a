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
