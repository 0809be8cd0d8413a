// Drop-in declarations of the reference's sampling API (include/g4dense/sampling.hpp:9-27 in the
// reference checkout): same namespace, types, names and signatures, so callers compile and
// link against libtwd_head.so unchanged. The implementations run on the GPU
// (turbo-winfare-dense_amd/csrc/g4dense_api.cpp).
#pragma once

#if __has_include("g4dense/format.hpp")
#include "g4dense/format.hpp"  // the caller's tree provides G4DenseFormatError
#else
#include <stdexcept>
#include <string>
namespace g4dense {
// Thrown for rejected parameters and degenerate distributions (format.hpp:249-253).
class G4DenseFormatError : public std::runtime_error {
public:
    explicit G4DenseFormatError(const std::string& message) : std::runtime_error(message) {}
};
}  // namespace g4dense
#endif

#include <cstdint>
#include <vector>

namespace g4dense {

struct SamplingParams {
    float temperature{0.0f};         // 0 = greedy
    float top_p{1.0f};               // 1 = no nucleus truncation
    int top_k{0};                    // 0 = no top-k truncation
    float repetition_penalty{1.0f};  // 1 = disabled
    bool has_seed{false};
    uint64_t seed{0};

    bool is_greedy() const { return temperature <= 0.0f && repetition_penalty == 1.0f; }
};

void validate_sampling(const SamplingParams& p);
uint64_t splitmix64(uint64_t x);
uint64_t seed_for(const SamplingParams& p, int position);
void apply_repetition_penalty(float* logits, uint32_t vocab, const std::vector<uint32_t>& history,
                              float penalty, float softcap);
uint32_t sample_token(const float* logits, uint32_t vocab, const SamplingParams& p, uint64_t seed);

}  // namespace g4dense
