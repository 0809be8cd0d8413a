// Drop-in declarations of the reference's speculative verifier
// (include/g4dense/speculator.hpp:10-43 in the reference checkout). evaluate_verification runs
// on the GPU (turbo-winfare-dense_amd/csrc/g4dense_api.cpp).
#pragma once

#include <cstdint>
#include <vector>

#include "g4dense/sampling.hpp"

namespace g4dense {

struct SpeculativeEvaluation {
    std::vector<uint32_t> accepted_tokens;  // N accepted + 1 bonus token
    uint32_t num_accepted{0};
    uint32_t total_drafted{0};
    bool bonus_token_sampled{false};
    uint32_t bonus_token{0};
    double acceptance_rate{0.0};
};

class SpeculativeCoordinator {
public:
    SpeculativeCoordinator() = default;

    // Evaluates K draft tokens against K (+1 bonus) rows of target logits.
    SpeculativeEvaluation evaluate_verification(
        const std::vector<uint32_t>& draft_tokens,
        const std::vector<const float*>& target_logits_per_pos, uint32_t vocab_size,
        const SamplingParams& sampling, uint64_t base_seed,
        const std::vector<std::vector<float>>& draft_logits = {});

    uint64_t total_draft_tokens() const { return total_draft_tokens_; }
    uint64_t total_accepted_tokens() const { return total_accepted_tokens_; }
    double cumulative_acceptance_rate() const {
        return total_draft_tokens_ == 0 ? 0.0
                                        : (double)total_accepted_tokens_ / total_draft_tokens_;
    }

private:
    uint64_t total_draft_tokens_{0};
    uint64_t total_accepted_tokens_{0};
};

}  // namespace g4dense
