// C entry points over the REFERENCE's own sampling.cpp and speculator.cpp, compiled from
// /root/reference by this directory's Makefile (target `ref`) into oracle/_ref/libref.so.
// Used only by tests/ and tests/golden/make_golden.py to pin the C restatement in oracle.c
// against the real reference code, and optionally as bench.py's CPU baseline.
//
// TEST INFRASTRUCTURE ONLY. Every function returns 0 on success and a nonzero code when the
// reference threw (the message is copied into `err` when it is given).
#include "g4dense/format.hpp"
#include "g4dense/sampling.hpp"
#include "g4dense/speculator.hpp"

#include <cstring>
#include <exception>
#include <vector>

using namespace g4dense;

namespace {
SamplingParams make_params(float t, float p, int k, float rp, int has_seed, uint64_t seed) {
    SamplingParams sp;
    sp.temperature = t;
    sp.top_p = p;
    sp.top_k = k;
    sp.repetition_penalty = rp;
    sp.has_seed = has_seed != 0;
    sp.seed = seed;
    return sp;
}

void copy_err(const std::exception& e, char* err, size_t err_len) {
    if (err && err_len) {
        std::strncpy(err, e.what(), err_len - 1);
        err[err_len - 1] = '\0';
    }
}
}  // namespace

extern "C" {

uint64_t ref_splitmix64(uint64_t x) { return splitmix64(x); }

uint64_t ref_seed_for(float t, float p, int k, float rp, int has_seed, uint64_t seed, int pos) {
    return seed_for(make_params(t, p, k, rp, has_seed, seed), pos);
}

int ref_validate_sampling(float t, float p, int k, float rp, char* err, size_t err_len) {
    try {
        validate_sampling(make_params(t, p, k, rp, 0, 0));
        return 0;
    } catch (const std::exception& e) {
        copy_err(e, err, err_len);
        return 3;
    }
}

void ref_apply_repetition_penalty(float* logits, uint32_t vocab, const uint32_t* hist,
                                  size_t n, float penalty, float softcap) {
    std::vector<uint32_t> h(hist, hist + n);
    apply_repetition_penalty(logits, vocab, h, penalty, softcap);
}

int ref_sample_token(const float* logits, uint32_t vocab, float t, float p, int k, float rp,
                     uint64_t seed, uint32_t* out, char* err, size_t err_len) {
    try {
        *out = sample_token(logits, vocab, make_params(t, p, k, rp, 0, 0), seed);
        return 0;
    } catch (const std::exception& e) {
        copy_err(e, err, err_len);
        return 2;
    }
}

// evaluate_verification without draft logits. tokens_out must hold n_drafts + 1 entries;
// info_out receives {n_tokens, num_accepted, total_drafted, bonus_sampled, bonus_token}.
int ref_evaluate_verification(const uint32_t* drafts, size_t n_drafts, const float* const* rows,
                              size_t n_rows, uint32_t vocab, float t, float p, int k, float rp,
                              uint64_t base_seed, uint32_t* tokens_out, uint32_t* info_out,
                              double* rate_out, char* err, size_t err_len) {
    try {
        SpeculativeCoordinator sc;
        std::vector<uint32_t> d(drafts, drafts + n_drafts);
        std::vector<const float*> r(rows, rows + n_rows);
        SpeculativeEvaluation ev =
            sc.evaluate_verification(d, r, vocab, make_params(t, p, k, rp, 0, 0), base_seed);
        for (size_t i = 0; i < ev.accepted_tokens.size(); ++i) tokens_out[i] = ev.accepted_tokens[i];
        info_out[0] = static_cast<uint32_t>(ev.accepted_tokens.size());
        info_out[1] = ev.num_accepted;
        info_out[2] = ev.total_drafted;
        info_out[3] = ev.bonus_token_sampled ? 1u : 0u;
        info_out[4] = ev.bonus_token;
        *rate_out = ev.acceptance_rate;
        return 0;
    } catch (const std::exception& e) {
        copy_err(e, err, err_len);
        return 2;
    }
}

// validate_header (src/format.cpp:6-65) on a 4096-byte header image; 0 when accepted.
int ref_validate_header(const void* header, uint64_t file_size, char* err, size_t err_len) {
    try {
        G4DenseHeader h;
        std::memcpy(&h, header, sizeof(h));
        validate_header(h, file_size);
        return 0;
    } catch (const std::exception& e) {
        copy_err(e, err, err_len);
        return 4;
    }
}

// evaluate_verification with draft logits: draft_rows[i] (i < n_draft_rows) is position i's
// draft row, or NULL for an empty vector. Outputs as ref_evaluate_verification.
int ref_evaluate_verification_draft(const uint32_t* drafts, size_t n_drafts,
                                    const float* const* rows, size_t n_rows,
                                    const float* const* draft_rows, size_t n_draft_rows,
                                    uint32_t vocab, float t, float p, int k, float rp,
                                    uint64_t base_seed, uint32_t* tokens_out, uint32_t* info_out,
                                    double* rate_out, char* err, size_t err_len) {
    try {
        SpeculativeCoordinator sc;
        std::vector<uint32_t> d(drafts, drafts + n_drafts);
        std::vector<const float*> r(rows, rows + n_rows);
        std::vector<std::vector<float>> dl(n_draft_rows);
        for (size_t i = 0; i < n_draft_rows; ++i)
            if (draft_rows[i]) dl[i].assign(draft_rows[i], draft_rows[i] + vocab);
        SpeculativeEvaluation ev =
            sc.evaluate_verification(d, r, vocab, make_params(t, p, k, rp, 0, 0), base_seed, dl);
        for (size_t i = 0; i < ev.accepted_tokens.size(); ++i) tokens_out[i] = ev.accepted_tokens[i];
        info_out[0] = static_cast<uint32_t>(ev.accepted_tokens.size());
        info_out[1] = ev.num_accepted;
        info_out[2] = ev.total_drafted;
        info_out[3] = ev.bonus_token_sampled ? 1u : 0u;
        info_out[4] = ev.bonus_token;
        *rate_out = ev.acceptance_rate;
        return 0;
    } catch (const std::exception& e) {
        copy_err(e, err, err_len);
        return 2;
    }
}

}  // extern "C"
