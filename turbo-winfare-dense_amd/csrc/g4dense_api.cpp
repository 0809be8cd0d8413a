// The reference's C++ sampling/speculator API (include/g4dense/sampling.hpp:20-27,
// include/g4dense/speculator.hpp:24-31 in the reference checkout) implemented on the GPU.
//
// These entry points take HOST logits, as the reference's do. Each call stages the rows into
// device memory, runs the same selection kernel as the device C-ABI, and copies the result
// back, so the host-pointer API and twd_select give identical ids on identical logits. A
// caller that already holds logits in HBM should use twd_select / twd_head_* directly and skip
// the copies.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "g4dense/sampling.hpp"
#include "g4dense/speculator.hpp"
#include "twd_internal.h"

#define G4_API __attribute__((visibility("default")))

namespace {

// Device staging of the host-pointer entry points: a pool of areas, one per concurrent caller.
// A call leases an area (its selector, buffers and its own non-blocking stream), so calls from
// different threads run concurrently; an area is grown on demand and returned to the pool.
struct Staging {
    hipStream_t stream = nullptr;
    twd_selector* sel = nullptr;
    uint32_t sel_vocab = 0, sel_rows = 0;
    float* logits = nullptr;
    size_t logits_cap = 0;
    float* dlogits = nullptr;  // draft rows of evaluate_verification
    size_t dlogits_cap = 0;
    uint32_t* history = nullptr;
    size_t history_cap = 0;
    uint32_t* drafts = nullptr;
    uint32_t* tokens = nullptr;
    twd_verify_result* vres = nullptr;

    ~Staging() = default;  // released with the process, like the reference's device context
};

struct StagingPool {
    std::mutex mu;
    std::vector<Staging*> idle;  // areas are kept for the process, like the reference's device context
};

StagingPool& pool() {
    static StagingPool* p = new StagingPool();
    return *p;
}

// One staging area for the duration of a call.
class Lease {
  public:
    Lease() {
        StagingPool& p = pool();
        std::lock_guard<std::mutex> lock(p.mu);
        if (p.idle.empty()) {
            s_ = new Staging();
        } else {
            s_ = p.idle.back();
            p.idle.pop_back();
        }
    }
    ~Lease() {
        StagingPool& p = pool();
        std::lock_guard<std::mutex> lock(p.mu);
        p.idle.push_back(s_);
    }
    Lease(const Lease&) = delete;
    Lease& operator=(const Lease&) = delete;
    Staging& operator*() const { return *s_; }

  private:
    Staging* s_;
};

[[noreturn]] void throw_last(const char* what) {
    throw g4dense::G4DenseFormatError(std::string(what) + ": " + twd_last_error());
}

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw g4dense::G4DenseFormatError(std::string(what) + ": " + hipGetErrorString(e));
}

void ensure(Staging& s, uint32_t vocab, uint32_t rows, size_t history_len) {
    if (!s.stream) check_hip(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), "hipStreamCreate");
    if (!s.sel || s.sel_vocab < vocab || s.sel_rows < rows) {
        if (s.sel) twd_selector_destroy(s.sel);
        s.sel = nullptr;
        const uint32_t v = std::max(vocab, s.sel_vocab);
        const uint32_t r = std::max<uint32_t>(std::max(rows, s.sel_rows), 8);
        if (twd_selector_create(v, r, &s.sel) != TWD_OK) throw_last("twd_selector_create");
        s.sel_vocab = v;
        s.sel_rows = r;
    }
    const size_t need = static_cast<size_t>(vocab) * rows;
    if (s.logits_cap < need) {
        if (s.logits) check_hip(hipFree(s.logits), "hipFree");
        s.logits = nullptr;
        check_hip(hipMalloc(&s.logits, need * sizeof(float)), "hipMalloc logits");
        s.logits_cap = need;
    }
    if (s.history_cap < history_len) {
        if (s.history) check_hip(hipFree(s.history), "hipFree");
        s.history = nullptr;
        check_hip(hipMalloc(&s.history, history_len * sizeof(uint32_t)), "hipMalloc history");
        s.history_cap = history_len;
    }
    if (!s.tokens) {
        check_hip(hipMalloc(&s.tokens, (TWD_MAX_ROWS + 1) * sizeof(uint32_t)), "hipMalloc tokens");
        check_hip(hipMalloc(&s.drafts, (TWD_MAX_ROWS + 1) * sizeof(uint32_t)), "hipMalloc drafts");
        check_hip(hipMalloc(&s.vres, sizeof(twd_verify_result)), "hipMalloc verify result");
    }
}

void upload(Staging& s, void* dst, const void* src, size_t bytes, const char* what) {
    check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s.stream), what);
}

// waits for everything enqueued on the area's stream, then copies back
void download(Staging& s, void* dst, const void* src, size_t bytes, const char* what) {
    check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s.stream), what);
    check_hip(hipStreamSynchronize(s.stream), what);
}

twd_row_params row_params(const g4dense::SamplingParams& p, float uniform) {
    twd_row_params r{};
    r.temperature = p.temperature;
    r.top_p = p.top_p;
    r.top_k = p.top_k;
    r.repetition_penalty = 1.0f;  // sample_token itself never penalises
    r.uniform = uniform;
    r.softcap = 0.0f;
    r.history_offset = 0;
    r.history_len = 0;
    return r;
}

}  // namespace

namespace g4dense {

G4_API void validate_sampling(const SamplingParams& p) {
    if (twd_validate_sampling(p.temperature, p.top_p, p.top_k, p.repetition_penalty) != TWD_OK)
        throw G4DenseFormatError(twd_last_error());
}

G4_API uint64_t splitmix64(uint64_t x) { return twd_splitmix64(x); }

G4_API uint64_t seed_for(const SamplingParams& p, int position) {
    return twd_seed_for(p.has_seed ? 1 : 0, p.seed, position);
}

G4_API void apply_repetition_penalty(float* logits, uint32_t vocab,
                                     const std::vector<uint32_t>& history, float penalty,
                                     float softcap) {
    if (penalty == 1.0f || history.empty() || vocab == 0) return;
    Lease lease;
    Staging& s = *lease;
    ensure(s, vocab, 1, history.size());
    upload(s, s.logits, logits, vocab * sizeof(float), "upload");
    upload(s, s.history, history.data(), history.size() * sizeof(uint32_t), "upload history");
    twd_row_params r{};
    r.temperature = 0.0f;
    r.top_p = 1.0f;
    r.repetition_penalty = penalty;
    r.softcap = softcap;
    r.history_len = static_cast<uint32_t>(history.size());
    if (twd::launch_select(s.sel->scratch, s.logits, vocab, 1, vocab, &r, s.history, nullptr,
                           s.stream, /*penalty_only=*/true) != TWD_OK)
        throw_last("apply_repetition_penalty");
    download(s, logits, s.logits, vocab * sizeof(float), "download");
}

G4_API uint32_t sample_token(const float* logits, uint32_t vocab, const SamplingParams& p,
                             uint64_t seed) {
    if (vocab == 0) throw G4DenseFormatError("sample_token: empty vocabulary");
    Lease lease;
    Staging& s = *lease;
    ensure(s, vocab, 1, 0);
    upload(s, s.logits, logits, vocab * sizeof(float), "upload");
    const twd_row_params r = row_params(p, twd_uniform_from_seed(seed));
    if (twd_select(s.sel, s.logits, vocab, 1, vocab, &r, nullptr, s.tokens, s.stream) != TWD_OK)
        throw_last("sample_token");
    uint32_t tok = 0;
    download(s, &tok, s.tokens, sizeof(uint32_t), "download");
    if (tok == TWD_TOKEN_DEGENERATE)
        throw G4DenseFormatError("sample_token: logit distribution is degenerate");
    return tok;
}

// evaluate_verification (speculator.cpp:34-153) has no bound on the number of drafts; the
// device entry points take at most TWD_MAX_ROWS per call. Longer drafts are verified in batches
// of TWD_MAX_ROWS positions in order: a batch whose drafts are all accepted hands over to the
// next, whose positions keep their global index in the seeds (base_seed + i, speculator.cpp:56,
// 88) by passing base_seed + batch start. Only the last batch may add the bonus row.
G4_API SpeculativeEvaluation SpeculativeCoordinator::evaluate_verification(
    const std::vector<uint32_t>& draft_tokens, const std::vector<const float*>& target_logits_per_pos,
    uint32_t vocab_size, const SamplingParams& sampling, uint64_t base_seed,
    const std::vector<std::vector<float>>& draft_logits) {
    SpeculativeEvaluation eval{};
    eval.total_drafted = static_cast<uint32_t>(draft_tokens.size());
    total_draft_tokens_ += eval.total_drafted;
    if (draft_tokens.empty() || target_logits_per_pos.empty()) return eval;
    const size_t k = std::min(draft_tokens.size(), target_logits_per_pos.size());
    const size_t rows_all = std::min(target_logits_per_pos.size(), k + 1);
    if (!sampling.is_greedy()) {
        for (size_t i = 0; i < k && i < draft_logits.size(); ++i)
            if (!draft_logits[i].empty() && draft_logits[i].size() < vocab_size)
                throw G4DenseFormatError("evaluate_verification: a draft logit row is shorter than vocab_size");
    }

    Lease lease;
    Staging& s = *lease;
    for (size_t b0 = 0; b0 < k; b0 += TWD_MAX_ROWS) {
        const uint32_t kb = static_cast<uint32_t>(std::min<size_t>(TWD_MAX_ROWS, k - b0));
        const bool last = b0 + kb == k;
        // rows of this batch: its kb positions, plus the bonus row after the final draft
        const uint32_t rows = last ? static_cast<uint32_t>(rows_all - b0) : kb;
        // positions of this batch whose draft probabilities select the rejection branch
        // (speculator.cpp:72)
        uint32_t n_draft_rows = 0;
        if (!sampling.is_greedy()) {
            for (uint32_t i = 0; i < kb && b0 + i < draft_logits.size(); ++i)
                if (!draft_logits[b0 + i].empty()) n_draft_rows = i + 1;
        }
        ensure(s, vocab_size, rows, 0);
        for (uint32_t i = 0; i < rows; ++i)
            upload(s, s.logits + static_cast<size_t>(i) * vocab_size, target_logits_per_pos[b0 + i],
                   vocab_size * sizeof(float), "upload rows");
        upload(s, s.drafts, draft_tokens.data() + b0, kb * sizeof(uint32_t), "upload drafts");
        twd_row_params r = row_params(sampling, 0.0f);
        const uint64_t seed = base_seed + b0;
        if (n_draft_rows == 0) {
            if (twd_verify(s.sel, s.logits, vocab_size, rows, vocab_size, &r, seed, s.drafts, kb, s.vres,
                           s.stream) != TWD_OK)
                throw_last("evaluate_verification");
        } else {
            const size_t need = static_cast<size_t>(n_draft_rows) * vocab_size;
            if (s.dlogits_cap < need) {
                check_hip(hipStreamSynchronize(s.stream), "hipStreamSynchronize");  // earlier batches' copies
                if (s.dlogits) check_hip(hipFree(s.dlogits), "hipFree");
                s.dlogits = nullptr;
                check_hip(hipMalloc(&s.dlogits, need * sizeof(float)), "hipMalloc draft rows");
                s.dlogits_cap = need;
            }
            const float* dptr[TWD_MAX_ROWS] = {};
            for (uint32_t i = 0; i < n_draft_rows; ++i) {
                if (draft_logits[b0 + i].empty()) continue;
                float* dst = s.dlogits + static_cast<size_t>(i) * vocab_size;
                upload(s, dst, draft_logits[b0 + i].data(), vocab_size * sizeof(float), "upload draft rows");
                dptr[i] = dst;
            }
            r.repetition_penalty = sampling.repetition_penalty;  // is_greedy() needs it
            if (twd_verify_draft(s.sel, s.logits, vocab_size, rows, vocab_size, dptr, n_draft_rows, &r, seed,
                                 s.drafts, kb, s.vres, s.stream) != TWD_OK)
                throw_last("evaluate_verification");
        }
        twd_verify_result v{};
        download(s, &v, s.vres, sizeof(v), "download result");
        if (v.n_tokens == TWD_TOKEN_DEGENERATE)
            throw G4DenseFormatError("sample_token: logit distribution is degenerate");
        eval.accepted_tokens.insert(eval.accepted_tokens.end(), v.tokens, v.tokens + v.n_tokens);
        eval.num_accepted += v.num_accepted;
        eval.bonus_token_sampled = v.bonus_token_sampled != 0;
        eval.bonus_token = v.bonus_token;
        if (v.num_accepted < kb) break;  // a correction ended the verification
    }
    total_accepted_tokens_ += eval.num_accepted;
    eval.acceptance_rate =
        eval.total_drafted == 0 ? 0.0 : static_cast<double>(eval.num_accepted) / eval.total_drafted;
    return eval;
}

}  // namespace g4dense
