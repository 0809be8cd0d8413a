// The decode loop around the head: what ForwardRunner::generate does with each step's logits
// (src/runner.cpp:2312-2344) -- repetition penalty over the whole history, seed_for(position),
// sample_token, append to the history, the token callback, stop on a stop id or after
// max_tokens, and the cancel flag -- with the history kept in device memory, so that a step
// moves no logits to the host. The caller runs the model and hands each step's final hidden
// state over; the generator returns the token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <vector>

#include "twd_internal.h"

struct twd_generator {
    twd_head* head = nullptr;
    uint32_t vocab = 0;
    float softcap = 0.0f;
    twd_generation_params p{};
    uint32_t* history = nullptr;  // device, capacity `cap`; each step writes its token at [len]
    uint32_t len = 0, cap = 0;
    uint32_t prompt_len = 0;
    uint32_t checked = 0;            // history[0, checked) has passed the stop rules
    uint32_t* token_host = nullptr;  // pinned
    float* logits = nullptr;         // device [vocab]
    std::vector<uint32_t> stop_ids;
    G4DenseTokenCallback on_token = nullptr;
    void* user = nullptr;
    std::atomic<bool> cancel{false};
    int reason = TWD_STOP_NONE;
};

namespace twd {
namespace {

// The step's sampling parameters: the generation's, with the draw of seed_for(position)
// (src/runner.cpp:2325-2326) and the history's penalty clamp at the head's softcap (:2321-2322).
twd_row_params step_params(const twd_generator* g) {
    twd_row_params r{};
    r.temperature = g->p.temperature;
    r.top_p = g->p.top_p;
    r.top_k = g->p.top_k;
    r.repetition_penalty = g->p.repetition_penalty;
    const int pos = static_cast<int>(g->len) - 1;
    r.uniform = twd_uniform_from_seed(twd_seed_for(g->p.has_seed, g->p.seed, pos));
    r.softcap = g->softcap;
    r.history_offset = 0;
    r.history_len = g->len;
    return r;
}

bool is_stop(const twd_generator* g, uint32_t t) {
    return std::find(g->stop_ids.begin(), g->stop_ids.end(), t) != g->stop_ids.end();
}

uint32_t emitted(const twd_generator* g) { return g->len - g->prompt_len; }

// The stop rules of runner.cpp:2327-2336 for the emitted id t at history index `at`: the id is
// already in the history (:2328), the callback sees it (:2330-2333), then a stop id ends the
// generation (:2336). A degenerate draw is sample_token's throw: the id is not a token, so the
// history ends before it. Returns TWD_E_DEGENERATE for that case.
int apply_stop_rules(twd_generator* g, uint32_t at, uint32_t t) {
    if (t == TWD_TOKEN_DEGENERATE) {
        g->len = at;
        g->checked = at;
        g->reason = TWD_STOP_DEGENERATE;
        return fail(TWD_E_DEGENERATE, "sample_token: logit distribution is degenerate");
    }
    g->checked = at + 1;
    if (g->on_token && g->on_token(g->user, static_cast<int>(at - g->prompt_len), t, "") == 0) {
        g->len = at + 1;
        g->reason = TWD_STOP_CALLBACK;
        return TWD_OK;
    }
    if (is_stop(g, t)) {
        g->len = at + 1;
        g->reason = TWD_STOP_TOKEN;
    }
    return TWD_OK;
}

// Reads history[checked, len) back (ids of steps enqueued without readback, then the current
// one) and applies the stop rules to them in order. A stop ends the history there, discarding
// the steps queued after it. *id_at (when given) receives the id read at history index `at`.
int check_emitted(twd_generator* g, hipStream_t s, uint32_t at = 0, uint32_t* id_at = nullptr) {
    const uint32_t first = g->checked, end = g->len;
    int rc = TWD_OK;
    if (first < end) {
        const uint32_t n = end - first;
        std::vector<uint32_t> many;
        uint32_t* ids = g->token_host;  // pinned, for the usual single id
        if (n > 1) {
            many.resize(n);
            ids = many.data();
        }
        TWD_HIP(hipMemcpyAsync(ids, g->history + first, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        TWD_HIP(hipStreamSynchronize(s));
        if (id_at && at >= first && at < end) *id_at = ids[at - first];
        g->reason = TWD_STOP_NONE;  // max_tokens is judged below, on the ids that survive
        for (uint32_t i = first; i < end; ++i) {
            rc = apply_stop_rules(g, i, ids[i - first]);
            if (rc != TWD_OK || g->reason != TWD_STOP_NONE) break;
        }
    }
    if (g->reason == TWD_STOP_NONE && emitted(g) >= g->p.max_tokens) g->reason = TWD_STOP_MAX_TOKENS;
    return rc;
}

// After the head pass has written the step's token at history[len] (the selection of this step
// read history[0, len) only): count it in and, when asked (or when a callback wants every id),
// bring it to the host and apply the stop rules.
int finish_step(twd_generator* g, hipStream_t s, uint32_t* token_out, int* finished) {
    const uint32_t at = g->len;
    ++g->len;
    int rc = TWD_OK;
    if (token_out || finished || g->on_token) {
        uint32_t t = 0;
        rc = check_emitted(g, s, at, &t);
        if (rc == TWD_OK && token_out && at < g->len) *token_out = t;
    } else if (emitted(g) >= g->p.max_tokens) {
        g->reason = TWD_STOP_MAX_TOKENS;
    }
    if (finished) *finished = g->reason != TWD_STOP_NONE ? 1 : 0;
    return rc;
}

// Returns 1 when the step must not run (finished or cancelled; *finished is then set).
int check_step(twd_generator* g, int* finished, int* rc) {
    *rc = TWD_OK;
    if (!g) {
        *rc = fail(TWD_E_INVALID, "null generator");
        return 1;
    }
    if (g->reason == TWD_STOP_NONE && g->cancel.load(std::memory_order_acquire)) {
        g->reason = TWD_STOP_CANCELLED;  // runner.cpp:2315: nothing is sampled
        if (finished) *finished = 1;
        return 1;
    }
    if (g->reason != TWD_STOP_NONE) {
        *rc = fail(TWD_E_INVALID, "the generation has finished");
        return 1;
    }
    if (g->len >= g->cap) {
        *rc = fail(TWD_E_INVALID, "history capacity exhausted");
        return 1;
    }
    return 0;
}

// greedy with no penalty: the head's fused argmax; otherwise logits, then penalty + draw
bool fused_greedy(const twd_generator* g) {
    return g->p.temperature <= 0.0f && g->p.repetition_penalty == 1.0f;
}

int generator_new(twd_head* head, const twd_generation_params& params, const uint32_t* prompt,
                  uint32_t prompt_len, const uint32_t* stop_ids, uint32_t n_stop,
                  G4DenseTokenCallback on_token, void* user, twd_generator** out) {
    if (!head || !out) return fail(TWD_E_INVALID, "null head or out");
    *out = nullptr;
    if (prompt_len == 0 || !prompt) return fail(TWD_E_INVALID, "the prompt must hold at least one token");
    if (n_stop > 0 && !stop_ids) return fail(TWD_E_INVALID, "null stop_ids");
    if (params.max_tokens > UINT32_MAX - prompt_len)
        return fail(TWD_E_INVALID, "prompt_len + max_tokens must fit 32 bits");
    uint32_t vocab = 0, d = 0;
    float cap = 0.0f;
    uint64_t bytes = 0;
    int rc = twd_head_info(head, &vocab, &d, &cap, &bytes);
    if (rc) return rc;
    twd_generator* g = new twd_generator();
    g->head = head;
    g->vocab = vocab;
    g->softcap = cap;
    g->p = params;
    g->cap = prompt_len + params.max_tokens;
    g->len = prompt_len;
    g->prompt_len = prompt_len;
    g->checked = prompt_len;
    g->stop_ids.assign(stop_ids, stop_ids + n_stop);
    g->on_token = on_token;
    g->user = user;
    hipError_t e = hipMalloc(&g->history, std::max<size_t>(g->cap, 1) * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&g->logits, static_cast<size_t>(vocab) * sizeof(float));
    if (e == hipSuccess) e = hipHostMalloc(&g->token_host, sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) e = hipMemcpy(g->history, prompt, prompt_len * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        twd_generator_destroy(g);
        return hip_fail(e, "twd_generator_create");
    }
    if (params.max_tokens == 0) g->reason = TWD_STOP_MAX_TOKENS;
    *out = g;
    return TWD_OK;
}

}  // namespace
}  // namespace twd

using namespace twd;

extern "C" {

TWD_API int twd_generator_create(twd_head* head, const twd_generation_params* params,
                                 const uint32_t* prompt, uint32_t prompt_len,
                                 const uint32_t* stop_ids, uint32_t n_stop, twd_generator** out) {
    clear_error();
    if (!params) return fail(TWD_E_INVALID, "null params");
    return generator_new(head, *params, prompt, prompt_len, stop_ids, n_stop, nullptr, nullptr, out);
}

TWD_API int twd_generator_create_ex(twd_head* head, const G4DenseGenerationOptions* opts,
                                    const uint32_t* prompt, uint32_t prompt_len,
                                    const uint32_t* stop_ids, uint32_t n_stop,
                                    G4DenseTokenCallback on_token, void* user,
                                    twd_generator** out) {
    clear_error();
    // GenerationOptions{} with SamplingParams{} (runner.hpp:25-27, sampling.hpp:9-18) when the
    // caller passes no options; otherwise the fields c_api.cpp:132-140 copies
    twd_generation_params p{};
    p.temperature = 0.0f;
    p.top_p = 1.0f;
    p.top_k = 0;
    p.repetition_penalty = 1.0f;
    p.has_seed = 0;
    p.seed = 0;
    p.max_tokens = 512;
    if (opts) {
        p.temperature = opts->temperature;
        p.top_p = opts->top_p;
        p.top_k = opts->top_k;
        p.repetition_penalty = opts->repetition_penalty;
        p.has_seed = opts->has_seed != 0 ? 1 : 0;
        p.seed = opts->seed;
        p.max_tokens = opts->max_tokens > 0 ? static_cast<uint32_t>(opts->max_tokens) : 0u;
    }
    return generator_new(head, p, prompt, prompt_len, stop_ids, n_stop, on_token, user, out);
}

TWD_API void twd_generator_cancel(twd_generator* g) {
    if (g) g->cancel.store(true, std::memory_order_release);
}

TWD_API int twd_generator_stop_reason(const twd_generator* g) { return g ? g->reason : TWD_STOP_NONE; }

TWD_API void twd_generator_destroy(twd_generator* g) {
    if (!g) return;
    if (g->history) (void)hipFree(g->history);
    if (g->logits) (void)hipFree(g->logits);
    if (g->token_host) (void)hipHostFree(g->token_host);
    delete g;
}

TWD_API int twd_generator_step(twd_generator* g, const uint16_t* hidden_bf16, void* stream,
                               uint32_t* token_out, int* finished) {
    clear_error();
    int rc = TWD_OK;
    if (check_step(g, finished, &rc)) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t* slot = g->history + g->len;  // the token lands in the history directly
    if (fused_greedy(g)) {
        rc = twd_head_greedy(g->head, hidden_bf16, 1, nullptr, slot, stream);
    } else {
        const twd_row_params r = step_params(g);
        rc = twd_head_sample(g->head, hidden_bf16, 1, &r, g->history, g->logits, slot, stream);
    }
    if (rc) return rc;
    return finish_step(g, s, token_out, finished);
}

TWD_API int twd_generator_step_rmsnorm(twd_generator* g, const float* x, const uint16_t* norm_weight,
                                       float eps, void* stream, uint32_t* token_out, int* finished) {
    clear_error();
    int rc = TWD_OK;
    if (check_step(g, finished, &rc)) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t* slot = g->history + g->len;
    if (fused_greedy(g)) {
        rc = twd_head_greedy_rmsnorm(g->head, x, norm_weight, eps, 1, nullptr, slot, stream);
    } else {
        const twd_row_params r = step_params(g);
        rc = twd_head_sample_rmsnorm(g->head, x, norm_weight, eps, 1, &r, g->history, g->logits,
                                     slot, stream);
    }
    if (rc) return rc;
    return finish_step(g, s, token_out, finished);
}

TWD_API int twd_generator_sync(twd_generator* g, int* finished) {
    clear_error();
    if (!g) return fail(TWD_E_INVALID, "null generator");
    TWD_HIP(hipDeviceSynchronize());  // the steps may have run on any stream
    const int rc = (g->reason == TWD_STOP_CANCELLED || g->reason == TWD_STOP_DEGENERATE)
                       ? TWD_OK
                       : check_emitted(g, nullptr);
    if (finished) *finished = g->reason != TWD_STOP_NONE ? 1 : 0;
    return rc;
}

TWD_API int twd_generator_history(const twd_generator* g, const uint32_t** history_dev,
                                  uint32_t* len) {
    clear_error();
    if (!g) return fail(TWD_E_INVALID, "null generator");
    if (history_dev) *history_dev = g->history;
    if (len) *len = g->len;
    return TWD_OK;
}

TWD_API int twd_generator_tokens(const twd_generator* g, uint32_t* host_out, uint32_t capacity,
                                 uint32_t* len) {
    clear_error();
    if (!g || !host_out) return fail(TWD_E_INVALID, "null generator or output");
    const uint32_t n = std::min(capacity, g->len);
    TWD_HIP(hipDeviceSynchronize());
    TWD_HIP(hipMemcpy(host_out, g->history, n * sizeof(uint32_t), hipMemcpyDeviceToHost));
    if (len) *len = g->len;
    return TWD_OK;
}

}  // extern "C"
