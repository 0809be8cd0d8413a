// The decode loop around the head: what ForwardRunner::generate does with each step's logits
// (src/runner.cpp:2312-2344) -- repetition penalty over the whole history, seed_for(position),
// sample_token, append to the history, stop on a stop id or after max_tokens -- with the
// history kept in device memory, so that a step moves no logits to the host. The caller runs
// the model and hands each step's final hidden state over; the generator returns the token.
#include <hip/hip_runtime.h>

#include <algorithm>
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
    uint32_t emitted = 0;
    uint32_t* token_host = nullptr;  // pinned
    float* logits = nullptr;         // device [vocab]
    std::vector<uint32_t> stop_ids;
    bool finished = false;
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

// After the head pass has written the step's token at history[len] (the selection of this step
// read history[0, len) only): count it in and, when asked, bring it to the host and apply the
// stop rules (src/runner.cpp:2327-2336).
int finish_step(twd_generator* g, hipStream_t s, uint32_t* token_out, int* finished) {
    const uint32_t* token_dev = g->history + g->len;
    ++g->len;
    ++g->emitted;
    bool done = g->emitted >= g->p.max_tokens;
    if (token_out || finished) {
        TWD_HIP(hipMemcpyAsync(g->token_host, token_dev, sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        TWD_HIP(hipStreamSynchronize(s));
        const uint32_t t = *g->token_host;
        if (t == TWD_TOKEN_DEGENERATE) {  // sample_token throws here; the generation ends
            g->finished = true;
            return fail(TWD_E_DEGENERATE, "sample_token: logit distribution is degenerate");
        }
        if (token_out) *token_out = t;
        done = done || std::find(g->stop_ids.begin(), g->stop_ids.end(), t) != g->stop_ids.end();
    }
    g->finished = done;
    if (finished) *finished = done ? 1 : 0;
    return TWD_OK;
}

int check_step(twd_generator* g) {
    if (!g) return fail(TWD_E_INVALID, "null generator");
    if (g->finished) return fail(TWD_E_INVALID, "the generation has finished");
    if (g->len >= g->cap) return fail(TWD_E_INVALID, "history capacity exhausted");
    return TWD_OK;
}

// greedy with no penalty: the head's fused argmax; otherwise logits, then penalty + draw
bool fused_greedy(const twd_generator* g) {
    return g->p.temperature <= 0.0f && g->p.repetition_penalty == 1.0f;
}

}  // namespace
}  // namespace twd

using namespace twd;

extern "C" {

TWD_API int twd_generator_create(twd_head* head, const twd_generation_params* params,
                                 const uint32_t* prompt, uint32_t prompt_len,
                                 const uint32_t* stop_ids, uint32_t n_stop, twd_generator** out) {
    clear_error();
    if (!head || !params || !out) return fail(TWD_E_INVALID, "null head, params or out");
    *out = nullptr;
    if (prompt_len == 0 || !prompt) return fail(TWD_E_INVALID, "the prompt must hold at least one token");
    if (n_stop > 0 && !stop_ids) return fail(TWD_E_INVALID, "null stop_ids");
    if (params->max_tokens > UINT32_MAX - prompt_len)
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
    g->p = *params;
    g->cap = prompt_len + params->max_tokens;
    g->len = prompt_len;
    g->stop_ids.assign(stop_ids, stop_ids + n_stop);
    hipError_t e = hipMalloc(&g->history, std::max<size_t>(g->cap, 1) * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&g->logits, static_cast<size_t>(vocab) * sizeof(float));
    if (e == hipSuccess) e = hipHostMalloc(&g->token_host, sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) e = hipMemcpy(g->history, prompt, prompt_len * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        twd_generator_destroy(g);
        return hip_fail(e, "twd_generator_create");
    }
    g->finished = params->max_tokens == 0;
    *out = g;
    return TWD_OK;
}

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
    int rc = check_step(g);
    if (rc) return rc;
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
    int rc = check_step(g);
    if (rc) return rc;
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
