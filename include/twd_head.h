/*
 * twd_head.h -- C-ABI of the MI355X (gfx950) token-selection path for Turbo-WinFare Dense.
 *
 * Covers the tied INT4 group-64 affine LM head and everything after it: the tanh logit softcap,
 * greedy argmax, the sampling chain (repetition penalty, then top-p over the full distribution,
 * then top-k, then the temperature draw), and greedy speculative verify/accept.
 *
 * Conventions (mirroring the reference's C-ABI, include/g4dense/c_api.h:18-49 and
 * src/c_api.cpp:82-93):
 *   - every entry point returns 0 on success and a negative TWD_E_* code on failure, never
 *     throws, and leaves a message for twd_last_error() (thread-local, valid until the next
 *     call on the same thread);
 *   - device pointers are plain pointers into HBM; `stream` is a hipStream_t passed as void*
 *     (NULL = the legacy default stream). Work is enqueued on that stream and the call returns
 *     without waiting, except where a comment says otherwise;
 *   - token ids are uint32; logits are fp32 rows of `vocab` entries; hidden states are bf16
 *     bit patterns (uint16) laid out [rows][d_model].
 *
 * A selected id of TWD_TOKEN_DEGENERATE (0xFFFFFFFF) in a token output marks a row whose
 * distribution the reference rejects: sample_token throws when sum(exp(l - max)) is not
 * > 0, e.g. NaN logits (src/sampling.cpp:112-118).
 */
#ifndef TWD_HEAD_H
#define TWD_HEAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TWD_API __attribute__((visibility("default")))

#define TWD_OK 0
#define TWD_E_INVALID (-1)  /* bad argument (null handle, size out of range, ...) */
#define TWD_E_HIP (-2)      /* a HIP runtime call failed */
#define TWD_E_DEGENERATE (-3)
#define TWD_E_UNSUPPORTED (-4)

#define TWD_TOKEN_DEGENERATE 0xFFFFFFFFu
#define TWD_MAX_ROWS 64u     /* rows per LM-head call (M) */
#define TWD_MAX_WANT 256u    /* largest shortlist (top_k, or 256 when top_k == 0) */

/* Per-row selection parameters. temperature/top_p/top_k/repetition_penalty have the meaning of
 * g4dense::SamplingParams (include/g4dense/sampling.hpp:9-18). `uniform` is the draw in [0,1):
 * sample_token derives it as next_uniform(seed) (src/sampling.cpp:25-28,161-162); the host
 * supplies it here (twd_uniform_from_seed computes the reference's value). `softcap` is the
 * clamp bound handed to apply_repetition_penalty (src/sampling.cpp:74-90). The history is
 * history_ids[history_offset .. history_offset + history_len). */
typedef struct {
    float temperature;
    float top_p;
    int32_t top_k;
    float repetition_penalty;
    float uniform;
    float softcap;
    uint32_t history_offset;
    uint32_t history_len;
} twd_row_params;

/* Greedy verify result, mirroring g4dense::SpeculativeEvaluation
 * (include/g4dense/speculator.hpp:10-17). Written to device memory. */
typedef struct {
    uint32_t n_tokens;             /* accepted drafts + 1 correction/bonus token */
    uint32_t num_accepted;
    uint32_t total_drafted;
    uint32_t bonus_token_sampled;
    uint32_t bonus_token;
    uint32_t tokens[TWD_MAX_ROWS + 1];
} twd_verify_result;

typedef struct twd_head twd_head;
typedef struct twd_selector twd_selector;

/* Message of the last failed call on this thread (g4dense_engine_last_error, c_api.h:47). */
TWD_API const char* twd_last_error(void);

/* ---- the LM head ---------------------------------------------------------------------------
 * Uploads the tied head once, as the runner does at load time (src/runner.cpp:423-443): `wsb`
 * is the container's contiguous LM-head slice [W u32 V x d/8 | S bf16 V x d/64 | B bf16 V x d/64]
 * (include/g4dense/format.hpp:60-61), element c of row r being nibble c%8 (low first) of word
 * r*d/8 + c/8 and w = q*s + b (shaders/Common.hlsli:163-222). The head is repacked once into
 * the HBM layout the kernels stream. group_size must be 64, d_model a multiple of 128, vocab at
 * most 2^30, and the call is synchronous. A head with a group scale above 2^100 in magnitude or an infinite group
 * bias is rejected with TWD_E_UNSUPPORTED. */
TWD_API int twd_head_create(const void* wsb_host, uint64_t wsb_bytes, uint32_t vocab,
                            uint32_t d_model, uint32_t group_size, float softcap,
                            twd_head** out);
/* Same, from a copy of the slice that is already in device memory (left untouched). */
TWD_API int twd_head_create_device(const void* wsb_dev, uint64_t wsb_bytes, uint32_t vocab,
                                   uint32_t d_model, uint32_t group_size, float softcap,
                                   void* stream, twd_head** out);
TWD_API void twd_head_destroy(twd_head* head);
TWD_API int twd_head_info(const twd_head* head, uint32_t* vocab, uint32_t* d_model,
                          float* softcap, uint64_t* device_bytes);

/* logits[m][v] = softcap(sum_c w[v][c] * h[m][c]) for m < rows, row stride `vocab`.
 * Replaces GemvInt4 (rows == 1) / GemmInt4Batch (rows > 1) followed by Softcap
 * (src/runner.cpp:1958-2022; shaders/GemvInt4.hlsl:31-53, GemmInt4Batch.hlsl:65-143,
 * Softcap.hlsl:16-30). rows <= TWD_MAX_ROWS. */
TWD_API int twd_head_logits(twd_head* head, const uint16_t* hidden_bf16, uint32_t rows,
                            float* logits, void* stream);

/* tokens[m] = greedy sample_token of row m's softcapped logits (strict '>' argmax, lowest index
 * on ties, -0 == +0), fused into the head pass. `logits` may be NULL (not materialised).
 * Replaces LMHeadGreedy + ArgmaxReduce (shaders/LMHeadGreedy.hlsl:28-72,
 * ArgmaxReduce.hlsl:21-61) with the softcap the reference's sample_token sees
 * (src/sampling.cpp:97-104). */
TWD_API int twd_head_greedy(twd_head* head, const uint16_t* hidden_bf16, uint32_t rows,
                            float* logits, uint32_t* tokens, void* stream);

/* The decode-loop order of src/runner.cpp:2314-2326 per row m: softcapped logits, then
 * apply_repetition_penalty over the row's history (in place on `logits`, when
 * repetition_penalty != 1), then sample_token with params[m].uniform as the draw.
 * `params` is a host array of `rows` entries; `history_ids` is device memory. `logits` is
 * required (rows x vocab). */
TWD_API int twd_head_sample(twd_head* head, const uint16_t* hidden_bf16, uint32_t rows,
                            const twd_row_params* params, const uint32_t* history_ids,
                            float* logits, uint32_t* tokens, void* stream);

/* Greedy speculative verify over rows = n_drafts + 1 target rows [pending, d1..dK]:
 * SpeculativeCoordinator::evaluate_verification's greedy branch (src/speculator.cpp:50-69,
 * 138-150) fused into the head pass. `drafts` is device memory (n_drafts ids), `result` a
 * device twd_verify_result. `logits` may be NULL. */
TWD_API int twd_head_verify_greedy(twd_head* head, const uint16_t* hidden_bf16, uint32_t rows,
                                   const uint32_t* drafts, uint32_t n_drafts, float* logits,
                                   twd_verify_result* result, void* stream);

/* ---- calls on several streams, and the grid-finish state -------------------------------------
 * The greedy and verify passes finish on the device: every block folds its per-row maxima into
 * the head's finish state with atomics and the last block to arrive writes the result. That
 * state, the M > 8 staging of h and the head's selection scratch are shared by the head's calls,
 * so calls that arrive on another stream than the previous call are ordered after it (the
 * first change of stream waits for the device once; after that each call records an event
 * and a call on another stream waits for it). A head is driven by one host thread at a time.
 * Each launch counts its blocks in under its own epoch, and its last block arms the counter for
 * the next launch. A launch repeated with the same arguments (a captured graph replayed) counts
 * in on a replay slot armed by its previous replay, and a launch that finds neither armed for it
 * (the first replay, a write from outside) counts in on a fallback word, so a count left behind
 * never decides which block finishes.
 *
 * Stream capture: the head's calls (and a selector's) may be captured into a HIP graph on any
 * stream; a captured call waits for nothing and records nothing. Replays of such a graph share
 * the object's state with its other calls, so the caller orders them against those calls (one
 * stream, or its own events), as it orders the replays themselves.
 *
 * No counterpart in the reference: the device address of that state, for diagnostics and
 * tests: 64 per-row uint64 maxima, then the arrival counter's six uint64 words
 * {arrivals << 32 | epoch}: the word armed for the next launch, four replay slots and the
 * fallback word. */
TWD_API void* twd_head_finish_state(const twd_head* head);

/* ---- the same passes with the final RMSNorm as their prologue --------------------------------
 * h[m] = x[m] * (1 / sqrt(mean(x[m]^2) + eps)) * norm_weight, the model's last step before the
 * head (src/runner.cpp:1889-1918, shaders/RMSNormK.hlsl with has_weight = 1, eps = 1e-6 there;
 * CPU form src/cpu_reference.cpp:141-150), computed inside the head pass: x is fp32 [rows][d]
 * (16-byte aligned, rows <= 8, the reference's verify batch limit), norm_weight bf16 [d], and h
 * is carried at fp32 precision (as two bf16 halves) into the head, as the reference's fp32 GEMV
 * consumes it. Outputs and their meaning as the bf16-h entry points above. */
TWD_API int twd_head_logits_rmsnorm(twd_head* head, const float* x, const uint16_t* norm_weight,
                                    float eps, uint32_t rows, float* logits, void* stream);
TWD_API int twd_head_greedy_rmsnorm(twd_head* head, const float* x, const uint16_t* norm_weight,
                                    float eps, uint32_t rows, float* logits, uint32_t* tokens,
                                    void* stream);
TWD_API int twd_head_verify_greedy_rmsnorm(twd_head* head, const float* x,
                                           const uint16_t* norm_weight, float eps, uint32_t rows,
                                           const uint32_t* drafts, uint32_t n_drafts,
                                           float* logits, twd_verify_result* result, void* stream);
TWD_API int twd_head_sample_rmsnorm(twd_head* head, const float* x, const uint16_t* norm_weight,
                                    float eps, uint32_t rows, const twd_row_params* params,
                                    const uint32_t* history_ids, float* logits, uint32_t* tokens,
                                    void* stream);

/* ---- the .g4dense container ----------------------------------------------------------------
 * The fields of the container header (include/g4dense/format.hpp:26-110) this path uses. */
typedef struct {
    uint32_t version;
    uint32_t quant_type;
    uint32_t num_layers;
    uint32_t d_model;
    uint32_t d_ff;
    uint32_t vocab_size;
    uint32_t quant_group_size;
    uint32_t scale_dtype;
    uint32_t tied_embeddings;
    float final_logit_softcapping;
    uint64_t embed_offset;
    uint64_t embed_size;
    uint64_t lm_head_offset;
    uint64_t lm_head_size;
    uint64_t file_size;
} twd_container_info;

/* Reads and validates a container's 4096-byte header as validate_header(header, file_size)
 * does (src/format.cpp:6-65): the same checks, in the same order, with the same messages
 * (TWD_E_INVALID). Host only. */
TWD_API int twd_container_inspect(const char* path, twd_container_info* info);
/* Validates the header, then loads the LM head as the runner does at start-up: the tied head's
 * [W|S|B] slice at lm_head_offset (src/runner.cpp:423-443, rejected when it exceeds
 * lm_head_size) with the header's final_logit_softcapping as the softcap, and the final
 * RMSNorm weight stored after the embedding table (src/runner.cpp:488-497), kept on the head
 * for the *_rmsnorm entry points (twd_head_norm_weight). The head must be affine INT4 with
 * 64-wide groups and bf16 scales (TWD_E_UNSUPPORTED otherwise). Synchronous. */
TWD_API int twd_head_load(const char* path, void* stream, twd_head** out);
/* Device copy of the final RMSNorm weight (bf16 [d_model]) of a head loaded by twd_head_load,
 * NULL for heads created from a bare [W|S|B] slice. */
TWD_API const uint16_t* twd_head_norm_weight(const twd_head* head);

/* ---- the decode loop around the head -------------------------------------------------------
 * ForwardRunner::generate's per-step glue (src/runner.cpp:2312-2344) with the history in device
 * memory: per step, the head pass over the step's hidden state, then apply_repetition_penalty
 * over the whole history (when repetition_penalty != 1, clamped at the head's softcap), then
 * sample_token with the draw of seed_for(position = history length - 1), then the token is
 * appended; the generation finishes after max_tokens or on a stop id. The caller runs the
 * model between steps. The sampling fields mean what G4DenseGenerationOptions' do
 * (include/g4dense/c_api.h:24-36). */
typedef struct {
    float temperature;
    float top_p;
    int32_t top_k;
    float repetition_penalty;
    int32_t has_seed;
    uint64_t seed;
    uint32_t max_tokens;
} twd_generation_params;

typedef struct twd_generator twd_generator;

/* `prompt` (host, prompt_len >= 1 ids) starts the history; stop_ids (host) end the generation
 * when sampled. Allocates the history (prompt_len + max_tokens ids) and one logit row. */
TWD_API int twd_generator_create(twd_head* head, const twd_generation_params* params,
                                 const uint32_t* prompt, uint32_t prompt_len,
                                 const uint32_t* stop_ids, uint32_t n_stop, twd_generator** out);

/* The reference's own generation options and token callback, layout-identical to
 * include/g4dense/c_api.h:24-40 of the reference. They are declared here only when that header
 * has not been included first, so a caller that already holds the reference's struct passes it
 * unchanged (include c_api.h before this header). */
#ifndef G4DENSE_C_API_H
typedef struct {
    int max_tokens;
    float temperature;
    float top_p;
    int top_k;
    float repetition_penalty;
    int has_seed;
    unsigned long long seed;
    const char* system_prompt;
    const char* const* stop_strings;
    int stop_count;
    int tier_id;
} G4DenseGenerationOptions;
typedef int (*G4DenseTokenCallback)(void* user, int index, unsigned int token_id, const char* delta);
#endif

/* Why a generation finished (twd_generator_stop_reason). */
#define TWD_STOP_NONE 0        /* still running */
#define TWD_STOP_MAX_TOKENS 1  /* max_tokens ids emitted */
#define TWD_STOP_TOKEN 2       /* a stop id was sampled (it is the history's last id) */
#define TWD_STOP_CALLBACK 3    /* the token callback returned 0 (its id is the last one) */
#define TWD_STOP_CANCELLED 4   /* twd_generator_cancel; the step sampled nothing */
#define TWD_STOP_DEGENERATE 5  /* sample_token's degenerate-distribution error */

/* twd_generator_create with the options g4dense_engine_generate_ex receives
 * (src/c_api.cpp:121-162): max_tokens and the sampling fields are taken as c_api.cpp:132-140
 * maps them (a NULL opts means GenerationOptions' defaults: 512 tokens, greedy). system_prompt,
 * stop_strings, stop_count and tier_id are ignored, as generate_ex ignores the first three and
 * the memory tiers are not on this path. max_tokens <= 0 emits nothing. on_token (may be NULL)
 * is called once per emitted id, on the thread that runs the step, with (user, index, id, "")
 * where index counts emitted ids from 0 and the text piece is empty (detokenising is not on
 * this path); a return of 0 ends the generation after that id (runner.cpp:2330-2333,
 * c_api.cpp:148-155). With a callback every step reads its id back. Stop ids are checked after
 * the callback, as runner.cpp:2336 does. */
TWD_API int twd_generator_create_ex(twd_head* head, const G4DenseGenerationOptions* opts,
                                    const uint32_t* prompt, uint32_t prompt_len,
                                    const uint32_t* stop_ids, uint32_t n_stop,
                                    G4DenseTokenCallback on_token, void* user,
                                    twd_generator** out);
/* The cancel flag of ForwardRunner::generate (src/runner.cpp:2064, tested at the start of each
 * step, :2315). Safe to call from any thread while another runs steps: the next step samples
 * nothing and finishes the generation with TWD_STOP_CANCELLED (it returns TWD_OK, sets
 * *finished and leaves *token_out untouched). */
TWD_API void twd_generator_cancel(twd_generator* gen);
/* TWD_STOP_* of the generation (TWD_STOP_NONE while it runs). */
TWD_API int twd_generator_stop_reason(const twd_generator* gen);
TWD_API void twd_generator_destroy(twd_generator* gen);
/* One step on a bf16 hidden state [d_model]. With token_out or finished given (or a token
 * callback registered), the token is brought to the host (4 bytes, the call then waits for the
 * stream) and the stop rules are applied; a degenerate distribution returns TWD_E_DEGENERATE.
 * Without them the call only enqueues: the stop rules see max_tokens alone until
 * twd_generator_sync applies them to the ids emitted so far. */
TWD_API int twd_generator_step(twd_generator* gen, const uint16_t* hidden_bf16, void* stream,
                               uint32_t* token_out, int* finished);
/* Waits for the device and applies the stop rules to the ids emitted since the last readback,
 * in order: the history is cut after the first stop id, or before the first degenerate draw
 * (returning TWD_E_DEGENERATE), and *finished (may be NULL) tells whether the generation is
 * over. Steps enqueued without readback past such an id are discarded this way. */
TWD_API int twd_generator_sync(twd_generator* gen, int* finished);
/* The same step with the final RMSNorm as the head's prologue (fp32 x [d_model]). */
TWD_API int twd_generator_step_rmsnorm(twd_generator* gen, const float* x,
                                       const uint16_t* norm_weight, float eps, void* stream,
                                       uint32_t* token_out, int* finished);
/* The device history (prompt then sampled ids) and its current length. */
TWD_API int twd_generator_history(const twd_generator* gen, const uint32_t** history_dev,
                                  uint32_t* len);
/* The history copied to host memory (at most `capacity` ids); waits for the device. Ids of
 * steps that were enqueued without readback are copied as they are: call twd_generator_sync
 * first to apply the stop rules to them. */
TWD_API int twd_generator_tokens(const twd_generator* gen, uint32_t* host_out, uint32_t capacity,
                                 uint32_t* len);

/* ---- selection over caller-owned logits ----------------------------------------------------
 * A selector owns the scratch for up to max_rows rows of up to max_vocab entries. */
TWD_API int twd_selector_create(uint32_t max_vocab, uint32_t max_rows, twd_selector** out);
TWD_API void twd_selector_destroy(twd_selector* sel);

/* Per row m of `logits` (device, row stride `row_stride` floats): apply_repetition_penalty in
 * place (src/sampling.cpp:74-90), then sample_token (src/sampling.cpp:92-169) with
 * params[m].uniform. tokens[m] receives the id (device). */
TWD_API int twd_select(twd_selector* sel, float* logits, uint32_t vocab, uint32_t rows,
                       uint64_t row_stride, const twd_row_params* params,
                       const uint32_t* history_ids, uint32_t* tokens, void* stream);

/* twd_select without a selector, allocating nothing: no counterpart in the reference. It is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The selection scratch is a fixed device array of
 * 4,252,208 bytes per GPU, kept for the life of the process: at most 64 rows of at most 262144
 * entries per call (TWD_E_INVALID beyond). Every call on one GPU uses that GPU's one array, so
 * calls that overlap on a GPU (other streams, other threads) race: order them. The first call on
 * each device looks the array's address up there. Results are those of twd_select. */
TWD_API int twd_select_noalloc(float* logits, uint32_t vocab, uint32_t rows, uint64_t row_stride,
                               const twd_row_params* params, const uint32_t* history_ids,
                               uint32_t* tokens, void* stream);

/* evaluate_verification without draft logits (src/speculator.cpp:34-153 minus :71-122): row i
 * is sampled with uniform next_uniform(splitmix64(base_seed + i)) and compared with draft i;
 * the first mismatch emits the target token, a full match adds the bonus row. Greedy params
 * (temperature <= 0) give the greedy branch. `params` applies to every row and its history
 * fields are ignored (the reference's verify applies no penalty). */
TWD_API int twd_verify(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                       uint64_t row_stride, const twd_row_params* params, uint64_t base_seed,
                       const uint32_t* drafts, uint32_t n_drafts, twd_verify_result* result,
                       void* stream);

/* evaluate_verification with draft logits, every branch (src/speculator.cpp:34-153). As
 * twd_verify, plus: `draft_rows` is a host array of n_draft_rows device pointers; a non-NULL
 * entry i is position i's draft logit row (vocab floats) and selects the rejection-sampling
 * branch (:71-122) there: fp32 softmaxes of both rows at params->temperature (compute_softmax,
 * :14-30, its sequential fp32 sums reproduced exactly), the ratio test p/q against u1 and, on
 * rejection, a draw from (p - q)+ with u2, where (u1, u2) are the first two
 * uniform_real_distribution<float> draws of mt19937_64(splitmix64(base_seed + i))
 * (twd_rejection_uniforms). NULL entries, positions >= n_draft_rows and greedy params
 * (temperature <= 0 and repetition_penalty == 1) sample-and-compare as twd_verify does. The
 * first call with draft rows allocates 8 * vocab bytes of scratch per such position on the
 * selector (kept, and grown when a later call needs more), and one side stream (default
 * priority) with two events: the target rows' selection runs there, forked from `stream` and
 * joined back into it before the call's last launch, so `stream` orders all of the call's work. */
TWD_API int twd_verify_draft(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                             uint64_t row_stride, const float* const* draft_rows,
                             uint32_t n_draft_rows, const twd_row_params* params,
                             uint64_t base_seed, const uint32_t* drafts, uint32_t n_drafts,
                             twd_verify_result* result, void* stream);

/* The exact sequential-sum engine of twd_verify_draft on its own. No counterpart in the
 * reference's API; it is for callers and tests that check the engine against an in-order fp32
 * loop (the sums of compute_softmax, src/speculator.cpp:22-26, and of the residual draw,
 * :104-116, are formed that way). terms: n finite values >= 0 in device memory, 16-byte
 * aligned and readable up to n rounded up to a multiple of 16 floats. With stop_out NULL,
 * *sum_out (device) receives the full in-order fp32 sum ((t0 + t1) + t2) + ... . With stop_out
 * (device) given, the sum stops at the first index i whose prefix sum t0 + ... + ti is >= thr:
 * *stop_out receives i and *sum_out that prefix sum; when no prefix reaches thr, *stop_out
 * receives n and *sum_out the full sum. Asynchronous on `stream`. */
TWD_API int twd_sequential_sum(const float* terms, uint32_t n, float thr, float* sum_out,
                               uint32_t* stop_out, void* stream);

/* No counterpart in the reference: the device address of the selector's draft-verify finish
 * counter, for diagnostics and tests (NULL before the first twd_verify_draft call that had
 * draft rows): the six uint64 words {arrivals << 32 | epoch} of its arrival counter (the word
 * armed for the next call, four replay slots, the fallback word). The residual launch's blocks
 * count in on it and its last block runs the accept chain; each call arms it for the next, and a
 * call that finds it not armed for itself (a write from outside) counts in on another word. */
TWD_API void* twd_selector_verify_state(const twd_selector* sel);
/* No counterpart in the reference: the fp32 softmax sums (compute_softmax, speculator.cpp:22-26)
 * of the last twd_verify_draft call on this selector that ran the rejection branch, for
 * diagnostics and tests. *n receives the number of positions that had draft rows; for each,
 * positions[i] is the position and sums[2i], sums[2i + 1] the target and draft rows' sums (at
 * most `capacity` positions). Waits for the device. */
TWD_API int twd_verify_draft_sums(const twd_selector* sel, float* sums, uint32_t* positions,
                                  uint32_t capacity, uint32_t* n);

/* ---- the reference's seeding, for callers that keep seeds (src/sampling.cpp:18-72) -------- */
TWD_API uint64_t twd_splitmix64(uint64_t x);
TWD_API uint64_t twd_seed_for(int has_seed, uint64_t seed, int position);
TWD_API float twd_uniform_from_seed(uint64_t seed);
/* The two draws of src/speculator.cpp:87-89,105 for a step seed: the host C++ standard
 * library's std::uniform_real_distribution<float>(0, 1) over std::mt19937_64(step_seed). */
TWD_API void twd_rejection_uniforms(uint64_t step_seed, float* u1, float* u2);
/* 0 when validate_sampling accepts the parameters, TWD_E_INVALID (with a message) otherwise
 * (src/sampling.cpp:32-54). */
TWD_API int twd_validate_sampling(float temperature, float top_p, int32_t top_k,
                                  float repetition_penalty);

/* ---- synthetic data (benchmarks and tests) -------------------------------------------------
 * Fills a device buffer with the reference layout [W|S|B] of a V x d head, rows drawn from the
 * counter formula: W[i] = hi32(splitmix64(seed + 2^60 + i)), u_j = (splitmix64(seed + 2^61 + j)
 * >> 40) / 2^24, S[j] = bf16_rne(fmaf(9e-3, u_j, 1e-3)), B[j] = -8 * S[j]. */
TWD_API int twd_generate_head(void* wsb_dev, uint32_t vocab, uint32_t d_model,
                              uint32_t group_size, uint64_t seed, void* stream);
/* A pure-read probe with no counterpart in the reference, for measurement: `waves` (a multiple
 * of 8) each stream a contiguous stripe of `bytes / waves` bytes (rounded down to 1 KB) of `buf`
 * with 16-byte non-temporal loads, 8 KB in flight per wave -- the head kernels' access pattern
 * with no arithmetic. Times `launches` launches after 5 warm-up ones on `stream`. */
TWD_API int twd_probe_read_bandwidth(const void* buf, uint64_t bytes, uint32_t waves,
                                     uint32_t launches, void* stream, float* us_per_launch,
                                     uint64_t* bytes_read);
/* No counterpart in the reference: out[i] = the device expf the draft-logits verify uses
 * (glibc's expf method, bit-exact with the x86-64 host library) of x[i], for tests. Device
 * buffers of n floats; asynchronous on `stream`. */
TWD_API int twd_probe_expf(const float* x, float* out, uint64_t n, void* stream);
/* No counterpart in the reference: out[i] = the device exp(double) the sampled shortlist uses for
 * its terms exp(l - max) and exp((l - max) / T) (glibc's exp method, bit-exact with the x86-64
 * host library) of x[i], for tests. Device buffers of n doubles; asynchronous on `stream`. */
TWD_API int twd_probe_exp(const double* x, double* out, uint64_t n, void* stream);
/* Bytes of the reference layout for a V x d head with 64-wide groups. */
TWD_API uint64_t twd_head_bytes(uint32_t vocab, uint32_t d_model, uint32_t group_size);

#ifdef __cplusplus
}
#endif

#endif /* TWD_HEAD_H */
