/*
 * CPU oracle for the Turbo-WinFare Dense token-selection path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a scalar restatement of the reference's algorithm, used by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker. Nothing in the
 * product library links, loads or calls it, and the product fails loudly when its HIP library
 * is missing instead of falling back to this code.
 *
 * Reference files restated (paths relative to the reference checkout):
 *   src/sampling.cpp:15-169      seeding, validation, repetition penalty, sample_token
 *   src/speculator.cpp:34-153    evaluate_verification (every branch except the draft-logits
 *                                rejection branch, :71-122)
 *   src/cpu_reference.cpp:635-665 scalar INT4 g64 LM head + tanh softcap
 *   shaders/Common.hlsli:163-222 weight layout (low nibble first, group = c / 64)
 *
 * Pinning status of each function is listed in the header comment of oracle.c.
 */
#ifndef TWD_ORACLE_H
#define TWD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OR_OK = 0,
    OR_ERR_EMPTY_VOCAB = 1,   /* sampling.cpp:94 */
    OR_ERR_DEGENERATE = 2,    /* sampling.cpp:116-118 */
    OR_ERR_INVALID = 3        /* validate_sampling rejections, sampling.cpp:32-54 */
};

/* Diagnostics of one sampled draw: how far the decisions were from flipping. */
typedef struct {
    double max_logit;    /* fp32 max promoted to double */
    double total;        /* sum_i exp(l_i - max) over the whole vocabulary, index order */
    uint32_t want;       /* shortlist size */
    uint32_t cut;        /* survivors after top-p, top-k, >=1 */
    double cut_margin;   /* |run - p| at the cut (top-p active), else +inf */
    double draw_r;       /* u * denom */
    double draw_margin;  /* min_i |acc_i - r| over the survivors */
    float u;             /* the uniform actually used */
} or_sample_diag;

typedef struct {
    uint32_t tokens[65];      /* accepted drafts + the correction or bonus token */
    uint32_t n_tokens;
    uint32_t num_accepted;
    uint32_t total_drafted;
    int bonus_token_sampled;
    uint32_t bonus_token;
    double acceptance_rate;
} or_verify_result;

uint64_t or_splitmix64(uint64_t x);
uint64_t or_seed_for(int has_seed, uint64_t seed, int position);
uint64_t or_next_random(uint64_t* state);
float or_next_uniform(uint64_t* state);
float or_uniform_from_seed(uint64_t seed);

int or_validate_sampling(float temperature, float top_p, int top_k, float repetition_penalty);

void or_apply_repetition_penalty(float* logits, uint32_t vocab, const uint32_t* history,
                                 size_t history_len, float penalty, float softcap);

/* sample_token with the seed path (sampling.cpp:92-169). */
int or_sample_token(const float* logits, uint32_t vocab, float temperature, float top_p,
                    int top_k, uint64_t seed, uint32_t* out, or_sample_diag* diag);
/* Same algorithm with the uniform injected directly instead of drawn from the seed. */
int or_sample_token_u(const float* logits, uint32_t vocab, float temperature, float top_p,
                      int top_k, float u, uint32_t* out, or_sample_diag* diag);

/* Greedy argmax: strict '>' so ties keep the lower index (sampling.cpp:96-104). */
uint32_t or_argmax(const float* logits, uint32_t vocab);

/* Sorted shortlist of `want` indices under (value desc, index asc). Returns its length. */
uint32_t or_shortlist(const float* logits, uint32_t vocab, uint32_t want, uint32_t* idx_out);

/* evaluate_verification without draft logits (speculator.cpp:34-153, the greedy branch and
 * the sample-and-compare branch; both call sample_token identically). */
int or_verify(const uint32_t* drafts, size_t n_drafts, const float* const* rows, size_t n_rows,
              uint32_t vocab, float temperature, float top_p, int top_k,
              uint64_t base_seed, or_verify_result* out);

/* Scalar INT4 g64 LM head (cpu_reference.cpp:643-665): fp32 sequential dot over c, then
 * softcap*tanhf(sum/softcap) when softcap > 0. W is [V][d/8] u32, S/B are [V][d/G] bf16 bits,
 * hidden is fp32 [d]. Computes rows [row0, row0+nrows). */
void or_lm_head(const uint32_t* W, const uint16_t* S, const uint16_t* B, const float* hidden,
                uint32_t d, uint32_t group, uint32_t row0, uint32_t nrows, float softcap,
                float* out);
/* The same dot in double precision with no softcap: an accuracy yardstick for both the scalar
 * fp32 loop and the device kernels. */
void or_lm_head_f64(const uint32_t* W, const uint16_t* S, const uint16_t* B, const float* hidden,
                    uint32_t d, uint32_t group, uint32_t row0, uint32_t nrows, double* out);
/* softcap*tanhf(z/softcap) elementwise, identity for softcap <= 0 (Softcap.hlsl:16-30). */
void or_softcap(float* z, size_t n, float softcap);

/* Synthetic LM-head generator (counter based, identical to the product's device generator):
 *   W[i] = hi32(splitmix64(seed + 0x1000000000000000 + i))
 *   u_j  = (splitmix64(seed + 0x2000000000000000 + j) >> 40) * 2^-24
 *   S[j] = bf16_rne(fmaf(9e-3f, u_j, 1e-3f)),  B[j] = bf16(-8 * S[j])  (exact)
 * Fills rows [row0, row0+nrows) of a [V][d] head with groups of `group`. */
void or_gen_lm_head(uint64_t seed, uint32_t d, uint32_t group, uint32_t row0, uint32_t nrows,
                    uint32_t* W, uint16_t* S, uint16_t* B);

/* Logits of the reference's own sampling test: std::mt19937(seed) with
 * std::normal_distribution<float>(mean, sd) (tests/test_sampling.cpp:177-180,238-242).
 * Implemented in gen_std.cpp against libstdc++. */
void or_gen_mt19937_normal(uint32_t seed, float mean, float sd, size_t n, float* out);

#ifdef __cplusplus
}
#endif

#endif /* TWD_ORACLE_H */
