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
 *   src/speculator.cpp:14-153    compute_softmax and evaluate_verification, every branch
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

/* The verify entry points take at most OR_MAX_DRAFTS drafts (OR_ERR_INVALID beyond). */
#define OR_MAX_DRAFTS 1024

typedef struct {
    uint32_t tokens[OR_MAX_DRAFTS + 1]; /* accepted drafts + the correction or bonus token */
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

/* ---- the draft-logits (rejection sampling) branch of evaluate_verification ---------------- */

/* std::mt19937_64 (the C++ standard's definition, [rand.predef]: Matsumoto-Nishimura MT19937-64
 * parameters, default seed 5489). */
typedef struct {
    uint64_t mt[312];
    int idx;
} or_mt64;
void or_mt64_seed(or_mt64* g, uint64_t seed);
uint64_t or_mt64_next(or_mt64* g);

/* libstdc++'s std::uniform_real_distribution<float>(0, 1) over a 64-bit engine: one engine call,
 * generate_canonical<float, 24>: float(x) / 2^64 in float, values that round to 1 replaced by
 * nextafter(1, 0); then 0 + 1 * c. */
float or_canonical_float(uint64_t x);
/* The two draws of speculator.cpp:87-89,105: rng = mt19937_64(step_seed); u1 = udist(rng) for the
 * ratio test, u2 = udist(rng) for the residual draw. */
void or_rejection_uniforms(uint64_t step_seed, float* u1, float* u2);

/* compute_softmax of speculator.cpp:14-30, in place: divide by temp (1 when temp <= 0), max from
 * -1e9f with '>', expf(l - max) summed in index order in float, times 1/sum (sum > 1e-12f, else
 * 1). */
void or_softmax(float* logits, uint32_t n, float temp);

/* Per-position diagnostics of the rejection branch. */
typedef struct {
    float r;            /* p_val / q_val (1 when q_val <= 1e-12f) */
    float u1;           /* ratio-test draw */
    float u2;           /* residual draw */
    float sum_p, sum_q; /* compute_softmax sums */
    float sum_diff;     /* sum of (p - q)+, or -1 when accepted */
    float r_val;        /* u2 * sum_diff, or -1 */
    uint32_t corr;      /* residual token, or 0xFFFFFFFF when the fallback sample_token ran */
    int accepted;
} or_reject_diag;

/* evaluate_verification, every branch (speculator.cpp:34-153). draft_rows[i] (i < n_draft_rows)
 * holds position i's draft logits, or NULL for "no draft probabilities" (an empty vector in the
 * reference); positions >= n_draft_rows have none. diag (optional) receives one entry per
 * position that ran the rejection branch, indexed by position. */
int or_verify_draft(const uint32_t* drafts, size_t n_drafts, const float* const* rows,
                    size_t n_rows, const float* const* draft_rows, size_t n_draft_rows,
                    uint32_t vocab, float temperature, float top_p, int top_k,
                    float repetition_penalty, uint64_t base_seed, or_verify_result* out,
                    or_reject_diag* diag);

/* out[i] = expf(x[i]) of the host C library: std::exp(float) as compute_softmax calls it
 * (speculator.cpp:23). */
void or_expf(const float* x, float* out, size_t n);
/* out[i] = exp(x[i]) of the host C library: std::exp(double) as sample_token calls it
 * (sampling.cpp:114,145,157) */
void or_exp(const double* x, double* out, size_t n);

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
/* The final RMSNorm, cpu_reference.cpp:141-150: sum of squares in index order (fp32),
 * rms = 1 / sqrt(sum / dim + eps), out = x * rms * weight; the bf16 weight widened to fp32 as
 * cpu_reference.cpp:614-618 does. */
void or_rmsnorm(const float* x, const uint16_t* weight_bf16, uint32_t dim, float eps, float* out);
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
/* libstdc++'s std::uniform_real_distribution<float>(0, 1) over std::mt19937_64(seeds[i]), two
 * draws per seed; and the 10000th output of a default-seeded std::mt19937_64. gen_std.cpp. */
void or_std_rejection_uniforms(const uint64_t* seeds, size_t n, float* out);
uint64_t or_std_mt64_10000th(void);

#ifdef __cplusplus
}
#endif

#endif /* TWD_ORACLE_H */
