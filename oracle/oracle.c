/*
 * CPU oracle: scalar restatement of the reference's token-selection path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with -O3 -ffp-contract=off so every float
 * expression is evaluated exactly as written, in the order written.
 *
 * What pins each function (tests/test_oracle.py):
 *   or_splitmix64         known answers from tests/test_sampling.cpp:118-121; reference build
 *   or_seed_for           reference build (oracle/_ref) over 10^4 positions x seeds; golden file
 *   or_next_uniform       reference build: or_sample_token(seed) == g4dense::sample_token(seed)
 *   or_validate_sampling  accept/reject matrix of tests/test_sampling.cpp:92-112; reference build
 *   or_apply_repetition_penalty  known answers tests/test_sampling.cpp:198-228; brute force for
 *                         duplicates; bit-exact against the reference build; golden file
 *   or_argmax             {1,5,3,5,2} -> 1 (test_sampling.cpp:141-148); numpy brute force
 *   or_shortlist          numpy full lexsort (independent algorithm) at V=262144
 *   or_sample_token(_u)   the full-sort restatement of test_sampling.cpp:36-84 re-derived in
 *                         numpy; truncation-order case (:161-172); 200 golden ids at V=262144
 *                         from the reference build; the u seam equals the seed path for
 *                         seed-derived u
 *   or_verify             the three cases of tests/test_speculative.cpp:48-76; reference build
 *   or_mt64_*             the standard's known answer ([rand.predef]: the 10000th output of a
 *                         default-seeded mt19937_64 is 9981545732273789042)
 *   or_canonical_float,   against libstdc++'s std::uniform_real_distribution<float> over
 *   or_rejection_uniforms std::mt19937_64 (gen_std.cpp) for 10^4 seeds; closed forms at the
 *                         extremes (x = 0, x >= 2^64 - 2^39 -> nextafter(1, 0))
 *   or_softmax,           reference build (oracle/_ref) on random rows, every branch incl.
 *   or_verify_draft       rejections and forced fallbacks; golden file; identical draft and
 *                         target rows always accept (r == 1)
 *   or_lm_head(_f64)      numpy float64 dequant + matmul (closed form w = q*s + b)
 *   or_rmsnorm            closed forms (constant rows, zero rows, unit weight) and numpy
 *                         float64 within the reference test's 1e-4/1e-3 (test_gpu_kernels.cpp:197)
 *   or_gen_lm_head        numpy restatement of the documented counter formula
 * Parity is unpinned at the libm layer: exp(double) and tanhf are glibc's here, and no
 * reference test fixes their last-ulp behaviour (the reference toolchain is unpinned).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* sampling.cpp:56-61 */
uint64_t or_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

/* sampling.cpp:63-72 */
uint64_t or_seed_for(int has_seed, uint64_t seed, int position) {
    const uint64_t pos = (uint64_t)(int64_t)position;
    const uint64_t base = has_seed ? seed + pos
                                   : (0x9E3779B97F4A7C15ULL ^ (pos * 0xD1B54A32D192ED03ULL));
    const uint64_t s = or_splitmix64(base);
    return s ? s : 0x9E3779B97F4A7C15ULL;
}

/* xorshift64*, sampling.cpp:18-23 */
uint64_t or_next_random(uint64_t* state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    return s * 0x2545F4914F6CDD1DULL;
}

/* sampling.cpp:25-28: the top 24 bits of the draw as an exact fraction of 2^24 */
float or_next_uniform(uint64_t* state) {
    return (float)((or_next_random(state) >> 40) & 0xFFFFFFu) / 16777216.0f;
}

float or_uniform_from_seed(uint64_t seed) {
    uint64_t s = seed;
    return or_next_uniform(&s);
}

/* sampling.cpp:32-54, kMaxTopK = 256 (:15) */
int or_validate_sampling(float t, float p, int k, float rp) {
    if (!isfinite(t) || t < 0.0f) return OR_ERR_INVALID;
    if (!isfinite(p) || p <= 0.0f || p > 1.0f) return OR_ERR_INVALID;
    if (k < 0 || k > 256) return OR_ERR_INVALID;
    if (!isfinite(rp) || rp <= 0.0f) return OR_ERR_INVALID;
    if (t > 0.0f && p < 1.0f && k == 0) return OR_ERR_INVALID;
    return OR_OK;
}

/* sampling.cpp:74-90: every occurrence applies the op again, so duplicates compound */
void or_apply_repetition_penalty(float* logits, uint32_t vocab, const uint32_t* history,
                                 size_t n, float penalty, float softcap) {
    if (penalty == 1.0f || n == 0) return;
    const float limit = (softcap > 0.0f) ? softcap * 0.9999f : 0.0f;
    for (size_t j = 0; j < n; ++j) {
        const uint32_t id = history[j];
        if (id >= vocab) continue;
        float v = logits[id];
        v = (v > 0.0f) ? (v / penalty) : (v * penalty);
        if (limit > 0.0f) {
            /* std::clamp(v, lo, hi) == (v < lo) ? lo : (hi < v) ? hi : v */
            const float lo = -limit;
            v = (v < lo) ? lo : ((limit < v) ? limit : v);
        }
        logits[id] = v;
    }
}

/* sampling.cpp:97-104 */
uint32_t or_argmax(const float* logits, uint32_t vocab) {
    uint32_t best = 0;
    float best_v = logits[0];
    for (uint32_t i = 1; i < vocab; ++i) {
        if (logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    }
    return best;
}

/* The shortlist order of sampling.cpp:128-131: value descending, index ascending; '!=' makes
 * -0 and +0 equal so they fall through to the index. */
static int ranks_before(const float* l, uint32_t a, uint32_t b) {
    if (l[a] != l[b]) return l[a] > l[b];
    return a < b;
}

static int cmp_rank(const void* pa, const void* pb, void* ctx) {
    const float* l = (const float*)ctx;
    const uint32_t a = *(const uint32_t*)pa, b = *(const uint32_t*)pb;
    if (a == b) return 0;
    return ranks_before(l, a, b) ? -1 : 1;
}

/* Bounded heap whose root is the worst kept index. Any correct selection under a strict total
 * order yields the same set as std::nth_element (sampling.cpp:132-137). */
static void sift_down(const float* l, uint32_t* h, uint32_t n, uint32_t i) {
    for (;;) {
        uint32_t worst = i;
        const uint32_t a = 2 * i + 1, b = 2 * i + 2;
        if (a < n && ranks_before(l, h[worst], h[a])) worst = a;
        if (b < n && ranks_before(l, h[worst], h[b])) worst = b;
        if (worst == i) return;
        const uint32_t t = h[i];
        h[i] = h[worst];
        h[worst] = t;
        i = worst;
    }
}

static void sift_up(const float* l, uint32_t* h, uint32_t i) {
    while (i > 0) {
        const uint32_t p = (i - 1) / 2;
        if (!ranks_before(l, h[p], h[i])) return;
        const uint32_t t = h[i];
        h[i] = h[p];
        h[p] = t;
        i = p;
    }
}

uint32_t or_shortlist(const float* logits, uint32_t vocab, uint32_t want, uint32_t* idx) {
    if (want > vocab) want = vocab;
    uint32_t n = 0;
    for (uint32_t i = 0; i < vocab; ++i) {
        if (n < want) {
            idx[n] = i;
            sift_up(logits, idx, n);
            ++n;
        } else if (want > 0 && ranks_before(logits, i, idx[0])) {
            idx[0] = i;
            sift_down(logits, idx, n, 0);
        }
    }
    qsort_r(idx, n, sizeof(uint32_t), cmp_rank, (void*)logits);
    return n;
}

/* sampling.cpp:92-169 with the uniform supplied by the caller */
int or_sample_token_u(const float* logits, uint32_t vocab, float temperature, float top_p,
                      int top_k, float u, uint32_t* out, or_sample_diag* diag) {
    if (vocab == 0) return OR_ERR_EMPTY_VOCAB;
    if (diag) {
        memset(diag, 0, sizeof(*diag));
        diag->u = u;
        diag->cut_margin = INFINITY;
        diag->draw_margin = INFINITY;
    }
    if (temperature <= 0.0f) {
        *out = or_argmax(logits, vocab);
        return OR_OK;
    }

    /* std::max(a, b) returns (a < b) ? b : a */
    float max_logit = logits[0];
    for (uint32_t i = 1; i < vocab; ++i) max_logit = (max_logit < logits[i]) ? logits[i] : max_logit;
    const double mx = (double)max_logit;

    double total = 0.0;
    for (uint32_t i = 0; i < vocab; ++i) total += exp((double)logits[i] - mx);
    if (!(total > 0.0)) return OR_ERR_DEGENERATE;

    const uint32_t want = (top_k > 0) ? ((uint32_t)top_k < vocab ? (uint32_t)top_k : vocab)
                                      : (256u < vocab ? 256u : vocab);
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * (want ? want : 1));
    const uint32_t n = or_shortlist(logits, vocab, want, idx);

    size_t cut = n;
    double cut_margin = INFINITY;
    if (top_p < 1.0f) {
        double run = 0.0;
        const double pp = (double)top_p;
        for (size_t i = 0; i < n; ++i) {
            run += exp((double)logits[idx[i]] - mx) / total;
            const double m = fabs(run - pp);
            if (m < cut_margin) cut_margin = m;
            if (run >= pp) {
                cut = i + 1;
                break;
            }
        }
    }
    if (top_k > 0 && cut > (size_t)top_k) cut = (size_t)top_k;
    if (cut < 1) cut = 1;

    double* q = (double*)malloc(sizeof(double) * cut);
    double denom = 0.0;
    const double td = (double)temperature;
    for (size_t i = 0; i < cut; ++i) {
        q[i] = exp(((double)logits[idx[i]] - mx) / td);
        denom += q[i];
    }
    const double r = (double)u * denom;
    double acc = 0.0;
    uint32_t tok = idx[cut - 1];
    double draw_margin = INFINITY;
    int found = 0;
    for (size_t i = 0; i < cut; ++i) {
        acc += q[i];
        const double m = fabs(acc - r);
        if (m < draw_margin) draw_margin = m;
        if (!found && acc >= r) {
            tok = idx[i];
            found = 1;
        }
    }
    *out = tok;
    if (diag) {
        diag->max_logit = mx;
        diag->total = total;
        diag->want = want;
        diag->cut = (uint32_t)cut;
        diag->cut_margin = cut_margin;
        diag->draw_r = r;
        diag->draw_margin = draw_margin;
    }
    free(q);
    free(idx);
    return OR_OK;
}

int or_sample_token(const float* logits, uint32_t vocab, float temperature, float top_p,
                    int top_k, uint64_t seed, uint32_t* out, or_sample_diag* diag) {
    return or_sample_token_u(logits, vocab, temperature, top_p, top_k, or_uniform_from_seed(seed),
                             out, diag);
}

/* speculator.cpp:34-153; the greedy branch (:58-69) and the no-draft-logits branch
 * (:123-134) both call sample_token(row_i, splitmix64(base_seed + i)) and compare. */
int or_verify(const uint32_t* drafts, size_t n_drafts, const float* const* rows, size_t n_rows,
              uint32_t vocab, float temperature, float top_p, int top_k, uint64_t base_seed,
              or_verify_result* out) {
    memset(out, 0, sizeof(*out));
    if (n_drafts > OR_MAX_DRAFTS) return OR_ERR_INVALID;
    out->total_drafted = (uint32_t)n_drafts;
    if (n_drafts == 0 || n_rows == 0) return OR_OK;
    const size_t k = n_drafts < n_rows ? n_drafts : n_rows;
    size_t accepted = 0;
    for (size_t i = 0; i < k; ++i) {
        uint32_t tok = 0;
        const int rc = or_sample_token(rows[i], vocab, temperature, top_p, top_k,
                                       or_splitmix64(base_seed + i), &tok, NULL);
        if (rc != OR_OK) return rc;
        if (drafts[i] == tok) {
            out->tokens[out->n_tokens++] = tok;
            ++accepted;
        } else {
            out->bonus_token = tok;
            out->bonus_token_sampled = 1;
            out->tokens[out->n_tokens++] = tok;
            break;
        }
    }
    if (accepted == k && n_rows > k) {
        uint32_t tok = 0;
        const int rc = or_sample_token(rows[k], vocab, temperature, top_p, top_k,
                                       or_splitmix64(base_seed + k), &tok, NULL);
        if (rc != OR_OK) return rc;
        out->bonus_token = tok;
        out->bonus_token_sampled = 1;
        out->tokens[out->n_tokens++] = tok;
    }
    out->num_accepted = (uint32_t)accepted;
    out->acceptance_rate = out->total_drafted == 0 ? 0.0
                                                   : (double)out->num_accepted / out->total_drafted;
    return OR_OK;
}

/* ---- rejection-sampling verify (speculator.cpp:14-30, :71-122) ------------------------------ */

/* MT19937-64 as the C++ standard defines std::mt19937_64: w=64, n=312, m=156, r=31,
 * a=0xB5026F5AA96619E9, u=29, d=0x5555555555555555, s=17, b=0x71D67FFFEDA60000, t=37,
 * c=0xFFF7EEE000000000, l=43, f=6364136223846793005. */
void or_mt64_seed(or_mt64* g, uint64_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
    g->idx = 312;
}

uint64_t or_mt64_next(or_mt64* g) {
    if (g->idx >= 312) {
        for (int i = 0; i < 312; ++i) {
            const uint64_t x = (g->mt[i] & 0xFFFFFFFF80000000ULL) | (g->mt[(i + 1) % 312] & 0x7FFFFFFFULL);
            uint64_t xa = x >> 1;
            if (x & 1) xa ^= 0xB5026F5AA96619E9ULL;
            g->mt[i] = g->mt[(i + 156) % 312] ^ xa;
        }
        g->idx = 0;
    }
    uint64_t y = g->mt[g->idx++];
    y ^= (y >> 29) & 0x5555555555555555ULL;
    y ^= (y << 17) & 0x71D67FFFEDA60000ULL;
    y ^= (y << 37) & 0xFFF7EEE000000000ULL;
    y ^= y >> 43;
    return y;
}

float or_canonical_float(uint64_t x) {
    const float sum = (float)x;                  /* _RealType(g() - g.min()) * 1 */
    float r = sum / 18446744073709551616.0f;     /* / 2^64, exact in float */
    if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
    return 0.0f + r * (1.0f - 0.0f);             /* uniform_real_distribution: a + c (b - a) */
}

void or_rejection_uniforms(uint64_t step_seed, float* u1, float* u2) {
    or_mt64 g;
    or_mt64_seed(&g, step_seed);
    *u1 = or_canonical_float(or_mt64_next(&g));
    *u2 = or_canonical_float(or_mt64_next(&g));
}

/* sampling.cpp:114,145,157: std::exp(double) is the C library's exp */
void or_exp(const double* x, double* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = exp(x[i]);
}

/* speculator.cpp:23: std::exp(float) is the C library's expf */
void or_expf(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(x[i]);
}

/* speculator.cpp:14-30 */
void or_softmax(float* l, uint32_t n, float temp) {
    if (temp <= 0.0f) temp = 1.0f;
    float max_l = -1e9f;
    for (uint32_t i = 0; i < n; ++i) {
        l[i] /= temp;
        if (l[i] > max_l) max_l = l[i];
    }
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        l[i] = expf(l[i] - max_l);
        sum += l[i];
    }
    const float inv = 1.0f / (sum > 1e-12f ? sum : 1.0f);
    for (uint32_t i = 0; i < n; ++i) l[i] *= inv;
}

static float softmax_sum(const float* l, uint32_t n, float temp) {
    /* the sum compute_softmax forms, for the diagnostics */
    if (temp <= 0.0f) temp = 1.0f;
    float max_l = -1e9f;
    for (uint32_t i = 0; i < n; ++i) {
        const float x = l[i] / temp;
        if (x > max_l) max_l = x;
    }
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; ++i) sum += expf(l[i] / temp - max_l);
    return sum;
}

/* speculator.cpp:34-153, all branches */
int or_verify_draft(const uint32_t* drafts, size_t n_drafts, const float* const* rows,
                    size_t n_rows, const float* const* draft_rows, size_t n_draft_rows,
                    uint32_t vocab, float temperature, float top_p, int top_k,
                    float repetition_penalty, uint64_t base_seed, or_verify_result* out,
                    or_reject_diag* diag) {
    memset(out, 0, sizeof(*out));
    if (n_drafts > OR_MAX_DRAFTS) return OR_ERR_INVALID;
    out->total_drafted = (uint32_t)n_drafts;
    if (n_drafts == 0 || n_rows == 0) return OR_OK;
    const int greedy = temperature <= 0.0f && repetition_penalty == 1.0f; /* sampling.hpp:17 */
    const size_t k = n_drafts < n_rows ? n_drafts : n_rows;
    size_t accepted = 0;
    float* p = NULL;
    float* q = NULL;
    int rc = OR_OK;
    for (size_t i = 0; i < k; ++i) {
        const uint32_t draft = drafts[i];
        const uint64_t step_seed = or_splitmix64(base_seed + i);
        const int has_draft = !greedy && i < n_draft_rows && draft_rows[i] != NULL;
        if (!has_draft) {
            uint32_t tok = 0;
            rc = or_sample_token(rows[i], vocab, temperature, top_p, top_k, step_seed, &tok, NULL);
            if (rc != OR_OK) break;
            if (draft == tok) {
                out->tokens[out->n_tokens++] = tok;
                ++accepted;
                continue;
            }
            out->bonus_token = tok;
            out->bonus_token_sampled = 1;
            out->tokens[out->n_tokens++] = tok;
            break;
        }
        if (!p) {
            p = (float*)malloc(sizeof(float) * vocab);
            q = (float*)malloc(sizeof(float) * vocab);
        }
        memcpy(p, rows[i], sizeof(float) * vocab);
        or_softmax(p, vocab, temperature);
        memcpy(q, draft_rows[i], sizeof(float) * vocab);
        or_softmax(q, vocab, temperature);
        const float p_val = draft < vocab ? p[draft] : 0.0f;
        const float q_val = draft < vocab ? q[draft] : 0.0f;
        const float r = (q_val > 1e-12f) ? (p_val / q_val) : 1.0f;
        float u1, u2;
        or_rejection_uniforms(step_seed, &u1, &u2);
        or_reject_diag dg = {r, u1, u2, softmax_sum(rows[i], vocab, temperature),
                             softmax_sum(draft_rows[i], vocab, temperature), -1.0f, -1.0f, 0, 0};
        if (u1 <= r) {
            dg.accepted = 1;
            if (diag) diag[i] = dg;
            out->tokens[out->n_tokens++] = draft;
            ++accepted;
            continue;
        }
        /* rejection: draw from (p - q)+ */
        float sum_diff = 0.0f;
        for (uint32_t v = 0; v < vocab; ++v) {
            const float x = p[v] - q[v];
            sum_diff += (0.0f < x) ? x : 0.0f;  /* std::max(0.0f, x) */
        }
        uint32_t corr = 0;
        dg.sum_diff = sum_diff;
        if (sum_diff > 1e-9f) {
            const float r_val = u2 * sum_diff;
            dg.r_val = r_val;
            float acc = 0.0f;
            for (uint32_t v = 0; v < vocab; ++v) {
                const float x = p[v] - q[v];
                acc += (0.0f < x) ? x : 0.0f;
                if (acc >= r_val) {
                    corr = v;
                    break;
                }
            }
            dg.corr = corr;
        } else {
            rc = or_sample_token(rows[i], vocab, temperature, top_p, top_k, step_seed, &corr, NULL);
            dg.corr = 0xFFFFFFFFu;
            if (rc != OR_OK) break;
        }
        if (diag) diag[i] = dg;
        out->bonus_token = corr;
        out->bonus_token_sampled = 1;
        out->tokens[out->n_tokens++] = corr;
        break;
    }
    free(p);
    free(q);
    if (rc != OR_OK) return rc;
    if (accepted == k && n_rows > k) {
        uint32_t tok = 0;
        rc = or_sample_token(rows[k], vocab, temperature, top_p, top_k, or_splitmix64(base_seed + k),
                             &tok, NULL);
        if (rc != OR_OK) return rc;
        out->bonus_token = tok;
        out->bonus_token_sampled = 1;
        out->tokens[out->n_tokens++] = tok;
    }
    out->num_accepted = (uint32_t)accepted;
    out->acceptance_rate = out->total_drafted == 0 ? 0.0
                                                   : (double)out->num_accepted / out->total_drafted;
    return OR_OK;
}

static float bf16_to_f32(uint16_t v);

/* cpu_reference.cpp:141-150 */
void or_rmsnorm(const float* x, const uint16_t* weight_bf16, uint32_t dim, float eps, float* out) {
    float sum_sq = 0.0f;
    for (uint32_t i = 0; i < dim; ++i) sum_sq += x[i] * x[i];
    const float rms = 1.0f / sqrtf((sum_sq / (float)dim) + eps);
    for (uint32_t i = 0; i < dim; ++i) out[i] = x[i] * rms * bf16_to_f32(weight_bf16[i]);
}

static float bf16_to_f32(uint16_t v) {
    const uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

/* cpu_reference.cpp:643-665 */
void or_lm_head(const uint32_t* W, const uint16_t* S, const uint16_t* B, const float* hidden,
                uint32_t d, uint32_t group, uint32_t row0, uint32_t nrows, float softcap,
                float* out) {
    const uint32_t packed_cols = d / 8, groups = d / group;
    for (uint32_t v = row0; v < row0 + nrows; ++v) {
        const uint32_t* rw = W + (size_t)v * packed_cols;
        const uint16_t* rs = S + (size_t)v * groups;
        const uint16_t* rb = B + (size_t)v * groups;
        float sum = 0.0f;
        for (uint32_t c = 0; c < d; ++c) {
            const uint32_t q = (rw[c / 8] >> ((c % 8) * 4)) & 0x0Fu;
            const uint32_t g = c / group;
            const float w = (float)q * bf16_to_f32(rs[g]) + bf16_to_f32(rb[g]);
            sum += w * hidden[c];
        }
        if (softcap > 0.0f) sum = softcap * tanhf(sum / softcap);
        out[v - row0] = sum;
    }
}

void or_lm_head_f64(const uint32_t* W, const uint16_t* S, const uint16_t* B, const float* hidden,
                    uint32_t d, uint32_t group, uint32_t row0, uint32_t nrows, double* out) {
    const uint32_t packed_cols = d / 8, groups = d / group;
    for (uint32_t v = row0; v < row0 + nrows; ++v) {
        const uint32_t* rw = W + (size_t)v * packed_cols;
        const uint16_t* rs = S + (size_t)v * groups;
        const uint16_t* rb = B + (size_t)v * groups;
        double sum = 0.0;
        for (uint32_t c = 0; c < d; ++c) {
            const uint32_t q = (rw[c / 8] >> ((c % 8) * 4)) & 0x0Fu;
            const uint32_t g = c / group;
            const double w = (double)q * bf16_to_f32(rs[g]) + bf16_to_f32(rb[g]);
            sum += w * (double)hidden[c];
        }
        out[v - row0] = sum;
    }
}

/* Softcap.hlsl:16-30 and cpu_reference.cpp:661-663 */
void or_softcap(float* z, size_t n, float softcap) {
    if (!(softcap > 0.0f)) return;
    for (size_t i = 0; i < n; ++i) z[i] = softcap * tanhf(z[i] / softcap);
}

static uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void or_gen_lm_head(uint64_t seed, uint32_t d, uint32_t group, uint32_t row0, uint32_t nrows,
                    uint32_t* W, uint16_t* S, uint16_t* B) {
    const uint64_t words = (uint64_t)(d / 8), groups = (uint64_t)(d / group);
    for (uint64_t r = 0; r < nrows; ++r) {
        const uint64_t grow = row0 + r;
        for (uint64_t w = 0; w < words; ++w) {
            const uint64_t i = grow * words + w;
            W[r * words + w] = (uint32_t)(or_splitmix64(seed + 0x1000000000000000ULL + i) >> 32);
        }
        for (uint64_t g = 0; g < groups; ++g) {
            const uint64_t j = grow * groups + g;
            const float u = (float)(or_splitmix64(seed + 0x2000000000000000ULL + j) >> 40) *
                            (1.0f / 16777216.0f);
            const uint16_t s = f32_to_bf16_rne(fmaf(9e-3f, u, 1e-3f));
            S[r * groups + g] = s;
            B[r * groups + g] = f32_to_bf16_rne(-8.0f * bf16_to_f32(s));
        }
    }
}
