// Speculative verify with draft logits on gfx950: the rejection-sampling branch of
// SpeculativeCoordinator::evaluate_verification (src/speculator.cpp:71-122, with compute_softmax
// of :14-30), composed with the sample-and-compare and bonus steps the selector already runs.
//
// The reference computes, per position with draft probabilities, two fp32 softmaxes whose sums
// run sequentially in index order, a ratio test p/q against a uniform, and on rejection a draw
// from (p - q)+ by a sequential fp32 prefix sum. Token ids only match the reference if those
// sequential float sums are reproduced bit for bit, so the device recomputes them exactly
// (block_seq_sum below) instead of summing in a tree.
//
// Kernels, all on the caller's stream:
//   draft_max_kernel     grid (parts, 2P): per row, partial maxima of l / T (T = 1 when <= 0)
//   draft_exp_kernel     grid (parts, 2P): e = expf(l / T - max) to scratch, NaN flags
//   draft_reject_kernel  grid P, 1024 threads: the two sums, the ratio test, the residual draw
//   draft_finish_kernel  one thread: the accept chain over all positions, bonus, result
// where P is the number of positions with a draft row; the target tokens of the other
// positions, of the fallback and of the bonus row come from the selector (launch_select).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "twd_internal.h"

// Every float expression in this file rounds each operation on its own: hipcc would otherwise
// fuse a * b - c * d into an fma, which the reference's x86-64 build never does.
#pragma clang fp contract(off)

namespace twd {

constexpr int kDraftThreads = 256;   // max / exp kernels
constexpr int kDraftPer = 16;
constexpr uint32_t kDraftChunk = kDraftThreads * kDraftPer;  // entries per block and row
constexpr uint32_t kDraftMaxParts = 128;                     // vocab <= 524288
constexpr int kRejThreads = 1024;    // one block per position
constexpr int kRejWaves = kRejThreads / 64;
constexpr int kRejPer = 8;           // terms per thread per window
constexpr uint32_t kRejWin = kRejThreads * kRejPer;
constexpr uint32_t kNoEvent = 0xFFFFFFFFu;

struct DraftPos {
    const float* target;  // row of vocab logits
    const float* draft;
    uint32_t position;    // index i in the draft chain
    float u1, u2;         // the two mt19937_64 draws of step_seed (speculator.cpp:87-89,105)
};

struct DraftArgs {
    uint32_t vocab;
    uint32_t parts;
    uint32_t npos;
    float temp;                   // compute_softmax's temperature (1 when <= 0)
    const uint32_t* drafts;       // device, draft ids by position
    float* part;                  // [2P][parts] partial maxima
    float* e;                     // [2P][vocab] expf(l / T - max)
    uint32_t* flags;              // [2P] bit 0: a NaN term
    uint32_t* rej;                // [64][4] {accepted, token, fallback, valid}
    DraftPos pos[TWD_MAX_ROWS];
};

// (float)exp((double)x): correctly rounded except where exp's double result lies within an ulp
// of a float rounding boundary. The reference calls the host libm's expf.
__device__ __forceinline__ float expf_cr(float x) {
    return static_cast<float>(exp(static_cast<double>(x)));
}

__device__ __forceinline__ const float* draft_row(const DraftArgs& a, uint32_t r) {
    return (r & 1) ? a.pos[r >> 1].draft : a.pos[r >> 1].target;
}

__global__ __launch_bounds__(kDraftThreads) void draft_max_kernel(DraftArgs a) {
    const uint32_t r = blockIdx.y;
    const float* l = draft_row(a, r);
    const uint32_t base = blockIdx.x * kDraftChunk + threadIdx.x;
    float m = -1e9f;
#pragma unroll
    for (int it = 0; it < kDraftPer; ++it) {
        const uint32_t j = base + it * kDraftThreads;
        if (j < a.vocab) {
            const float x = l[j] / a.temp;
            if (x > m) m = x;  // NaN never wins, as in the reference's '>' scan
        }
    }
    __shared__ float red[kDraftThreads / 64];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float y = __shfl_xor(m, o);
        m = y > m ? y : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kDraftThreads / 64; ++w) m = red[w] > m ? red[w] : m;
        a.part[r * a.parts + blockIdx.x] = m;
        if (blockIdx.x == 0) a.flags[r] = 0u;
    }
}

__global__ __launch_bounds__(kDraftThreads) void draft_exp_kernel(DraftArgs a) {
    const uint32_t r = blockIdx.y;
    const float* l = draft_row(a, r);
    // the row maximum; max over the partial maxima equals the reference's running '>' maximum
    // (both ignore NaN, start from -1e9f, and equal values are interchangeable)
    float mx = -1e9f;
    for (uint32_t p = 0; p < a.parts; ++p) {
        const float y = a.part[r * a.parts + p];
        mx = y > mx ? y : mx;
    }
    const uint32_t base = blockIdx.x * kDraftChunk + threadIdx.x;
    bool nan = false;
    float* e = a.e + static_cast<size_t>(r) * a.vocab;
#pragma unroll
    for (int it = 0; it < kDraftPer; ++it) {
        const uint32_t j = base + it * kDraftThreads;
        if (j < a.vocab) {
            const float x = l[j] / a.temp;
            const float v = expf_cr(x - mx);
            nan |= (v != v);
            e[j] = v;
        }
    }
    if (__syncthreads_or(nan) && threadIdx.x == 0)
        __hip_atomic_fetch_or(a.flags + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- exact sequential fp32 summation ---------------------------------------------------------
//
// block_seq_sum reproduces `float s = 0; for (j = 0; j < n; ++j) s += a(j);` bit for bit for
// non-negative, non-NaN terms, and optionally the first j whose prefix reaches `thr`.
//
// While the running sum S stays inside one binade [2^E, 2^(E+1)) (or below 2^-125, where the
// spacing is 2^-149 throughout), every representable S is an integer multiple of u = 2^(E-23)
// and fl(S + a) = S + RN(a / u) * u: the increment is a's value in units of u, rounded to
// nearest, except that an exact half-way case rounds so that the new S / u is even. So within
// a binade the sums are integer prefix sums whose only data dependence is the parity of S / u
// at each tie, which a scan over 2-state transfer functions resolves in parallel. The first
// term whose sum leaves the binade (S / u reaching 2^24) is added with one real fp32 add, and
// the scan restarts from there with the new binade's unit.

struct Xfer {  // input parity p -> (total increment, output parity)
    uint64_t inc0, inc1;
    uint32_t out0, out1;
};

__device__ __forceinline__ Xfer xfer_id() { return Xfer{0, 0, 0u, 1u}; }

// f, then g
__device__ __forceinline__ Xfer xfer_then(const Xfer& f, const Xfer& g) {
    Xfer h;
    h.inc0 = f.inc0 + (f.out0 ? g.inc1 : g.inc0);
    h.out0 = f.out0 ? g.out1 : g.out0;
    h.inc1 = f.inc1 + (f.out1 ? g.inc1 : g.inc0);
    h.out1 = f.out1 ? g.out1 : g.out0;
    return h;
}

__device__ __forceinline__ Xfer xfer_shfl_up(const Xfer& x, int d) {
    Xfer y;
    y.inc0 = (static_cast<uint64_t>(__shfl_up(static_cast<uint32_t>(x.inc0 >> 32), d)) << 32) |
             __shfl_up(static_cast<uint32_t>(x.inc0), d);
    y.inc1 = (static_cast<uint64_t>(__shfl_up(static_cast<uint32_t>(x.inc1 >> 32), d)) << 32) |
             __shfl_up(static_cast<uint32_t>(x.inc1), d);
    const uint32_t o = __shfl_up(x.out0 | (x.out1 << 1), d);
    y.out0 = o & 1u;
    y.out1 = o >> 1;
    return y;
}

// Term a >= 0 in units of u = 2^(E - 23): floor k, and kind 0 exact/rounds down, 1 rounds up,
// 2 exactly half-way.
__device__ __forceinline__ void split_term(float a, int E, uint64_t& k, uint32_t& kind) {
    const uint32_t b = __float_as_uint(a);
    const uint32_t f = b >> 23;
    uint32_t m = b & 0x7FFFFFu;
    int ea = -126;
    if (f) {
        m |= 0x800000u;
        ea = static_cast<int>(f) - 127;
    }
    const int sh = E - ea;
    kind = 0;
    if (m == 0) {
        k = 0;
    } else if (sh <= 0) {
        k = static_cast<uint64_t>(m) << min(-sh, 39);  // >= 2^24 from -sh >= 1: leaves the binade
    } else if (sh >= 25) {
        k = 0;  // a < u / 2
    } else {
        k = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
        kind = rem > half ? 1u : (rem == half ? 2u : 0u);
    }
}

__device__ __forceinline__ Xfer term_xfer(uint64_t k, uint32_t kind) {
    if (kind == 2) {
        const uint32_t kp = static_cast<uint32_t>(k & 1);
        return Xfer{k + kp, k + (kp ^ 1u), 0u, 0u};  // ties go to the even neighbour
    }
    const uint64_t c = k + kind;
    const uint32_t cp = static_cast<uint32_t>(c & 1);
    return Xfer{c, c, cp, cp ^ 1u};
}

__device__ __forceinline__ uint64_t term_inc(uint64_t k, uint32_t kind, uint32_t par) {
    if (kind == 2) return k + ((par + static_cast<uint32_t>(k)) & 1u);
    return k + kind;
}

struct SeqShared {
    Xfer wave_total[kRejWaves];
    uint32_t event;
    float S;
    uint32_t k0;
    uint32_t stop;
};

// Returns the sequential sum of term(0..n); *stop_at (when non-null) receives the first index
// whose prefix is >= thr, or n when none is.
template <typename Term>
__device__ float block_seq_sum(Term term, uint32_t n, float thr, uint32_t* stop_at, SeqShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool want_stop = stop_at != nullptr;
    float S = 0.0f;
    uint32_t k0 = 0;
    uint32_t stop = n;
    while (k0 < n) {
        // the binade of S: S = B * 2^(E - 23) with B < 2^24
        const uint32_t sb = __float_as_uint(S);
        const uint32_t sf = sb >> 23;
        const int E = sf ? static_cast<int>(sf) - 127 : -126;
        const uint64_t B = sf ? ((sb & 0x7FFFFFu) | 0x800000u) : sb;
        const uint32_t p0 = static_cast<uint32_t>(B & 1);
        const double Tu = want_stop ? ldexp(static_cast<double>(thr), 23 - E) : 0.0;
        constexpr uint64_t L = 1ull << 24;

        // this thread's terms of the window
        const uint32_t j0 = k0 + static_cast<uint32_t>(tid) * kRejPer;
        uint64_t kk[kRejPer];
        uint32_t kd[kRejPer];
        Xfer t = xfer_id();
#pragma unroll
        for (int q = 0; q < kRejPer; ++q) {
            const uint32_t j = j0 + q;
            const float a = j < n ? term(j) : 0.0f;
            split_term(a, E, kk[q], kd[q]);
            t = xfer_then(t, term_xfer(kk[q], kd[q]));
        }
        // wave inclusive scan, then exclusive
        Xfer inc = t;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const Xfer o = xfer_shfl_up(inc, d);
            if (lane >= d) inc = xfer_then(o, inc);
        }
        Xfer ex = xfer_shfl_up(inc, 1);
        if (lane == 0) ex = xfer_id();
        if (lane == 63) sh.wave_total[wave] = inc;
        if (tid == 0) sh.event = kNoEvent;
        __syncthreads();
        Xfer wp = xfer_id();
        for (int w = 0; w < wave; ++w) wp = xfer_then(wp, sh.wave_total[w]);
        const Xfer in = xfer_then(wp, ex);

        // replay: the first term that leaves the binade, or reaches thr
        uint64_t R = B + (p0 ? in.inc1 : in.inc0);
        uint32_t par = p0 ? in.out1 : in.out0;
        uint32_t my_event = kNoEvent;
        uint64_t R_before = R;
#pragma unroll
        for (int q = 0; q < kRejPer; ++q) {
            if (my_event != kNoEvent) break;
            const uint32_t j = j0 + q;
            if (j >= n) break;
            const uint64_t d = term_inc(kk[q], kd[q], par);
            if (R + d >= L) {
                my_event = 2 * j;  // crossing: exact add
                R_before = R;
                break;
            }
            R += d;
            par = (par + static_cast<uint32_t>(d)) & 1u;
            if (want_stop && static_cast<double>(R) >= Tu) my_event = 2 * j + 1;
        }
        if (my_event != kNoEvent) atomicMin(&sh.event, my_event);
        __syncthreads();
        const uint32_t ev = sh.event;
        if (ev == kNoEvent) {
            if (tid == kRejThreads - 1) {
                sh.S = ldexpf(static_cast<float>(R), E - 23);
                sh.k0 = min(n, k0 + kRejWin);
                sh.stop = n;
            }
        } else if (my_event == ev) {
            const uint32_t j = ev >> 1;
            if (ev & 1) {  // stop, no crossing before it
                sh.S = ldexpf(static_cast<float>(R), E - 23);
                sh.k0 = n;
                sh.stop = j;
            } else {
                const float prev = ldexpf(static_cast<float>(R_before), E - 23);
                const float s_new = prev + term(j);
                sh.S = s_new;
                sh.k0 = j + 1;
                sh.stop = (want_stop && s_new >= thr) ? j : n;
                if (sh.stop != n) sh.k0 = n;
            }
        }
        __syncthreads();
        S = sh.S;
        k0 = sh.k0;
        stop = sh.stop;
        __syncthreads();  // sh is rewritten by the next window
    }
    if (want_stop) *stop_at = stop;
    return S;
}

// One block per position with draft probabilities (speculator.cpp:74-121).
__global__ __launch_bounds__(kRejThreads) void draft_reject_kernel(DraftArgs a) {
    __shared__ SeqShared sh;
    const uint32_t pi = blockIdx.x;
    const DraftPos& P = a.pos[pi];
    const uint32_t V = a.vocab;
    const float* et = a.e + static_cast<size_t>(2 * pi) * V;
    const float* ed = a.e + static_cast<size_t>(2 * pi + 1) * V;
    const float nanf_ = __uint_as_float(0x7FC00000u);

    // compute_softmax sums (:22-26): NaN as soon as one term is NaN
    float sp = (a.flags[2 * pi] & 1u) ? nanf_
                                      : block_seq_sum([&](uint32_t j) { return et[j]; }, V, 0.0f, nullptr, sh);
    float sq = (a.flags[2 * pi + 1] & 1u) ? nanf_
                                          : block_seq_sum([&](uint32_t j) { return ed[j]; }, V, 0.0f, nullptr, sh);
    const float inv_p = 1.0f / (sp > 1e-12f ? sp : 1.0f);
    const float inv_q = 1.0f / (sq > 1e-12f ? sq : 1.0f);

    // ratio test (:83-92)
    const uint32_t dt = a.drafts[P.position];
    const float p_val = dt < V ? et[dt] * inv_p : 0.0f;
    const float q_val = dt < V ? ed[dt] * inv_q : 0.0f;
    const float r = (q_val > 1e-12f) ? (p_val / q_val) : 1.0f;
    uint32_t* out = a.rej + P.position * 4;
    if (P.u1 <= r) {
        if (threadIdx.x == 0) {
            out[0] = 1u;
            out[1] = dt;
            out[2] = 0u;
            out[3] = 1u;
        }
        return;
    }
    // residual (p - q)+ (:94-112): std::max(0.0f, x) keeps 0 for x <= 0 and for NaN
    // p[v] - q[v], each product rounded on its own as in the reference's separate loops
    auto diff = [&](uint32_t j) {
        const float x = et[j] * inv_p - ed[j] * inv_q;
        return (0.0f < x) ? x : 0.0f;
    };
    const float sum_diff = block_seq_sum(diff, V, 0.0f, nullptr, sh);
    uint32_t corr = 0;
    uint32_t fallback = 0;
    if (sum_diff > 1e-9f) {
        const float r_val = P.u2 * sum_diff;
        uint32_t at = V;
        block_seq_sum(diff, V, r_val, &at, sh);
        corr = at < V ? at : 0u;  // corr_tok starts at 0 (:101)
    } else {
        fallback = 1;  // sample_token on the target row (:114): the selector's token
    }
    if (threadIdx.x == 0) {
        out[0] = 0u;
        out[1] = corr;
        out[2] = fallback;
        out[3] = 1u;
    }
}

// The accept chain of speculator.cpp:53-146 over per-position outcomes: rej[i] for positions
// with draft rows (has_draft bit i), the selector's sampled token row_tok[i] otherwise, for the
// fallback, and for the bonus row k.
__global__ void draft_finish_kernel(const uint32_t* row_tokens, uint32_t rows, const uint32_t* drafts,
                                    uint32_t nd, uint64_t has_draft, const uint32_t* rej,
                                    twd_verify_result* v) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    uint32_t n = 0, acc = 0, bonus = 0, sampled = 0;
    bool bad = false;
    const uint32_t k = nd < rows ? nd : rows;
    bool rejected = false;
    for (uint32_t i = 0; i < k; ++i) {
        uint32_t t;
        bool ok;
        if ((has_draft >> i) & 1ull) {
            const uint32_t* o = rej + 4 * i;
            if (o[0]) {
                t = drafts[i];
                ok = true;
            } else {
                t = o[2] ? row_tokens[i] : o[1];
                ok = false;
            }
        } else {
            t = row_tokens[i];
            ok = drafts[i] == t;
        }
        if (t == TWD_TOKEN_DEGENERATE) {
            bad = true;
            break;
        }
        v->tokens[n++] = t;
        if (ok) {
            ++acc;
        } else {
            bonus = t;
            sampled = 1;
            rejected = true;
            break;
        }
    }
    if (!bad && !rejected && rows > k) {
        bonus = row_tokens[k];
        if (bonus == TWD_TOKEN_DEGENERATE) bad = true;
        sampled = 1;
        v->tokens[n++] = bonus;
    }
    v->n_tokens = bad ? TWD_TOKEN_DEGENERATE : n;
    v->num_accepted = acc;
    v->total_drafted = nd;
    v->bonus_token_sampled = sampled;
    v->bonus_token = bonus;
}

int draft_scratch_reserve(DraftScratch* d, uint32_t vocab, uint32_t npos) {
    const uint32_t parts = (vocab + kDraftChunk - 1) / kDraftChunk;
    const size_t need_e = static_cast<size_t>(2) * npos * vocab;
    if (d->e && d->e_capacity >= need_e && d->part_capacity >= static_cast<size_t>(2) * npos * parts)
        return TWD_OK;
    draft_scratch_free(d);  // grows: later calls with as many positions reuse it
    TWD_HIP(hipMalloc(&d->e, need_e * sizeof(float)));
    d->e_capacity = need_e;
    TWD_HIP(hipMalloc(&d->part, static_cast<size_t>(2) * npos * parts * sizeof(float)));
    d->part_capacity = static_cast<size_t>(2) * npos * parts;
    TWD_HIP(hipMalloc(&d->flags, 2 * TWD_MAX_ROWS * sizeof(uint32_t)));
    TWD_HIP(hipMalloc(&d->rej, 4 * TWD_MAX_ROWS * sizeof(uint32_t)));
    return TWD_OK;
}

void draft_scratch_free(DraftScratch* d) {
    if (d->e) (void)hipFree(d->e);
    if (d->part) (void)hipFree(d->part);
    if (d->flags) (void)hipFree(d->flags);
    if (d->rej) (void)hipFree(d->rej);
    *d = DraftScratch{};
}

}  // namespace twd

using namespace twd;

extern "C" {

TWD_API int twd_verify_draft(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                             uint64_t row_stride, const float* const* draft_rows,
                             uint32_t n_draft_rows, const twd_row_params* params,
                             uint64_t base_seed, const uint32_t* drafts, uint32_t n_drafts,
                             twd_verify_result* result, void* stream) {
    clear_error();
    if (!sel || !params || !result) return fail(TWD_E_INVALID, "null selector, params or result");
    if (n_drafts > 0 && !drafts) return fail(TWD_E_INVALID, "null drafts");
    if (n_drafts > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "n_drafts must be <= 64");
    if (rows > sel->scratch.max_rows) return fail(TWD_E_INVALID, "rows out of range for this selector");
    if (n_draft_rows > 0 && !draft_rows) return fail(TWD_E_INVALID, "null draft_rows");
    if (vocab > sel->max_vocab) return fail(TWD_E_INVALID, "vocab above the selector's max_vocab");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool greedy = params->temperature <= 0.0f && params->repetition_penalty == 1.0f;
    const uint32_t k = std::min(n_drafts, rows);
    uint64_t has = 0;
    DraftArgs a{};
    if (!greedy) {
        for (uint32_t i = 0; i < k && i < n_draft_rows; ++i) {
            if (!draft_rows[i]) continue;
            has |= 1ull << i;
            DraftPos& P = a.pos[a.npos++];
            P.target = logits + static_cast<size_t>(i) * row_stride;
            P.draft = draft_rows[i];
            P.position = i;
            twd_rejection_uniforms(twd_splitmix64(base_seed + i), &P.u1, &P.u2);
        }
    }
    if (a.npos == 0)  // greedy, or no draft probabilities anywhere: sample-and-compare
        return twd_verify(sel, logits, vocab, rows, row_stride, params, base_seed, drafts, n_drafts,
                          result, stream);
    if (vocab == 0) return fail(TWD_E_INVALID, "vocab must be > 0");

    // target tokens for the positions without draft rows, the fallback and the bonus row
    const uint32_t used = (rows > k) ? k + 1 : k;
    twd_row_params rp[TWD_MAX_ROWS + 1];
    for (uint32_t i = 0; i < used; ++i) {
        rp[i] = *params;
        rp[i].repetition_penalty = 1.0f;
        rp[i].history_len = 0;
        rp[i].uniform = twd_uniform_from_seed(twd_splitmix64(base_seed + i));
    }
    int rc = launch_select(sel->scratch, const_cast<float*>(logits), vocab, used, row_stride, rp,
                           nullptr, sel->scratch.verify_tokens, s);
    if (rc) return rc;

    if ((rc = draft_scratch_reserve(&sel->draft, vocab, a.npos))) return rc;
    a.vocab = vocab;
    a.parts = (vocab + kDraftChunk - 1) / kDraftChunk;
    a.temp = params->temperature <= 0.0f ? 1.0f : params->temperature;
    a.drafts = drafts;
    a.part = sel->draft.part;
    a.e = sel->draft.e;
    a.flags = sel->draft.flags;
    a.rej = sel->draft.rej;
    const dim3 grid(a.parts, 2 * a.npos);
    draft_max_kernel<<<grid, kDraftThreads, 0, s>>>(a);
    draft_exp_kernel<<<grid, kDraftThreads, 0, s>>>(a);
    draft_reject_kernel<<<a.npos, kRejThreads, 0, s>>>(a);
    draft_finish_kernel<<<1, 64, 0, s>>>(sel->scratch.verify_tokens, used, drafts, n_drafts, has,
                                         a.rej, result);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

}  // extern "C"
