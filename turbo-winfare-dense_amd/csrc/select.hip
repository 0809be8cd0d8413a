// Token selection over device logit rows on gfx950: repetition penalty, greedy argmax and the
// sampled chain of sample_token (src/sampling.cpp:103-198), plus verify bookkeeping.
//
// select_slice_kernel covers all rows: grid (parts, rows), each block owns a 16384-entry slice
// of one row. Per block: penalty on the slice's history ids (occurrence counts in LDS, each
// applied one occurrence at a time like the reference loop), then either the greedy rank
// maximum or {slice max, sum exp(l - slice max) in double, the slice's top-`want` ranks by a
// radix select on 64-bit (value desc, index asc) ranks}. A row held by one slice finishes in
// the same block; otherwise select_merge_kernel (one block per row, second launch) merges the
// slices, sorts the global top-`want`, and runs top-p, top-k and the draw in reference order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "twd_internal.h"

namespace twd {

constexpr uint32_t kMaxParts = 32;  // vocab <= 32 * 16384 = 524288
constexpr uint32_t kMergePerThread = kMaxParts * kMaxWant / kSelThreads;  // 8
constexpr int kSelWaves = kSelThreads / 64;

struct SelectArgs {
    uint32_t rows;
    uint32_t parts;
    uint32_t penalty_only;  // stop after the repetition penalty
    twd_row_params p[TWD_MAX_ROWS + 1];  // verify samples up to K+1 rows
};

struct SelectBufs {
    float* logits;
    uint32_t vocab;
    uint64_t stride;
    const uint32_t* history;
    uint32_t* tokens;
    float* part_max;
    double* part_sum;
    uint32_t* part_flag;
    uint32_t* part_count;
    uint64_t* part_key;
    uint64_t* cand;
};

struct SelectShared {
    union {
        uint32_t cnt[kSlice];                 // penalty occurrence counts of the slice
        float val[kSlice];                    // then the slice's penalised values
        uint64_t cand[kMaxParts * kMaxWant];  // then, in the merge kernel, every slice's ranks
    } u;
    uint32_t hist[256];         // radix digit histogram
    uint32_t misc[8];
    uint64_t red64[kSelWaves];
    double redd[kSelWaves];
    float redf[kSelWaves];
    uint32_t redu[kSelWaves];
    uint64_t top[kMaxWant];     // selected ranks, sorted in place
    double e[kMaxWant];         // exp(l - max) / total
    double q[kMaxWant];         // exp((l - max) / T), then the running sum
    float gmax;
    double total;
    uint32_t flag;
};

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, SelectShared& sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max_u64(v);
    if (lane == 0) sh.red64[wave] = v;
    __syncthreads();
    uint64_t r = sh.red64[0];
    for (int w = 1; w < kSelWaves; ++w) r = sh.red64[w] > r ? sh.red64[w] : r;
    __syncthreads();
    return r;
}

__device__ __forceinline__ float block_max_f32(float v, SelectShared& sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float o = __shfl_xor(v, m);
        v = (v < o) ? o : v;
    }
    if (lane == 0) sh.redf[wave] = v;
    __syncthreads();
    float r = sh.redf[0];
    for (int w = 1; w < kSelWaves; ++w) r = (r < sh.redf[w]) ? sh.redf[w] : r;
    __syncthreads();
    return r;
}

__device__ __forceinline__ double block_sum_f64(double v, SelectShared& sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    if (lane == 0) sh.redd[wave] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < kSelWaves; ++w) r += sh.redd[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ uint32_t block_or_u32(uint32_t v, SelectShared& sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v |= __shfl_xor(v, m);
    if (lane == 0) sh.redu[wave] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int w = 0; w < kSelWaves; ++w) r |= sh.redu[w];
    __syncthreads();
    return r;
}

// The smallest rank T with exactly `want` of the block's ranks >= T (ranks are distinct; rank
// 0 marks an empty slot and is never selected while want <= number of real ranks). Radix
// descent over 8-bit digits from the top, stopping once a digit bin is taken whole.
template <typename KeyAt>
__device__ uint64_t block_select(uint32_t per_thread, KeyAt key_at, uint32_t want,
                                 SelectShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t prefix = 0, mask = 0;
    uint32_t need = want;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += kSelThreads) sh.hist[i] = 0;
        __syncthreads();
#pragma unroll 4
        for (uint32_t e = 0; e < per_thread; ++e) {
            const uint64_t k = key_at(e);
            if (k != 0 && (k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            uint32_t c[4];
            uint32_t t = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = sh.hist[4 * lane + j];
                t += c[j];
            }
            uint32_t x = t;  // inclusive suffix sum over lanes >= lane
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t y = __shfl_down(x, off);
                if (lane + off < 64) x += y;
            }
            uint32_t above = x - t;
#pragma unroll
            for (int j = 3; j >= 0; --j) {
                if (above < need && need <= above + c[j]) {
                    sh.misc[0] = 4 * lane + j;
                    sh.misc[1] = above;
                    sh.misc[2] = c[j];
                }
                above += c[j];
            }
        }
        __syncthreads();
        const uint32_t d = sh.misc[0], above = sh.misc[1], cnt = sh.misc[2];
        need -= above;
        prefix |= static_cast<uint64_t>(d) << shift;
        mask |= 255ull << shift;
        if (cnt == need) break;
    }
    return prefix;
}

// Bitonic sort of sh.top[0..n2) into descending order, n2 a power of two <= 256.
__device__ void block_sort_desc(SelectShared& sh, uint32_t n2) {
    const int tid = threadIdx.x;
    for (uint32_t k = 2; k <= n2; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            if (static_cast<uint32_t>(tid) < n2) {
                const uint32_t i = tid, x = i ^ j;
                if (x > i) {
                    const uint64_t a = sh.top[i], b = sh.top[x];
                    const bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) {
                        sh.top[i] = b;
                        sh.top[x] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Steps 5-7 of sample_token on the sorted shortlist sh.top[0..want) (sampling.cpp:168-197).
__device__ uint32_t finish_sampled(SelectShared& sh, uint32_t want, const twd_row_params& p) {
    const int tid = threadIdx.x;
    const double mx = static_cast<double>(sh.gmax);
    const double total = sh.total;
    const double td = static_cast<double>(p.temperature);
    if (static_cast<uint32_t>(tid) < want) {
        const double l = static_cast<double>(rank_value(sh.top[tid]));
        sh.e[tid] = exp(l - mx) / total;
        sh.q[tid] = exp((l - mx) / td);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t cut = want;
        if (p.top_p < 1.0f) {
            const double pp = static_cast<double>(p.top_p);
            double run = 0.0;
            for (uint32_t i = 0; i < want; ++i) {
                run += sh.e[i];
                if (run >= pp) {
                    cut = i + 1;
                    break;
                }
            }
        }
        if (p.top_k > 0 && cut > static_cast<uint32_t>(p.top_k)) cut = static_cast<uint32_t>(p.top_k);
        if (cut < 1) cut = 1;
        double denom = 0.0;
        for (uint32_t i = 0; i < cut; ++i) {
            denom += sh.q[i];
            sh.q[i] = denom;  // the running sums acc_i of the draw loop
        }
        const double r = static_cast<double>(p.uniform) * denom;
        uint32_t tok = rank_index(sh.top[cut - 1]);
        for (uint32_t i = 0; i < cut; ++i) {
            if (sh.q[i] >= r) {
                tok = rank_index(sh.top[i]);
                break;
            }
        }
        sh.misc[4] = tok;
    }
    __syncthreads();
    return sh.misc[4];
}

// After sh.top[0..want) holds the row's shortlist and sh.gmax/total/flag its statistics:
// the degenerate check of sampling.cpp:145-147, the shortlist sort, and steps 5-7.
__device__ void finish_row(SelectShared& sh, uint32_t want, const twd_row_params& p,
                           uint32_t* token_out) {
    const int tid = threadIdx.x;
    if (sh.flag != 0 || !(sh.total > 0.0)) {
        if (tid == 0) *token_out = TWD_TOKEN_DEGENERATE;
        return;
    }
    uint32_t n2 = 1;
    while (n2 < want) n2 <<= 1;
    if (static_cast<uint32_t>(tid) >= want && static_cast<uint32_t>(tid) < n2) sh.top[tid] = 0;
    __syncthreads();
    block_sort_desc(sh, n2);
    const uint32_t tok = finish_sampled(sh, want, p);
    if (tid == 0) *token_out = tok;
}

// SelectArgs is the first kernel argument, so it sits at offset 0 of the kernarg segment. The
// row's parameters are read through that pointer: indexing the by-value argument with
// blockIdx.y would make the compiler copy all of it into per-lane scratch memory.
__global__ __launch_bounds__(kSelThreads) void select_slice_kernel(SelectArgs args_by_value, SelectBufs b) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    SelectShared& sh = *reinterpret_cast<SelectShared*>(smem_raw);
#if __HIP_DEVICE_COMPILE__
    const SelectArgs& args =
        *reinterpret_cast<const SelectArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
#else
    const SelectArgs& args = args_by_value;  // the host pass only parses kernel bodies
#endif
    const int tid = threadIdx.x;
    const uint32_t part = blockIdx.x, row = blockIdx.y;
    const uint32_t parts = args.parts;
    const twd_row_params p = args.p[row];
    float* lg = b.logits + static_cast<size_t>(row) * b.stride;
    const uint32_t lo = part * kSlice;
    const uint32_t hi = min(b.vocab, lo + kSlice);

    float v[kSelPerThread];
#pragma unroll
    for (int e = 0; e < kSelPerThread; ++e) {
        const uint32_t i = lo + tid + kSelThreads * e;
        v[e] = i < hi ? lg[i] : 0.0f;
    }

    // ---- repetition penalty, sampling.cpp:103-119 ----
    if (p.repetition_penalty != 1.0f && p.history_len > 0) {
#pragma unroll
        for (int e = 0; e < kSelPerThread; ++e) sh.u.cnt[tid + kSelThreads * e] = 0;
        __syncthreads();
        const uint32_t* hist = b.history + p.history_offset;
        for (uint32_t j = tid; j < p.history_len; j += kSelThreads) {
            const uint32_t id = hist[j];
            if (id >= lo && id < hi) atomicAdd(&sh.u.cnt[id - lo], 1u);
        }
        __syncthreads();
        const float rp = p.repetition_penalty;
        const float limit = (p.softcap > 0.0f) ? p.softcap * 0.9999f : 0.0f;
#pragma unroll
        for (int e = 0; e < kSelPerThread; ++e) {
            const uint32_t n = sh.u.cnt[tid + kSelThreads * e];
            if (n == 0) continue;
            float x = v[e];
            for (uint32_t t = 0; t < n; ++t) {
                x = (x > 0.0f) ? (x / rp) : (x * rp);
                if (limit > 0.0f) {
                    const float lo_b = -limit;
                    x = (x < lo_b) ? lo_b : ((limit < x) ? limit : x);
                }
            }
            v[e] = x;
            lg[lo + tid + kSelThreads * e] = x;
        }
    }
    if (args.penalty_only) return;

    const bool greedy = !(p.temperature > 0.0f);
    if (greedy) {
        // ---- sampling.cpp:126-133 ----
        uint64_t k = 0;
#pragma unroll
        for (int e = 0; e < kSelPerThread; ++e) {
            const uint32_t i = lo + tid + kSelThreads * e;
            if (i < hi) {
                const uint64_t r = rank_key(v[e], i);
                k = r > k ? r : k;
            }
        }
        k = block_max_u64(k, sh);
        if (parts == 1) {
            if (tid == 0) b.tokens[row] = rank_index(k);
            return;
        }
        if (tid == 0) b.part_key[static_cast<size_t>(row) * parts + part] = k;
        return;
    }

    // ---- sampled: slice statistics, sampling.cpp:138-147 ----
    uint32_t nan_seen = 0;
    float mx = -INFINITY;
    bool any = false;
#pragma unroll
    for (int e = 0; e < kSelPerThread; ++e) {
        const uint32_t i = lo + tid + kSelThreads * e;
        if (i < hi) {
            if (v[e] != v[e]) nan_seen = 1;
            mx = any ? ((mx < v[e]) ? v[e] : mx) : v[e];
            any = true;
        }
    }
    __syncthreads();  // the penalty's counts are dead from here on: the region now holds values
#pragma unroll
    for (int e = 0; e < kSelPerThread; ++e) sh.u.val[tid + kSelThreads * e] = v[e];
    nan_seen = block_or_u32(nan_seen, sh);
    mx = block_max_f32(any ? mx : -INFINITY, sh);
    const double dmx = static_cast<double>(mx);
    double s = 0.0;
    const uint32_t n_here = hi - lo;
#pragma unroll 2
    for (uint32_t e = 0; e < kSelPerThread; ++e) {
        const uint32_t i = tid + kSelThreads * e;
        if (i < n_here) s += exp(static_cast<double>(sh.u.val[i]) - dmx);
    }
    s = block_sum_f64(s, sh);

    // ---- shortlist of this slice, sampling.cpp:149-166 ----
    const uint32_t want_row = (p.top_k > 0) ? min(static_cast<uint32_t>(p.top_k), b.vocab)
                                            : min(kMaxWant, b.vocab);
    const uint32_t want = min(want_row, n_here);
    auto local_key = [&](uint32_t e) -> uint64_t {
        const uint32_t i = tid + kSelThreads * e;
        return i < n_here ? rank_key(sh.u.val[i], lo + i) : 0ull;
    };
    const uint64_t thr = block_select(kSelPerThread, local_key, want, sh);
    if (tid == 0) sh.misc[3] = 0;
    __syncthreads();
    uint64_t* out = (parts == 1) ? sh.top : b.cand + (static_cast<size_t>(row) * parts + part) * kMaxWant;
#pragma unroll 4
    for (uint32_t e = 0; e < kSelPerThread; ++e) {
        const uint64_t k = local_key(e);
        if (k != 0 && k >= thr) {
            const uint32_t pos = atomicAdd(&sh.misc[3], 1u);
            if (pos < want) out[pos] = k;  // exactly `want` ranks pass; the bound is a guard
        }
    }

    if (parts > 1) {
        if (tid == 0) {
            const size_t o = static_cast<size_t>(row) * parts + part;
            b.part_max[o] = mx;
            b.part_sum[o] = s;
            b.part_flag[o] = nan_seen;
            b.part_count[o] = want;
        }
        return;  // select_merge_kernel finishes the row
    }
    if (tid == 0) {
        sh.gmax = mx;
        sh.total = s;
        sh.flag = nan_seen;
    }
    __syncthreads();
    finish_row(sh, want_row, p, b.tokens + row);
}

// Second launch when a row spans several slices: global max, the rescaled sum of exponentials,
// the global shortlist from every slice's candidates, then the draw. One block per row.
__global__ __launch_bounds__(kSelThreads) void select_merge_kernel(SelectArgs args_by_value, SelectBufs b) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    SelectShared& sh = *reinterpret_cast<SelectShared*>(smem_raw);
#if __HIP_DEVICE_COMPILE__
    const SelectArgs& args =
        *reinterpret_cast<const SelectArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
#else
    const SelectArgs& args = args_by_value;
#endif
    const int tid = threadIdx.x;
    const uint32_t row = blockIdx.x;
    const uint32_t parts = args.parts;
    const twd_row_params p = args.p[row];
    const size_t o = static_cast<size_t>(row) * parts;

    if (!(p.temperature > 0.0f)) {  // greedy: the best rank over the slices
        uint64_t m = 0;
        for (uint32_t q = tid; q < parts; q += kSelThreads) {
            const uint64_t x = b.part_key[o + q];
            m = x > m ? x : m;
        }
        m = block_max_u64(m, sh);
        if (tid == 0) b.tokens[row] = rank_index(m);
        return;
    }
    const uint32_t want_row = (p.top_k > 0) ? min(static_cast<uint32_t>(p.top_k), b.vocab)
                                            : min(kMaxWant, b.vocab);
    if (tid == 0) {
        float gm = b.part_max[o];
        uint32_t fl = b.part_flag[o];
        for (uint32_t q = 1; q < parts; ++q) {
            const float x = b.part_max[o + q];
            gm = (gm < x) ? x : gm;
            fl |= b.part_flag[o + q];
        }
        double tot = 0.0;
        for (uint32_t q = 0; q < parts; ++q)
            tot += b.part_sum[o + q] *
                   exp(static_cast<double>(b.part_max[o + q]) - static_cast<double>(gm));
        sh.gmax = gm;
        sh.total = tot;
        sh.flag = fl;
    }
    for (uint32_t f = tid; f < kMaxParts * kMaxWant; f += kSelThreads) {
        const uint32_t q = f / kMaxWant, slot = f % kMaxWant;
        uint64_t k = 0;
        if (q < parts && slot < b.part_count[o + q]) k = b.cand[(o + q) * kMaxWant + slot];
        sh.u.cand[f] = k;
    }
    __syncthreads();
    auto merge_key = [&](uint32_t e) -> uint64_t { return sh.u.cand[tid + kSelThreads * e]; };
    const uint64_t thr = block_select(kMergePerThread, merge_key, want_row, sh);
    if (tid == 0) sh.misc[3] = 0;
    __syncthreads();
#pragma unroll 4
    for (uint32_t e = 0; e < kMergePerThread; ++e) {
        const uint64_t k = merge_key(e);
        if (k != 0 && k >= thr) {
            const uint32_t pos = atomicAdd(&sh.misc[3], 1u);
            if (pos < want_row) sh.top[pos] = k;
        }
    }
    __syncthreads();
    finish_row(sh, want_row, p, b.tokens + row);
}

__global__ void verify_compare_kernel(const uint32_t* row_tokens, uint32_t rows,
                                      const uint32_t* drafts, uint32_t nd,
                                      twd_verify_result* v) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    uint32_t n = 0, acc = 0, bonus = 0, sampled = 0;
    bool bad = false;
    if (nd != 0 && rows != 0) {
        const uint32_t k = nd < rows ? nd : rows;
        bool rejected = false;
        for (uint32_t i = 0; i < k; ++i) {
            const uint32_t t = row_tokens[i];
            if (t == TWD_TOKEN_DEGENERATE) {
                bad = true;
                break;
            }
            if (drafts[i] == t) {
                v->tokens[n++] = t;
                ++acc;
            } else {
                bonus = t;
                sampled = 1;
                v->tokens[n++] = t;
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
    }
    v->n_tokens = bad ? TWD_TOKEN_DEGENERATE : n;
    v->num_accepted = acc;
    v->total_drafted = nd;
    v->bonus_token_sampled = sampled;
    v->bonus_token = bonus;
}

// ---- scratch and launch helpers ----------------------------------------------------------------

static uint32_t parts_for(uint32_t vocab) { return (vocab + kSlice - 1) / kSlice; }

int scratch_alloc(SelectScratch* s, uint32_t max_vocab, uint32_t max_rows) {
    s->max_rows = max_rows;
    s->max_parts = parts_for(max_vocab);
    const size_t n = static_cast<size_t>(max_rows) * s->max_parts;
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = hipMalloc(&s->part_max, n * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&s->part_sum, n * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&s->part_flag, n * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&s->part_count, n * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&s->part_key, n * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc(&s->cand, n * kMaxWant * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc(&s->verify_tokens, (max_rows + 1) * sizeof(uint32_t));
    if (e != hipSuccess) {
        scratch_free(s);
        return hip_fail(e, "allocating selection scratch");
    }
    return TWD_OK;
}

void scratch_free(SelectScratch* s) {
    (void)hipFree(s->part_max);
    (void)hipFree(s->part_sum);
    (void)hipFree(s->part_flag);
    (void)hipFree(s->part_count);
    (void)hipFree(s->part_key);
    (void)hipFree(s->cand);
    (void)hipFree(s->verify_tokens);
    *s = SelectScratch{};
}

int launch_select(const SelectScratch& s, float* logits, uint32_t vocab, uint32_t rows,
                  uint64_t stride, const twd_row_params* params, const uint32_t* history,
                  uint32_t* tokens, hipStream_t stream, bool penalty_only) {
    if (!logits || !params || (!tokens && !penalty_only))
        return fail(TWD_E_INVALID, "null logits, tokens or params");
    if (vocab == 0) return fail(TWD_E_INVALID, "sample_token: empty vocabulary");
    if (rows == 0 || rows > s.max_rows) return fail(TWD_E_INVALID, "rows out of range for this selector");
    const uint32_t parts = parts_for(vocab);
    if (parts > s.max_parts || parts > kMaxParts) return fail(TWD_E_INVALID, "vocab larger than this selector's max_vocab");
    if (stride < vocab) return fail(TWD_E_INVALID, "row_stride < vocab");
    SelectArgs a{};
    a.rows = rows;
    a.parts = parts;
    a.penalty_only = penalty_only ? 1u : 0u;
    for (uint32_t r = 0; r < rows; ++r) {
        const twd_row_params& p = params[r];
        if (p.temperature > 0.0f && p.top_k > static_cast<int32_t>(kMaxWant))
            return fail(TWD_E_UNSUPPORTED, "top_k > 256 is not supported on the device path (validate_sampling rejects it)");
        if (p.repetition_penalty != 1.0f && p.history_len > 0 && !history)
            return fail(TWD_E_INVALID, "null history with a non-empty history_len");
        a.p[r] = p;
    }
    SelectBufs b{};
    b.logits = logits;
    b.vocab = vocab;
    b.stride = stride;
    b.history = history;
    b.tokens = tokens;
    b.part_max = s.part_max;
    b.part_sum = s.part_sum;
    b.part_flag = s.part_flag;
    b.part_count = s.part_count;
    b.part_key = s.part_key;
    b.cand = s.cand;
    const size_t smem = sizeof(SelectShared);
    select_slice_kernel<<<dim3(parts, rows), kSelThreads, smem, stream>>>(a, b);
    TWD_HIP(hipGetLastError());
    if (parts > 1 && !penalty_only) {
        select_merge_kernel<<<rows, kSelThreads, smem, stream>>>(a, b);
        TWD_HIP(hipGetLastError());
    }
    return TWD_OK;
}

int launch_verify_compare(const uint32_t* row_tokens, uint32_t rows, const uint32_t* drafts,
                          uint32_t n_drafts, twd_verify_result* result, hipStream_t stream) {
    verify_compare_kernel<<<1, 64, 0, stream>>>(row_tokens, rows, drafts, n_drafts, result);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

}  // namespace twd

using namespace twd;

extern "C" {

TWD_API int twd_selector_create(uint32_t max_vocab, uint32_t max_rows, twd_selector** out) {
    clear_error();
    if (!out) return fail(TWD_E_INVALID, "null out");
    *out = nullptr;
    if (max_vocab == 0 || max_rows == 0 || max_rows > TWD_MAX_ROWS + 1)
        return fail(TWD_E_INVALID, "max_vocab must be > 0 and max_rows in 1..65");
    if (parts_for(max_vocab) > kMaxParts) return fail(TWD_E_UNSUPPORTED, "max_vocab above 1048576");
    static bool attr_done = false;
    if (!attr_done) {
        TWD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(select_slice_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(sizeof(SelectShared))));
        TWD_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(select_merge_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(sizeof(SelectShared))));
        attr_done = true;
    }
    twd_selector* s = new twd_selector();
    s->max_vocab = max_vocab;
    const int rc = scratch_alloc(&s->scratch, max_vocab, max_rows);
    if (rc) {
        delete s;
        return rc;
    }
    *out = s;
    return TWD_OK;
}

TWD_API void twd_selector_destroy(twd_selector* s) {
    if (!s) return;
    scratch_free(&s->scratch);
    delete s;
}

TWD_API int twd_select(twd_selector* sel, float* logits, uint32_t vocab, uint32_t rows,
                       uint64_t row_stride, const twd_row_params* params,
                       const uint32_t* history, uint32_t* tokens, void* stream) {
    clear_error();
    if (!sel) return fail(TWD_E_INVALID, "null selector");
    if (vocab > sel->max_vocab) return fail(TWD_E_INVALID, "vocab larger than this selector's max_vocab");
    return launch_select(sel->scratch, logits, vocab, rows, row_stride, params, history, tokens,
                         static_cast<hipStream_t>(stream));
}

TWD_API int twd_verify(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                       uint64_t row_stride, const twd_row_params* params, uint64_t base_seed,
                       const uint32_t* drafts, uint32_t n_drafts, twd_verify_result* result,
                       void* stream) {
    clear_error();
    if (!sel || !params || !result) return fail(TWD_E_INVALID, "null selector, params or result");
    if (n_drafts > 0 && !drafts) return fail(TWD_E_INVALID, "null drafts");
    if (n_drafts > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "n_drafts must be <= 64");
    if (rows > sel->scratch.max_rows) return fail(TWD_E_INVALID, "rows out of range for this selector");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_drafts == 0 || rows == 0)
        return launch_verify_compare(sel->scratch.verify_tokens, 0, drafts, n_drafts, result, s);
    // Only rows 0..min(n_drafts, rows) can be consulted; sample them all, as the reference
    // would on the path it takes.
    const uint32_t k = std::min(n_drafts, rows);
    const uint32_t used = (rows > k) ? k + 1 : k;
    twd_row_params rp[TWD_MAX_ROWS + 1];
    for (uint32_t i = 0; i < used; ++i) {
        rp[i] = *params;
        rp[i].repetition_penalty = 1.0f;
        rp[i].history_len = 0;
        rp[i].uniform = twd_uniform_from_seed(twd_splitmix64(base_seed + i));
    }
    // The selector only reads the rows (penalty is off), so the const cast does not write.
    int rc = launch_select(sel->scratch, const_cast<float*>(logits), vocab, used, row_stride, rp,
                           nullptr, sel->scratch.verify_tokens, s);
    if (rc) return rc;
    return launch_verify_compare(sel->scratch.verify_tokens, used, drafts, n_drafts, result, s);
}

}  // extern "C"
