// Device code shared by the selection kernels (select.hip) and the draft verify (verify.hip):
// the block-level reductions, the exact top-`want` selection (block_top), steps 5-7 of
// sample_token (finish_sampled), the per-64-entry selection records of a row (the wave-record
// path) and the one-block-per-row merge that finishes sample_token from them. Every function
// here is the same code in both files, so a row gets the same token from either.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "exp_libm.h"
#include "twd_internal.h"

namespace twd {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxWaves = 16;
constexpr uint32_t kBins = 256;         // distance-from-max bins of block_top
constexpr uint32_t kReps = 8;           // histogram replicas: lane l counts into replica l % 8
constexpr uint32_t kGatherMax = 512;    // boundary-bin entries ranked directly
constexpr float kBinRange = 64.0f;      // widest span of values the bins resolve

// Shared memory: what every block needs (reductions, the row's shortlist and its sums)...
struct SelCommon {
    uint32_t misc[8];
    uint64_t red64[kMaxWaves];
    double redd[kMaxWaves];
    float redf[kMaxWaves];
    float redf2[kMaxWaves];
    uint32_t redu[kMaxWaves];
    uint64_t top[kMaxWant];     // selected ranks
    uint64_t sorted[kMaxWant];  // the same, in descending order
    alignas(16) double e[kMaxWant];  // exp(l - max) / total
    alignas(16) double q[kMaxWant];  // exp((l - max) / T), then the running sum
    double exp2_tbl[64];        // 2^(j/64), for the row sum's exponentials
    float gmax;
    double total;
    uint32_t flag;
};

// ... block_top's work space ...
struct TopScratch {
    uint32_t hist[kReps * kBins];  // radix digit histogram / replicated bin histogram [bin][rep]
    uint64_t gath[kGatherMax];     // the boundary bin's ranks
};

template <int NT>
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, SelCommon& c) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max_u64(v);
    if (lane == 0) c.red64[wave] = v;
    __syncthreads();
    uint64_t r = c.red64[0];
    for (int w = 1; w < NT / 64; ++w) r = c.red64[w] > r ? c.red64[w] : r;
    __syncthreads();
    return r;
}

template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, SelCommon& c) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_reduce(v, 0.0, [](double a, double b) { return a + b; });
    if (lane == 0) c.redd[wave] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < NT / 64; ++w) r += c.redd[w];
    __syncthreads();
    return r;
}

// One exchange for three block reductions: OR of the NaN flags, max and min (NaN-ignoring).
// kReuse false: the caller passes another barrier before c.redu/redf/redf2 are written again,
// so the trailing barrier that protects them is left out.
template <int NT, bool kReuse = true>
__device__ __forceinline__ void block_stats(uint32_t& flag, float& mx, float& mn, SelCommon& c) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    flag = wave_reduce(flag, 0u, [](uint32_t a, uint32_t b) { return a | b; });
    mx = wave_reduce(mx, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
    mn = wave_reduce(mn, INFINITY, [](float a, float b) { return fminf(a, b); });
    if (lane == 0) {
        c.redu[wave] = flag;
        c.redf[wave] = mx;
        c.redf2[wave] = mn;
    }
    __syncthreads();
    flag = 0;
    mx = -INFINITY;
    mn = INFINITY;
    for (int w = 0; w < NT / 64; ++w) {
        flag |= c.redu[w];
        mx = fmaxf(mx, c.redf[w]);
        mn = fminf(mn, c.redf2[w]);
    }
    if constexpr (kReuse) __syncthreads();
}

// The smallest rank T with exactly `want` of the block's ranks >= T (ranks are distinct; rank
// 0 marks an empty slot and is never selected while want <= number of real ranks). Radix
// descent over 8-bit digits from the top, stopping once a digit bin is taken whole.
// PER = 0: `per` entries per thread with a loop that is not unrolled (entries read from memory).
template <int NT, int PER, typename KeyAt>
__device__ __forceinline__ uint64_t block_select(KeyAt key_at, int per, uint32_t want, uint32_t* hist,
                                                 SelCommon& c) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t prefix = 0, mask = 0;
    uint32_t need = want;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += NT) hist[i] = 0;
        __syncthreads();
        // keys read from memory (the merge's overflow over whole candidate waves, where heavy
        // ties are the usual cause): one wave's keys into the digit histogram, and where every
        // counted key of the wave has the same digit, one atomic adds them all. Every lane of
        // the wave calls.
        auto count_key = [&](uint64_t k) {
            const bool live = k != 0 && (k & mask) == prefix;
            const uint32_t dg = static_cast<uint32_t>(k >> shift) & 255u;
            const uint64_t m = __ballot(live);
            if (m == 0) return;
            const int first = __ffsll(static_cast<long long>(m)) - 1;
            const uint32_t d0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(dg), first));
            if (__ballot(live && dg == d0) == m) {
                if (lane == first) atomicAdd(&hist[d0], static_cast<uint32_t>(__popcll(m)));
            } else if (live) {
                atomicAdd(&hist[dg], 1u);
            }
        };
        if constexpr (PER > 0) {  // keys in registers: a plain atomic per key
#pragma unroll
            for (int e = 0; e < PER; ++e) {
                if (e >= per) break;
                const uint64_t k = key_at(e);
                if (k != 0 && (k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
            }
        } else {
            // eight keys requested before any is counted: key_at may read memory
            constexpr int kB = 8;
            int e = 0;
            for (; e + kB <= per; e += kB) {
                uint64_t kk[kB];
#pragma unroll
                for (int j = 0; j < kB; ++j) kk[j] = key_at(e + j);
#pragma unroll
                for (int j = 0; j < kB; ++j) count_key(kk[j]);
            }
            for (; e < per; ++e) count_key(key_at(e));
        }
        __syncthreads();
        if (wave == 0) {
            uint32_t cc[4];
            uint32_t t = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                cc[j] = hist[4 * lane + j];
                t += cc[j];
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
                if (above < need && need <= above + cc[j]) {
                    c.misc[0] = 4 * lane + j;
                    c.misc[1] = above;
                    c.misc[2] = cc[j];
                }
                above += cc[j];
            }
        }
        __syncthreads();
        const uint32_t d = c.misc[0], above = c.misc[1], cnt = c.misc[2];
        need -= above;
        prefix |= static_cast<uint64_t>(d) << shift;
        mask |= 255ull << shift;
        if (cnt == need) break;
    }
    return prefix;
}

// Appends k (where pred holds) to dst through the shared counter, one atomic per wave: the
// wave's slots are reserved by its first active lane and handed out in lane order. Slots at
// or beyond cap are dropped (a guard: callers reserve exactly what they need).
__device__ __forceinline__ void wave_put(bool pred, uint64_t k, uint32_t* counter, uint64_t* dst,
                                         uint32_t cap) {
    const uint64_t mask = __ballot(pred);
    if (mask == 0) return;
    const int lane = threadIdx.x & 63;
    const int leader = __ffsll(static_cast<long long>(mask)) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(counter, static_cast<uint32_t>(__popcll(mask)));
    base = __builtin_amdgcn_readlane(base, leader);
    if (pred) {
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
        if (base + below < cap) dst[base + below] = k;
    }
}

// wave_put_n for pairs: item q goes to dst[at] and its companion to dst2[at], one slot for both.
template <uint32_t N, typename T, typename U>
__device__ __forceinline__ void wave_put_n2(const bool (&pred)[N], const T (&k)[N], const U (&k2)[N],
                                            uint32_t* counter, T* dst, U* dst2, uint32_t cap) {
    uint64_t mask[N];
    uint32_t total = 0;
#pragma unroll
    for (uint32_t q = 0; q < N; ++q) {
        mask[q] = __ballot(pred[q]);
        total += static_cast<uint32_t>(__popcll(mask[q]));
    }
    if (total == 0) return;
    const int lane = threadIdx.x & 63;
    const int leader = __ffsll(static_cast<long long>(__ballot(true))) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(counter, total);
    base = __builtin_amdgcn_readlane(base, leader);
#pragma unroll
    for (uint32_t q = 0; q < N; ++q) {
        if (pred[q]) {
            const uint32_t at = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask[q] >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask[q]), 0u));
            if (at < cap) {
                dst[at] = k[q];
                dst2[at] = k2[q];
            }
        }
        base += static_cast<uint32_t>(__popcll(mask[q]));
    }
}

// wave_put for N items per lane: one atomic reserves the wave's slots for all N, handed out in
// (item, lane) order.
template <uint32_t N, typename T>
__device__ __forceinline__ void wave_put_n(const bool (&pred)[N], const T (&k)[N], uint32_t* counter, T* dst,
                                           uint32_t cap) {
    uint64_t mask[N];
    uint32_t total = 0;
#pragma unroll
    for (uint32_t q = 0; q < N; ++q) {
        mask[q] = __ballot(pred[q]);
        total += static_cast<uint32_t>(__popcll(mask[q]));
    }
    if (total == 0) return;
    const int lane = threadIdx.x & 63;
    const int leader = __ffsll(static_cast<long long>(__ballot(true))) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(counter, total);
    base = __builtin_amdgcn_readlane(base, leader);
#pragma unroll
    for (uint32_t q = 0; q < N; ++q) {
        if (pred[q]) {
            const uint32_t at = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask[q] >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask[q]), 0u));
            if (at < cap) dst[at] = k[q];
        }
        base += static_cast<uint32_t>(__popcll(mask[q]));
    }
}

// The block's top-`want` ranks (value desc, index asc), appended to out[0..want) in no
// particular order; every thread returns once out is complete, with c.misc[4] holding how
// many were found (want, unless fewer entries carry a rank). Entry e < per (per <= PER, the
// same in every thread) of the calling thread has value val_at(e) and rank key_at(e) (0 = no
// entry); slow_key(e) gives the same rank for the radix fallback, from memory the compiler
// cannot keep in registers across its passes. mx / mn are the largest and smallest finite
// values among the entries. ts.hist must be zero on entry (cleared behind an earlier barrier).
//
// bin(v) = floor((mx - v) * 255 / min(mx - mn, kBinRange)), capped at 254, is monotone in v,
// so every entry of a bin nearer than the boundary bin bt outranks every entry of bt, which
// outranks every farther one. The boundary bin's entries are ranked against each other.
template <int NT, int PER, typename ValAt, typename KeyAt, typename SlowVal, typename SlowKey>
__device__ __forceinline__ void block_top(ValAt val_at, KeyAt key_at, SlowVal slow_val, SlowKey slow_key,
                                          int per, float mx, float mn, uint32_t want, uint64_t* out,
                                          TopScratch& ts, SelCommon& c) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float span = mx - mn;
    // 0: take every entry; 1: rank the gathered boundary bin; 2: radix inside the boundary bin;
    // 3: radix over the whole block
    int mode = 3;
    uint32_t bt = kBins, above = 0, nbt = 0;
    float scale = 0.0f;
    auto bin_of_value = [&](float x) -> uint32_t {
        const float dist = (mx - x) * scale;
        return dist < static_cast<float>(kBins - 2) ? static_cast<uint32_t>(dist) : kBins - 2;
    };
    // each entry's bin, computed once: 8 bits per entry, 0xFF for entries without a rank
    uint32_t bins[(PER + 3) / 4];
#pragma unroll
    for (int j = 0; j < (PER + 3) / 4; ++j) bins[j] = 0;
    auto bin_at = [&](int e) -> uint32_t { return (bins[e / 4] >> (8 * (e % 4))) & 0xFFu; };
    if (__builtin_isfinite(mx) && __builtin_isfinite(mn) && span > 0.0f) {
        scale = static_cast<float>(kBins - 1) / (span < kBinRange ? span : kBinRange);
        const uint32_t rep = lane & (kReps - 1);
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            if (e >= per) break;
            if (key_at(e) != 0) {
                const uint32_t b = bin_of_value(val_at(e));
                atomicAdd(&ts.hist[b * kReps + rep], 1u);
                bins[e / 4] |= b << (8 * (e % 4));
            } else {
                bins[e / 4] |= 0xFFu << (8 * (e % 4));  // no rank: never gathered or taken
            }
        }
        __syncthreads();
        if (wave == 0) {  // lane l owns bins 4l .. 4l+3: their replicas are 32 consecutive words
            uint32_t cc[4], t = 0;
            const u32x4* h4 = reinterpret_cast<const u32x4*>(ts.hist) + lane * (4 * kReps / 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 a = h4[2 * j], b2 = h4[2 * j + 1];
                cc[j] = a.x + a.y + a.z + a.w + b2.x + b2.y + b2.z + b2.w;
                t += cc[j];
            }
            const uint32_t x = wave_incl_scan_u32(t);  // over lanes <= lane
            uint32_t before = x - t;
            if (lane == 63) {
                c.misc[0] = kBins;  // no boundary: fewer ranked entries than want
                c.misc[3] = 0;
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (before < want && want <= before + cc[j]) {
                    c.misc[0] = 4 * lane + j;
                    c.misc[1] = before;
                    c.misc[2] = cc[j];
                }
                before += cc[j];
            }
        }
        __syncthreads();
        bt = c.misc[0];
        above = c.misc[1];
        nbt = c.misc[2];
        mode = (bt == kBins) ? 0 : (nbt <= kGatherMax ? 1 : 2);
    }

    uint64_t thr = 0;
    if (mode == 1) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            if (e >= per) break;
            const bool in_bt = bin_at(e) == bt;
            wave_put(in_bt, in_bt ? key_at(e) : 0ull, &c.misc[3], ts.gath, kGatherMax);
        }
    } else if (mode == 2) {
        auto key_in_bin = [&](int e) -> uint64_t {
            return bin_of_value(slow_val(e)) == bt ? slow_key(e) : 0ull;
        };
        thr = block_select<NT, PER>(key_in_bin, per, want - above, ts.hist, c);
    } else if (mode == 3) {
        thr = block_select<NT, PER>(slow_key, per, want, ts.hist, c);
    }
    if (tid == 0) c.misc[4] = 0;
    __syncthreads();
    // every entry that is taken whole, then (mode 1) the boundary bin's top `want - above`;
    // exactly `want` ranks are written
    if (mode == 0 || mode == 1) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            if (e >= per) break;
            const bool take = bin_at(e) < (mode == 0 ? kBins - 1 : bt);  // 0xFF: no rank
            wave_put(take, take ? key_at(e) : 0ull, &c.misc[4], out, want);
        }
    } else {
        for (int e = 0; e < per; ++e) {
            const uint64_t k = slow_key(e);
            bool take = k != 0;
            if (take && mode == 3) take = k >= thr;
            if (take && mode == 2) {
                const uint32_t b = bin_of_value(slow_val(e));
                take = b < bt || (b == bt && k >= thr);
            }
            wave_put(take, k, &c.misc[4], out, want);
        }
    }
    if (mode == 1) {
        const uint32_t need = want - above;
        for (uint32_t i0 = 0; i0 < nbt; i0 += NT) {  // the same trip count in every thread
            const uint32_t i = i0 + tid;
            uint64_t k = 0;
            uint32_t higher = need;
            if (i < nbt) {
                k = ts.gath[i];
                higher = 0;
                for (uint32_t j = 0; j < nbt; ++j) higher += ts.gath[j] > k ? 1u : 0u;
            }
            wave_put(higher < need, k, &c.misc[4], out, want);
        }
    }
    __syncthreads();
}

// c.sorted[0..n) = c.top[0..n) in descending order (ranks are distinct): each entry's
// position is the number of entries above it.
__device__ __forceinline__ void block_sort_desc(SelCommon& c, uint32_t n) {
    const int tid = threadIdx.x;
    if (static_cast<uint32_t>(tid) < n) {
        const uint64_t k = c.top[tid];
        uint32_t higher = 0;
        for (uint32_t j = 0; j < n; ++j) higher += c.top[j] > k ? 1u : 0u;
        c.sorted[higher] = k;
    }
    __syncthreads();
}

// Steps 5-7 of sample_token on the sorted shortlist c.sorted[0..want) (sampling.cpp:139-168).
// Every thread i < want computes its two terms as the reference does: e_i = exp(l_i - max) /
// total (top-p, at T = 1) and q_i = exp((l_i - max) / T); threads want .. want rounded up to
// kChunk write zeros, which leave a running sum unchanged. The two sequential double sums then
// run in reference order on two lanes of wave 0, one v_add per term for both: lane 0 forms the
// running sums acc_i of q (stored back), lane 1 the top-p running sum, kChunk terms at a time,
// until lane 1's sum reaches p (the cut). The sums of non-negative terms never decrease, so a
// chunk holds the cut exactly when its last sum reaches p: one compare per chunk, then the
// chunk's own compares find the term. Both lanes issue every instruction of a full wave, so
// the loop is held to the sums' adds, 16-byte LDS accesses and that one compare. denom is acc
// at the cut (the additions of the reference's denom loop), and the draw -- the first i < cut
// with acc_i >= u * denom, else cut - 1 -- is a ballot over the stored sums in wave 0. Needs
// want <= blockDim.x and c.e, c.q 16-byte aligned. gmax and total are the row's maximum and sum
// of exponentials, the same in every thread. The id is returned to the threads of wave 0
// (callers store it from thread 0).
constexpr uint32_t kFinishChunk = 16;  // terms per step of the sequential sums

// The two terms of shortlist entry i (rank k) as the reference forms them (sampling.cpp:145,157).
__device__ __forceinline__ void shortlist_terms(SelCommon& c, uint32_t i, uint64_t k, float gmax, double total,
                                                const twd_row_params& p) {
    const double mx = static_cast<double>(gmax);
    const double l = static_cast<double>(rank_value(k));
    c.e[i] = exp_libm(l - mx) / total;
    c.q[i] = exp_libm((l - mx) / static_cast<double>(p.temperature));
}

// Zero terms past the shortlist, up to the sums' next whole chunk: they leave a running sum
// unchanged.
__device__ __forceinline__ void shortlist_pad(SelCommon& c, uint32_t want) {
    const uint32_t tid = threadIdx.x;
    const uint32_t padded = (want + kFinishChunk - 1) & ~(kFinishChunk - 1);  // <= kMaxWant
    if (tid >= want && tid < padded) {
        c.e[tid] = 0.0;
        c.q[tid] = 0.0;
    }
}

// The row a shortlist was taken from: its (penalised) logits and maximum, for the reference's
// own row total when a top-p cut lies within that total's rounding of p.
struct RowSrc {
    const float* logits;
    uint32_t vocab;
    float gmax;
    uint32_t nterms;  // the shortlist entries known by rank (c.sorted); the rest have zero terms
};

// How far (relative) a top-p prefix formed with this build's row total may lie from the
// reference's. The reference adds the row's vocab exponentials one after another, and a
// recursive sum of n non-negative terms lies within (n - 1) 2^-53 of their exact sum (terms
// under half an ulp of the running sum are dropped, so the bound is reached on rows with long
// tails); this build's total (partial sums at most a few dozen additions deep, rescaled once or
// twice, table exponentials within 2 ulp) within 256 2^-53, and the prefixes' own additions (at
// most 256 per prefix, each term one division) within 512 2^-53. Doubled, with room to spare,
// for the margin the decisions keep.
__device__ __forceinline__ double total_tol(uint32_t vocab) {
    return static_cast<double>(vocab + 2048u) * 0x1p-52;
}

// The reference's row total (sampling.cpp:113-115): exp((double)l - max) over the row in index
// order, each term glibc's exp, added one after another. Wave 0 only (every lane calls): the
// lanes form kTotStep terms at a time into stage[0..kTotStep), with the next step's logits
// already requested, and lane 0 adds them in order, 16 LDS reads ahead of its additions. About
// 3.6 ms at V = 262,144 (the additions are one dependent chain): taken only for a top-p cut
// within total_tol of p.
constexpr uint32_t kTotStep = 512;
__device__ __forceinline__ double exact_row_total(const RowSrc& src, double* stage) {
    constexpr uint32_t kPer = kTotStep / 64;
    const int lane = threadIdx.x & 63;
    const double mx = static_cast<double>(src.gmax);
    auto fetch = [&](float (&x)[kPer], uint32_t i0) {
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t i = i0 + 64 * j + static_cast<uint32_t>(lane);
            x[j] = src.logits[i < src.vocab ? i : src.vocab - 1];
        }
    };
    float xn[kPer];
    fetch(xn, 0);
    double run = 0.0;
    for (uint32_t i0 = 0; i0 < src.vocab; i0 += kTotStep) {
        float x[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) x[j] = xn[j];
        if (i0 + kTotStep < src.vocab) fetch(xn, i0 + kTotStep);
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) {
            const uint32_t i = i0 + 64 * j + static_cast<uint32_t>(lane);
            stage[64 * j + lane] = i < src.vocab ? exp_libm(static_cast<double>(x[j]) - mx) : 0.0;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) {
            // all kTotStep in order (past the row they are +0, which leaves a sum >= +0
            // unchanged), 16 at a time, the next 16 requested before these are added
            double a[16], b[16];
#pragma unroll
            for (uint32_t j = 0; j < 16; ++j) a[j] = stage[j];
#pragma unroll 1
            for (uint32_t k = 0; k < kTotStep; k += 32) {
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j) b[j] = stage[k + 16 + j];
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j) run += a[j];
                if (k + 32 < kTotStep) {
#pragma unroll
                    for (uint32_t j = 0; j < 16; ++j) a[j] = stage[k + 32 + j];
                }
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j) run += b[j];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return readlane_f64(run, 0);
}

__device__ __forceinline__ uint32_t finish_sums(SelCommon& c, uint32_t want, const twd_row_params& p,
                                                const RowSrc& src);
__device__ __noinline__ uint32_t finish_sums_exact(SelCommon& c, uint32_t want, const twd_row_params& p,
                                                   const RowSrc& src);

// src.nterms <= want: only c.sorted[0..nterms) is known; the shortlist's other entries are ones
// whose two terms are 0 (they can be neither cut nor drawn), so zero terms stand in for them.
__device__ __forceinline__ uint32_t finish_sampled(SelCommon& c, uint32_t want, const twd_row_params& p,
                                                   double total, const RowSrc& src) {
    const uint32_t tid = threadIdx.x;
    if (tid < src.nterms) {
        shortlist_terms(c, tid, c.sorted[tid], src.gmax, total, p);
    } else if (tid < want) {
        c.e[tid] = 0.0;
        c.q[tid] = 0.0;
    }
    shortlist_pad(c, want);
    __syncthreads();
    return finish_sums(c, want, p, src);
}

// Steps 5-7 after the terms c.e[0..want), c.q[0..want) (zero-padded) have been published.
//
// First on wave 0 by parallel prefix sums: lane l sums terms 4l .. 4l + 3 in order (one term per
// lane for shortlists of up to 64), a wave scan adds the lanes' totals, so every prefix is formed
// by at most ten additions of non-negative terms, against up to 255 in the reference's running sum: the two differ by less than 3e-14 of
// the prefix. Each decision of steps 5-7 compares a prefix with a threshold (the top-p cut: the
// first running sum >= p; the draw: the first running sum of q >= u * the sum at the cut), and
// the prefixes never decrease, so a decision is the reference's whenever the prefixes on both
// sides of it lie further than kSumTol (relative) from its threshold, and for the top-p cut
// further than kSumTol + total_tol, since its terms are divided by this build's row total.
// Otherwise (a prefix that close, e.g. an exact tie) finish_sums_exact repeats steps 5-7 with the
// reference's additions.
constexpr double kSumTol = 0x1p-36;

// TPL terms per lane of wave 0: lane l holds terms TPL l .. TPL l + TPL - 1 and their running
// sums (TPL = 1 for shortlists of up to 64 terms: each prefix is then the scan's own value).
template <uint32_t TPL>
__device__ __forceinline__ uint32_t finish_sums_par(SelCommon& c, uint32_t want, const twd_row_params& p,
                                                    const RowSrc& src) {
    const int lane = threadIdx.x & 63;
    const uint32_t padded = (want + kFinishChunk - 1) & ~(kFinishChunk - 1);  // <= 64 * TPL
    const uint32_t i0 = TPL * static_cast<uint32_t>(lane);
    double pe[TPL], pq[TPL];
#pragma unroll
    for (uint32_t j = 0; j < TPL; ++j) pe[j] = pq[j] = 0.0;
    if (i0 < padded) {  // padded is a multiple of 16: the lane's terms all lie below it
#pragma unroll
        for (uint32_t j = 0; j < TPL; ++j) {
            pe[j] = c.e[i0 + j];
            pq[j] = c.q[i0 + j];
        }
    }
#pragma unroll
    for (uint32_t j = 1; j < TPL; ++j) {
        pe[j] = pe[j - 1] + pe[j];
        pq[j] = pq[j - 1] + pq[j];
    }
    const double se = wave_incl_scan_f64(pe[TPL - 1]), sq = wave_incl_scan_f64(pq[TPL - 1]);
    if constexpr (TPL == 1) {
        pe[0] = se;
        pq[0] = sq;
    } else {
        // the lanes below: wave_shr:1 (lane 0 takes 0)
        const double xe = dpp_move<0x138>(0.0, se), xq = dpp_move<0x138>(0.0, sq);
#pragma unroll
        for (uint32_t j = 0; j < TPL; ++j) {
            pe[j] = xe + pe[j];
            pq[j] = xq + pq[j];
        }
    }
    auto at = [&](const double (&a)[TPL], uint32_t i) {
        double v = a[0];
#pragma unroll
        for (uint32_t j = 1; j < TPL; ++j) v = (i % TPL) == j ? a[j] : v;
        return readlane_f64(v, static_cast<int>(i / TPL));
    };
    // the first index i < lim whose prefix reaches x, as (found, i)
    auto first = [&](const double (&a)[TPL], uint32_t lim, double x, uint32_t& i) -> bool {
        uint32_t hit = 0;
#pragma unroll
        for (uint32_t j = 0; j < TPL; ++j) hit |= (i0 + j < lim && a[j] >= x ? 1u : 0u) << j;
        const uint64_t lanes = __ballot(hit != 0);
        if (lanes == 0) return false;
        const int L = __ffsll(static_cast<long long>(lanes)) - 1;
        i = TPL * static_cast<uint32_t>(L) +
            static_cast<uint32_t>(__builtin_ctz(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(hit), L))));
        return true;
    };
    bool ok = true;
    uint32_t cut = want;
    if (p.top_p < 1.0f) {
        const double pp = static_cast<double>(p.top_p);
        const double tc = kSumTol + total_tol(src.vocab);
        uint32_t i = 0;
        if (first(pe, want, pp, i)) {
            cut = i + 1;
            ok = at(pe, i) >= pp * (1.0 + tc) && (i == 0 || at(pe, i - 1) < pp * (1.0 - tc));
        } else {
            ok = at(pe, want - 1) < pp * (1.0 - tc);
        }
    }
    if (p.top_k > 0 && cut > static_cast<uint32_t>(p.top_k)) cut = static_cast<uint32_t>(p.top_k);
    if (cut < 1) cut = 1;
    const double r = static_cast<double>(p.uniform) * at(pq, cut - 1);
    uint32_t pick = cut - 1;
    if (first(pq, cut, r, pick))
        ok = ok && at(pq, pick) >= r * (1.0 + kSumTol) && (pick == 0 || at(pq, pick - 1) < r * (1.0 - kSumTol));
    else
        ok = false;
    if (ok) return rank_index(c.sorted[pick]);
    return finish_sums_exact(c, want, p, src);
}

__device__ __forceinline__ uint32_t finish_sums(SelCommon& c, uint32_t want, const twd_row_params& p,
                                                const RowSrc& src) {
    if (threadIdx.x >= 64) return 0;
    return want <= 64 ? finish_sums_par<1>(c, want, p, src) : finish_sums_par<4>(c, want, p, src);
}

// Steps 5-7 with the reference's running sums: lanes 0 and 1 of wave 0 (every lane of it calls).
// When a prefix on either side of the top-p cut lies within total_tol of p, the terms are formed
// again with the reference's own row total (exact_row_total) and the sums repeated.
__device__ __noinline__ uint32_t finish_sums_exact(SelCommon& c, uint32_t want, const twd_row_params& p,
                                                   const RowSrc& src) {
    const int tid = threadIdx.x, lane = tid & 63;
    constexpr uint32_t kChunk = kFinishChunk;
    if (tid >= 64) return 0;
    const bool topp = p.top_p < 1.0f;
    const double pp = static_cast<double>(p.top_p);
    uint32_t cut = want;
    for (int pass = 0;; ++pass) {
        cut = want;
        if (lane < 2) {
            // lane 0 reads q and stores its running sums over q; lane 1 reads e and stores its own
            // over e, so that no store needs a branch
            double* srcv = lane == 0 ? c.q : c.e;
            double run = 0.0;
            auto load = [&](double (&x)[kChunk], uint32_t i0) {
                const double2* s2 = reinterpret_cast<const double2*>(srcv + i0);
#pragma unroll
                for (uint32_t j = 0; j < kChunk / 2; ++j) {
                    const double2 v = s2[j];
                    x[2 * j] = v.x;
                    x[2 * j + 1] = v.y;
                }
            };
            // the running sums of chunk i0, stored over its terms; true when it holds the cut
            auto step = [&](const double (&x)[kChunk], uint32_t i0) -> bool {
                double pre[kChunk];
#pragma unroll
                for (uint32_t j = 0; j < kChunk; ++j) {
                    run += x[j];
                    pre[j] = run;
                }
                double2* d2 = reinterpret_cast<double2*>(srcv + i0);
#pragma unroll
                for (uint32_t j = 0; j < kChunk / 2; ++j) d2[j] = make_double2(pre[2 * j], pre[2 * j + 1]);
                // lane 1's sums decide; past want they repeat the sum at want - 1
                if (!topp || __builtin_amdgcn_readlane(pre[kChunk - 1] >= pp ? 1u : 0u, 1) == 0) return false;
                uint32_t hit = 0;
#pragma unroll
                for (uint32_t j = 0; j < kChunk; ++j) hit |= (pre[j] >= pp ? 1u : 0u) << j;
                const uint32_t h1 = __builtin_amdgcn_readlane(hit, 1);
                cut = i0 + static_cast<uint32_t>(__builtin_ctz(h1)) + 1;  // h1 != 0: its top bit is set
                return true;
            };
            // two chunks in flight: the next chunk's terms are read before this chunk's sums are
            // stored (it lies at i0 + kChunk, below padded when i0 + kChunk < want)
            double xa[kChunk], xb[kChunk];
            load(xa, 0);
            for (uint32_t i0 = 0; i0 < want; i0 += 2 * kChunk) {
                if (i0 + kChunk < want) load(xb, i0 + kChunk);
                if (step(xa, i0) || i0 + kChunk >= want) break;
                if (i0 + 2 * kChunk < want) load(xa, i0 + 2 * kChunk);
                if (step(xb, i0 + kChunk)) break;
            }
        }
        cut = __builtin_amdgcn_readfirstlane(cut);
        if (!topp || pass > 0 || !src.logits) break;
        // c.e holds the top-p running sums up to the cut (all of them when there is none): the
        // one at the cut (when it reached p; a last sum below p gives the same cut, want, either
        // way) and the one before it decide
        const double tc = total_tol(src.vocab);
        const double hi = c.e[cut - 1], lo = cut >= 2 ? c.e[cut - 2] : 0.0;
        const bool near = (hi >= pp && hi <= pp * (1.0 + tc)) ||
                          (cut >= 2 && lo >= pp * (1.0 - tc) && lo <= pp * (1.0 + tc));
        if (!near) break;
        // c.e and c.q, adjacent, stage the terms (both are formed again below)
        static_assert(offsetof(SelCommon, q) == offsetof(SelCommon, e) + sizeof(SelCommon::e) &&
                          2 * kMaxWant >= kTotStep, "the exact total's stage spans e and q");
        const double total = exact_row_total(src, c.e);
        for (uint32_t i = static_cast<uint32_t>(lane); i < want; i += 64) {
            if (i < src.nterms) {
                shortlist_terms(c, i, c.sorted[i], src.gmax, total, p);
            } else {
                c.e[i] = 0.0;
                c.q[i] = 0.0;
            }
        }
        for (uint32_t i = want + static_cast<uint32_t>(lane); i < ((want + kChunk - 1) & ~(kChunk - 1)); i += 64) {
            c.e[i] = 0.0;
            c.q[i] = 0.0;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (p.top_k > 0 && cut > static_cast<uint32_t>(p.top_k)) cut = static_cast<uint32_t>(p.top_k);
    if (cut < 1) cut = 1;
    const double r = static_cast<double>(p.uniform) * c.q[cut - 1];  // r = u * denom
    uint32_t pick = cut - 1;  // the reference's fallback: the last survivor
    for (uint32_t i0 = 0; i0 < cut; i0 += 64) {
        const uint32_t i = i0 + static_cast<uint32_t>(lane);
        const uint64_t m = __ballot(i < cut && c.q[min(i, cut - 1)] >= r);
        if (m != 0) {
            pick = i0 + static_cast<uint32_t>(__ffsll(static_cast<long long>(m)) - 1);
            break;
        }
    }
    return rank_index(c.sorted[pick]);
}

// ---- the merge after the wave records: one block per row -------------------------------------------
//
// The records are one per 64 vocabulary entries of a row: the best rank (value desc, index asc)
// and the sum of exp(v - that value) in double, NaN when a NaN was seen. The head's sample mode
// publishes them, and so does the wave-record pass over logits in memory (wave_records_block).
// sample_merge_row finishes sample_token (sampling.cpp:92-169) per row:
//   * greedy rows take the best rank over the waves;
//   * the row max and the rescaled sum of exponentials come from the records (a NaN sum makes
//     the row degenerate, as the reference's NaN total does);
//   * the shortlist only needs the waves that can hold a top-`want` entry. The wave maxima are
//     binned by distance from the row max (256 bins, monotone in the value) and b* is the first
//     bin at which `want` maxima have been counted: `want` entries lie in bins <= b*, so the
//     want-th largest entry X does too, every top-`want` entry is in a bin <= b*, and it lives in
//     a wave whose maximum is in a bin <= b*. Only those waves' rows are read, and only entries
//     in bins <= b* are kept;
//   * the survivors are ranked exactly (by counting when they fit one per thread, else by
//     block_top; by a radix select over the candidate waves' rows in memory if they overflow
//     the LDS list), then steps 5-7 run on one wave from registers.
constexpr int kSmThreads = 1024;
constexpr uint32_t kSmPer = kSampleMaxWaves / kSmThreads;  // wave records per thread
constexpr uint32_t kSmCap = 2048;     // survivors kept in LDS
constexpr uint32_t kSmMaxCand = 2048; // candidate waves listed in LDS

// A sampled row's statistics from its wave records, and b*: the row max, the sum of
// exp(l - max) over the row, the binning of wave maxima by distance from the row max
// (block_top's monotone bins) and the first bin b* at which `want` wave maxima have been
// counted. Every top-`want` entry lies in a bin <= b*, in a wave whose maximum is in a bin
// <= b*. One block of kSmThreads threads; thread tid holds records tid + kSmThreads q in key /
// wsum (0 / 0.0 past the row's records) and receives their maxima in wm. t.hist must be zero
// and c.exp2_tbl loaded, both published by the barriers inside. `degenerate` (the same in every
// thread, which then return together) marks a row whose total is NaN or not > 0
// (sampling.cpp:116-118). Every caller runs this code, so rows finished by different kernels
// see the same max and total. With kTotal false the total is left to the caller (records_part,
// then the waves' sums in order after a barrier of its own), and a row max that is not finite
// marks the row degenerate here: the reference's total is then NaN (+inf - +inf, or -inf -
// -inf, in every term), and with a finite max it is at least exp(0) = 1.
struct RecStats {
    float gm;
    double total;
    float scale;   // bins per unit of distance from gm
    bool binned;   // false: every value in bin 0
    uint32_t bstar;
    bool degenerate;
    double dead;   // a record whose maximum lies further than this below gm holds no live entry
};

// sampling.cpp:145,157: an entry l with l - max below -746 and (l - max) / T below -746 has both
// terms 0 (exp(x) = 0 below -745.14): it adds nothing to any running sum and is never drawn
// (the draw's threshold u * denom lies below denom), so which such entries fill a shortlist
// cannot change the token. The distance below the row max past which an entry is so, for a row
// at temperature T > 0.
// A NaN or infinite temperature has none: its weights can be NaN (every one, or those of -inf
// entries), and then the draw falls back to the cut's last survivor, whose identity matters.
__device__ __forceinline__ double dead_distance(const twd_row_params& p) {
    const double t = static_cast<double>(p.temperature);
    if (!(t < INFINITY)) return -INFINITY;
    return -746.0 * (t > 1.0 ? t : 1.0);
}

__device__ __forceinline__ uint32_t rec_bin(const RecStats& r, float x) {
    if (!r.binned) return 0u;
    const float dist = (r.gm - x) * r.scale;
    return dist < static_cast<float>(kBins - 2) ? static_cast<uint32_t>(dist) : kBins - 2;
}

// The calling wave's share of the row's sum of exp(l - max): its records' sums rescaled to the
// row max gm, summed in the thread's record order and then over the wave (wave_reduce's
// tree); the waves' shares summed in wave order give the row total. A record adds nothing when
// its sum is 0 (no live entry, every entry -inf, or past the row's records). With a fixed
// reference ref (finite; every record's sum is of exp(v - ref)) the share is the records' sums,
// times exp(ref - gm) once.
template <uint32_t PER = kSmPer>
__device__ __forceinline__ double records_part(const double (&wsum)[PER], const float (&wm)[PER], float gm,
                                               float ref, const double* tbl) {
    double part = 0.0;
    if (ref == ref) {
#pragma unroll
        for (uint32_t q = 0; q < PER; ++q) part += wsum[q];
        part = wave_reduce(part, 0.0, [](double u, double v) { return u + v; });
        return part * exp_for_sum(static_cast<double>(ref) - static_cast<double>(gm), tbl);
    }
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q)
        if (wsum[q] != 0.0) {
            // exp_core is exp_for_sum's value on [-700, 0] without its special cases
            const double x = static_cast<double>(wm[q]) - static_cast<double>(gm);
            part += wsum[q] * (x >= -700.0 ? exp_core(x, tbl) : exp_for_sum(x, tbl));
        }
    return wave_reduce(part, 0.0, [](double u, double v) { return u + v; });
}

// The records as records_stats takes them: live[q] for a record that counts among the row's
// wave maxima, wm[q] its maximum (-inf otherwise), and `flag` set when a record saw a NaN.
template <bool kTotal = true, uint32_t PER = kSmPer>
// dead: records whose maximum lies further below the row max than this (dead_distance; -inf:
// none) are left out of the bins, so that b* and the candidates are those of the live entries.
__device__ __forceinline__ RecStats records_stats(const bool (&live)[PER], const float (&wm)[PER],
                                                  uint32_t flag, const double (&wsum)[PER], float ref, uint32_t want,
                                                  TopScratch& t, SelCommon& c, double dead = -INFINITY) {
    constexpr int NT = kSmThreads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    RecStats rs{};
    float gm = -INFINITY, mn = INFINITY;
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q) {
        gm = fmaxf(gm, wm[q]);
        if (live[q] && __builtin_isfinite(wm[q])) mn = fminf(mn, wm[q]);
    }
    // NaN seen, row max, smallest finite wave max; the histogram's barrier below comes before
    // any reuse of the exchange
    block_stats<NT, false>(flag, gm, mn, c);
    rs.gm = gm;
    if (flag != 0 || (!kTotal && !__builtin_isfinite(gm))) {  // a NaN term makes the total NaN
        rs.degenerate = true;
        return rs;
    }
    if constexpr (kTotal) {
        // the waves' partial sums cross the histogram's barrier below (block_sum_f64's order)
        const double part = records_part<PER>(wsum, wm, gm, ref, c.exp2_tbl);
        if (lane == 0) c.redd[wave] = part;
    }

    // ---- b*: bins of distance from the row max (block_top's binning), 8 replicas
    const float span = gm - mn;
    rs.binned = __builtin_isfinite(gm) && __builtin_isfinite(mn) && span > 0.0f;
    rs.scale = rs.binned ? static_cast<float>(kBins - 1) / (span < kBinRange ? span : kBinRange) : 0.0f;
    rs.dead = dead;
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q)
        if (live[q] && !(static_cast<double>(wm[q]) - static_cast<double>(gm) < dead))
            atomicAdd(&t.hist[rec_bin(rs, wm[q]) * kReps + (lane & (kReps - 1))], 1u);
    __syncthreads();
    if constexpr (kTotal) {
        double total = 0.0;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) total += c.redd[w];
        rs.total = total;
        if (!(total > 0.0)) {  // every thread sums the same values
            rs.degenerate = true;
            return rs;
        }
    }
    if (wave == 0) {  // lane l owns bins 4l .. 4l + 3
        uint32_t cc[4], tsum = 0;
        const u32x4* h4 = reinterpret_cast<const u32x4*>(t.hist) + lane * (4 * kReps / 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 x = h4[2 * j], y = h4[2 * j + 1];
            cc[j] = x.x + x.y + x.z + x.w + y.x + y.y + y.z + y.w;
            tsum += cc[j];
        }
        uint32_t before = wave_incl_scan_u32(tsum) - tsum;
        if (lane == 63) c.misc[0] = kBins - 1;  // fewer maxima than want: every bin
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (before < want && want <= before + cc[j]) c.misc[0] = 4 * lane + j;
            before += cc[j];
        }
        if (lane == 0) {
            c.misc[3] = 0;  // candidate waves read whole
            c.misc[4] = 0;  // survivors
            c.misc[5] = 0;  // candidate waves with one survivor
        }
    }
    __syncthreads();
    rs.bstar = c.misc[0];
    return rs;
}

struct SampleMergeBufs {
    const float* logits;  // [rows][stride], penalised
    uint64_t stride;
    uint32_t vocab;
    uint32_t waves;       // head waves (records per row)
    SampleStats st;
    uint32_t* tokens;
};

struct SampleMergeShared {
    uint32_t cwave[kSmMaxCand];   // the candidate waves read whole
    uint16_t cwave1[kSmMaxCand];  // the candidate waves whose one survivor is their best rank
    alignas(16) uint64_t cand[kSmCap];  // surviving ranks
    uint64_t warm[32];           // sink of the loads that bring exp_libm's table into the caches
    TopScratch t;
    SelCommon c;
};

// One row of the merge after the wave records (select_sample_merge_kernel's block, kSmThreads
// threads): sample_token of row `row` with parameters p from its records and its penalised
// logits (see the kernel's comment). Every thread of the block calls it.
template <uint32_t PER>
__device__ __forceinline__ void sample_merge_row_per(const twd_row_params& p, uint32_t row, const SampleMergeBufs& b,
                                                     SampleMergeShared& sh) {
    constexpr int NT = kSmThreads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t W = b.waves;
    const size_t o = static_cast<size_t>(row) * W;
    const float* lg = b.logits + static_cast<size_t>(row) * b.stride;

    // the exp2 table first, so that its load overlaps the records' (the first barrier publishes it)
    if (tid < 64) sh.c.exp2_tbl[tid] = kExp2Table[tid];
    // ---- the wave records: thread tid holds waves tid + NT * q
    if (p.temperature <= 0.0f) {  // greedy (sampling.cpp:97; a NaN temperature samples): the best rank over the waves
        uint64_t key[PER];
#pragma unroll
        for (uint32_t q = 0; q < PER; ++q) {
            const uint32_t i = tid + NT * q;
            key[q] = i < W ? b.st.key[o + i] : 0ull;
        }
        uint64_t k = 0;
#pragma unroll
        for (uint32_t q = 0; q < PER; ++q) k = key[q] > k ? key[q] : k;
        k = block_max_u64<NT>(k, sh.c);
        if (tid == 0) b.tokens[row] = rank_index(k);
        return;
    }
    const uint32_t want = (p.top_k > 0) ? min(static_cast<uint32_t>(p.top_k), b.vocab)
                                        : min(kMaxWant, b.vocab);
    if (want > kMaxWant) return;  // a longer shortlist: the long path finishes the row
    // Sampled: the records' maxima first (4 bytes each: the row max, the bins and the
    // candidates need nothing else), then their sums, which arrive while the maxima are binned
    // and are first used by the row total. A record of the grid whose waves had no live entry
    // counts as a -inf maximum: -inf maxima land in the last bin, which every entry's bin is at
    // most, so they change neither b* nor the survivors, and their rows are past the vocabulary.
    float wm[PER];
    double wsum[PER];
    bool live[PER];
    uint32_t aux[PER];
    const bool have_aux = b.st.aux != nullptr;  // the records' words (else every candidate is read)
    const float ref = fixed_ref(b.st.cap, p);    // the records' sums' reference (NaN: each wave's max)
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q) {
        const uint32_t i = tid + NT * q;
        live[q] = i < W;
        wm[q] = live[q] ? b.st.max[o + i] : -INFINITY;
        aux[q] = (live[q] && have_aux) ? b.st.aux[o + i] : 0u;
    }
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q) {
        const uint32_t i = tid + NT * q;
        wsum[q] = i < W ? b.st.sum[o + i] : 0.0;
    }
    // one load per 64-byte line of exp_libm's table, in flight with the records': the finish's
    // exponentials then find it in the caches
    if (tid < 32) sh.warm[tid] = kExpTab[8 * tid];
    for (uint32_t i = tid; i < kReps * kBins; i += NT) sh.t.hist[i] = 0;
    uint32_t nan = 0;
#pragma unroll
    for (uint32_t q = 0; q < PER; ++q) nan |= wm[q] != wm[q] ? 1u : 0u;
    const RecStats rs = records_stats<false, PER>(live, wm, nan, wsum, ref, want, sh.t, sh.c, dead_distance(p));
    if (rs.degenerate) {  // sampling.cpp:116-118
        if (tid == 0) b.tokens[row] = TWD_TOKEN_DEGENERATE;
        return;
    }
    const float gm = rs.gm;
    const uint32_t bstar = rs.bstar;
    auto bin_of = [&](float x) -> uint32_t { return rec_bin(rs, x); };
    // The candidate waves, in any order. A record's entries other than its best two ranks rank
    // below its second, so they lie in bins at least the second's (the bins are monotone): a
    // candidate whose second (rounded up, which can only lower its bin) lies past b* holds one
    // survivor, its best rank, rebuilt here from the record's maximum and row; the others are
    // read whole below. Most rows of a short shortlist then read no logits at all.
    float smn = INFINITY;  // the survivors' smallest finite value
    {
        bool whole[PER], one[PER];
        uint32_t wid[PER];
        uint16_t wid1[PER];
        uint64_t bk[PER];
#pragma unroll
        for (uint32_t q = 0; q < PER; ++q) {
            const uint32_t w = tid + NT * q;
            const bool cand = live[q] && bin_of(wm[q]) <= bstar &&
                              !(static_cast<double>(wm[q]) - static_cast<double>(gm) < rs.dead);
            whole[q] = cand && (!have_aux || bin_of(fminf(aux_second(aux[q]), gm)) <= bstar);
            one[q] = cand && !whole[q];
            wid[q] = w;
            wid1[q] = static_cast<uint16_t>(w);  // w < kSampleMaxWaves
            bk[q] = rank_key(wm[q], w * kSampleWaveRows + (aux[q] & 63u));
            if (one[q] && __builtin_isfinite(wm[q])) smn = fminf(smn, wm[q]);
        }
        wave_put_n(whole, wid, &sh.c.misc[3], sh.cwave, kSmMaxCand);
        // the one-survivor waves' best ranks are the first survivors; cwave1[i] is cand[i]'s wave
        wave_put_n2(one, bk, wid1, &sh.c.misc[5], sh.cand, sh.cwave1, kSmMaxCand);
    }
    __syncthreads();
    const uint32_t ncw = sh.c.misc[3], ncw1 = sh.c.misc[5];
    // a candidate list this long only comes from values that barely bin (huge ties): the
    // two-launch path's kernels are not reachable from here, so rank over every wave, its
    // survivors listed afresh (each best rank is read again with the rest of its wave)
    const bool all_waves = ncw + ncw1 > kSmMaxCand;
    if (all_waves) smn = INFINITY;
    // the gathered survivors follow the best ranks already listed (counted in misc[4] from 0)
    const uint32_t first = all_waves ? 0u : ncw1;
    const uint32_t nent = all_waves ? W * kSampleWaveRows : ncw * kSampleWaveRows;  // entries to scan
    // every candidate wave's entries, for the overflow path: the whole ones, then the others
    const uint32_t nent_all = all_waves ? nent : (ncw + ncw1) * kSampleWaveRows;
    auto entry_row = [&](uint32_t f) -> uint32_t {
        const uint32_t s = f / kSampleWaveRows;
        const uint32_t w = all_waves ? s : (s < ncw ? sh.cwave[s] : static_cast<uint32_t>(sh.cwave1[s - ncw]));
        return w * kSampleWaveRows + f % kSampleWaveRows;
    };

    // ---- survivors: entries in bins <= b* of the waves read whole, kGatherBatch loads at a time
    constexpr uint32_t kGatherBatch = 8;
    const uint32_t per = (nent + NT - 1) / NT;
    float v[kGatherBatch];
    uint32_t r[kGatherBatch];
    // the batch's list reads first, then its loads back to back (an entry past the list or the
    // vocabulary loads entry 0 and is dropped)
    auto issue = [&](uint32_t i0) {
        uint32_t w[kGatherBatch];
#pragma unroll
        for (uint32_t q = 0; q < kGatherBatch; ++q) {
            const uint32_t f = (i0 + q) * NT + static_cast<uint32_t>(tid);
            const uint32_t slot = min(f / kSampleWaveRows, kSmMaxCand - 1);
            w[q] = all_waves ? f / kSampleWaveRows : sh.cwave[slot];
        }
#pragma unroll
        for (uint32_t q = 0; q < kGatherBatch; ++q) {
            const uint32_t f = (i0 + q) * NT + static_cast<uint32_t>(tid);
            const uint32_t rr = w[q] * kSampleWaveRows + f % kSampleWaveRows;
            const bool ok = i0 + q < per && f < nent && rr < b.vocab;
            r[q] = ok ? rr : 0xFFFFFFFFu;
            v[q] = lg[ok ? rr : 0u];
        }
    };
    auto consume = [&]() {
        bool keep[kGatherBatch];
        uint64_t kk[kGatherBatch];
#pragma unroll
        for (uint32_t q = 0; q < kGatherBatch; ++q) {
            keep[q] = r[q] != 0xFFFFFFFFu && bin_of(v[q]) <= bstar;
            if (keep[q] && __builtin_isfinite(v[q])) smn = fminf(smn, v[q]);
            kk[q] = keep[q] ? rank_key(v[q], r[q]) : 0ull;
        }
        wave_put_n(keep, kk, &sh.c.misc[4], sh.cand + first, kSmCap - first);
    };
    if (per > 0) issue(0);  // per is the same in every thread
    // the row total's terms while the first loads are in flight (the empty asm keeps the loads
    // ahead of them); the barrier below publishes the waves' shares
    __asm__ volatile("" ::: "memory");
    const double part = records_part<PER>(wsum, wm, gm, ref, sh.c.exp2_tbl);
    if (lane == 0) sh.c.redd[wave] = part;
    if (per > 0) consume();
    for (uint32_t i0 = kGatherBatch; i0 < per; i0 += kGatherBatch) {
        issue(i0);
        consume();
    }
    __syncthreads();                  // the survivors are listed
    double total = 0.0;               // block_sum_f64's order
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) total += sh.c.redd[w];
    if (!(total > 0.0)) {  // sampling.cpp:116-118; every thread sums the same values
        if (tid == 0) b.tokens[row] = TWD_TOKEN_DEGENERATE;
        return;
    }
    const uint32_t n = first + sh.c.misc[4];  // may exceed kSmCap: then only counted
    if (n > static_cast<uint32_t>(NT)) {  // block_top needs the survivors' smallest finite value
        uint32_t no_flag = 0;
        float no_max = -INFINITY;
        block_stats<NT>(no_flag, no_max, smn, sh.c);
    }

    // ---- the shortlist, sorted (value desc, index asc)
    if (n <= static_cast<uint32_t>(NT / 4)) {
        // four lanes per survivor, each counting the larger ranks over every fourth pair of the
        // list (pair reads may take the slot at n, past the survivors: it is not counted)
        const uint32_t sv = static_cast<uint32_t>(tid) >> 2, part = static_cast<uint32_t>(tid) & 3;
        const uint64_t k = sv < n ? sh.cand[sv] : 0ull;
        const ulonglong2* c2 = reinterpret_cast<const ulonglong2*>(sh.cand);
        uint32_t higher = 0;
        for (uint32_t pi = part; 2 * pi < n; pi += 4) {
            const ulonglong2 x = c2[pi];
            higher += x.x > k ? 1u : 0u;
            higher += (2 * pi + 1 < n && x.y > k) ? 1u : 0u;
        }
        higher += dpp_move<0xB1>(0u, higher);  // quad_perm [1,0,3,2]
        higher += dpp_move<0x4E>(0u, higher);  // quad_perm [2,3,0,1]
        // the survivor's place in the shortlist, and there its two terms: steps 5-7 then need
        // only the sums, after one barrier
        if (sv < n && part == 0 && higher < want) {
            sh.c.sorted[higher] = k;
            shortlist_terms(sh.c, higher, k, gm, total, p);
        }
        // fewer survivors than want only when the rest of the row is dead (dead_distance): zero
        // terms stand in for the dead entries that fill the reference's shortlist
        if (static_cast<uint32_t>(tid) >= n && static_cast<uint32_t>(tid) < want) {
            sh.c.e[tid] = 0.0;
            sh.c.q[tid] = 0.0;
        }
        shortlist_pad(sh.c, want);
        __syncthreads();
        const uint32_t tok = finish_sums(sh.c, want, p, RowSrc{lg, b.vocab, gm, min(n, want)});
        if (tid == 0) b.tokens[row] = tok;
        return;
    } else if (n <= static_cast<uint32_t>(NT)) {
        if (static_cast<uint32_t>(tid) < n) {
            const uint64_t k = sh.cand[tid];
            uint32_t higher = 0;
#pragma unroll 8
            for (uint32_t j = 0; j < n; ++j) higher += sh.cand[j] > k ? 1u : 0u;
            if (higher < want) sh.c.sorted[higher] = k;
        }
        __syncthreads();
    } else if (n <= kSmCap) {
        auto merge_key = [&](int e) -> uint64_t {
            const uint32_t f = tid + NT * e;
            return f < n ? sh.cand[f] : 0ull;
        };
        auto merge_val = [&](int e) -> float { return rank_value(merge_key(e)); };
        for (uint32_t i = tid; i < kReps * kBins; i += NT) sh.t.hist[i] = 0;
        __syncthreads();
        block_top<NT, kSmCap / NT>(merge_val, merge_key, merge_val, merge_key, static_cast<int>((n + NT - 1) / NT),
                                   gm, smn, want, sh.c.top, sh.t, sh.c);
        block_sort_desc(sh.c, want);
    } else {
        // overflow (heavy ties): a radix select over every candidate wave's rows in memory
        const uint32_t per_all = (nent_all + NT - 1) / NT;
        // branch-free, so that a batch's loads issue back to back: an index past the list or
        // the row reads a valid entry and is dropped
        auto cand_key = [&](int e) -> uint64_t {
            const uint32_t f = static_cast<uint32_t>(e) * NT + static_cast<uint32_t>(tid);
            const uint32_t rr = entry_row(f < nent_all ? f : nent_all - 1);
            const float x = lg[rr < b.vocab ? rr : b.vocab - 1];
            return (f < nent_all && rr < b.vocab && bin_of(x) <= bstar) ? rank_key(x, rr) : 0ull;
        };
        // Entries whose two terms, exp(l - max) and exp((l - max) / T), are both 0 can be neither
        // cut nor drawn (sampling.cpp:145,157: they add 0 to every running sum, and the draw's
        // threshold u * denom lies below denom). Which value is live is monotone in the value, so
        // when fewer than want entries are live they are the shortlist's first entries and zero
        // terms the rest, whichever tied entries fill it: a vocabulary masked to one value (-inf
        // or a large negative number) then needs one pass over the candidates, not a radix select
        // through every digit of the ties.
        {
            const double dead = dead_distance(p), dgm = static_cast<double>(gm);
            auto live_key = [&](uint32_t e) -> uint64_t {
                const uint64_t k = cand_key(static_cast<int>(e));
                if (k == 0) return 0ull;
                return static_cast<double>(rank_value(k)) - dgm < dead ? 0ull : k;
            };
            if (tid == 0) sh.c.misc[4] = 0;
            __syncthreads();
            uint32_t e = 0;
            for (; e + 8 <= per_all; e += 8) {  // eight rows requested before any is kept
                uint64_t kk[8];
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) kk[j] = live_key(e + j);
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) wave_put(kk[j] != 0, kk[j], &sh.c.misc[4], sh.c.top, want);
            }
            for (; e < per_all; ++e) {
                const uint64_t k = live_key(e);
                wave_put(k != 0, k, &sh.c.misc[4], sh.c.top, want);
            }
            __syncthreads();
            const uint32_t nlive = sh.c.misc[4];  // every live entry counted, at most want kept
            if (nlive < want) {
                block_sort_desc(sh.c, nlive);
                const uint32_t tok = finish_sampled(sh.c, want, p, total, RowSrc{lg, b.vocab, gm, nlive});
                if (tid == 0) b.tokens[row] = tok;
                return;
            }
        }
        const uint64_t thr = block_select<NT, 0>(cand_key, static_cast<int>(per_all), want, sh.t.hist, sh.c);
        if (tid == 0) sh.c.misc[4] = 0;
        __syncthreads();
        uint32_t e = 0;
        for (; e + 8 <= per_all; e += 8) {  // eight rows requested before any is kept
            uint64_t kk[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) kk[j] = cand_key(static_cast<int>(e + j));
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) wave_put(kk[j] != 0 && kk[j] >= thr, kk[j], &sh.c.misc[4], sh.c.top, want);
        }
        for (; e < per_all; ++e) {
            const uint64_t k = cand_key(static_cast<int>(e));
            wave_put(k != 0 && k >= thr, k, &sh.c.misc[4], sh.c.top, want);
        }
        __syncthreads();
        block_sort_desc(sh.c, want);
    }
    const uint32_t tok = finish_sampled(sh.c, want, p, total, RowSrc{lg, b.vocab, gm, want});
    if (tid == 0) b.tokens[row] = tok;
}

// One row of the merge: the records per thread sized to the row's record count, so that rows of
// at most 4,096 records (V <= 262,144) run no code for records that do not exist.
__device__ __forceinline__ void sample_merge_row(const twd_row_params& p, uint32_t row, const SampleMergeBufs& b,
                                                 SampleMergeShared& sh) {
    if (b.waves <= kSmThreads * (kSmPer / 2))
        sample_merge_row_per<kSmPer / 2>(p, row, b, sh);
    else
        sample_merge_row_per<kSmPer>(p, row, b, sh);
}

// ---- the wave records of logits in memory ------------------------------------------------------------
//
// Per 64 entries of a row, the record the head's sample mode publishes: the best rank (value
// desc, index asc) and the sum of exp(v - that value) in double, NaN when a NaN was seen. Eight
// lanes hold one record's 64 entries, eight each.
constexpr int kWsThreads = 256;
constexpr uint32_t kWsEntries = kWsThreads * 8;         // entries of one batch of a block

struct WaveStatsBufs {
    const float* logits;
    uint64_t stride;
    uint32_t vocab;
    uint32_t waves;  // records per row, ceil(vocab / 64)
    uint32_t vec;    // rows 16-byte aligned: 16 B loads
    SampleStats st;
};

// The records of one block of kWsThreads threads: row `row`, its NB * kWsEntries entries from
// chunk * NB * kWsEntries. tbl: 64 doubles of LDS for the exp table (loaded here, published by
// the barrier below). Every thread of the block calls it.
// AUX: also the record word (record_aux); without it the merge reads every candidate wave whole
// (b.st.aux is then null), which costs many-row launches less than forming the words.
template <uint32_t NB, bool AUX = true>
__device__ __forceinline__ void wave_records_block(const WaveStatsBufs& b, uint32_t chunk, uint32_t row,
                                                   double* tbl) {
    constexpr uint32_t kWsBatches = NB;
    constexpr uint32_t kWsBlockEntries = kWsEntries * NB;
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) tbl[tid] = kExp2Table[tid];
    const float* lg = b.logits + static_cast<size_t>(row) * b.stride;
    // batch k of this lane: entries e0 + 8 * 256 * k .. + 7; all loads requested at once
    const uint32_t e0 = chunk * kWsBlockEntries + static_cast<uint32_t>(tid) * 8;
    float v[kWsBatches][8];
#pragma unroll
    for (uint32_t k = 0; k < kWsBatches; ++k) {
        const uint32_t e = e0 + kWsEntries * k;
        if (b.vec && e + 8 <= b.vocab) {
            const float4 x0 = *reinterpret_cast<const float4*>(lg + e);
            const float4 x1 = *reinterpret_cast<const float4*>(lg + e + 4);
            v[k][0] = x0.x; v[k][1] = x0.y; v[k][2] = x0.z; v[k][3] = x0.w;
            v[k][4] = x1.x; v[k][5] = x1.y; v[k][6] = x1.z; v[k][7] = x1.w;
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[k][q] = e + q < b.vocab ? lg[e + q] : -INFINITY;
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < kWsBatches; ++k) {
        const uint32_t e = e0 + kWsEntries * k;
        // common case, decided per wave: every entry of the wave finite and live, and every
        // exp argument v - (record best) in [-700, 0]. The lane's best rank is its largest value
        // at its lowest index (equal values, -0 and +0 included, rank by index), and exp_core
        // needs no special cases.
        float hi = v[k][0], lo = v[k][0];
        bool ok = e + 8 <= b.vocab;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            ok &= __builtin_isfinite(v[k][q]);
            hi = fmaxf(hi, v[k][q]);
            lo = fminf(lo, v[k][q]);
        }
        if (__ballot(!ok) == 0) {
            uint32_t qi = 7;
#pragma unroll
            for (int q = 6; q >= 0; --q) qi = v[k][q] == hi ? static_cast<uint32_t>(q) : qi;
            // the lane's second value: the largest of its other entries (hi again if it repeats)
            float h2 = -INFINITY;
            if constexpr (AUX) {
#pragma unroll
                for (int q = 0; q < 8; ++q) h2 = static_cast<uint32_t>(q) != qi ? fmaxf(h2, v[k][q]) : h2;
            }
            uint64_t best = rank_key(hi, e + qi);
            float h1 = hi;
            // the record's 64 entries are the 8 lanes with the same lane >> 3: the best rank, and
            // the two largest values (a value held twice counts twice)
            auto step = [&](auto ctrl) {
                constexpr int C = decltype(ctrl)::value;
                const uint64_t ob = dpp_move<C>(best, best);
                best = ob > best ? ob : best;
                if constexpr (AUX) {
                    const float o1 = dpp_move<C>(h1, h1), o2 = dpp_move<C>(h2, h2);
                    h2 = fmaxf(fminf(h1, o1), fmaxf(h2, o2));
                    h1 = fmaxf(h1, o1);
                }
            };
            step(std::integral_constant<int, 0xB1>{});
            step(std::integral_constant<int, 0x4E>{});
            step(std::integral_constant<int, 0x141>{});
            const float wm = rank_value(best);
            if (__ballot(lo < wm - 700.0f) == 0) {
                const double dwm = static_cast<double>(wm);
                double sum = 0.0;
#pragma unroll
                for (int q = 0; q < 8; ++q) sum += exp_core(static_cast<double>(v[k][q]) - dwm, tbl);
#pragma unroll
                for (int m = 1; m < 8; m <<= 1) sum += __shfl_xor(sum, m);
                const uint32_t w = e / kSampleWaveRows;
                if ((lane & 7) == 0) {
                    const size_t o = static_cast<size_t>(row) * b.waves + w;
                    b.st.key[o] = best;
                    b.st.sum[o] = sum;
                    b.st.max[o] = wm;
                    if constexpr (AUX) b.st.aux[o] = record_aux_value(best, h2);
                }
                continue;
            }
        }
        // entries past the vocabulary hold -inf and no rank: they add nothing
        uint64_t best = 0, second = 0;
        uint32_t nan = 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            top2_insert(best, second, e + q < b.vocab ? rank_key(v[k][q], e + q) : 0ull);
            nan |= v[k][q] != v[k][q] ? 1u : 0u;
        }
        // the record's 64 entries are the 8 lanes with the same lane >> 3
        top2_step<0xB1>(best, second);
        top2_step<0x4E>(best, second);
        top2_step<0x141>(best, second);
        nan |= dpp_move<0xB1>(nan, nan);
        nan |= dpp_move<0x4E>(nan, nan);
        nan |= dpp_move<0x141>(nan, nan);
        // a record of -inf entries only (best value -inf, or no entry) adds nothing
        const float wm = best != 0 ? rank_value(best) : -INFINITY;
        const double dwm = wm != -INFINITY ? static_cast<double>(wm) : 0.0;
        double sum = 0.0;
#pragma unroll
        for (int q = 0; q < 8; ++q) sum += exp_for_sum(static_cast<double>(v[k][q]) - dwm, tbl);
        if (wm == -INFINITY) sum = 0.0;
#pragma unroll
        for (int m = 1; m < 8; m <<= 1) sum += __shfl_xor(sum, m);
        if (nan) sum = __builtin_nan("");
        const uint32_t w = e / kSampleWaveRows;
        if ((lane & 7) == 0 && w < b.waves) {
            const size_t o = static_cast<size_t>(row) * b.waves + w;
            b.st.key[o] = best;
            b.st.sum[o] = sum;
            b.st.max[o] = nan ? __builtin_nanf("") : wm;
            if constexpr (AUX) b.st.aux[o] = record_aux(best, second);
        }
    }
}


}  // namespace twd
