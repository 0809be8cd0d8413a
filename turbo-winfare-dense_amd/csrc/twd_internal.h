// Shared definitions of the gfx950 token-selection library: the HBM layout of the LM head, the
// orderable selection keys, small wave-level helpers and the error plumbing of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "twd_head.h"

namespace twd {

// ---- LM-head layout in HBM ---------------------------------------------------------------------
//
// The reference keeps the tied head as three row-major arrays [W | S | B]
// (src/runner.cpp:423-443). The kernels stream it as "units": one unit is 16 vocabulary rows x
// 128 columns (two 64-wide groups) and is 1152 contiguous bytes:
//
//   bytes [0, 1024)     64 lanes x 16 B of packed nibbles. Lane l = 16*kg + r holds row r of the
//                       tile and the four words 16U + 4t + kg (t = 0..3) of that row, i.e. the
//                       8 columns 128U + 32t + 8kg .. +7 for each of the four MFMA k-steps t.
//   bytes [1024, 1152)  16 rows x 8 B: two words, one per group g = 2U, 2U+1 of the row, each
//                       bf16 {b(g), t(g)} (low half b) with t = -128 * s(g), which is exact.
//
// Units are ordered [row tile T][chunk U], so a wave working through one row tile reads one
// contiguous 48 KB stripe, and every load instruction moves 1 KB (nibbles) or 128 B (scales)
// of contiguous memory. The total is exactly the reference's byte count: 3024 B per row.
// Storing t instead of s lets the word {b, t} serve directly as an MFMA operand for the group's
// bias term (b - 128 s) * X; s itself is t * (-1/128), folded into h ahead of time.
constexpr float kMaxScale = 0x1p100f;  // |s| above this is rejected at load (t would overflow)
constexpr uint32_t kGroup = 64;
constexpr uint32_t kChunkK = 128;
constexpr uint32_t kTileRows = 16;
constexpr uint32_t kUnitNibbleBytes = 1024;
constexpr uint32_t kUnitBytes = 1152;

// ---- selection -----------------------------------------------------------------------------------
constexpr uint32_t kMaxWant = TWD_MAX_WANT;

// Orderable 32-bit key of a float: larger float -> larger key, -0 folded into +0. NaN maps to 0
// (below -inf) so it never wins a comparison, except at index 0 where the reference's argmax
// returns 0 when logits[0] is NaN (every later '>' test against NaN fails, sampling.cpp:97-104).
__device__ __forceinline__ uint32_t float_key(float v) {
    v = v + 0.0f;  // -0 + 0 == +0 under round-to-nearest; +0 and every other value unchanged
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// 64-bit rank: value descending, then index ascending -- the total order of sample_token's
// shortlist comparator (sampling.cpp:128-131). Distinct indices make every rank distinct.
__device__ __forceinline__ uint64_t rank_key(float v, uint32_t idx) {
    uint32_t k = float_key(v);
    if (v != v) k = (idx == 0) ? 0xFFFFFFFFu : 0u;
    return (static_cast<uint64_t>(k) << 32) | static_cast<uint64_t>(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ uint32_t rank_index(uint64_t r) {
    return 0xFFFFFFFFu - static_cast<uint32_t>(r);
}

__device__ __forceinline__ float rank_value(uint64_t r) {
    return key_float(static_cast<uint32_t>(r >> 32));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), mask);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), mask);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One DPP move of a 32- or 64-bit value (a 64-bit one as two 32-bit moves): lanes of rows
// outside ROWS keep `old`.
template <int CTRL, int ROWS = 0xF, typename T>
__device__ __forceinline__ T dpp_move(T old, T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
    } else {
        const uint64_t o = __builtin_bit_cast(uint64_t, old), x = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            static_cast<int>(static_cast<uint32_t>(o)), static_cast<int>(static_cast<uint32_t>(x)), CTRL, ROWS, 0xF,
            false));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
            static_cast<int>(static_cast<uint32_t>(o >> 32)), static_cast<int>(static_cast<uint32_t>(x >> 32)), CTRL,
            ROWS, 0xF, false));
        return __builtin_bit_cast(T, (static_cast<uint64_t>(hi) << 32) | lo);
    }
}

// The two largest of a set of distinct ranks (0 stands for none). Merging another such pair
// keeps the larger first, and as second the larger of the smaller first and the larger second.
__device__ __forceinline__ void top2_merge(uint64_t& b1, uint64_t& b2, uint64_t o1, uint64_t o2) {
    const uint64_t lo = b1 < o1 ? b1 : o1;
    const uint64_t hi2 = b2 > o2 ? b2 : o2;
    b1 = b1 > o1 ? b1 : o1;
    b2 = lo > hi2 ? lo : hi2;
}

__device__ __forceinline__ void top2_insert(uint64_t& b1, uint64_t& b2, uint64_t k) { top2_merge(b1, b2, k, 0ull); }

// One exchange of a top-two reduction inside a DPP row, every lane active: CTRL pairs the lanes
// (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror), and both lanes of a pair
// end with the pair's merge (the pairs hold disjoint ranks).
template <int CTRL>
__device__ __forceinline__ void top2_step(uint64_t& b1, uint64_t& b2) {
    const uint64_t o1 = dpp_move<CTRL>(b1, b1), o2 = dpp_move<CTRL>(b2, b2);
    top2_merge(b1, b2, o1, o2);
}

// A record's second word: the best rank's row within the record's 64 (bits 0-5), and the
// second-best rank's value rounded up to bf16 (bits 16-31; -inf when there is none). Rounding up
// keeps the merge's test conservative: a second value whose bin lies past b* rounds to one that
// does too only when the exact one does.
// second: the second-best value (-inf when there is none).
__device__ __forceinline__ uint32_t record_aux_value(uint64_t best, float second) {
    const uint32_t b = __float_as_uint(second + 0.0f);  // -0 as +0
    const uint32_t t = b >> 16;                        // truncation: toward zero
    // toward +inf: a positive value with bits below the bf16 cut goes up one bf16 step
    uint32_t up = (second > 0.0f && (b & 0xFFFFu) != 0) ? t + 1 : t;
    if (second != second) up = 0x7FC0u;
    return (up << 16) | (rank_index(best) & 63u);
}

__device__ __forceinline__ uint32_t record_aux(uint64_t best, uint64_t second) {
    return record_aux_value(best, second != 0 ? rank_value(second) : -INFINITY);
}

__device__ __forceinline__ float aux_second(uint32_t aux) { return __uint_as_float(aux & 0xFFFF0000u); }

template <typename T>
__device__ __forceinline__ T readlane63(T v) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    } else {
        const uint64_t x = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(x)), 63));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(x >> 32)), 63));
        return __builtin_bit_cast(T, (static_cast<uint64_t>(hi) << 32) | lo);
    }
}

// Reduction of a full wave (every lane active) under an associative, commutative op, returned
// wave-uniform. Inside each row of 16 lanes: quad_perm [1,0,3,2] and [2,3,0,1], then
// row_half_mirror and row_mirror, after which every lane holds its row's value; row_bcast:15
// into rows 1 and 3 and row_bcast:31 into rows 2 and 3 leave the wave's value in lane 63. Each
// step is a register move, where a shuffle is an LDS round trip. For max, min and OR the
// result is the same as any other order; a floating-point sum is rounded in this tree's order.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, T ident, Op op) {
    v = op(v, dpp_move<0xB1>(ident, v));
    v = op(v, dpp_move<0x4E>(ident, v));
    v = op(v, dpp_move<0x141>(ident, v));
    v = op(v, dpp_move<0x140>(ident, v));
    v = op(v, dpp_move<0x142, 0xA>(ident, v));
    v = op(v, dpp_move<0x143, 0xC>(ident, v));
    return readlane63(v);
}

// Inclusive prefix sum over the lanes of a full wave (every lane active): row_shr:1, 2, 4, 8
// inside each row of 16 lanes (lanes without a source add 0), then row_bcast:15 adds row 0's
// total to row 1 and row 2's to row 3, and row_bcast:31 adds rows 0-1's total to rows 2 and 3.
// Register moves only, where a shuffle is an LDS round trip per step.
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x) {
    x += dpp_move<0x111>(0u, x);
    x += dpp_move<0x112>(0u, x);
    x += dpp_move<0x114>(0u, x);
    x += dpp_move<0x118>(0u, x);
    x += dpp_move<0x142, 0xA>(0u, x);
    x += dpp_move<0x143, 0xC>(0u, x);
    return x;
}

// The same inclusive prefix sum of doubles (each lane's value formed by at most six additions).
__device__ __forceinline__ double wave_incl_scan_f64(double x) {
    x += dpp_move<0x111>(0.0, x);
    x += dpp_move<0x112>(0.0, x);
    x += dpp_move<0x114>(0.0, x);
    x += dpp_move<0x118>(0.0, x);
    x += dpp_move<0x142, 0xA>(0.0, x);
    x += dpp_move<0x143, 0xC>(0.0, x);
    return x;
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
    const uint64_t x = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(x)), l));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(x >> 32)), l));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    return wave_reduce(v, uint64_t{0}, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}

// 2^(j/64), j = 0..63, each the double nearest the exact value: the table of exp_for_sum.
static __constant__ double kExp2Table[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

// exp(x) for the row sum, x = l - max <= 0 with l and max floats (so x is exact in double).
// Tang's table method: x = k ln2/64 + r with |r| <= ln2/128 (Cody-Waite split of ln2/64),
// exp(x) = 2^(k>>6) * 2^((k&63)/64) * e^r, e^r by its degree-5 Taylor polynomial (truncation
// below 4e-17 relative). tbl holds 2^(j/64), j = 0..63. Within 2 ulp; only the sum over the
// row uses it, whose summation order already differs from the reference's in the last bits.
__device__ __forceinline__ double exp_for_sum(double x, const double* tbl) {
    // branch-free: the polynomial runs on a safe argument, then NaN (+inf - +inf) stays NaN
    // and anything below -745.5 (also -inf) gives 0
    const bool nan = x != x, tiny = x < -745.5;
    const double xs = (nan || tiny) ? 0.0 : x;
    const double kInvL = 92.332482616893656;             // 64 / ln2
    const double kLHi = 6.93147180369123816490e-01 / 64;  // ln2 / 64, high part (exact products)
    const double kLLo = 1.90821492927058770002e-10 / 64;  // ln2 / 64, low part
    const double kd = __builtin_rint(xs * kInvL);
    const int k = static_cast<int>(kd);
    double r = fma(-kd, kLHi, xs);
    r = fma(-kd, kLLo, r);
    double p = fma(r, 1.0 / 120.0, 1.0 / 24.0);
    p = fma(r, p, 1.0 / 6.0);
    p = fma(r, p, 0.5);
    p = fma(r, p, 1.0);
    p = fma(r, p, 1.0);
    const double v = ldexp(tbl[k & 63] * p, k >> 6);
    return nan ? x : (tiny ? 0.0 : v);
}

// exp_for_sum without its special cases, for finite x in [-700, 0]: the same reduction,
// polynomial and table, so the same value there. k is read from the bits of fl(x * 64/ln2) +
// 1.5 * 2^52 (that addition rounds to the nearest integer, ties to even, as rint does) and
// 2^(k >> 6) is added to the table entry's exponent, which is exact because the result stays
// normal: no rint, conversion or ldexp instruction.
__device__ __forceinline__ double exp_core(double x, const double* tbl) {
#pragma clang fp contract(off)
    const double kInvL = 92.332482616893656;             // 64 / ln2
    const double kLHi = 6.93147180369123816490e-01 / 64;  // ln2 / 64, high part
    const double kLLo = 1.90821492927058770002e-10 / 64;  // ln2 / 64, low part
    const double kShift = 0x1.8p52;
    const double t = x * kInvL + kShift;  // two roundings, as rint(x * kInvL)
    const int k = static_cast<int>(static_cast<uint32_t>(__builtin_bit_cast(uint64_t, t)));
    const double kd = t - kShift;
    double r = fma(-kd, kLHi, x);
    r = fma(-kd, kLLo, r);
    double p = fma(r, 1.0 / 120.0, 1.0 / 24.0);
    p = fma(r, p, 1.0 / 6.0);
    p = fma(r, p, 0.5);
    p = fma(r, p, 1.0);
    p = fma(r, p, 1.0);
    const uint64_t tb = __builtin_bit_cast(uint64_t, tbl[k & 63]) +
                        (static_cast<uint64_t>(static_cast<int64_t>(k >> 6)) << 52);
    return __builtin_bit_cast(double, tb) * p;
}

// ---- which block of a launch arrives last ----------------------------------------------------
//
// Launches whose last block finishes the work (the head's greedy finish, the one-pass greedy
// selection, the draft verify's accept chain) count their blocks in on an arrival counter of
// kArriveWords uint64 words, each {arrivals (high 32 bits), epoch (low 32 bits)}. The host gives
// every launch an epoch (1 .. 2^31 - 1, never 0) and the next one's; a block adds 1 to the high
// half of a word, which never carries into the epoch, so every block of a launch sees the same
// epoch in a word until the launch's last block rewrites it.
//   * word 0, the eager word: armed {0, epoch} for the launch by the previous launch's last
//     block (or at allocation for the first). Every launch of a host thread's call sequence
//     finishes on it with one atomic add per block.
//   * words 1 .. kArriveSlots, the replay slots: a launch repeated with frozen arguments (a
//     captured graph replayed) carries an epoch that word 0 is no longer armed for. It counts in
//     on slot (epoch % kArriveSlots), which the previous launch of the same arguments armed with
//     its epoch; its last block re-arms the slot and takes this launch's adds back out of word 0,
//     leaving word 0 armed for the next eager launch.
//   * the last word, the fallback: a launch that finds neither armed for it (the first replay of
//     a captured launch, another capture's epoch in the slot, a count written from outside) counts
//     in by compare-and-swap with its epoch attached, starting afresh over any other epoch or a
//     count that already reached nb. Every failed swap means another block counted itself in, so
//     that loop ends after at most nb tries. Its last block arms word 0 for the next launch and
//     the slot for this launch's arguments.
// Every block of a launch takes the same word: the words' epochs do not change until all nb
// blocks have counted in, and a word's count is 0 when it is armed. Exactly one block returns
// true, after every other block of the launch has counted in.
constexpr uint32_t kArriveSlots = 4;
constexpr uint32_t kArriveWords = 2 + kArriveSlots;

// First epoch of a counter; allocation arms word 0 with it.
constexpr uint32_t kFirstEpoch = 1;
inline uint32_t epoch_after(uint32_t e) { return e % 0x7FFFFFFFu + 1u; }

__device__ __forceinline__ bool grid_arrive(unsigned long long* ctr, uint32_t nb, uint32_t epoch,
                                            uint32_t next_epoch) {
    constexpr unsigned long long kOne = 1ull << 32, kLo = 0xFFFFFFFFull;
    const unsigned long long ep = epoch;
    const unsigned long long o0 = __hip_atomic_fetch_add(ctr, kOne, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((o0 & kLo) == ep && (o0 >> 32) < nb) {
        const bool last = (o0 >> 32) == nb - 1;
        if (last)
            __hip_atomic_exchange(ctr, static_cast<unsigned long long>(next_epoch), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        return last;
    }
    unsigned long long* slot = ctr + 1 + epoch % kArriveSlots;
    const unsigned long long o1 = __hip_atomic_fetch_add(slot, kOne, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((o1 & kLo) == ep && (o1 >> 32) < nb) {
        const bool last = (o1 >> 32) == nb - 1;
        if (last) {  // every block has added to word 0 and the slot by now
            __hip_atomic_exchange(ctr, o0 & kLo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_exchange(slot, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return last;
    }
    unsigned long long* fb = ctr + 1 + kArriveSlots;
    unsigned long long cur = __hip_atomic_load(fb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), want;
    do {
        want = ((cur & kLo) == ep && (cur >> 32) < nb) ? cur + kOne : (ep | kOne);
    } while (!__hip_atomic_compare_exchange_strong(fb, &cur, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
    const bool last = (want >> 32) == nb;
    if (last) {  // every block has added to word 0 and the slot by now
        __hip_atomic_exchange(ctr, static_cast<unsigned long long>(next_epoch), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_exchange(slot, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return last;
}

// bf16 bit patterns <-> float
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// ---- error plumbing --------------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define TWD_HIP(call)                                  \
    do {                                               \
        hipError_t e_ = (call);                        \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

// ---- calls on several streams ------------------------------------------------------------------------
// An object whose calls share device state (a head's grid-finish state and staging buffers, a
// selector's scratch) orders them when they arrive on different streams: the first change of
// stream waits for the device once; from then on every call records an event on its stream and
// a call on another stream waits for that event first. Calls on one stream cost nothing extra.
// Not thread-safe: one host thread drives an object at a time, as the reference's runner does.
struct StreamOrder {
    hipStream_t last = nullptr;
    bool used = false;
    bool multi = false;
    hipEvent_t ev = nullptr;
};
int order_before(StreamOrder& o, hipStream_t s);  // before enqueueing work that uses the state
int order_after(StreamOrder& o, hipStream_t s);   // after enqueueing it
void order_release(StreamOrder& o);

// ---- the fused sample pass ------------------------------------------------------------------------
// The resident-h head kernel's sample mode publishes, per row m and wave w of the grid (index
// m * waves + w), the selection statistics of the wave's 64 vocabulary rows [64 w, 64 w + 64);
// select_sample_merge_kernel finishes the rows from them and the penalised logits.
struct SampleStats {
    uint64_t* key;  // best rank (value desc, index asc) of the wave's rows (0: none live)
    double* sum;    // sum of exp(v - best value) over them in double; NaN when a NaN was seen
    float* max;     // the best rank's value (-inf: none live, or every one -inf); NaN when a NaN
                    // was seen. The merge of a sampled row reads these 4 bytes per record first.
    uint32_t* aux;  // record_aux of the best two ranks, read with max
    // The head's softcap when its records were formed by the head's sample mode, NaN otherwise.
    // For a row whose values fixed_ref bounds (finite result), sum holds the sum of exp(v - ref)
    // against that fixed reference instead of the wave's max, so the row total is one
    // exponential times the sum of the records' sums.
    float cap;
};

// The fixed reference of a head row's record sums: a bound C >= |v| of every value the row can
// hold after the softcap (|cap tanh(x / cap)| <= cap) and the repetition penalty (whose clamp
// bounds the entries it changes by the row's softcap * 0.9999; without a clamp they are not
// bounded), when C <= kFixedRefMaxCap, so that exp(v - C) >= exp(-2 C) stays a normal double;
// NaN otherwise (the records are then summed against each wave's max).
constexpr float kFixedRefMaxCap = 300.0f;
__host__ __device__ inline float fixed_ref(float cap, const twd_row_params& p) {
    if (!(cap > 0.0f)) return __builtin_nanf("");
    float c = cap;
    if (p.repetition_penalty != 1.0f && p.history_len != 0) {
        if (!(p.softcap > 0.0f)) return __builtin_nanf("");
        const float lim = p.softcap * 0.9999f;
        c = lim > c ? lim : c;
    }
    return c <= kFixedRefMaxCap ? c : __builtin_nanf("");
}
constexpr uint32_t kSampleMaxWaves = 8192;  // waves a fused sample pass may have
constexpr uint32_t kSampleWaveRows = 64;    // vocabulary rows per wave

// Sort and finish buffers of the rows whose shortlist is longer than kMaxWant (top_k > 256),
// grown on demand by the calls that have such rows.
struct LongScratch {
    uint64_t* keys = nullptr;  // [rows][npad] ranks to sort
    double* pre = nullptr;     // [rows][npad] running sums of the temperature weights
    uint32_t* len = nullptr;   // [rows] sort length
    float* gmax = nullptr;     // [rows] row max
    double* total = nullptr;   // [rows] sum of exp(l - max)
    uint32_t rows_cap = 0;
    uint64_t npad_cap = 0;
};
void long_free(LongScratch* l);

// True for a row that the long path finishes: temperature > 0 and min(top_k, vocab) > kMaxWant.
inline bool long_row(const twd_row_params& p, uint32_t vocab) {
    return !(p.temperature <= 0.0f) && p.top_k > static_cast<int32_t>(kMaxWant) && vocab > kMaxWant;
}

// Enqueues the long path for those of `rows` rows that need it, after their penalised logits
// and wave records (`waves` per row, row stride of the records) are in place. `lng` may be
// null only when no row needs it.
int launch_long(LongScratch* lng, const SampleStats& st, uint32_t waves, const float* logits, uint64_t stride,
                uint32_t vocab, uint32_t rows, const twd_row_params* params, uint32_t* tokens,
                hipStream_t stream);

// Enqueues the merge after a sample-mode head pass over `rows` rows (params: host array), and
// the long path for rows with top_k > 256 (lng: their scratch).
int launch_sample_merge(const SampleStats& st, uint32_t waves, const float* logits, uint32_t vocab,
                        uint32_t rows, const twd_row_params* params, uint32_t* tokens,
                        LongScratch* lng, hipStream_t stream);

// ---- device scratch shared by the launch helpers ------------------------------------------------------
struct SelectScratch {
    uint32_t max_rows = 0;
    uint32_t max_parts = 0;
    float* part_max = nullptr;      // [rows][parts]
    double* part_sum = nullptr;     // [rows][parts]
    uint32_t* part_flag = nullptr;  // [rows][parts] bit0: NaN seen
    uint32_t* part_count = nullptr; // [rows][parts] candidates written
    uint64_t* part_key = nullptr;   // [rows][parts] greedy best rank
    uint64_t* cand = nullptr;       // [rows][parts][kMaxWant]
    uint32_t* verify_tokens = nullptr;  // [max_rows] scratch for twd_verify
    uint32_t wave_cap = 0;              // wave records per row (0: no wave-record path)
    uint64_t* wkey = nullptr;           // [rows][wave_cap] best rank per 64 entries
    double* wsum = nullptr;             // [rows][wave_cap] sum of exp(v - best value)
    float* wmax = nullptr;              // [rows][wave_cap] best value (NaN: a NaN seen)
    uint32_t* waux = nullptr;           // [rows][wave_cap] record_aux
    // one-pass greedy launches: per-row best ranks (zero between launches), the arrival counter
    // {arrivals, epoch} and its fallback word, and the host's epoch of the last such launch
    uint64_t* gbest = nullptr;          // [max_rows]
    uint64_t* gctr = nullptr;           // [kArriveWords]
    uint32_t* epoch = nullptr;          // host memory
    LongScratch* lng = nullptr;         // rows with top_k > 256 (null: not supported)
};

int scratch_alloc(SelectScratch* s, uint32_t max_vocab, uint32_t max_rows);
void scratch_free(SelectScratch* s);

// Scratch of the draft-logits verify, allocated on its first use by a selector.
struct DraftScratch {
    float* e = nullptr;        // [2 positions][vocab] expf(l / T - max)
    float* part = nullptr;     // [2 positions][parts] partial maxima
    uint32_t* flags = nullptr; // [2 * TWD_MAX_ROWS] NaN flags
    uint32_t* rej = nullptr;   // [TWD_MAX_ROWS][4] per-position outcome
    float* sums = nullptr;     // [2 * TWD_MAX_ROWS] softmax sums
    double* seg_d = nullptr;   // [2 * TWD_MAX_ROWS][segments + 1] double sums of the exact-sum pipeline
    void* seg_rec = nullptr;   // [2 * TWD_MAX_ROWS][segments] segment records
    void* seg_head = nullptr;  // [2 * TWD_MAX_ROWS] the serial heads' sums
    uint32_t* xin = nullptr;   // [2 positions][segments][128] the segments' crossing data
    uint32_t* live = nullptr;  // [TWD_MAX_ROWS] 1: the position's draft was rejected
    uint64_t* fin_ctr = nullptr;  // [2] the residual launch's arrival counter (epoch-armed)
    uint32_t fin_epoch = 0;       // the last call's epoch
    hipStream_t side = nullptr;  // twd_verify_draft's selection runs here, beside the draft chain
    hipEvent_t fork = nullptr, join = nullptr;
    size_t e_capacity = 0;
    size_t part_capacity = 0;
    size_t x_capacity = 0;
    uint32_t last_npos = 0;               // positions of the last call with draft rows
    uint32_t last_pos[TWD_MAX_ROWS] = {};
};

int draft_scratch_reserve(DraftScratch* d, uint32_t vocab, uint32_t npos);
// Gives the head a device copy of the final RMSNorm weight (bf16 [d]), freed with the head.
int head_set_norm_weight(twd_head* h, const uint16_t* host_w, uint32_t d);
void draft_scratch_free(DraftScratch* d);  // the buffers; the side stream stays
void draft_side_free(DraftScratch* d);     // the side stream and its events

// Enqueues penalty + selection over `rows` rows. `params` is a host array.
int launch_select(const SelectScratch& s, float* logits, uint32_t vocab, uint32_t rows,
                  uint64_t stride, const twd_row_params* params, const uint32_t* history,
                  uint32_t* tokens, hipStream_t stream, bool penalty_only = false);

// Greedy-verify bookkeeping over already selected per-row tokens (device).
int launch_verify_compare(const uint32_t* row_tokens, uint32_t rows, const uint32_t* drafts,
                          uint32_t n_drafts, twd_verify_result* result, hipStream_t stream);

}  // namespace twd

struct twd_selector;
namespace twd {
// twd_verify's launches, without the selector's stream ordering (callers that hold it already).
int verify_launches(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                    uint64_t row_stride, const twd_row_params* params, uint64_t base_seed,
                    const uint32_t* drafts, uint32_t n_drafts, twd_verify_result* result,
                    hipStream_t s);
// twd_verify_draft's launches, likewise.
int verify_draft_launches(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                          uint64_t row_stride, const float* const* draft_rows, uint32_t n_draft_rows,
                          const twd_row_params* params, uint64_t base_seed, const uint32_t* drafts,
                          uint32_t n_drafts, twd_verify_result* result, hipStream_t s);
}  // namespace twd

struct twd_selector {
    twd::StreamOrder order;
    twd::SelectScratch scratch;
    twd::DraftScratch draft;
    uint32_t max_vocab = 0;
};
