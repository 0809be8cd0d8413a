// The tied INT4 group-64 LM head on gfx950: layout repack, synthetic generator, and the fused
// dequant-GEMM kernels (softcap, greedy argmax and greedy verify in their epilogue).
//
// Arithmetic (reference: shaders/Common.hlsli:163-222, src/cpu_reference.cpp:643-665):
//   logit[m][r] = sum_g s[r][g] * sum_{c in g} q[r][c] * h[m][c]  +  b[r][g] * X[m][g],
//   X[m][g] = sum_{c in g} h[m][c],  then softcap*tanh(logit/softcap).
// Both sums run on MFMA (v_mfma_f32_16x16x32_bf16) with fp32 accumulation and exact products:
//   * weights: a nibble pair becomes the exact bf16 values 128 + q with one and-or;
//   * h enters as -h/128 (exact), so one group's MFMA chain gives acc = -(128 X + sum q h)/128
//     and, with t = -128 s stored in the unit, t * acc = s * sum q h + 128 s X;
//   * the bias term (b - 128 s) X runs as a second MFMA stream: X is split into three bf16
//     slices hi + mid + lo (exact to fp32), paired against the stored word {b, t}, four groups
//     per K=32 MFMA.
// Per group and output element that leaves one fp32 FMA on the VALU: tot += t * acc.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <cstring>
#include <string>

#include "twd_internal.h"

namespace twd {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// greedy: also the grid-wide rank maximum; sample (M <= 8, resident-h kernel only): the
// repetition penalty in place and each wave's selection statistics
enum HeadMode { kModeLogits = 0, kModeGreedy = 1, kModeSample = 2 };

constexpr uint32_t kSampleRows = 8;  // rows of the sample mode: four apart up to 4, two apart up to 8

constexpr int kHeadThreads = 256;
constexpr int kHeadWaves = 4;

struct HeadArgs {
    const uint8_t* tiled;
    uint32_t ntiles, nunits;
    const uint16_t* h;
    uint32_t M, d;
    float softcap;
    float* logits;
    uint32_t vocab;
    // greedy finish: running per-row maxima (zero between launches), the arrival counter
    // {epoch, count} and this launch's epoch, and where the last block puts its results
    uint64_t* gbest;    // [TWD_MAX_ROWS]
    uint64_t* gctr;     // [kArriveWords]: grid_arrive's counter
    uint32_t epoch, next_epoch;
    uint32_t* tokens;
    const uint32_t* drafts;
    uint32_t n_drafts;
    twd_verify_result* vres;
    // 1: MFMA rows 8..15 hold the low halves of rows 0..7 (the fp32 h of the RMSNorm prologue
    // split into two bf16 parts); the epilogue adds them to their rows first
    uint32_t fold;
    // the RMSNorm prologue of the resident-h kernel: fp32 rows x [M][d], bf16 weight [d]
    const float* x;
    const uint16_t* norm_w;
    float eps;
    // sample mode: per row m, the penalty over history[hist_off[m], + hist_len[m]) (rp != 1)
    // clamped to +-clamp[m] (0.9999 softcap; 0: no clamp), and where each block's statistics go
    // (index m * gridDim.x + block)
    const uint32_t* history;
    uint32_t hist_off[kSampleRows], hist_len[kSampleRows];
    float rp[kSampleRows], clamp[kSampleRows];
    float ref[kSampleRows];  // fixed_ref of each row (NaN: its records are summed against each wave's max)
    SampleStats stats;
};

// speculator.cpp:46-69 and :138-150, greedy branch, over per-row target tokens tok[0..rows)
// (in LDS). Called by every lane of wave 0: lane i reads draft i, so the drafts cost one memory
// round trip, and a ballot finds the first mismatch. The reference's loop accepts drafts while
// they equal the target tokens and then emits the target token at the first mismatch (or, with
// every draft accepted and a row past them, that row's token as the bonus), so the emitted
// tokens are tok[0..n). n <= rows <= 64 (a bonus needs rows > the accepted count).
__device__ void verify_bookkeeping(const uint32_t* tok, uint32_t rows, const uint32_t* drafts,
                                   uint32_t nd, twd_verify_result* v) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t k = (nd != 0 && rows != 0) ? (nd < rows ? nd : rows) : 0u;  // <= 64
    const bool live = lane < k;
    const uint32_t d = live ? drafts[lane] : 0u;
    const uint32_t t = live ? tok[lane] : 0u;
    const uint64_t miss = __ballot(live && d != t);
    uint32_t n = 0, acc = 0, bonus = 0, sampled = 0;
    if (miss != 0) {
        acc = static_cast<uint32_t>(__ffsll(static_cast<long long>(miss)) - 1);
        n = acc + 1;
        bonus = tok[acc];
        sampled = 1;
    } else if (k != 0) {
        acc = k;
        n = k;
        if (rows > k) {
            bonus = tok[k];
            sampled = 1;
            n = k + 1;
        }
    }
    if (lane < n) v->tokens[lane] = tok[lane];
    if (lane == 0) {
        v->n_tokens = n;
        v->num_accepted = acc;
        v->total_drafted = nd;
        v->bonus_token_sampled = sampled;
        v->bonus_token = bonus;
    }
}

__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    if (f != f) return 0x7FC0u;
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// A VGPR holding c, opaque to constant folding. (w & mask) | c only becomes a single
// v_and_or_b32 when c sits in a register: a VOP3 op on this target encodes no literal.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
    return r;
}

// 8 nibbles of one word -> 8 bf16 values 128+q, in k-slot order [0,4,1,5,2,6,3,7]. magic holds
// 0x43004300 (bf16 128.0 twice).
__device__ __forceinline__ bf16x8_t nibbles_to_bf16(uint32_t w, uint32_t magic) {
    const uint32_t m = 0x000F000Fu;
    u32x4_t p;
    p.x = (w & m) | magic;
    p.y = ((w >> 4) & m) | magic;
    p.z = ((w >> 8) & m) | magic;
    p.w = ((w >> 12) & m) | magic;
    return __builtin_bit_cast(bf16x8_t, p);
}

// -h/128 of a bf16 pair, exact for every |h| >= 2^-119.
__device__ __forceinline__ uint32_t neg_over_128(uint32_t v) {
    const uint32_t lo = f32_to_bf16_rne(bf16_lo(v) * -0.0078125f);
    const uint32_t hi = f32_to_bf16_rne(bf16_hi(v) * -0.0078125f);
    return lo | (hi << 16);
}

// One 16-byte slice of h (8 bf16 values e0..e7) as an A-fragment entry: permuted into the
// nibbles' k-slot order and multiplied by -1/128.
__device__ __forceinline__ u32x4_t prep_h(u32x4_t v) {
    u32x4_t o;
    o.x = neg_over_128((v.x & 0xFFFFu) | (v.z << 16));
    o.y = neg_over_128((v.x >> 16) | (v.z & 0xFFFF0000u));
    o.z = neg_over_128((v.y & 0xFFFFu) | (v.w << 16));
    o.w = neg_over_128((v.y >> 16) | (v.w & 0xFFFF0000u));
    return o;
}

__device__ __forceinline__ float sum8_bf16(u32x4_t v) {
    float s = bf16_lo(v.x);
    s += bf16_hi(v.x);
    s += bf16_lo(v.y);
    s += bf16_hi(v.y);
    s += bf16_lo(v.z);
    s += bf16_hi(v.z);
    s += bf16_lo(v.w);
    s += bf16_hi(v.w);
    return s;
}

// The bias MFMA of one super-unit (two chunks, groups 4P + c, c = 0..3).
//   B fragment, lane (row r, k-group kg): the four {b, t} words of row r, one per group c,
//     the same for every kg -- i.e. the two units' scale words side by side.
//   A fragment, lane (row m, k-group kg): dword c = slice kg of X[m][4P + c], duplicated into
//     a bf16 pair, with X = hi + mid + lo (slices kg = 0, 1, 2; slice 3 is zero).
// Summed over k that is sum_c X_c * (b_c + t_c) = sum_c X_c * (b_c - 128 s_c).
// bias_slices writes the four slice dwords of one (m, group) entry; at(kg) addresses them.
template <typename At>
__device__ __forceinline__ void bias_slices(float x, At at) {
    const uint32_t hi = f32_to_bf16_rne(x);
    const float r1 = x - __uint_as_float(hi << 16);  // exact
    const uint32_t mid = f32_to_bf16_rne(r1);
    const float r2 = r1 - __uint_as_float(mid << 16);  // exact
    const uint32_t lo = f32_to_bf16_rne(r2);
    *at(0) = hi * 0x10001u;
    *at(1) = mid * 0x10001u;
    *at(2) = lo * 0x10001u;
    *at(3) = 0u;
}

// Shared memory of the head epilogue (cross-wave greedy reduction).
template <int NW>
struct EpiSharedT {
    uint64_t red[NW][TWD_MAX_ROWS];
    uint64_t seen[TWD_MAX_ROWS];
    uint32_t tok[TWD_MAX_ROWS];
    int last;
};
using EpiShared = EpiSharedT<kHeadWaves>;

// Softcap, logits store, and -- for the greedy modes -- the per-row rank maximum over the
// whole grid, finished by the last block to arrive (tokens, then greedy verify bookkeeping).
//
// Cross-block publication uses device-scope atomics only: each block folds its ranks into
// gbest[m] with a returning atomic max, then counts itself in on the arrival counter; the block
// that completes the count reads and clears gbest with atomic exchanges. Returning atomics are
// performed at the memory-side coherence point before they return, so every block's maxima
// precede its arrival, and the last block observes all of them. No data travels through plain
// stores, so no device-scope fence is needed: on this part such a fence writes back the XCD's
// L2 and, paid by each of ~1000 blocks, costs more than the streaming pass itself.
//
// Arrivals are counted by grid_arrive on gctr (an epoch per launch, armed by the previous
// launch's last block; replays of a captured launch count in on a replay slot, and only a launch
// that finds neither armed for it pays for contended compare-and-swap retries).
// tot[j][mt][i] holds row r = (tile0 + j) * 16 + lane % 16 of MFMA row 16 mt + 4 (lane / 16) + i,
// which carries h row m = (16 mt + 4 (lane / 16) + i) / MS when i is a multiple of MS (MS > 1:
// the rows are spread over the MFMA rows, see head_small_kernel); other entries are not outputs.
template <int NW>
__device__ __forceinline__ void grid_finish(const HeadArgs& a, EpiSharedT<NW>& se);

template <int NMT, int NI, int RT, int MODE, int NW, int MS = 1>
__device__ __forceinline__ void head_epilogue(const HeadArgs& a, f32x4_t (&tot)[RT][NMT],
                                              uint32_t tile0, EpiSharedT<NW>& se) {
    static_assert(MS == 1 || (NMT == 1 && NI == 4), "spread rows live in one m tile");
    if (NMT == 1 && a.fold) {  // rows r and r + 8 sit in lanes l and l + 32
#pragma unroll
        for (int j = 0; j < RT; ++j)
#pragma unroll
            for (int i = 0; i < NI; ++i) tot[j][0][i] += __shfl_xor(tot[j][0][i], 32);
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    uint64_t best[NMT][NI];
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int i = 0; i < NI; ++i) best[mt][i] = 0;

#pragma unroll
    for (int j = 0; j < RT; ++j) {
        const uint32_t r = (tile0 + j) * kTileRows + (lane & 15);
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
            for (int i = 0; i < NI; i += MS) {
                const uint32_t m = (mt * 16 + 4 * (lane >> 4) + i) / MS;
                float v = tot[j][mt][i];
                if (a.softcap > 0.0f) v = a.softcap * tanhf(v / a.softcap);
                const bool live = (m < a.M) && (r < a.vocab);
                if (live && a.logits) a.logits[static_cast<size_t>(m) * a.vocab + r] = v;
                if (MODE != kModeLogits) {
                    const uint64_t k = live ? rank_key(v, r) : 0ull;
                    best[mt][i] = k > best[mt][i] ? k : best[mt][i];
                }
            }
    }
    if (MODE == kModeLogits) return;

    // rows sharing m are the 16 lanes with the same lane >> 4, one DPP row: quad_perm [1,0,3,2]
    // and [2,3,0,1], row_half_mirror, row_mirror (register moves, where a shuffle is an LDS
    // round trip at the end of every wave)
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int i = 0; i < NI; i += MS) {
            uint64_t k = best[mt][i];
            auto step = [&](auto ctrl) {
                const uint64_t o = dpp_move<decltype(ctrl)::value>(k, k);
                k = o > k ? o : k;
            };
            step(std::integral_constant<int, 0xB1>{});
            step(std::integral_constant<int, 0x4E>{});
            step(std::integral_constant<int, 0x141>{});
            step(std::integral_constant<int, 0x140>{});
            const uint32_t m = (mt * 16 + 4 * (lane >> 4) + i) / MS;
            if ((lane & 15) == 0 && m < TWD_MAX_ROWS) se.red[wave][m] = k;
        }
    grid_finish<NW>(a, se);
}

// The greedy finish shared by the head kernels, once every wave has written its per-row maxima
// to se.red[wave][m]: the block's maxima go to gbest, the block counts itself in, and the last
// block of the launch writes the tokens (and the greedy verify bookkeeping).
template <int NW>
__device__ __forceinline__ void grid_finish(const HeadArgs& a, EpiSharedT<NW>& se) {
    const int tid = threadIdx.x;
    __syncthreads();
    const uint32_t nb = gridDim.x;
    if (static_cast<uint32_t>(tid) < a.M) {
        uint64_t k = se.red[0][tid];
#pragma unroll
        for (int w = 1; w < NW; ++w) k = se.red[w][tid] > k ? se.red[w][tid] : k;
        // the returning form: the maximum is performed before this block counts itself in
        se.seen[tid] = __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(a.gbest + tid),
                                              static_cast<unsigned long long>(k), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
        const bool last = grid_arrive(reinterpret_cast<unsigned long long*>(a.gctr), nb, a.epoch, a.next_epoch);
        se.last = last;
    }
    __syncthreads();
    if (!se.last) return;
    // every other block's maximum was performed before its arrival was counted
    if (static_cast<uint32_t>(tid) < a.M) {
        const uint64_t k = __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(a.gbest + tid),
                                                 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t t = rank_index(k);
        se.tok[tid] = t;
        if (a.tokens) a.tokens[tid] = t;
    }
    __syncthreads();
    if (tid < 64 && a.vres) verify_bookkeeping(se.tok, a.M, a.drafts, a.n_drafts, a.vres);
}

// Sample mode of the resident-h kernel. With rows spread four apart (MS = 4, M <= 4) row m's
// outputs are accumulator entry 0 of lanes 16m .. 16m + 15; two apart (MS = 2, M <= 8) rows 2g
// and 2g + 1 are entries 0 and 2 of lanes 16g .. 16g + 15. Per live entry: the softcap, then
// apply_repetition_penalty (sampling.cpp:74-90) with the entry's occurrence count from the
// block's LDS counts, one occurrence at a time (divide or multiply, then clamp), then the store.
// Each wave then publishes, per row, the statistics of its 64 vocabulary rows that
// select_sample_merge_kernel needs -- its best rank (value desc, index asc) and the sum of
// exp(v - that value) in double, NaN when the wave saw a NaN (the row is then degenerate, as a
// NaN makes the reference's total NaN) -- with no barrier and no cross-wave step. tbl holds
// 2^(j/64), j < 64, for exp_for_sum.
template <int RT, int NW, int MS>
__device__ __forceinline__ void head_epilogue_sample(const HeadArgs& a, f32x4_t (&tot)[RT][1],
                                                     uint32_t tile0, uint32_t block_row0,
                                                     const uint32_t* cnt, const double* tbl,
                                                     const float* prm) {
    constexpr uint32_t kRowsPerBlock = NW * RT * kTileRows;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int e = 0; e < 4 / MS; ++e) {  // entry MS * e: h row (4 (lane / 16) + MS * e) / MS
        const uint32_t m = (4 * (lane >> 4) + MS * e) / MS;
        const bool mlive = m < a.M;
        const uint32_t mm = mlive ? m : 0u;
        const float rp = prm[mm], lim = prm[kSampleRows + mm], ref = prm[2 * kSampleRows + mm];
        float v[RT];
        uint64_t best = 0, second = 0;
        uint32_t nan = 0;
#pragma unroll
        for (int j = 0; j < RT; ++j) {
            const uint32_t r = (tile0 + j) * kTileRows + (lane & 15);
            const bool live = mlive && r < a.vocab;
            float x = tot[j][0][MS * e];
            if (a.softcap > 0.0f) x = a.softcap * tanhf(x / a.softcap);
            if (live && rp != 1.0f) {
                const uint32_t n = cnt[mm * kRowsPerBlock + (r - block_row0)];
                for (uint32_t t = 0; t < n; ++t) {
                    x = (x > 0.0f) ? (x / rp) : (x * rp);
                    if (lim > 0.0f) x = (x < -lim) ? -lim : ((lim < x) ? lim : x);
                }
            }
            if (live) {
                a.logits[static_cast<size_t>(m) * a.vocab + r] = x;
                top2_insert(best, second, rank_key(x, r));
                if (x != x) nan = 1;
            }
            v[j] = live ? x : -INFINITY;
        }
        // the 16 lanes of a row, one DPP row: its two best ranks and the NaN flag
        top2_step<0xB1>(best, second);
        top2_step<0x4E>(best, second);
        top2_step<0x141>(best, second);
        top2_step<0x140>(best, second);
        nan |= dpp_move<0xB1>(nan, nan);
        nan |= dpp_move<0x4E>(nan, nan);
        nan |= dpp_move<0x141>(nan, nan);
        nan |= dpp_move<0x140>(nan, nan);
        // the wave's largest value (exact: the best rank's value, -0 read as +0); a wave of -inf
        // entries adds nothing to the row's sum
        const float wm = best != 0 ? rank_value(best) : -INFINITY;
        double sum = 0.0;
        if (wm != -INFINITY) {
            // the sum's reference: the row's fixed one (a bound of every value) or the wave's max
            const double dwm = static_cast<double>(ref == ref ? ref : wm);
            // exp_core where every argument of the lane is finite and in [-700, 0]: the value
            // exp_for_sum gives there, without its special cases
            bool core = true;
#pragma unroll
            for (int j = 0; j < RT; ++j)
                core = core && __builtin_isfinite(v[j]) && static_cast<double>(v[j]) - dwm >= -700.0;
            if (core) {
#pragma unroll
                for (int j = 0; j < RT; ++j) sum += exp_core(static_cast<double>(v[j]) - dwm, tbl);
            } else {
#pragma unroll
                for (int j = 0; j < RT; ++j) sum += exp_for_sum(static_cast<double>(v[j]) - dwm, tbl);
            }
        }
#pragma unroll
        for (int msk = 1; msk < 16; msk <<= 1) sum += __shfl_xor(sum, msk);
        if (nan) sum = __builtin_nan("");
        if ((lane & 15) == 0 && mlive) {
            const size_t o = static_cast<size_t>(m) * (gridDim.x * NW) + blockIdx.x * NW + (threadIdx.x >> 6);
            a.stats.key[o] = best;
            a.stats.sum[o] = sum;
            a.stats.max[o] = nan ? __builtin_nanf("") : wm;
            a.stats.aux[o] = record_aux(best, second);
        }
    }
}

// Weight streams: one buffer descriptor per row tile covering its stripe of units, so a unit
// load is one buffer_load with the unit offset in a scalar register and a fixed per-lane offset
// -- no per-lane address arithmetic in the streaming loop. Tiles past the end (tile0 is
// wave-uniform) re-read the last tile: their rows are >= vocab and never stored.
constexpr int kBufferWord3 = 0x00020000;  // descriptor word 3: 32-bit data format
constexpr int kNonTemporal = 2;           // cache-policy bit of a streaming load
constexpr int kWaitVm0 = 0x0F70;          // s_waitcnt vmcnt(0), other counters not waited on

template <int RT>
__device__ __forceinline__ void tile_streams(const HeadArgs& a, uint32_t tile0,
                                             __amdgpu_buffer_rsrc_t (&rs)[RT]) {
    const uint32_t stripe = a.nunits * kUnitBytes;
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        const uint32_t T = min(tile0 + j, a.ntiles - 1);
        rs[j] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.tiled) + static_cast<size_t>(T) * stripe,
                                                  0, static_cast<int>(stripe), kBufferWord3);
    }
}

// Unit U of the RT row tiles, in two halves: 16 B of nibbles per lane (lane offset lane * 16),
// and the 8 B {b, t} pair of the lane's row (lane offset 1024 + (lane % 16) * 8). Each half is
// issued in a fixed order and fenced from the surrounding code. A ring whose prologue and loop
// issue their loads in the same order lets the wait before each slot's first use count only
// that slot's loads; any other order makes the wait at the loop head cover the worst case of
// both.
template <int RT>
__device__ __forceinline__ void load_nibbles_ordered(const __amdgpu_buffer_rsrc_t (&rs)[RT], uint32_t U,
                                                     uint32_t vo_w, u32x4_t (&w)[RT]) {
    const int so = static_cast<int>(U * kUnitBytes);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        w[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs[j], vo_w, so, kNonTemporal));
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int RT>
__device__ __forceinline__ void load_scales_ordered(const __amdgpu_buffer_rsrc_t (&rs)[RT], uint32_t U,
                                                    uint32_t vo_s, u32x2_t (&sb)[RT]) {
    const int so = static_cast<int>(U * kUnitBytes);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        sb[j] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs[j], vo_s, so, kNonTemporal));
        __builtin_amdgcn_sched_barrier(0);
    }
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), in order.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// Wave index as a scalar: keeps tile and address arithmetic on the scalar unit.
__device__ __forceinline__ uint32_t wave_id() {
    return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// ---- M <= 8: the whole h resident in LDS, no barrier in the streaming loop ---------------------
//
// LDS holds the prepared h in A-fragment order, [m][chunk U][k-step t][kg] of 16 B, and the bias
// A-fragment entries [super-unit P][slice kg][m] of 16 B, both over npad = nunits rounded up to
// the ring depth PF; the chunks past nunits hold zeros, so the streaming loop runs whole ring
// cycles with no branch: its weight loads are clamped to the last unit, whose contribution the
// zero h and zero bias entries cancel exactly (the loader rejects infinite biases and scales
// above 2^100, so every product with those zeros is zero). A-fragment rows m >= M only feed
// output rows that are never stored, so their lanes simply read row 0. Each wave streams its
// RT row tiles through the PF-deep register ring with no synchronisation until the epilogue.
template <int PF>
__host__ __device__ constexpr uint32_t small_pad_units(uint32_t nunits) {
    return (nunits + PF - 1) / PF * PF;
}

//
// MS spreads the rows over the MFMA's 16 A rows: h row m sits in A row MS * m, so its outputs
// land in accumulator entry i = (MS * m) % 4 of the lanes with lane / 16 = MS * m / 4. With
// MS = 4 (M <= 4) every output is entry 0 and each group costs one scale FMA per accumulator
// instead of four; MS = 2 (M <= 8) uses entries 0 and 2. A rows that carry no h row read row 0;
// their outputs are never stored.
//
// NORM: the final RMSNorm as the prologue (M <= 4). Each block computes the rows' mean squares
// itself and stages h = (x * rms) * w, which is fp32, as two bf16 halves hi = bf16(h) and
// lo = bf16(h - hi) (|h - hi - lo| <= 2^-18 |h|) in LDS rows 2m and 2m + 1, fed as A rows 4m
// and 4m + 1; their outputs, entries 0 and 1 of one lane, are added before the softcap. The
// bias term uses the group sums of hi + lo (what the MFMA rows carry), on the hi rows only.
template <int MS, int RT, int PF, int NW, int MODE, bool NORM = false>
__global__ __launch_bounds__(NW * 64) void head_small_kernel(HeadArgs a) {
    static_assert(PF % 2 == 0, "the ring holds whole super-units");
    static_assert(MS == 2 || MS == 4, "rows spread over 16 MFMA rows with stride 2 or 4");
    static_assert(!NORM || MS == 4, "the RMSNorm prologue takes two MFMA rows per h row");
    constexpr int NT = NW * 64;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ EpiSharedT<NW> se;
    u32x4_t* sH = reinterpret_cast<u32x4_t*>(smem_raw);
    const uint32_t row_vecs = a.d / 8;  // 16 B vectors per h row
    const uint32_t npad = small_pad_units<PF>(a.nunits);
    const uint32_t pad_vecs = npad * 16;  // 16 B vectors per padded LDS row
    const uint32_t lrows = NORM ? 2 * a.M : a.M;  // LDS rows of prepared h
    u32x4_t* sXF = sH + lrows * pad_vecs;          // [super-units][4][lrows]
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t tile0 = (blockIdx.x * NW + wave_id()) * RT;
    const uint32_t magic = vgpr_const(0x43004300u);

    __amdgpu_buffer_rsrc_t rs[RT];
    tile_streams<RT>(a, tile0, rs);
    const uint32_t vo_w = lane * 16, vo_s = kUnitNibbleBytes + (lane & 15) * 8;
    const uint32_t last = a.nunits - 1;
    u32x4_t wq[PF][RT];
    u32x2_t sq[PF][RT];
    // sample mode: occurrence counts of the block's rows in each row's history (16 / MS rows)
    constexpr uint32_t kRowsPerBlock = NW * RT * kTileRows;
    constexpr uint32_t kCntRows = 16 / MS;
    __shared__ uint32_t cnt[MODE == kModeSample ? kCntRows * kRowsPerBlock : 1];
    __shared__ double exp2_tbl[MODE == kModeSample ? 64 : 1];
    // the rows' penalty factors and clamps, read per lane in the epilogue: staged here, where the
    // load overlaps the ring fill, instead of a memory round trip at the end of every block
    __shared__ float prm[MODE == kModeSample ? 3 * kSampleRows : 1];
    const uint32_t block_row0 = blockIdx.x * kRowsPerBlock;
    if constexpr (MODE == kModeSample) {
        for (uint32_t i = tid; i < kCntRows * kRowsPerBlock; i += NT) cnt[i] = 0;
        if (tid < 64) exp2_tbl[tid] = kExp2Table[tid];
        if (tid < static_cast<int>(kSampleRows)) {
            prm[tid] = a.rp[tid];
            prm[kSampleRows + tid] = a.clamp[tid];
            prm[2 * kSampleRows + tid] = a.ref[tid];
        }
    }
    // sample mode: the history's first batch (kHistBatch ids per thread of the first row with a
    // penalty) is requested first, so that its round trip overlaps the ring fill and the staging
    // of h
    constexpr int kHistBatch = 8;
    uint32_t hids[MODE == kModeSample ? kHistBatch : 1];
    uint32_t m_first = kSampleRows;
    if constexpr (MODE == kModeSample) {
        for (uint32_t m = 0; m < a.M; ++m)
            if (a.rp[m] != 1.0f && a.hist_len[m] != 0) {
                m_first = m;
                break;
            }
        if (m_first < a.M) {
            const uint32_t* hs = a.history + a.hist_off[m_first];
#pragma unroll
            for (int q = 0; q < kHistBatch; ++q) {
                const uint32_t j = tid + NT * q;
                hids[q] = j < a.hist_len[m_first] ? hs[j] : 0xFFFFFFFFu;
            }
        }
    }

    // The ring is filled before h is staged, so the two memory round trips overlap. Ring order,
    // the same in the prologue and in every cycle: per super-unit, the even unit's nibbles, then
    // its {b, t} words, then the odd unit's nibbles and words. The even unit's words are refilled
    // only after the odd step's bias MFMA has read them, so the bias fragment needs no copy that
    // outlives the refill.
#pragma unroll
    for (int s = 0; s < PF; ++s) {
        const uint32_t U = min(static_cast<uint32_t>(s), last);
        load_nibbles_ordered<RT>(rs, U, vo_w, wq[s]);
        load_scales_ordered<RT>(rs, U, vo_s, sq[s]);
    }

    // ---- stage h: 8 consecutive threads cover one 64-column group; padding chunks get zeros.
    // Each thread issues kBatch loads before it waits, so a block pays about one round trip per
    // kBatch * NT vectors.
    constexpr int kBatch = 4;
    const uint32_t tasks = a.M * pad_vecs;
    // NORM: the per-row scale 1 / sqrt(mean(x^2) + eps) is common to every term of a row's
    // logit, so h' = x * w is staged and the sum is scaled once in the epilogue; the mean
    // squares are gathered from the same loads (partial sums per wave in ss_red).
    __shared__ float ss_red[NORM ? NW : 1][4];
    if constexpr (NORM) {
        // row by row, so each thread's square sum belongs to one row; one vector per thread in
        // flight (its temporaries share the registers with the filled weight ring: two would
        // cost a wave per SIMD)
        constexpr int kBatchN = 1;
        uint32_t* xo = reinterpret_cast<uint32_t*>(sXF);
        for (uint32_t m = 0; m < a.M; ++m) {
            const float* xrow = a.x + static_cast<size_t>(m) * a.d;
            float ssm = 0.0f;
            for (uint32_t base = 0; base < pad_vecs; base += NT * kBatchN) {
                float4 x0[kBatchN], x1[kBatchN];
                u32x4_t wv[kBatchN];
#pragma unroll
                for (int b = 0; b < kBatchN; ++b) {
                    const uint32_t c8 = base + b * NT + tid;
                    x0[b] = x1[b] = float4{0.f, 0.f, 0.f, 0.f};
                    wv[b] = u32x4_t{0u, 0u, 0u, 0u};
                    if (c8 < row_vecs) {
                        x0[b] = *reinterpret_cast<const float4*>(xrow + c8 * 8);
                        x1[b] = *reinterpret_cast<const float4*>(xrow + c8 * 8 + 4);
                        wv[b] = *reinterpret_cast<const u32x4_t*>(a.norm_w + c8 * 8);
                    }
                }
#pragma unroll
                for (int b = 0; b < kBatchN; ++b) {
                    const uint32_t c8 = base + b * NT + tid;
                    const float xs[8] = {x0[b].x, x0[b].y, x0[b].z, x0[b].w, x1[b].x, x1[b].y, x1[b].z, x1[b].w};
                    const uint32_t ws[4] = {wv[b].x, wv[b].y, wv[b].z, wv[b].w};
                    uint32_t hi[8], lo[8];
                    float sum = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t wb = (ws[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                        const float he = xs[e] * __uint_as_float(wb << 16);  // x * weight
                        hi[e] = f32_to_bf16_rne(he);
                        lo[e] = f32_to_bf16_rne(he - __uint_as_float(hi[e] << 16));
                        // the sum of what the MFMA rows carry (hi + lo, exact in fp32), so that
                        // the bias term cancels their 128 X exactly
                        sum += __uint_as_float(hi[e] << 16) + __uint_as_float(lo[e] << 16);
                        ssm += xs[e] * xs[e];
                    }
                    sum += __shfl_xor(sum, 1);
                    sum += __shfl_xor(sum, 2);
                    sum += __shfl_xor(sum, 4);
                    if (c8 < pad_vecs) {
                        const uint32_t U = c8 >> 4, c = c8 & 15;
                        const u32x4_t vh = u32x4_t{hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16),
                                                   hi[4] | (hi[5] << 16), hi[6] | (hi[7] << 16)};
                        const u32x4_t vl = u32x4_t{lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16),
                                                   lo[4] | (lo[5] << 16), lo[6] | (lo[7] << 16)};
                        sH[(((2 * m) * npad + U) * 4 + (c >> 2)) * 4 + (c & 3)] = prep_h(vh);
                        sH[(((2 * m + 1) * npad + U) * 4 + (c >> 2)) * 4 + (c & 3)] = prep_h(vl);
                        if ((c8 & 7) == 0) {
                            const uint32_t g = c8 >> 3;
                            bias_slices(sum, [&](int kg) {
                                return xo + (((g >> 2) * 4 + kg) * lrows + 2 * m) * 4 + (g & 3);
                            });
                            bias_slices(0.0f, [&](int kg) {
                                return xo + (((g >> 2) * 4 + kg) * lrows + 2 * m + 1) * 4 + (g & 3);
                            });
                        }
                    }
                }
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ssm += __shfl_xor(ssm, o);
            if (lane == 0) ss_red[tid >> 6][m] = ssm;
        }
    } else
    for (uint32_t base = 0; base < tasks; base += NT * kBatch) {
        u32x4_t v[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const uint32_t task = base + b * NT + tid;
            const uint32_t m = task / pad_vecs, c8 = task % pad_vecs;
            v[b] = u32x4_t{0u, 0u, 0u, 0u};
            if (task < tasks && c8 < row_vecs)
                v[b] = *reinterpret_cast<const u32x4_t*>(a.h + (static_cast<size_t>(m) * row_vecs + c8) * 8);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const uint32_t task = base + b * NT + tid;
            const uint32_t m = task / pad_vecs, c8 = task % pad_vecs;
            float s = sum8_bf16(v[b]);
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            s += __shfl_xor(s, 4);
            if (task < tasks) {
                const uint32_t U = c8 >> 4, c = c8 & 15;
                sH[((m * npad + U) * 4 + (c >> 2)) * 4 + (c & 3)] = prep_h(v[b]);
                if ((c8 & 7) == 0) {
                    const uint32_t g = c8 >> 3;
                    uint32_t* x = reinterpret_cast<uint32_t*>(sXF);
                    bias_slices(s, [&](int kg) { return x + (((g >> 2) * 4 + kg) * a.M + m) * 4 + (g & 3); });
                }
            }
        }
    }
    if constexpr (MODE == kModeSample) {
        // every wave's zeros are in place; then the occurrence counts of the block's rows, each
        // history id of this block counted once (ids >= vocab never match a live row)
        __syncthreads();
        auto count = [&](uint32_t m, const uint32_t (&ids)[kHistBatch]) {
#pragma unroll
            for (int q = 0; q < kHistBatch; ++q) {
                const uint32_t lr = ids[q] - block_row0;
                if (lr < kRowsPerBlock) atomicAdd(&cnt[m * kRowsPerBlock + lr], 1u);
            }
        };
        if (m_first < a.M) count(m_first, hids);
        for (uint32_t m = m_first; m < a.M; ++m) {
            if (a.rp[m] == 1.0f || a.hist_len[m] == 0) continue;
            const uint32_t* hs = a.history + a.hist_off[m];
            const uint32_t len = a.hist_len[m];
            for (uint32_t j0 = (m == m_first) ? NT * kHistBatch : 0; j0 < len; j0 += NT * kHistBatch) {
                uint32_t ids[kHistBatch];
#pragma unroll
                for (int q = 0; q < kHistBatch; ++q) {
                    const uint32_t j = j0 + tid + NT * q;
                    ids[q] = j < len ? hs[j] : 0xFFFFFFFFu;
                }
                count(m, ids);
            }
        }
    }
    __syncthreads();

    // this lane's A row rho: h row rho / MS when rho % MS is 0 (NORM: its hi half, and its lo
    // half when rho % MS is 1); any other A row reads LDS row 0
    const uint32_t rho = lane & 15, part = rho % MS, m_of = rho / MS;
    const uint32_t lrow = NORM ? ((part < 2 && m_of < a.M) ? 2 * m_of + part : 0u)
                               : ((part == 0 && m_of < a.M) ? m_of : 0u);
    const u32x4_t* aRow = sH + lrow * pad_vecs + (lane >> 4);
    const u32x4_t* xRow = sXF + (lane >> 4) * lrows + lrow;

    f32x4_t tot[RT][1], bacc[RT];
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        tot[j][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        bacc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }


    // One unit of the ring: slot s holds chunk U0 + s; RELOAD refills the slot PF chunks ahead.
    auto step = [&](uint32_t U0, auto slot, auto reload) {
        constexpr int s = decltype(slot)::value;
        const uint32_t U = U0 + s;
        bf16x8_t av[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) av[t] = __builtin_bit_cast(bf16x8_t, aRow[(U * 4 + t) * 4]);
        f32x4_t acc[RT][2];
#pragma unroll
        for (int j = 0; j < RT; ++j)
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const bf16x8_t b0 = nibbles_to_bf16(wq[s][j][2 * g], magic);
                const bf16x8_t b1 = nibbles_to_bf16(wq[s][j][2 * g + 1], magic);
                acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[2 * g], b0,
                                                                    f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                acc[j][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[2 * g + 1], b1, acc[j][g], 0, 0, 0);
            }
#pragma unroll
        for (int j = 0; j < RT; ++j)
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                const float t = bf16_hi(g ? sq[s][j].y : sq[s][j].x);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (i % MS == 0 || (NORM && i % MS == 1)) tot[j][0][i] = fmaf(t, acc[j][g][i], tot[j][0][i]);
            }
        // the fences in the loads keep each refill inside its step: the scheduler would otherwise
        // sink every refill of the cycle below the last MFMA, leaving no loads in flight while
        // the cycle computes
        constexpr bool kReload = decltype(reload)::value;
        const uint32_t Un = min(U + PF, last);
        if constexpr ((s & 1) == 0) {
            if constexpr (kReload) load_nibbles_ordered<RT>(rs, Un, vo_w, wq[s]);
        } else {
            // {b, t} words of the super-unit's four groups: the bias B fragment
            const bf16x8_t xa = __builtin_bit_cast(bf16x8_t, xRow[(U >> 1) * 4 * lrows]);
#pragma unroll
            for (int j = 0; j < RT; ++j) {
                const u32x4_t bp = u32x4_t{sq[s - 1][j].x, sq[s - 1][j].y, sq[s][j].x, sq[s][j].y};
                bacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(bf16x8_t, bp),
                                                                  bacc[j], 0, 0, 0);
            }
            if constexpr (kReload) {
                load_scales_ordered<RT>(rs, min(U - 1 + PF, last), vo_s, sq[s - 1]);
                load_nibbles_ordered<RT>(rs, Un, vo_w, wq[s]);
                load_scales_ordered<RT>(rs, Un, vo_s, sq[s]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto cycle = [&](uint32_t U0, auto reload) {
        static_for<PF>([&](auto slot) { step(U0, slot, reload); });
    };
    for (uint32_t U0 = 0; U0 + PF < npad; U0 += PF) cycle(U0, std::true_type{});
    cycle(npad - PF, std::false_type{});
#pragma unroll
    for (int j = 0; j < RT; ++j) tot[j][0] += bacc[j];
    if constexpr (NORM) {
        // row lane / 16: the two halves' sums, times the row's 1 / sqrt(mean(x^2) + eps)
        const uint32_t m = (lane >> 4) < a.M ? (lane >> 4) : 0u;
        float t = 0.0f;
        for (int w2 = 0; w2 < NW; ++w2) t += ss_red[w2][m];
        const float rms = 1.0f / sqrtf(t / static_cast<float>(a.d) + a.eps);
#pragma unroll
        for (int j = 0; j < RT; ++j) tot[j][0][0] = (tot[j][0][0] + tot[j][0][1]) * rms;
    }
    if constexpr (MODE == kModeSample) {
        head_epilogue_sample<RT, NW, MS>(a, tot, tile0, block_row0, cnt, exp2_tbl, prm);
    } else {
        head_epilogue<1, 4, RT, MODE, NW, MS>(a, tot, tile0, se);
    }
}

// ---- 9 <= M <= 16 (and the RMSNorm prologue's 5 <= M <= 8): h prepared once per call, ------
// staged through LDS by plain copies; M > 16 runs head_wide32_kernel below
//
// prep_hidden_kernel writes, once per call, the prepared h in A-fragment order,
// hp[U][mt][t][lane] (16 B each, rows m >= M zero), and the bias A-fragment entries
// hx[P][mt][lane] of super-unit P (groups past the end zero).
template <int NMT>
__global__ __launch_bounds__(kHeadThreads) void prep_hidden_kernel(const uint16_t* __restrict__ h,
                                                                   uint32_t M, uint32_t d,
                                                                   u32x4_t* __restrict__ hp,
                                                                   u32x4_t* __restrict__ hx) {
    const uint32_t per_chunk = NMT * 256;  // 16 B vectors per chunk (NMT*16 rows x 16)
    const uint32_t nunits = d / kChunkK;
    // an odd chunk count is padded with one zero chunk: the kernel always computes both
    // chunks of a stage, and a zero h makes the padding add exactly nothing
    const uint32_t padded = nunits + (nunits & 1);
    const uint32_t task = blockIdx.x * kHeadThreads + threadIdx.x;  // grid covers padded chunks
    const uint32_t U = task / per_chunk, rem = task % per_chunk;
    const uint32_t m = rem >> 4, c = rem & 15;
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    if (U < nunits && m < M)
        v = *reinterpret_cast<const u32x4_t*>(h + static_cast<size_t>(m) * d + U * kChunkK + c * 8);
    float s = sum8_bf16(v);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (U < padded) {
        hp[((static_cast<size_t>(U) * NMT + (m >> 4)) * 4 + (c >> 2)) * 64 + (c & 3) * 16 + (m & 15)] =
            prep_h(v);
        if ((c & 7) == 0) {
            const uint32_t g = 2 * U + (c >> 3);
            uint32_t* x = reinterpret_cast<uint32_t*>(hx);
            auto at = [&](int kg) {
                return x + (((static_cast<size_t>(g >> 2) * NMT + (m >> 4)) * 4 + kg) * 16 + (m & 15)) * 4 +
                       (g & 3);
            };
            bias_slices(s, at);  // zero slices for the padding chunk's two groups
        }
    }
}

// The final RMSNorm as the head's prologue (src/runner.cpp:1889-1918, shaders/RMSNormK.hlsl;
// CPU: src/cpu_reference.cpp:141-150): h[m] = x[m] * (1 / sqrt(mean(x[m]^2) + eps)) * w, fp32
// x rows, bf16 weight, for rows <= 8. h is fp32, which the bf16 MFMA operands cannot hold, so
// it is split into h_hi = bf16(h) and h_lo = bf16(h - h_hi) (|h - h_hi - h_lo| <= 2^-18 |h|),
// placed as MFMA rows m and m + 8 of one 16-row tile; the kernel's epilogue adds row m + 8 to
// row m (HeadArgs::fold). The bias term uses the group sums of hi + lo, on rows < 8 only.
// Every block recomputes the rows' mean squares itself (M x d fp32 from L2), so the prologue
// needs no launch of its own. Output: the hp / hx layout of prep_hidden_kernel<1>.
__global__ __launch_bounds__(kHeadThreads) void prep_rmsnorm_kernel(const float* __restrict__ x,
                                                                    const uint16_t* __restrict__ w,
                                                                    float eps, uint32_t M, uint32_t d,
                                                                    u32x4_t* __restrict__ hp,
                                                                    u32x4_t* __restrict__ hx) {
    __shared__ float red[kHeadWaves][8];
    __shared__ float rms[8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // mean squares: thread t sums the float4 chunks t, t + 256, ... of every row
    float ss[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        ss[r] = 0.0f;
        if (static_cast<uint32_t>(r) < M) {
            const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(r) * d);
            for (uint32_t q = tid; q < d / 4; q += kHeadThreads) {
                const float4 v = xr[q];
                ss[r] += v.x * v.x;
                ss[r] += v.y * v.y;
                ss[r] += v.z * v.z;
                ss[r] += v.w * v.w;
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss[r] += __shfl_xor(ss[r], o);
        if (lane == 0) red[wave][r] = ss[r];
    }
    __syncthreads();
    if (tid < 8) {
        float t = 0.0f;
        for (int w2 = 0; w2 < kHeadWaves; ++w2) t += red[w2][tid];
        rms[tid] = 1.0f / sqrtf(t / static_cast<float>(d) + eps);
    }
    __syncthreads();

    const uint32_t nunits = d / kChunkK;
    const uint32_t padded = nunits + (nunits & 1);
    const uint32_t task = blockIdx.x * kHeadThreads + tid;  // grid covers padded chunks
    const uint32_t U = task / 256, rem = task % 256;
    const uint32_t m = rem >> 4, c = rem & 15;
    const uint32_t row = m & 7, lo_plane = m >> 3;
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    float s = 0.0f;
    if (U < nunits && row < M) {
        const size_t col = static_cast<size_t>(U) * kChunkK + c * 8;
        const float4 x0 = *reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * d + col);
        const float4 x1 = *reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * d + col + 4);
        const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(w + col);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
        const float r = rms[row];
        uint32_t half[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t wb = (ws[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            const float he = (xs[e] * r) * __uint_as_float(wb << 16);  // x * rms * weight
            const uint32_t hi = f32_to_bf16_rne(he);
            const uint32_t lo = f32_to_bf16_rne(he - __uint_as_float(hi << 16));
            half[e] = lo_plane ? lo : hi;
            // the group sum of what the MFMA rows carry, hi + lo (exact in fp32): the bias
            // term's X must cancel the MFMA's 128 X to the last bit, or the 2^-18 gap between
            // h and hi + lo comes back multiplied by 128 s
            s += __uint_as_float(hi << 16) + __uint_as_float(lo << 16);
        }
        v = u32x4_t{half[0] | (half[1] << 16), half[2] | (half[3] << 16), half[4] | (half[5] << 16),
                    half[6] | (half[7] << 16)};
        if (lo_plane) s = 0.0f;  // the bias is added once, on the high rows
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (U < padded) {
        hp[((static_cast<size_t>(U) * 1 + 0) * 4 + (c >> 2)) * 64 + (c & 3) * 16 + m] = prep_h(v);
        if ((c & 7) == 0) {
            const uint32_t g = 2 * U + (c >> 3);
            uint32_t* xo = reinterpret_cast<uint32_t*>(hx);
            bias_slices(s, [&](int kg) { return xo + ((static_cast<size_t>(g >> 2) * 4 + kg) * 16 + m) * 4 + (g & 3); });
        }
    }
}

// Block = NW waves; wave w owns RT consecutive 16-row tiles. NMT = number of 16-wide m tiles
// (1: this kernel serves M <= 16). A stage is one chunk (two groups). Each stage: one barrier;
// the next chunk's prepared h copied straight from global memory into the other LDS buffer
// (for an even chunk also the next super-unit's bias fragment); the weights of the next chunk
// requested into the other half of a two-deep register ring. One chunk per stage keeps the LDS
// small; measured on MI355X at V = 262144, d = 5376 against a two-chunk register-staged form:
// M = 16 143.8 -> 136.2 us.
//
// Per group step the MFMA chains of all RT x NMT accumulators run first; the scales are
// applied (tot += t * acc) right after, while the next step's nibbles are converted.
template <int NMT, int RT, int MODE, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(3)))
void head_wide_kernel(HeadArgs a, const u32x4_t* __restrict__ hp, const u32x4_t* __restrict__ hx) {
    constexpr int kVec = NMT * 4 * 64;  // 16 B A-fragment vectors per chunk
    constexpr int kXA = NMT * 64;       // 16 B bias vectors per super-unit
    constexpr int kCopies = kVec / 64 / NW;  // 1 KB pieces each wave copies per chunk
    static_assert(kCopies >= 1 && kXA / 64 <= NW, "copy split");
    // two buffers as separate arrays: each LDS read names the buffer it reads
    __shared__ u32x4_t sA0[kVec], sA1[kVec];  // [mt][t][lane] of one chunk
    __shared__ u32x4_t sXA0[kXA], sXA1[kXA];  // [mt][lane] of one super-unit
    __shared__ EpiSharedT<NW> se;

    const int lane = threadIdx.x & 63;
    const uint32_t wave = wave_id();
    const uint32_t tile0 = (blockIdx.x * NW + wave) * RT;
    const uint32_t magic = vgpr_const(0x43004300u);
    // an odd chunk count ends with hp's zero chunk; its weight loads re-read the last unit
    const uint32_t nchunks = a.nunits + (a.nunits & 1);

    __amdgpu_buffer_rsrc_t rs[RT];
    tile_streams<RT>(a, tile0, rs);
    const uint32_t vo_w = lane * 16, vo_s = kUnitNibbleBytes + (lane & 15) * 8;

    // 16 B per lane from global memory into LDS at l + 16 * lane (global_load_lds_dwordx4 with
    // the wave's LDS base in M0). Issued by inline asm, so the compiler neither holds its LDS
    // reads of the other buffer behind these copies nor counts them: the wait and barrier at
    // each stage's start cover them. hp and hx hold one chunk and one super-unit past the end,
    // so the copies need no branch.
    auto copy16 = [&](const u32x4_t* g, u32x4_t* l) {
        // the LDS offset of l: an address-space cast, not the low bits of the flat address
        const uint32_t la = static_cast<uint32_t>(
            reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) u32x4_t*)l));
        // M0 is reserved to the compiler, which sets it next to each instruction of its own that
        // reads it; this kernel has no such instruction, so the value left here is never read
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(la), "v"(g) : "memory");
    };
    auto chunk_copy = [&](uint32_t C, auto parity) {
        constexpr int P = decltype(parity)::value;
        u32x4_t* dst = P ? sA1 : sA0;
        const u32x4_t* src = hp + static_cast<size_t>(C) * kVec;
#pragma unroll
        for (int it = 0; it < kCopies; ++it) {
            const uint32_t piece = wave * kCopies + it;
            copy16(src + piece * 64 + lane, dst + piece * 64);
        }
        // chunk C opens super-unit C / 2 when even; its bias buffer is (C / 2) & 1
        if constexpr (P == 0) {
            if (wave < static_cast<uint32_t>(kXA / 64)) {
                copy16(hx + static_cast<size_t>(C >> 1) * kXA + wave * 64 + lane,
                       (((C >> 1) & 1) ? sXA1 : sXA0) + wave * 64);
            }
        }
    };
    // chunk C's weights into ring slot B: the lane's 16 B of nibbles and its row's two {b, t} words
    u32x4_t wr[2][RT];
    u32x2_t sc[2][RT];
    auto chunk_w = [&](uint32_t C, auto slot) {
        constexpr int B = decltype(slot)::value;
        const int so = static_cast<int>(min(C, a.nunits - 1) * kUnitBytes);
#pragma unroll
        for (int j = 0; j < RT; ++j) {
            wr[B][j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs[j], vo_w, so, kNonTemporal));
            sc[B][j] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs[j], vo_s, so, kNonTemporal));
        }
    };

    f32x4_t tot[RT][NMT];
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) tot[j][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    bf16x8_t bq[2][RT][2];  // converted nibbles of the current and the next group step
    u32x2_t sc_even[RT];    // the even chunk's {b, t} words, for the super-unit's bias MFMA

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    chunk_copy(0, I0{});
    chunk_w(0, I0{});
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        bq[0][j][0] = nibbles_to_bf16(wr[0][j].x, magic);
        bq[0][j][1] = nibbles_to_bf16(wr[0][j].y, magic);
    }

    // chunk C in LDS buffer and ring slot P = C & 1
    auto stage = [&](uint32_t C, auto parity) {
        constexpr int P = decltype(parity)::value;
        const u32x4_t* sA = P ? sA1 : sA0;
        __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this wave's copies of chunk C, its weights
        __syncthreads();                        // every wave's copies; buffer P ^ 1 is free
        chunk_copy(C + 1, std::integral_constant<int, P ^ 1>{});
        chunk_w(C + 1, std::integral_constant<int, P ^ 1>{});
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            bf16x8_t av[NMT][2];
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    av[mt][t] = __builtin_bit_cast(bf16x8_t, sA[(mt * 4 + 2 * g + t) * 64 + lane]);
            f32x4_t acc[RT][NMT];
#pragma unroll
            for (int j = 0; j < RT; ++j)
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt) {
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][0], bq[g][j][0],
                                                                         f32x4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][1], bq[g][j][1], acc[j][mt], 0, 0, 0);
                }
            // the next step's nibbles: this chunk's second group, or the next chunk's first
#pragma unroll
            for (int j = 0; j < RT; ++j) {
                const u32x4_t& nx = (g == 0) ? wr[P][j] : wr[P ^ 1][j];
                bq[g ^ 1][j][0] = nibbles_to_bf16(g == 0 ? nx.z : nx.x, magic);
                bq[g ^ 1][j][1] = nibbles_to_bf16(g == 0 ? nx.w : nx.y, magic);
            }
#pragma unroll
            for (int j = 0; j < RT; ++j) {
                const float t = bf16_hi(g == 0 ? sc[P][j].x : sc[P][j].y);
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) tot[j][mt][i] = fmaf(t, acc[j][mt][i], tot[j][mt][i]);
            }
        }
        if constexpr (P == 0) {
#pragma unroll
            for (int j = 0; j < RT; ++j) sc_even[j] = sc[0][j];
        } else {
            // the super-unit's bias after its odd chunk: one K=32 MFMA per row tile and m tile
            const u32x4_t* sXA = ((C >> 1) & 1) ? sXA1 : sXA0;
            bf16x8_t xa[NMT];
#pragma unroll
            for (int mt = 0; mt < NMT; ++mt) xa[mt] = __builtin_bit_cast(bf16x8_t, sXA[mt * 64 + lane]);
#pragma unroll
            for (int j = 0; j < RT; ++j) {
                const u32x4_t bw = u32x4_t{sc_even[j].x, sc_even[j].y, sc[1][j].x, sc[1][j].y};
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt)
                    tot[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[mt], __builtin_bit_cast(bf16x8_t, bw),
                                                                         tot[j][mt], 0, 0, 0);
            }
        }
    };
    for (uint32_t C = 0; C < nchunks; C += 2) {
        stage(C, I0{});
        stage(C + 1, I1{});
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the last (unused) copies land before LDS is reused
    __syncthreads();
    head_epilogue<NMT, 4, RT, MODE>(a, tot, tile0, se);
}

// ---- 33 <= M <= 64: 32x32x16 MFMAs, weights and h streamed into LDS two chunks ahead ----------
//
// Lane l = 32 kh + n of a 32 x 32 x 16 MFMA carries B column n (a vocabulary row of the wave's
// tile pair: tile n / 16, row n % 16) and k half kh. For k-step s of group g (64 columns) it
// takes one nibble word of row n: the unit's lane 16 kg + n % 16, kg = kh for s = 0, 1 and
// kh + 2 for s = 2, 3, word 2 g + (s & 1), i.e. columns 64 g + {0, 32, 16, 48}[s] + 8 kh + 0..7.
// prep_hidden32_kernel lays the A entries (h rows) out in the same column order:
// hp[U][mt][g][s][lane] is prep_h of h[32 mt + l % 32][128 U + 64 g + koff[s] + 8 (l / 32) ..+8]
// (rows >= M zero), and hx[P][mt][f][lane] holds, in dword c, slice 2 f + l / 32 (hi, mid, lo,
// zero) of X[32 mt + l % 32][4 P + c] duplicated into a bf16 pair. The group sums X are taken in
// the order of prep_hidden_kernel: eight-column pieces summed in column order, then a
// three-level pairwise tree over the pieces.
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int NM>
__global__ __launch_bounds__(kHeadThreads) void prep_hidden32_kernel(const uint16_t* __restrict__ h,
                                                                     uint32_t M, uint32_t d,
                                                                     u32x4_t* __restrict__ hp,
                                                                     u32x4_t* __restrict__ hx) {
    constexpr uint32_t per_chunk = NM * 512;  // tasks per chunk: [mt][g][row i][piece p]
    const uint32_t nunits = d / kChunkK;
    const uint32_t padded = nunits + (nunits & 1);
    const uint32_t task = blockIdx.x * kHeadThreads + threadIdx.x;  // grid covers padded chunks
    const uint32_t U = task / per_chunk, rem = task % per_chunk;
    const uint32_t p = rem & 7, i = (rem >> 3) & 31, g = (rem >> 8) & 1, mt = rem >> 9;
    const uint32_t m = 32 * mt + i;
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    if (U < nunits && m < M)
        v = *reinterpret_cast<const u32x4_t*>(h + static_cast<size_t>(m) * d + U * kChunkK + g * kGroup + p * 8);
    float s = sum8_bf16(v);
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (U < padded) {
        // piece p holds columns 8 p of the group: k-step {0, 2, 1, 3}[p / 2], k half p % 2
        const uint32_t ks = ((p >> 1) == 1) ? 2u : ((p >> 1) == 2) ? 1u : (p >> 1);
        hp[(((static_cast<size_t>(U) * NM + mt) * 2 + g) * 4 + ks) * 64 + (p & 1) * 32 + i] = prep_h(v);
        if (p == 0) {
            const uint32_t G = 2 * U + g;
            uint32_t* x = reinterpret_cast<uint32_t*>(hx);
            auto at = [&](int sl) {
                return x + ((((static_cast<size_t>(G >> 2) * NM + mt) * 2 + (sl >> 1)) * 64 + (sl & 1) * 32 + i) * 4 +
                            (G & 3));
            };
            bias_slices(s, at);  // zero slices for the padding chunk's two groups
        }
    }
}

// Softcap, logits store and, for the greedy modes, the per-row maxima of the 32 x 32 layout:
// tot[mt][v] of lane l is vocabulary row 16 T0 + l % 32 and h row 32 mt + 8 (v / 4) + 4 (l / 32)
// + v % 4.
template <int NP, int NM, int MODE, int NW>
__device__ __forceinline__ void head_epilogue32(const HeadArgs& a, f32x16_t (&tot)[NP][NM], uint32_t T0,
                                                EpiSharedT<NW>& se) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t mb = 4 * (lane >> 5);
    uint64_t best[NM][16];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) best[mt][v] = 0;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const uint32_t r = (T0 + 2 * p) * kTileRows + (lane & 31);
#pragma unroll
        for (int mt = 0; mt < NM; ++mt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t m = 32 * mt + 8 * (v >> 2) + mb + (v & 3);
                float x = tot[p][mt][v];
                if (a.softcap > 0.0f) x = a.softcap * tanhf(x / a.softcap);
                const bool live = (m < a.M) && (r < a.vocab);
                if (live && a.logits) a.logits[static_cast<size_t>(m) * a.vocab + r] = x;
                if (MODE != kModeLogits) {
                    const uint64_t k = live ? rank_key(x, r) : 0ull;
                    best[mt][v] = k > best[mt][v] ? k : best[mt][v];
                }
            }
    }
    if (MODE == kModeLogits) return;
    // The rows sharing m are the 32 lanes with the same lane / 32, and each lane holds NM * 16
    // maxima (index j = 16 mt + v, padded to 32 with zero keys). A transposed butterfly reduces
    // all of them at once: at the step over lane bit b, the lanes with that bit set keep the
    // upper half of their indices and send the lower half to their partner, which keeps the
    // lower half, so each step halves the values per lane. After five steps lane l holds the
    // maximum of index j = l % 32 over its 32 lanes: 31 exchanges instead of 32 x 5.
    uint64_t k[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) k[j] = j < NM * 16 ? best[j / 16 % NM][j % 16] : 0ull;
    static_for<5>([&](auto st) {
        constexpr int kHalf = 16 >> decltype(st)::value;  // values kept after this step
        const bool up = (lane & kHalf) != 0;
#pragma unroll
        for (int i = 0; i < kHalf; ++i) {
            const uint64_t send = up ? k[i] : k[i + kHalf];
            const uint64_t keep = up ? k[i + kHalf] : k[i];
            const uint64_t o = shfl_xor_u64(send, kHalf);
            k[i] = o > keep ? o : keep;
        }
    });
    const uint32_t j = lane & 31;
    const uint32_t m = 32 * (j / 16) + 8 * ((j % 16) >> 2) + mb + (j & 3);
    if (j < NM * 16 && m < TWD_MAX_ROWS) se.red[wave][m] = k[0];
    grid_finish<NW>(a, se);
}

// Block = NW waves; wave w owns NP tile pairs (32 vocabulary rows each, tiles T0 + 2 p and
// T0 + 2 p + 1, T0 = 2 NP (blockIdx.x * NW + w)) and all rows as NM m tiles of 32. Every
// vector-memory access of the streaming loop is a DMA into LDS: the wave's own weights (per pair
// and chunk, two 16 B nibble vectors and one scale dword per lane) two chunks ahead into a
// private two-slot ring, and the block's share of the prepared h (with each even chunk also the
// super-unit's bias entries) one chunk ahead into a two-slot ring -- h comes from L2, the weights
// from HBM. At 79 KB two blocks share a CU, so one block's epilogue and pipeline fill overlap the
// other's stream. A stage (one chunk, two groups):
//   1. wait until only the weight DMAs of chunk C + 1 are outstanding; barrier (chunk C's h is in
//      LDS for every wave, and every wave is done with chunk C - 1); the DMAs of chunk C + 1's h
//      into the slot chunk C - 1 used;
//   2. read the wave's weights of chunk C out of its ring slot into registers;
//   3. per group: the A entries of the group once, then per pair 4 k-steps x NM m tiles of
//      MFMAs into acc and tot += t * acc; before the second group, once the weight reads have
//      landed, the DMAs of chunk C + 2's weights into the slot just read;
//   4. after an odd chunk, the super-unit's bias MFMAs (two per pair and m tile: slices
//      hi + mid, lo).
// The loop issues no vector-memory instruction the compiler can see, so the one explicit wait
// per stage is exact: it counts the youngest DMAs, chunk C + 1's weights.
constexpr int kW32Waves = 8;
constexpr int kW32Pairs = 1;

template <int NP, int NM, int NW, int MODE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NP == 1 ? 4 : 2)))
void head_wide32_kernel(HeadArgs a, const u32x4_t* __restrict__ hp, const u32x4_t* __restrict__ hx) {
    constexpr int kVec = NM * 512;              // 16 B A vectors per chunk
    constexpr int kXA = NM * 128;               // 16 B bias vectors per super-unit
    constexpr int kHCopies = kVec / (64 * NW);  // 1 KB pieces of h each wave copies per chunk
    constexpr int kXPieces = kXA / 64;
    static_assert(kHCopies >= 1 && kVec % (64 * NW) == 0 && kXPieces <= NW, "copy split");
    constexpr int kOpsW = 3 * NP;  // weight DMAs a wave issues per chunk
    __shared__ u32x4_t sH[2][kVec];
    __shared__ u32x4_t sX[2][kXA];
    __shared__ u32x4_t sWn[NW][2][NP][2][64];
    __shared__ uint32_t sWs[NW][2][NP][64];
    // the greedy finish's shared state lives in the h staging, dead once the stream has ended:
    // a block stays within the LDS that lets two share a CU
    static_assert(sizeof(EpiSharedT<NW>) <= sizeof(sH), "the finish's state fits the h staging");

    const int lane = threadIdx.x & 63;
    const uint32_t wave = wave_id();
    const uint32_t T0 = (blockIdx.x * NW + wave) * 2 * NP;
    const uint32_t magic = vgpr_const(0x43004300u);
    const uint32_t nchunks = a.nunits + (a.nunits & 1);
    const uint32_t stripe = a.nunits * kUnitBytes;

    // weights: SGPR base at the wave's first tile (clamped; tiles past the end re-read the last
    // tile and their rows are never stored), per-lane offsets to the lane's tile of each pair
    const uint32_t Tb = min(T0, a.ntiles - 1);
    const uint32_t kh = lane >> 5, n = lane & 31;
    uint32_t vo_n[NP], vo_s[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        vo_n[p] = (min(T0 + 2 * p + (n >> 4), a.ntiles - 1) - Tb) * stripe + (16 * kh + (n & 15)) * 16;
        vo_s[p] = (min(T0 + 2 * p + kh, a.ntiles - 1) - Tb) * stripe + kUnitNibbleBytes + n * 4;
    }
    const uint8_t* wbase = a.tiled + static_cast<size_t>(Tb) * stripe;
    const uint32_t vo_h = lane * 16;

    auto lds_off = [](const void* q) {
        return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)q));
    };
    // One DMA: 16 B (or 4 B) per lane from base + voff into LDS at dst + 16 * lane (4 * lane).
    // No instruction offset: it would move the LDS address as well. Issued by inline asm,
    // invisible to the compiler's wait insertion; M0 is reserved to the compiler, which sets it
    // next to each instruction of its own that reads it, and this kernel has none, so the value
    // left here is never read.
    auto dma16 = [&](const void* base, uint32_t voff, uint32_t dst) {
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"(voff), "s"(base)
                     : "memory");
    };
    // the weights stream once: non-temporal, so they do not push h out of L2
    auto dma16_nt = [&](const void* base, uint32_t voff, uint32_t dst) {
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2 nt" ::"s"(dst), "v"(voff), "s"(base)
                     : "memory");
    };
    auto dma4_nt = [&](const void* base, uint32_t voff, uint32_t dst) {
        asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2 nt" ::"s"(dst), "v"(voff), "s"(base)
                     : "memory");
    };
    // chunk C's h pieces into slot C & 1, with an even C also super-unit C / 2's bias pieces
    auto issue_h = [&](uint32_t C) {
        const u32x4_t* src = hp + static_cast<size_t>(C) * kVec;
#pragma unroll
        for (int it = 0; it < kHCopies; ++it) {
            const uint32_t piece = wave * kHCopies + it;
            dma16(src + piece * 64, vo_h, lds_off(&sH[C & 1][piece * 64]));
        }
        if ((C & 1) == 0) {
            const uint32_t xp = wave % kXPieces, P = C >> 1;
            dma16(hx + static_cast<size_t>(P) * kXA + xp * 64, vo_h, lds_off(&sX[P & 1][xp * 64]));
        }
    };
    // chunk C's weights into the wave's slot C & 1
    auto issue_w = [&](uint32_t C) {
        const uint32_t ws = C & 1;
        const uint8_t* wb = wbase + static_cast<size_t>(min(C, a.nunits - 1)) * kUnitBytes;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            dma16_nt(wb, vo_n[p], lds_off(&sWn[wave][ws][p][0][0]));
            dma16_nt(wb + 512, vo_n[p], lds_off(&sWn[wave][ws][p][1][0]));  // unit lanes 16 (kh + 2) + r
            dma4_nt(wb, vo_s[p], lds_off(&sWs[wave][ws][p][0]));
        }
    };

    f32x16_t tot[NP][NM];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int mt = 0; mt < NM; ++mt)
#pragma unroll
            for (int v = 0; v < 16; ++v) tot[p][mt][v] = 0.0f;
    u32x2_t sc_even[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) sc_even[p] = u32x2_t{0u, 0u};

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    issue_h(0);
    issue_w(0);
    issue_w(1);

    auto stage = [&](uint32_t C, auto parity) {
        constexpr int P = decltype(parity)::value;
        __builtin_amdgcn_s_waitcnt(0x0F70 | kOpsW);  // outstanding now: chunk C + 1's weights
        __syncthreads();
        issue_h(C + 1);  // slot (C + 1) & 1: every wave is done with chunk C - 1
        u32x4_t w0[NP], w1[NP];
        u32x2_t sc[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            w0[p] = sWn[wave][P][p][0][lane];
            w1[p] = sWn[wave][P][p][1][lane];
            sc[p] = u32x2_t{sWs[wave][P][p][2 * n], sWs[wave][P][p][2 * n + 1]};
        }
        const u32x4_t* sA = sH[P];
        // unit u = NP g + p: the MFMA chains of pair p over group g into acc[u & 1]; its scale
        // FMAs are placed after the next unit's chains, so each wave has MFMA and VALU work
        // that do not depend on each other
        f32x16_t acc[2][NM];
        bf16x8_t av[NM][4];
        auto load_a = [&](int g) {
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    av[mt][s] = __builtin_bit_cast(bf16x8_t, sA[((mt * 2 + g) * 4 + s) * 64 + lane]);
        };
        auto chain = [&](int g, int p) {
            const int u = (NP * g + p) & 1;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint32_t word = (s < 2) ? w0[p][2 * g + (s & 1)] : w1[p][2 * g + (s & 1)];
                const bf16x8_t b = nibbles_to_bf16(word, magic);
#pragma unroll
                for (int mt = 0; mt < NM; ++mt) {
                    if (s == 0)
                        acc[u][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[mt][s], b, f32x16_t{}, 0, 0, 0);
                    else
                        acc[u][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[mt][s], b, acc[u][mt], 0, 0, 0);
                }
            }
        };
        auto scale = [&](int g, int p) {
            const int u = (NP * g + p) & 1;
            const float t = bf16_hi(g == 0 ? sc[p].x : sc[p].y);
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) tot[p][mt][v] = fmaf(t, acc[u][mt][v], tot[p][mt][v]);
        };
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            load_a(g);
            if (g == 1) {
                // every LDS read of this wave's weight slot (and the group's A entries) has
                // landed: the slot can take chunk C + 2
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                issue_w(C + 2);
            }
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                chain(g, p);
                if (p > 0) scale(g, p - 1);
                else if (g > 0) scale(g - 1, NP - 1);
            }
        }
        scale(1, NP - 1);
        if constexpr (P == 0) {
#pragma unroll
            for (int p = 0; p < NP; ++p) sc_even[p] = sc[p];
        } else {
            // the super-unit's bias: B = the four groups' {b, t} words of row n (both k halves),
            // A = X slices hi + mid, then lo + zero
            const u32x4_t* sXA = sX[(C >> 1) & 1];
            bf16x8_t xa[NM][2];
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
#pragma unroll
                for (int f = 0; f < 2; ++f) xa[mt][f] = __builtin_bit_cast(bf16x8_t, sXA[(mt * 2 + f) * 64 + lane]);
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const bf16x8_t bb =
                    __builtin_bit_cast(bf16x8_t, u32x4_t{sc_even[p].x, sc_even[p].y, sc[p].x, sc[p].y});
#pragma unroll
                for (int mt = 0; mt < NM; ++mt)
#pragma unroll
                    for (int f = 0; f < 2; ++f)
                        tot[p][mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[mt][f], bb, tot[p][mt], 0, 0, 0);
            }
        }
    };
    for (uint32_t C = 0; C < nchunks; C += 2) {
        stage(C, I0{});
        stage(C + 1, I1{});
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the last (unused) DMAs land before LDS is reused
    __syncthreads();
    head_epilogue32<NP, NM, MODE, NW>(a, tot, T0, *reinterpret_cast<EpiSharedT<NW>*>(&sH[0][0]));
}

// ---- layout repack: reference [W|S|B] -> units ----------------------------------------------
// Sets *bad when a scale's magnitude exceeds kMaxScale (t = -128 s would not be finite) or a bias
// is infinite: the kernels multiply every bias and t by bf16 slices and padding entries that can
// be exactly zero, which would turn such a term into NaN where the reference's sum is infinite.
__global__ void repack_kernel(const uint32_t* __restrict__ W, const uint16_t* __restrict__ S,
                              const uint16_t* __restrict__ B, uint32_t vocab, uint32_t d,
                              uint32_t ntiles, uint32_t nunits, uint8_t* __restrict__ out,
                              uint32_t* __restrict__ bad) {
    const uint64_t total = static_cast<uint64_t>(ntiles) * nunits * 64;
    const uint32_t wpr = d / 8, gpr = d / kGroup;
    for (uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < total;
         g += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint32_t lane = static_cast<uint32_t>(g & 63);
        const uint64_t unit = g >> 6;
        const uint32_t U = static_cast<uint32_t>(unit % nunits);
        const uint32_t T = static_cast<uint32_t>(unit / nunits);
        const uint32_t r = T * kTileRows + (lane & 15), kg = lane >> 4;
        u32x4_t w = u32x4_t{0u, 0u, 0u, 0u};
        if (r < vocab) {
            const uint32_t* row = W + static_cast<size_t>(r) * wpr + 16 * U + kg;
            w = u32x4_t{row[0], row[4], row[8], row[12]};
        }
        uint8_t* ub = out + unit * kUnitBytes;
        *reinterpret_cast<u32x4_t*>(ub + lane * 16) = w;
        if (lane < 16) {
            u32x2_t sb = u32x2_t{0u, 0u};
            if (r < vocab) {
                const uint16_t* sr = S + static_cast<size_t>(r) * gpr + 2 * U;
                const uint16_t* br = B + static_cast<size_t>(r) * gpr + 2 * U;
                uint32_t word[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const float s = __uint_as_float(static_cast<uint32_t>(sr[k]) << 16);
                    const float b = __uint_as_float(static_cast<uint32_t>(br[k]) << 16);
                    if (fabsf(s) > kMaxScale || __builtin_isinf(b))
                        __hip_atomic_fetch_or(bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    word[k] = static_cast<uint32_t>(br[k]) | (f32_to_bf16_rne(-128.0f * s) << 16);
                }
                sb = u32x2_t{word[0], word[1]};
            }
            *reinterpret_cast<u32x2_t*>(ub + kUnitNibbleBytes + lane * 8) = sb;
        }
    }
}

// ---- synthetic head in the reference layout (formula in twd_head.h) ---------------------------
__device__ __forceinline__ uint64_t splitmix64_dev(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

__global__ void generate_kernel(uint32_t* __restrict__ W, uint16_t* __restrict__ S,
                                uint16_t* __restrict__ B, uint64_t n_words, uint64_t n_groups,
                                uint64_t seed) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_words;
         i += stride)
        W[i] = static_cast<uint32_t>(splitmix64_dev(seed + 0x1000000000000000ULL + i) >> 32);
    for (uint64_t j = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < n_groups;
         j += stride) {
        const float u = static_cast<float>(splitmix64_dev(seed + 0x2000000000000000ULL + j) >> 40) *
                        (1.0f / 16777216.0f);
        const uint16_t s = static_cast<uint16_t>(f32_to_bf16_rne(fmaf(9e-3f, u, 1e-3f)));
        S[j] = s;
        B[j] = static_cast<uint16_t>(f32_to_bf16_rne(-8.0f * __uint_as_float(static_cast<uint32_t>(s) << 16)));
    }
}

}  // namespace twd

// =================================================================================================
// C-ABI: the head object
// =================================================================================================

using namespace twd;

struct twd_head {
    uint32_t vocab = 0, d = 0, ntiles = 0, nunits = 0;
    float softcap = 0.f;
    uint8_t* tiled = nullptr;
    uint64_t tiled_bytes = 0;
    // [TWD_MAX_ROWS] per-row maxima (zero between launches), the arrival counter, and the
    // repack's flag
    uint64_t* gbest = nullptr;
    uint32_t epoch = kFirstEpoch - 1;  // of the last launch; the next is epoch_after(epoch)
    StreamOrder order;            // calls on several streams share gbest, hp/hx and sel
    u32x4_t* hp = nullptr;        // prepared h in A-fragment order for M > 8 (prep_hidden_kernel)
    u32x4_t* hx = nullptr;        // its bias A-fragment entries
    twd_selector* sel = nullptr;
    uint16_t* norm_w = nullptr;   // final RMSNorm weight, when loaded from a container
    SampleStats stats{};          // per-wave statistics of the fused sample pass (M <= 8)
    uint32_t sample_blocks = 0;   // its head blocks for M <= 4 (0: no fused sample pass)
    uint32_t sample_blocks8 = 0;  // for 5 <= M <= 8 (0: none, e.g. h and the counts exceed LDS)
};

namespace {

// staged-h kernel (M <= 16): row tiles per wave, measured best on MI355X
constexpr int kRT1 = 4;
// resident-h kernel: row tiles per wave and weight units in flight, measured best on MI355X at
// V = 262144, d = 5376: 4096 waves, 16 resident per CU, one round on 256 CUs. M <= 4: 512 blocks
// of 8 waves, two per CU. 5 <= M <= 8: 256 blocks of 16 waves, one per CU (one LDS copy of h
// serves 16 waves; M = 8 leaves no room for a second block's h anyway).
constexpr int kRTS = 4, kPFS = 2;
constexpr int kNWS4 = 8, kNWS8 = 16;
constexpr size_t kLdsBytes = 160 * 1024;
constexpr uint32_t kSmallMaxRows = 8;
// static LDS of the 16-wave sample mode (its occurrence counts, 8 rows x 1,024 block rows, and
// the exp table), beside the dynamic h staging
constexpr size_t kSample8StaticLds = kSampleRows * kNWS8 * kRTS * kTileRows * 4 + 64 * 8 + 1024;

uint32_t blocks_for(uint32_t ntiles, int rt, int nw = kHeadWaves) {
    const uint32_t per = nw * rt;
    return (ntiles + per - 1) / per;
}

uint32_t super_units(uint32_t nunits) { return (nunits + 1) / 2; }
uint32_t padded_units(uint32_t nunits) { return nunits + (nunits & 1); }

int check_geometry(uint32_t vocab, uint32_t d, uint32_t group) {
    if (group != kGroup) return fail(TWD_E_UNSUPPORTED, "group_size must be 64");
    if (vocab == 0) return fail(TWD_E_INVALID, "vocab must be > 0");
    // tile counts and row indices stay far from 32-bit wrap-around
    if (vocab > (1u << 30)) return fail(TWD_E_UNSUPPORTED, "vocab must be at most 2^30");
    if (d == 0 || d % kChunkK != 0) return fail(TWD_E_UNSUPPORTED, "d_model must be a positive multiple of 128");
    return TWD_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Dynamic LDS of the resident-h kernel with ring depth PF: prepared h (M rows of npad chunks of
// 256 B) + bias entries (npad / 2 super-units x 4 slices x M of 16 B).
template <int PF>
size_t small_smem_bytes(uint32_t rows, uint32_t d) {
    const size_t npad = small_pad_units<PF>(d / kChunkK);
    return static_cast<size_t>(rows) * npad * (256 + 32);
}

template <typename K>
hipError_t allow_smem(K kernel, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

// Lets every resident-h instantiation use the LDS it needs for kSmallMaxRows rows of d.
int enable_small_kernels(uint32_t d) {
    const size_t bytes4 = small_smem_bytes<kPFS>(4, d);
    const size_t bytes8 = small_smem_bytes<kPFS>(kSmallMaxRows, d);
    if (bytes4 + sizeof(EpiSharedT<kNWS4>) > kLdsBytes || bytes8 + sizeof(EpiSharedT<kNWS8>) > kLdsBytes)
        return fail(TWD_E_UNSUPPORTED, "d_model too large for the LDS-resident head");
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS4, kModeLogits>, bytes4);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS4, kModeGreedy>, bytes4);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<2, kRTS, kPFS, kNWS8, kModeLogits>, bytes8);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<2, kRTS, kPFS, kNWS8, kModeGreedy>, bytes8);
    // the RMSNorm prologue variant: two LDS rows per h row, M <= 4
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS4, kModeLogits, true>, bytes8);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS4, kModeGreedy, true>, bytes8);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS8, kModeLogits, true>, bytes8);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS8, kModeGreedy, true>, bytes8);
    // the fused sample pass (M <= 4), with and without the RMSNorm prologue, and 5 <= M <= 8
    // where its counts fit beside h
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS4, kModeSample>, bytes4);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS, kPFS, kNWS4, kModeSample, true>, bytes8);
    if (e == hipSuccess && bytes8 + kSample8StaticLds <= kLdsBytes)
        e = allow_smem(head_small_kernel<2, kRTS, kPFS, kNWS8, kModeSample>, bytes8);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    return TWD_OK;
}

int head_alloc(uint32_t vocab, uint32_t d, float softcap, twd_head** out) {
    twd_head* h = new twd_head();
    h->vocab = vocab;
    h->d = d;
    h->softcap = softcap;
    h->ntiles = (vocab + kTileRows - 1) / kTileRows;
    h->nunits = d / kChunkK;
    h->tiled_bytes = static_cast<uint64_t>(h->ntiles) * h->nunits * kUnitBytes;
    hipError_t e = hipMalloc(&h->tiled, h->tiled_bytes);
    // gbest: per-row maxima, the arrival counter's words, and the repack's bad-scale flag; the
    // counter starts armed for the first launch's epoch
    const uint64_t armed = kFirstEpoch;
    constexpr size_t kWords = TWD_MAX_ROWS + kArriveWords + 1;
    if (e == hipSuccess) e = hipMalloc(&h->gbest, sizeof(uint64_t) * kWords);
    if (e == hipSuccess) e = hipMemset(h->gbest, 0, sizeof(uint64_t) * kWords);
    if (e == hipSuccess) e = hipMemcpy(h->gbest + TWD_MAX_ROWS, &armed, sizeof(armed), hipMemcpyHostToDevice);
    // hp / hx: room past the last chunk and super-unit (each stage copies the next one
    // unconditionally)
    if (e == hipSuccess) e = hipMalloc(&h->hp, sizeof(u32x4_t) * (h->nunits + 3) * 4 * 4 * 64);
    if (e == hipSuccess) e = hipMalloc(&h->hx, sizeof(u32x4_t) * (super_units(h->nunits) + 1) * 4 * 64);
    // the fused sample pass's wave records: rows <= 4 on 8-wave blocks, 5..8 on 16-wave blocks
    // (the two grids' wave counts differ by less than a block); the 16-wave form also needs its
    // occurrence counts beside h in LDS
    const uint32_t sb = blocks_for(h->ntiles, kRTS, kNWS4), sb8 = blocks_for(h->ntiles, kRTS, kNWS8);
    const uint32_t waves = std::max(sb * kNWS4, sb8 * kNWS8);
    if (waves <= kSampleMaxWaves) {
        h->sample_blocks = sb;
        if (small_smem_bytes<kPFS>(kSampleRows, d) + kSample8StaticLds <= kLdsBytes) h->sample_blocks8 = sb8;
        const size_t n = static_cast<size_t>(kSampleRows) * waves;
        if (e == hipSuccess) e = hipMalloc(&h->stats.key, n * sizeof(uint64_t));
        if (e == hipSuccess) e = hipMalloc(&h->stats.sum, n * sizeof(double));
        if (e == hipSuccess) e = hipMalloc(&h->stats.max, n * sizeof(float));
        if (e == hipSuccess) e = hipMalloc(&h->stats.aux, n * sizeof(uint32_t));
    }
    h->stats.cap = softcap > 0.0f ? softcap : __builtin_nanf("");
    if (e != hipSuccess) {
        twd_head_destroy(h);
        return hip_fail(e, "allocating the LM head");
    }
    if (enable_small_kernels(d) != TWD_OK || twd_selector_create(vocab, TWD_MAX_ROWS, &h->sel) != TWD_OK) {
        twd_head_destroy(h);
        return TWD_E_HIP;
    }
    *out = h;
    return TWD_OK;
}

uint32_t* repack_flag(twd_head* h) { return reinterpret_cast<uint32_t*>(h->gbest + TWD_MAX_ROWS + kArriveWords); }

int head_repack(twd_head* h, const uint8_t* wsb_dev, hipStream_t stream) {
    const uint64_t w_bytes = static_cast<uint64_t>(h->vocab) * (h->d / 8) * 4;
    const uint64_t s_bytes = static_cast<uint64_t>(h->vocab) * (h->d / kGroup) * 2;
    const uint32_t* W = reinterpret_cast<const uint32_t*>(wsb_dev);
    const uint16_t* S = reinterpret_cast<const uint16_t*>(wsb_dev + w_bytes);
    const uint16_t* B = reinterpret_cast<const uint16_t*>(wsb_dev + w_bytes + s_bytes);
    const uint64_t work = static_cast<uint64_t>(h->ntiles) * h->nunits * 64;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((work + 255) / 256, 1u << 16));
    repack_kernel<<<grid, 256, 0, stream>>>(W, S, B, h->vocab, h->d, h->ntiles, h->nunits, h->tiled,
                                            repack_flag(h));
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

template <int MODE>
int launch_head(twd_head* h, const uint16_t* hidden, uint32_t rows, float* logits,
                uint32_t* tokens, const uint32_t* drafts, uint32_t n_drafts,
                twd_verify_result* vres, hipStream_t stream) {
    if (!h) return fail(TWD_E_INVALID, "null head");
    if (!hidden || !aligned16(hidden)) return fail(TWD_E_INVALID, "hidden must be a 16-byte aligned device pointer");
    if (rows == 0 || rows > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "rows must be in 1..64");
    HeadArgs a{};
    a.tiled = h->tiled;
    a.ntiles = h->ntiles;
    a.nunits = h->nunits;
    a.h = hidden;
    a.M = rows;
    a.d = h->d;
    a.softcap = h->softcap;
    a.logits = logits;
    a.vocab = h->vocab;
    a.gbest = h->gbest;
    a.gctr = h->gbest + TWD_MAX_ROWS;
    if (MODE != kModeLogits) h->epoch = epoch_after(h->epoch);  // only greedy launches count in
    a.epoch = h->epoch;
    a.next_epoch = epoch_after(h->epoch);
    a.tokens = tokens;
    a.drafts = drafts;
    a.n_drafts = n_drafts;
    a.vres = vres;
    if (rows <= 4) {
        head_small_kernel<4, kRTS, kPFS, kNWS4, MODE><<<blocks_for(h->ntiles, kRTS, kNWS4), kNWS4 * 64,
                                                      small_smem_bytes<kPFS>(rows, h->d), stream>>>(a);
    } else if (rows <= kSmallMaxRows) {
        head_small_kernel<2, kRTS, kPFS, kNWS8, MODE><<<blocks_for(h->ntiles, kRTS, kNWS8), kNWS8 * 64,
                                                      small_smem_bytes<kPFS>(rows, h->d), stream>>>(a);
    } else if (rows <= 16) {
        prep_hidden_kernel<1><<<padded_units(h->nunits) * 1, kHeadThreads, 0, stream>>>(hidden, rows, h->d,
                                                                                       h->hp, h->hx);
        head_wide_kernel<1, kRT1, MODE, kHeadWaves>
            <<<blocks_for(h->ntiles, kRT1), kHeadThreads, 0, stream>>>(a, h->hp, h->hx);
    } else if (rows <= 32) {
        prep_hidden32_kernel<1><<<padded_units(h->nunits) * 2, kHeadThreads, 0, stream>>>(hidden, rows, h->d,
                                                                                         h->hp, h->hx);
        head_wide32_kernel<kW32Pairs, 1, kW32Waves, MODE>
            <<<blocks_for(h->ntiles, 2 * kW32Pairs, kW32Waves), kW32Waves * 64, 0, stream>>>(a, h->hp, h->hx);
    } else {
        prep_hidden32_kernel<2><<<padded_units(h->nunits) * 4, kHeadThreads, 0, stream>>>(hidden, rows, h->d,
                                                                                         h->hp, h->hx);
        head_wide32_kernel<kW32Pairs, 2, kW32Waves, MODE>
            <<<blocks_for(h->ntiles, 2 * kW32Pairs, kW32Waves), kW32Waves * 64, 0, stream>>>(a, h->hp, h->hx);
    }
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

// The head pass with the final RMSNorm as its prologue: fp32 x rows (rows <= 8) and the bf16
// norm weight in, the same outputs as launch_head.
template <int MODE>
int launch_head_rmsnorm(twd_head* h, const float* x, const uint16_t* norm_w, float eps,
                        uint32_t rows, float* logits, uint32_t* tokens, const uint32_t* drafts,
                        uint32_t n_drafts, twd_verify_result* vres, hipStream_t stream) {
    if (!h) return fail(TWD_E_INVALID, "null head");
    if (!x || !aligned16(x)) return fail(TWD_E_INVALID, "x must be a 16-byte aligned device pointer");
    if (!norm_w || !aligned16(norm_w))
        return fail(TWD_E_INVALID, "norm_weight must be a 16-byte aligned device pointer");
    if (rows == 0 || rows > 8) return fail(TWD_E_INVALID, "rows must be in 1..8 with the RMSNorm prologue");
    if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(TWD_E_INVALID, "eps must be finite and >= 0");
    HeadArgs a{};
    a.tiled = h->tiled;
    a.ntiles = h->ntiles;
    a.nunits = h->nunits;
    a.h = nullptr;
    a.M = rows;
    a.d = h->d;
    a.softcap = h->softcap;
    a.logits = logits;
    a.vocab = h->vocab;
    a.gbest = h->gbest;
    a.gctr = h->gbest + TWD_MAX_ROWS;
    if (MODE != kModeLogits) h->epoch = epoch_after(h->epoch);  // only greedy launches count in
    a.epoch = h->epoch;
    a.next_epoch = epoch_after(h->epoch);
    a.tokens = tokens;
    a.drafts = drafts;
    a.n_drafts = n_drafts;
    a.vres = vres;
    if (rows <= 4) {
        // the resident-h kernel stages the normalised rows itself, two LDS rows each
        a.x = x;
        a.norm_w = norm_w;
        a.eps = eps;
        const size_t bytes = small_smem_bytes<kPFS>(2 * rows, h->d);
        if (2 * (bytes + sizeof(EpiSharedT<kNWS4>)) <= kLdsBytes)
            head_small_kernel<4, kRTS, kPFS, kNWS4, MODE, true>
                <<<blocks_for(h->ntiles, kRTS, kNWS4), kNWS4 * 64, bytes, stream>>>(a);
        else
            head_small_kernel<4, kRTS, kPFS, kNWS8, MODE, true>
                <<<blocks_for(h->ntiles, kRTS, kNWS8), kNWS8 * 64, bytes, stream>>>(a);
        TWD_HIP(hipGetLastError());
        return TWD_OK;
    }
    a.fold = 1;
    prep_rmsnorm_kernel<<<padded_units(h->nunits), kHeadThreads, 0, stream>>>(x, norm_w, eps, rows, h->d,
                                                                              h->hp, h->hx);
    head_wide_kernel<1, kRT1, MODE, kHeadWaves><<<blocks_for(h->ntiles, kRT1), kHeadThreads, 0, stream>>>(a, h->hp, h->hx);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

// The fused sample pass: the resident-h kernel in sample mode (softcap, penalty from LDS
// occurrence counts, logits store, per-wave statistics), then select_sample_merge_kernel. Used
// for rows <= 8 (rows <= 4 with the RMSNorm prologue) when the head's wave count allows it, the
// 16-wave form's counts fit beside h, and the rows' histories (where the penalty applies) hold
// at most kSampleMaxHistory ids together: every head block scans them.
constexpr uint32_t kSampleMaxHistory = 16384;

bool sample_fusable(const twd_head* h, uint32_t rows, const twd_row_params* params, bool norm) {
    if (rows == 0 || rows > kSampleRows || h->sample_blocks == 0) return false;
    if (rows > 4 && (norm || h->sample_blocks8 == 0)) return false;  // the RMSNorm form: rows <= 4
    uint64_t ids = 0;
    for (uint32_t m = 0; m < rows; ++m)
        if (params[m].repetition_penalty != 1.0f) ids += params[m].history_len;
    return ids <= kSampleMaxHistory;
}

// x/norm_w/eps select the RMSNorm prologue (x != nullptr) instead of bf16 hidden rows.
int launch_head_sample(twd_head* h, const uint16_t* hidden, const float* x, const uint16_t* norm_w,
                       float eps, uint32_t rows, const twd_row_params* params,
                       const uint32_t* history, float* logits, uint32_t* tokens, hipStream_t stream) {
    HeadArgs a{};
    a.tiled = h->tiled;
    a.ntiles = h->ntiles;
    a.nunits = h->nunits;
    a.h = hidden;
    a.M = rows;
    a.d = h->d;
    a.softcap = h->softcap;
    a.logits = logits;
    a.vocab = h->vocab;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.history = history;
    for (uint32_t m = 0; m < kSampleRows; ++m) {
        const bool live = m < rows;
        a.rp[m] = live ? params[m].repetition_penalty : 1.0f;
        // the bound apply_repetition_penalty clamps to (sampling.cpp:79), in the same fp32
        a.clamp[m] = (live && params[m].softcap > 0.0f) ? params[m].softcap * 0.9999f : 0.0f;
        a.hist_off[m] = live ? params[m].history_offset : 0u;
        a.hist_len[m] = live ? params[m].history_len : 0u;
        a.ref[m] = live ? fixed_ref(h->stats.cap, params[m]) : __builtin_nanf("");
        if (!live) continue;
        if (params[m].repetition_penalty != 1.0f && params[m].history_len > 0 && !history)
            return fail(TWD_E_INVALID, "null history with a non-empty history_len");
    }
    a.stats = h->stats;
    uint32_t waves = 0;
    if (x) {
        const size_t bytes = small_smem_bytes<kPFS>(2 * rows, h->d);
        head_small_kernel<4, kRTS, kPFS, kNWS4, kModeSample, true>
            <<<h->sample_blocks, kNWS4 * 64, bytes, stream>>>(a);
        waves = h->sample_blocks * kNWS4;
    } else if (rows <= 4) {
        head_small_kernel<4, kRTS, kPFS, kNWS4, kModeSample>
            <<<h->sample_blocks, kNWS4 * 64, small_smem_bytes<kPFS>(rows, h->d), stream>>>(a);
        waves = h->sample_blocks * kNWS4;
    } else {  // rows two apart in the MFMA's rows, one 16-wave block per CU
        head_small_kernel<2, kRTS, kPFS, kNWS8, kModeSample>
            <<<h->sample_blocks8, kNWS8 * 64, small_smem_bytes<kPFS>(rows, h->d), stream>>>(a);
        waves = h->sample_blocks8 * kNWS8;
    }
    TWD_HIP(hipGetLastError());
    static_assert(kRTS * kTileRows == kSampleWaveRows, "a wave of the sample pass owns 64 rows");
    return launch_sample_merge(h->stats, waves, logits, h->vocab, rows, params, tokens, h->sel->scratch.lng,
                               stream);
}

// Runs one call's launches with the head's cross-stream ordering around them.
template <typename F>
int ordered(twd_head* h, void* stream, F&& launches) {
    if (!h) return fail(TWD_E_INVALID, "null head");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = order_before(h->order, s);
    if (rc) return rc;
    rc = launches(s);
    const int rc2 = order_after(h->order, s);
    return rc ? rc : rc2;
}

}  // namespace

namespace twd {
int head_set_norm_weight(twd_head* h, const uint16_t* host_w, uint32_t d) {
    if (!h || !host_w || d != h->d) return fail(TWD_E_INVALID, "norm weight of the wrong length");
    if (!h->norm_w) TWD_HIP(hipMalloc(&h->norm_w, static_cast<size_t>(d) * sizeof(uint16_t)));
    TWD_HIP(hipMemcpy(h->norm_w, host_w, static_cast<size_t>(d) * sizeof(uint16_t), hipMemcpyHostToDevice));
    return TWD_OK;
}
}  // namespace twd

extern "C" {

TWD_API uint64_t twd_head_bytes(uint32_t vocab, uint32_t d_model, uint32_t group_size) {
    if (group_size == 0) return 0;
    return static_cast<uint64_t>(vocab) * (d_model / 8) * 4 +
           2ull * static_cast<uint64_t>(vocab) * (d_model / group_size) * 2;
}

TWD_API int twd_head_create_device(const void* wsb_dev, uint64_t wsb_bytes, uint32_t vocab,
                                   uint32_t d_model, uint32_t group_size, float softcap,
                                   void* stream, twd_head** out) {
    clear_error();
    if (!out || !wsb_dev) return fail(TWD_E_INVALID, "null argument");
    *out = nullptr;
    int rc = check_geometry(vocab, d_model, group_size);
    if (rc) return rc;
    if (wsb_bytes < twd_head_bytes(vocab, d_model, group_size))
        return fail(TWD_E_INVALID, "wsb_bytes is smaller than the [W|S|B] slice of this geometry");
    twd_head* h = nullptr;
    if ((rc = head_alloc(vocab, d_model, softcap, &h))) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if ((rc = head_repack(h, static_cast<const uint8_t*>(wsb_dev), s))) {
        twd_head_destroy(h);
        return rc;
    }
    uint32_t bad = 0;
    hipError_t e = hipMemcpyAsync(&bad, repack_flag(h), sizeof(bad), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        twd_head_destroy(h);
        return hip_fail(e, "repacking the LM head");
    }
    if (bad) {
        twd_head_destroy(h);
        return fail(TWD_E_UNSUPPORTED, "a group scale exceeds 2^100 in magnitude or a group bias is infinite");
    }
    *out = h;
    return TWD_OK;
}

TWD_API int twd_head_create(const void* wsb_host, uint64_t wsb_bytes, uint32_t vocab,
                            uint32_t d_model, uint32_t group_size, float softcap,
                            twd_head** out) {
    clear_error();
    if (!out || !wsb_host) return fail(TWD_E_INVALID, "null argument");
    *out = nullptr;
    int rc = check_geometry(vocab, d_model, group_size);
    if (rc) return rc;
    const uint64_t need = twd_head_bytes(vocab, d_model, group_size);
    if (wsb_bytes < need)
        return fail(TWD_E_INVALID, "wsb_bytes is smaller than the [W|S|B] slice of this geometry");
    void* staging = nullptr;
    TWD_HIP(hipMalloc(&staging, need));
    hipError_t e = hipMemcpy(staging, wsb_host, need, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(staging);
        return hip_fail(e, "uploading the LM head");
    }
    rc = twd_head_create_device(staging, need, vocab, d_model, group_size, softcap, nullptr, out);
    (void)hipFree(staging);
    return rc;
}

TWD_API void twd_head_destroy(twd_head* h) {
    if (!h) return;
    if (h->tiled) (void)hipFree(h->tiled);
    if (h->gbest) (void)hipFree(h->gbest);
    if (h->hp) (void)hipFree(h->hp);
    if (h->hx) (void)hipFree(h->hx);
    if (h->sel) twd_selector_destroy(h->sel);
    if (h->norm_w) (void)hipFree(h->norm_w);
    if (h->stats.key) (void)hipFree(h->stats.key);
    if (h->stats.sum) (void)hipFree(h->stats.sum);
    if (h->stats.max) (void)hipFree(h->stats.max);
    if (h->stats.aux) (void)hipFree(h->stats.aux);
    order_release(h->order);
    delete h;
}

TWD_API const uint16_t* twd_head_norm_weight(const twd_head* h) { return h ? h->norm_w : nullptr; }

TWD_API int twd_head_info(const twd_head* h, uint32_t* vocab, uint32_t* d_model, float* softcap,
                          uint64_t* device_bytes) {
    clear_error();
    if (!h) return fail(TWD_E_INVALID, "null head");
    if (vocab) *vocab = h->vocab;
    if (d_model) *d_model = h->d;
    if (softcap) *softcap = h->softcap;
    if (device_bytes) *device_bytes = h->tiled_bytes;
    return TWD_OK;
}

TWD_API int twd_head_logits(twd_head* h, const uint16_t* hidden, uint32_t rows, float* logits,
                            void* stream) {
    clear_error();
    if (!logits) return fail(TWD_E_INVALID, "null logits");
    return ordered(h, stream, [&](hipStream_t s) {
        return launch_head<kModeLogits>(h, hidden, rows, logits, nullptr, nullptr, 0, nullptr, s);
    });
}

TWD_API int twd_head_greedy(twd_head* h, const uint16_t* hidden, uint32_t rows, float* logits,
                            uint32_t* tokens, void* stream) {
    clear_error();
    if (!tokens) return fail(TWD_E_INVALID, "null tokens");
    return ordered(h, stream, [&](hipStream_t s) {
        return launch_head<kModeGreedy>(h, hidden, rows, logits, tokens, nullptr, 0, nullptr, s);
    });
}

TWD_API int twd_head_verify_greedy(twd_head* h, const uint16_t* hidden, uint32_t rows,
                                   const uint32_t* drafts, uint32_t n_drafts, float* logits,
                                   twd_verify_result* result, void* stream) {
    clear_error();
    if (!result) return fail(TWD_E_INVALID, "null result");
    if (n_drafts > 0 && !drafts) return fail(TWD_E_INVALID, "null drafts");
    if (n_drafts > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "n_drafts must be <= 64");
    return ordered(h, stream, [&](hipStream_t s) {
        return launch_head<kModeGreedy>(h, hidden, rows, logits, nullptr, drafts, n_drafts, result, s);
    });
}

TWD_API int twd_head_sample(twd_head* h, const uint16_t* hidden, uint32_t rows,
                            const twd_row_params* params, const uint32_t* history, float* logits,
                            uint32_t* tokens, void* stream) {
    clear_error();
    if (!logits || !tokens || !params) return fail(TWD_E_INVALID, "null logits, tokens or params");
    return ordered(h, stream, [&](hipStream_t s) {
        if (sample_fusable(h, rows, params, false)) {
            if (!hidden || !aligned16(hidden))
                return fail(TWD_E_INVALID, "hidden must be a 16-byte aligned device pointer");
            return launch_head_sample(h, hidden, nullptr, nullptr, 0.0f, rows, params, history, logits,
                                      tokens, s);
        }
        int rc = launch_head<kModeLogits>(h, hidden, rows, logits, nullptr, nullptr, 0, nullptr, s);
        if (rc) return rc;
        return launch_select(h->sel->scratch, logits, h->vocab, rows, h->vocab, params, history,
                             tokens, s);
    });
}

TWD_API int twd_head_logits_rmsnorm(twd_head* h, const float* x, const uint16_t* norm_w, float eps,
                                    uint32_t rows, float* logits, void* stream) {
    clear_error();
    if (!logits) return fail(TWD_E_INVALID, "null logits");
    return ordered(h, stream, [&](hipStream_t s) {
        return launch_head_rmsnorm<kModeLogits>(h, x, norm_w, eps, rows, logits, nullptr, nullptr, 0,
                                                nullptr, s);
    });
}

TWD_API int twd_head_greedy_rmsnorm(twd_head* h, const float* x, const uint16_t* norm_w, float eps,
                                    uint32_t rows, float* logits, uint32_t* tokens, void* stream) {
    clear_error();
    if (!tokens) return fail(TWD_E_INVALID, "null tokens");
    return ordered(h, stream, [&](hipStream_t s) {
        return launch_head_rmsnorm<kModeGreedy>(h, x, norm_w, eps, rows, logits, tokens, nullptr, 0,
                                                nullptr, s);
    });
}

TWD_API int twd_head_verify_greedy_rmsnorm(twd_head* h, const float* x, const uint16_t* norm_w,
                                           float eps, uint32_t rows, const uint32_t* drafts,
                                           uint32_t n_drafts, float* logits,
                                           twd_verify_result* result, void* stream) {
    clear_error();
    if (!result) return fail(TWD_E_INVALID, "null result");
    if (n_drafts > 0 && !drafts) return fail(TWD_E_INVALID, "null drafts");
    if (n_drafts > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "n_drafts must be <= 64");
    return ordered(h, stream, [&](hipStream_t s) {
        return launch_head_rmsnorm<kModeGreedy>(h, x, norm_w, eps, rows, logits, nullptr, drafts,
                                                n_drafts, result, s);
    });
}

TWD_API int twd_head_sample_rmsnorm(twd_head* h, const float* x, const uint16_t* norm_w, float eps,
                                    uint32_t rows, const twd_row_params* params,
                                    const uint32_t* history, float* logits, uint32_t* tokens,
                                    void* stream) {
    clear_error();
    if (!logits || !tokens || !params) return fail(TWD_E_INVALID, "null logits, tokens or params");
    return ordered(h, stream, [&](hipStream_t s) {
        if (sample_fusable(h, rows, params, true)) {
            if (!x || !aligned16(x)) return fail(TWD_E_INVALID, "x must be a 16-byte aligned device pointer");
            if (!norm_w || !aligned16(norm_w))
                return fail(TWD_E_INVALID, "norm_weight must be a 16-byte aligned device pointer");
            if (!(eps >= 0.0f) || !std::isfinite(eps)) return fail(TWD_E_INVALID, "eps must be finite and >= 0");
            return launch_head_sample(h, nullptr, x, norm_w, eps, rows, params, history, logits, tokens, s);
        }
        int rc = launch_head_rmsnorm<kModeLogits>(h, x, norm_w, eps, rows, logits, nullptr, nullptr, 0,
                                                  nullptr, s);
        if (rc) return rc;
        return launch_select(h->sel->scratch, logits, h->vocab, rows, h->vocab, params, history,
                             tokens, s);
    });
}

TWD_API void* twd_head_finish_state(const twd_head* h) {
    return h ? static_cast<void*>(h->gbest) : nullptr;
}

TWD_API int twd_generate_head(void* wsb_dev, uint32_t vocab, uint32_t d_model,
                              uint32_t group_size, uint64_t seed, void* stream) {
    clear_error();
    if (!wsb_dev) return fail(TWD_E_INVALID, "null buffer");
    if (group_size == 0 || d_model % group_size != 0 || d_model % 8 != 0)
        return fail(TWD_E_INVALID, "d_model must be a multiple of 8 and of group_size");
    const uint64_t n_words = static_cast<uint64_t>(vocab) * (d_model / 8);
    const uint64_t n_groups = static_cast<uint64_t>(vocab) * (d_model / group_size);
    uint32_t* W = static_cast<uint32_t*>(wsb_dev);
    uint16_t* S = reinterpret_cast<uint16_t*>(W + n_words);
    uint16_t* B = S + n_groups;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((n_words + 255) / 256, 1u << 16));
    generate_kernel<<<std::max(grid, 1u), 256, 0, static_cast<hipStream_t>(stream)>>>(W, S, B, n_words, n_groups, seed);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

}  // extern "C"
