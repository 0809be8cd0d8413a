// The tied INT4 group-64 LM head on gfx950: layout repack, synthetic generator, and the fused
// dequant-GEMM kernel (softcap, greedy argmax and greedy verify in its epilogue).
//
// Arithmetic (reference: shaders/Common.hlsli:163-222, src/cpu_reference.cpp:643-665):
//   logit[m][r] = sum_g s[r][g] * sum_{c in g} q[r][c] * h[m][c]  +  b[r][g] * X[m][g],
//   X[m][g] = sum_{c in g} h[m][c],  then softcap*tanh(logit/softcap).
// The inner sums run on MFMA (v_mfma_f32_16x16x32_bf16): nibbles become the exact bf16 values
// 128 + q with one and-or per pair, h is already bf16, so every product is exact and the
// accumulation is fp32. The +128 offset is removed per group through X:
//   sum (128+q) h = 128 X + sum q h  =>  logit += s * acc + (b - 128 s) * X.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>

#include "twd_internal.h"

namespace twd {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

enum HeadMode { kModeLogits = 0, kModeGreedy = 1 };  // greedy: also write block ranks

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
    // greedy finish: running per-row maxima and the arrival count, both zero between
    // launches, and where the last block puts its results
    uint64_t* gbest;    // [TWD_MAX_ROWS]
    uint32_t* gcount;
    uint32_t* tokens;
    const uint32_t* drafts;
    uint32_t n_drafts;
    twd_verify_result* vres;
};

// speculator.cpp:91-114 and :183-195, greedy branch, over per-row target tokens tok[0..rows).
__device__ void verify_bookkeeping(const uint32_t* tok, uint32_t rows, const uint32_t* drafts,
                                   uint32_t nd, twd_verify_result* v) {
    uint32_t n = 0, acc = 0, bonus = 0, sampled = 0;
    if (nd != 0 && rows != 0) {
        const uint32_t k = nd < rows ? nd : rows;
        bool rejected = false;
        for (uint32_t i = 0; i < k; ++i) {
            const uint32_t t = tok[i];
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
        if (!rejected && rows > k) {
            bonus = tok[k];
            sampled = 1;
            v->tokens[n++] = bonus;
        }
    }
    v->n_tokens = n;
    v->num_accepted = acc;
    v->total_drafted = nd;
    v->bonus_token_sampled = sampled;
    v->bonus_token = bonus;
}

// 8 nibbles of one word -> 8 bf16 values 128+q, in k-slot order [0,4,1,5,2,6,3,7].
__device__ __forceinline__ bf16x8_t nibbles_to_bf16(uint32_t w) {
    const uint32_t m = 0x000F000Fu, e = 0x43004300u;
    u32x4_t p;
    p.x = (w & m) | e;
    p.y = ((w >> 4) & m) | e;
    p.z = ((w >> 8) & m) | e;
    p.w = ((w >> 12) & m) | e;
    return __builtin_bit_cast(bf16x8_t, p);
}

// One 16-byte slice of h (8 bf16 values e0..e7) permuted into the same k-slot order.
__device__ __forceinline__ u32x4_t permute_h(u32x4_t v) {
    u32x4_t o;
    o.x = (v.x & 0xFFFFu) | (v.z << 16);
    o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
    o.z = (v.y & 0xFFFFu) | (v.w << 16);
    o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
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

// Shared memory of the head epilogue (cross-wave greedy reduction).
struct EpiShared {
    uint64_t red[kHeadWaves][TWD_MAX_ROWS];
    uint64_t seen[TWD_MAX_ROWS];
    uint32_t tok[TWD_MAX_ROWS];
    int last;
};

// Softcap, logits store, and -- for the greedy modes -- the per-row rank maximum over the
// whole grid, finished by the last block to arrive (tokens, then greedy verify bookkeeping).
//
// Cross-block publication uses device-scope atomics only: each block folds its ranks into
// gbest[m] with a returning atomic max, then counts itself in with an atomic add; the block that
// sees the final count reads and clears gbest with atomic exchanges. Returning atomics are
// performed at the memory-side coherence point before they return, so every block's maxima
// precede its arrival, and the last block observes all of them. No data travels through plain
// stores, so no device-scope fence is needed: on this part such a fence writes back the XCD's
// L2 and, paid by each of ~1000 blocks, costs more than the streaming pass itself.
// tot[j][mt][i] holds row r = (tile0 + j) * 16 + lane % 16 of m = 16 mt + 4 (lane / 16) + i.
template <int NMT, int NI, int RT, int MODE>
__device__ __forceinline__ void head_epilogue(const HeadArgs& a, f32x4_t (&tot)[RT][NMT],
                                              uint32_t tile0, EpiShared& se) {
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
            for (int i = 0; i < NI; ++i) {
                const uint32_t m = mt * 16 + 4 * (lane >> 4) + i;
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

    // rows sharing m are the 16 lanes with the same lane >> 4
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            uint64_t k = best[mt][i];
#pragma unroll
            for (int msk = 1; msk < 16; msk <<= 1) {
                const uint64_t o = shfl_xor_u64(k, msk);
                k = o > k ? o : k;
            }
            const uint32_t m = mt * 16 + 4 * (lane >> 4) + i;
            if ((lane & 15) == 0 && m < TWD_MAX_ROWS) se.red[wave][m] = k;
        }
    __syncthreads();
    const uint32_t nb = gridDim.x;
    if (static_cast<uint32_t>(tid) < a.M) {
        uint64_t k = se.red[0][tid];
#pragma unroll
        for (int w = 1; w < kHeadWaves; ++w) k = se.red[w][tid] > k ? se.red[w][tid] : k;
        // the returning form: the maximum is performed before this block counts itself in
        se.seen[tid] = __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(a.gbest + tid),
                                              static_cast<unsigned long long>(k), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0)
        se.last = __hip_atomic_fetch_add(a.gcount, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  nb - 1;
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
    if (tid == 0) {
        __hip_atomic_exchange(a.gcount, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.vres) verify_bookkeeping(se.tok, a.M, a.drafts, a.n_drafts, a.vres);
    }
}

// Per-chunk math shared by both kernels: one unit of one row tile (4 words per lane = 4 MFMA
// k-steps, two groups) against A fragments av[mt][t] and group sums xv[g][mt].
template <int NMT, int NI>
__device__ __forceinline__ void unit_mac(const u32x4_t& w, const u32x2_t& sb,
                                         const bf16x8_t (&av)[NMT][4],
                                         const f32x4_t (&xv)[2][NMT], f32x4_t (&tot)[NMT]) {
    bf16x8_t bv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) bv[t] = nibbles_to_bf16(w[t]);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const float s = g == 0 ? bf16_lo(sb.x) : bf16_hi(sb.x);
        const float b = g == 0 ? bf16_lo(sb.y) : bf16_hi(sb.y);
        const float tb = fmaf(-128.0f, s, b);
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) {
            f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][2 * g], bv[2 * g], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][2 * g + 1], bv[2 * g + 1], acc,
                                                          0, 0, 0);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                tot[mt][i] = fmaf(s, acc[i], fmaf(tb, xv[g][mt][i], tot[mt][i]));
        }
    }
}

// One 64-column group (two MFMA k-steps) of one row tile: words w0, w1 of the unit, the
// group's scale and bias from sb (g selects the half), A fragments av[mt][t] and X sums xv[mt].
template <int NMT, int NI>
__device__ __forceinline__ void group_mac(uint32_t w0, uint32_t w1, const u32x2_t& sb, int g,
                                          const bf16x8_t (&av)[NMT][2], const f32x4_t (&xv)[NMT],
                                          f32x4_t (&tot)[NMT]) {
    const bf16x8_t b0 = nibbles_to_bf16(w0), b1 = nibbles_to_bf16(w1);
    const float s = g == 0 ? bf16_lo(sb.x) : bf16_hi(sb.x);
    const float b = g == 0 ? bf16_lo(sb.y) : bf16_hi(sb.y);
    const float tb = fmaf(-128.0f, s, b);
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
        f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][0], b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][1], b1, acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < NI; ++i) tot[mt][i] = fmaf(s, acc[i], fmaf(tb, xv[mt][i], tot[mt][i]));
    }
}

template <int RT>
__device__ __forceinline__ void load_unit(const HeadArgs& a, uint32_t tile0, uint32_t U, int lane,
                                          u32x4_t (&w)[RT], u32x2_t (&sb)[RT]) {
#pragma unroll
    for (int j = 0; j < RT; ++j) {
        const uint32_t T = tile0 + j;
        if (T < a.ntiles) {
            const uint8_t* base = a.tiled + (static_cast<size_t>(T) * a.nunits + U) * kUnitBytes;
            w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base) + lane);
            sb[j] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x2_t*>(base + kUnitNibbleBytes) + (lane & 15));
        } else {
            w[j] = u32x4_t{0u, 0u, 0u, 0u};
            sb[j] = u32x2_t{0u, 0u};
        }
    }
}

// ---- M <= 8: the whole h resident in LDS, no barrier in the streaming loop ---------------------
//
// LDS holds h permuted into A-fragment order, [m][chunk U][k-step t][kg] of 16 B, plus the group
// sums [g][16]. A-fragment rows m >= M only feed output rows that are never stored, so their
// lanes simply read row 0. Each wave streams its RT row tiles through a PF-deep register ring
// of weight units, with no synchronisation until the epilogue.
template <int NI, int RT, int PF, int MODE>
__global__ __launch_bounds__(kHeadThreads) void head_small_kernel(HeadArgs a) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ EpiShared se;
    u32x4_t* sH = reinterpret_cast<u32x4_t*>(smem_raw);
    const uint32_t row_vecs = a.d / 8;  // 16 B vectors per h row
    float* sX = reinterpret_cast<float*>(sH + a.M * row_vecs);  // [groups][16]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t tile0 = (blockIdx.x * kHeadWaves + wave) * RT;
    const uint32_t groups = a.d / kGroup;

    // ---- stage h: 8 consecutive threads cover one 64-column group ----
    const uint32_t tasks = a.M * row_vecs;
    for (uint32_t base = 0; base < tasks; base += kHeadThreads) {
        const uint32_t task = base + tid;
        u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
        if (task < tasks) v = *reinterpret_cast<const u32x4_t*>(a.h + static_cast<size_t>(task) * 8);
        float s = sum8_bf16(v);
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        if (task < tasks) {
            const uint32_t m = task / row_vecs, c8 = task % row_vecs;
            const uint32_t U = c8 >> 4, c = c8 & 15;
            sH[((m * (a.d / kChunkK) + U) * 4 + (c >> 2)) * 4 + (c & 3)] = permute_h(v);
            if ((c8 & 7) == 0) sX[(c8 >> 3) * 16 + m] = s;
        }
    }
    for (uint32_t i = tid; i < groups * 16; i += kHeadThreads)
        if ((i & 15) >= a.M) sX[i] = 0.0f;
    __syncthreads();

    const uint32_t m_lane = lane & 15;
    const u32x4_t* aRow = sH + (m_lane < a.M ? m_lane : 0u) * row_vecs + (lane >> 4);
    const float* xLane = sX + 4 * (lane >> 4);

    f32x4_t tot[RT][1];
#pragma unroll
    for (int j = 0; j < RT; ++j) tot[j][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    u32x4_t wq[PF][RT];
    u32x2_t sq[PF][RT];
#pragma unroll
    for (int s = 0; s < PF; ++s)
        if (static_cast<uint32_t>(s) < a.nunits) load_unit<RT>(a, tile0, s, lane, wq[s], sq[s]);

    for (uint32_t U0 = 0; U0 < a.nunits; U0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const uint32_t U = U0 + s;
            if (U >= a.nunits) break;
            bf16x8_t av[1][4];
#pragma unroll
            for (int t = 0; t < 4; ++t) av[0][t] = __builtin_bit_cast(bf16x8_t, aRow[(U * 4 + t) * 4]);
            f32x4_t xv[2][1];
#pragma unroll
            for (int g = 0; g < 2; ++g)
                xv[g][0] = *reinterpret_cast<const f32x4_t*>(xLane + (2 * U + g) * 16);
#pragma unroll
            for (int j = 0; j < RT; ++j) unit_mac<1, NI>(wq[s][j], sq[s][j], av, xv, tot[j]);
            if (U + PF < a.nunits) load_unit<RT>(a, tile0, U + PF, lane, wq[s], sq[s]);
        }
    }
    head_epilogue<1, NI, RT, MODE>(a, tot, tile0, se);
}

// ---- any M <= 64: h staged through LDS, PF chunks of 128 columns at a time ---------------------
//
// Block = 4 waves; wave w owns RT consecutive 16-row tiles. NMT = number of 16-wide m tiles
// (1 for M <= 16, 4 for M <= 64); NI = accumulator lanes per m tile that can hold a live row.
// A stage is PF chunks: one barrier per stage, h for the next stage loaded into registers while
// this one computes, and a PF-deep register ring of weight units per row tile.
template <int NMT, int NI, int RT, int PF, int MODE>
__global__ __launch_bounds__(kHeadThreads) __attribute__((amdgpu_waves_per_eu(2)))
void head_kernel(HeadArgs a) {
    __shared__ u32x4_t sA[2][PF][NMT][4][64];
    __shared__ float sX[2][PF][2][NMT * 16];
    __shared__ EpiShared se;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const uint32_t tile0 = (blockIdx.x * kHeadWaves + wave) * RT;

    // ---- h staging: chunks [S*PF, S*PF + PF) of every live row, permuted, with group sums ----
    u32x4_t hv[PF][NMT];
    auto stage_load = [&](uint32_t S) {
#pragma unroll
        for (int u = 0; u < PF; ++u)
#pragma unroll
            for (int it = 0; it < NMT; ++it) {
                const int task = tid + kHeadThreads * it;
                const int m = task >> 4, c = task & 15;
                const uint32_t U = S * PF + u;
                hv[u][it] = u32x4_t{0u, 0u, 0u, 0u};
                if (m < static_cast<int>(a.M) && U < a.nunits)
                    hv[u][it] = *reinterpret_cast<const u32x4_t*>(
                        a.h + static_cast<size_t>(m) * a.d + U * kChunkK + c * 8);
            }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < PF; ++u)
#pragma unroll
            for (int it = 0; it < NMT; ++it) {
                const int task = tid + kHeadThreads * it;
                const int m = task >> 4, c = task & 15;
                float s = sum8_bf16(hv[u][it]);
                s += __shfl_xor(s, 1);
                s += __shfl_xor(s, 2);
                s += __shfl_xor(s, 4);
                sA[buf][u][m >> 4][c >> 2][(c & 3) * 16 + (m & 15)] = permute_h(hv[u][it]);
                if ((c & 7) == 0) sX[buf][u][c >> 3][m] = s;
            }
    };

    f32x4_t tot[RT][NMT];
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) tot[j][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    u32x4_t wq[PF][RT];
    u32x2_t sq[PF][RT];
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (static_cast<uint32_t>(u) < a.nunits) load_unit<RT>(a, tile0, u, lane, wq[u], sq[u]);
    stage_load(0);
    stage_store(0);

    const uint32_t nstages = (a.nunits + PF - 1) / PF;
    for (uint32_t S = 0; S < nstages; ++S) {
        __syncthreads();
        const int buf = S & 1;
        const bool more = (S + 1) < nstages;
        if (more) stage_load(S + 1);
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const uint32_t U = S * PF + u;
            if (U >= a.nunits) break;
            // one 64-column group at a time keeps only its two k-steps of A and X live
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                bf16x8_t av[NMT][2];
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        av[mt][t] = __builtin_bit_cast(bf16x8_t, sA[buf][u][mt][2 * g + t][lane]);
                f32x4_t xv[NMT];
#pragma unroll
                for (int mt = 0; mt < NMT; ++mt)
                    xv[mt] = *reinterpret_cast<const f32x4_t*>(&sX[buf][u][g][mt * 16 + 4 * (lane >> 4)]);
#pragma unroll
                for (int j = 0; j < RT; ++j)
                    group_mac<NMT, NI>(wq[u][j][2 * g], wq[u][j][2 * g + 1], sq[u][j], g, av, xv, tot[j]);
            }
            if (U + PF < a.nunits) load_unit<RT>(a, tile0, U + PF, lane, wq[u], sq[u]);
        }
        if (more) stage_store(buf ^ 1);
    }
    head_epilogue<NMT, NI, RT, MODE>(a, tot, tile0, se);
}

// ---- layout repack: reference [W|S|B] -> units ----------------------------------------------
__global__ void repack_kernel(const uint32_t* __restrict__ W, const uint16_t* __restrict__ S,
                              const uint16_t* __restrict__ B, uint32_t vocab, uint32_t d,
                              uint32_t ntiles, uint32_t nunits, uint8_t* __restrict__ out) {
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
                sb.x = static_cast<uint32_t>(sr[0]) | (static_cast<uint32_t>(sr[1]) << 16);
                sb.y = static_cast<uint32_t>(br[0]) | (static_cast<uint32_t>(br[1]) << 16);
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

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
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
        const uint16_t s = f32_to_bf16_rne(fmaf(9e-3f, u, 1e-3f));
        S[j] = s;
        B[j] = f32_to_bf16_rne(-8.0f * __uint_as_float(static_cast<uint32_t>(s) << 16));
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
    uint64_t* gbest = nullptr;    // [TWD_MAX_ROWS] + arrival counter, zero between launches
    twd_selector* sel = nullptr;
};

namespace {

// staged-h kernel: row tiles per wave, units per stage (measured: M = 16 -> 4 x 2, 155 us;
// M = 64 -> 2 x 2, 446 us greedy)
constexpr int kRT1 = 4, kPF1 = 2;  // M <= 16
constexpr int kRT4 = 2, kPF4 = 2;  // M <= 64
// resident-h kernel: row tiles per wave and weight units in flight (measured best on MI355X:
// M = 1 -> 2 tiles x 4 units, 122-136 us; M = 5 -> 4 tiles x 2 units, 155-165 us)
constexpr int kRTS1 = 2, kPFS1 = 4;  // M == 1
constexpr int kRTS4 = 4, kPFS4 = 2;  // 2 <= M <= 8
constexpr uint32_t kSmallMaxRows = 8;

uint32_t blocks_for(uint32_t ntiles, int rt) {
    const uint32_t per = kHeadWaves * rt;
    return (ntiles + per - 1) / per;
}

int check_geometry(uint32_t vocab, uint32_t d, uint32_t group) {
    if (group != kGroup) return fail(TWD_E_UNSUPPORTED, "group_size must be 64");
    if (vocab == 0) return fail(TWD_E_INVALID, "vocab must be > 0");
    if (d == 0 || d % kChunkK != 0) return fail(TWD_E_UNSUPPORTED, "d_model must be a positive multiple of 128");
    return TWD_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Dynamic LDS of the resident-h kernel: h permuted (M x d bf16) + group sums [d/64][16] fp32.
size_t small_smem_bytes(uint32_t rows, uint32_t d) {
    return static_cast<size_t>(rows) * d * 2 + static_cast<size_t>(d / kGroup) * 16 * 4;
}

template <typename K>
hipError_t allow_smem(K kernel, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

// Lets every resident-h instantiation use the LDS it needs for kSmallMaxRows rows of d.
int enable_small_kernels(uint32_t d) {
    const size_t bytes = small_smem_bytes(kSmallMaxRows, d);
    if (bytes > 160 * 1024) return fail(TWD_E_UNSUPPORTED, "d_model too large for the LDS-resident head");
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = allow_smem(head_small_kernel<1, kRTS1, kPFS1, kModeLogits>, bytes);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<1, kRTS1, kPFS1, kModeGreedy>, bytes);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS4, kPFS4, kModeLogits>, bytes);
    if (e == hipSuccess) e = allow_smem(head_small_kernel<4, kRTS4, kPFS4, kModeGreedy>, bytes);
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
    if (e == hipSuccess) e = hipMalloc(&h->gbest, sizeof(uint64_t) * (TWD_MAX_ROWS + 1));
    if (e == hipSuccess) e = hipMemset(h->gbest, 0, sizeof(uint64_t) * (TWD_MAX_ROWS + 1));
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

int head_repack(twd_head* h, const uint8_t* wsb_dev, hipStream_t stream) {
    const uint64_t w_bytes = static_cast<uint64_t>(h->vocab) * (h->d / 8) * 4;
    const uint64_t s_bytes = static_cast<uint64_t>(h->vocab) * (h->d / kGroup) * 2;
    const uint32_t* W = reinterpret_cast<const uint32_t*>(wsb_dev);
    const uint16_t* S = reinterpret_cast<const uint16_t*>(wsb_dev + w_bytes);
    const uint16_t* B = reinterpret_cast<const uint16_t*>(wsb_dev + w_bytes + s_bytes);
    const uint64_t work = static_cast<uint64_t>(h->ntiles) * h->nunits * 64;
    const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>((work + 255) / 256, 1u << 16));
    repack_kernel<<<grid, 256, 0, stream>>>(W, S, B, h->vocab, h->d, h->ntiles, h->nunits, h->tiled);
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
    a.gcount = reinterpret_cast<uint32_t*>(h->gbest + TWD_MAX_ROWS);
    a.tokens = tokens;
    a.drafts = drafts;
    a.n_drafts = n_drafts;
    a.vres = vres;
    if (rows == 1) {
        head_small_kernel<1, kRTS1, kPFS1, MODE><<<blocks_for(h->ntiles, kRTS1), kHeadThreads,
                                                   small_smem_bytes(rows, h->d), stream>>>(a);
    } else if (rows <= kSmallMaxRows) {
        head_small_kernel<4, kRTS4, kPFS4, MODE><<<blocks_for(h->ntiles, kRTS4), kHeadThreads,
                                                   small_smem_bytes(rows, h->d), stream>>>(a);
    } else if (rows <= 16) {
        head_kernel<1, 4, kRT1, kPF1, MODE><<<blocks_for(h->ntiles, kRT1), kHeadThreads, 0, stream>>>(a);
    } else {
        head_kernel<4, 4, kRT4, kPF4, MODE><<<blocks_for(h->ntiles, kRT4), kHeadThreads, 0, stream>>>(a);
    }
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

}  // namespace

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
    if ((rc = head_repack(h, static_cast<const uint8_t*>(wsb_dev), static_cast<hipStream_t>(stream)))) {
        twd_head_destroy(h);
        return rc;
    }
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        twd_head_destroy(h);
        return hip_fail(e, "repacking the LM head");
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
    if (h->sel) twd_selector_destroy(h->sel);
    delete h;
}

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
    return launch_head<kModeLogits>(h, hidden, rows, logits, nullptr, nullptr, 0, nullptr,
                                    static_cast<hipStream_t>(stream));
}

TWD_API int twd_head_greedy(twd_head* h, const uint16_t* hidden, uint32_t rows, float* logits,
                            uint32_t* tokens, void* stream) {
    clear_error();
    if (!tokens) return fail(TWD_E_INVALID, "null tokens");
    return launch_head<kModeGreedy>(h, hidden, rows, logits, tokens, nullptr, 0, nullptr,
                                    static_cast<hipStream_t>(stream));
}

TWD_API int twd_head_verify_greedy(twd_head* h, const uint16_t* hidden, uint32_t rows,
                                   const uint32_t* drafts, uint32_t n_drafts, float* logits,
                                   twd_verify_result* result, void* stream) {
    clear_error();
    if (!result) return fail(TWD_E_INVALID, "null result");
    if (n_drafts > 0 && !drafts) return fail(TWD_E_INVALID, "null drafts");
    if (n_drafts > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "n_drafts must be <= 64");
    return launch_head<kModeGreedy>(h, hidden, rows, logits, nullptr, drafts, n_drafts, result,
                                    static_cast<hipStream_t>(stream));
}

TWD_API int twd_head_sample(twd_head* h, const uint16_t* hidden, uint32_t rows,
                            const twd_row_params* params, const uint32_t* history, float* logits,
                            uint32_t* tokens, void* stream) {
    clear_error();
    if (!h) return fail(TWD_E_INVALID, "null head");
    if (!logits || !tokens || !params) return fail(TWD_E_INVALID, "null logits, tokens or params");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = launch_head<kModeLogits>(h, hidden, rows, logits, nullptr, nullptr, 0, nullptr, s);
    if (rc) return rc;
    return launch_select(h->sel->scratch, logits, h->vocab, rows, h->vocab, params, history,
                         tokens, s);
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
