// Speculative verify with draft logits on gfx950: the rejection-sampling branch of
// SpeculativeCoordinator::evaluate_verification (src/speculator.cpp:71-122, with compute_softmax
// of :14-30), composed with the sample-and-compare and bonus steps the selector already runs.
//
// The reference computes, per position with draft probabilities, two fp32 softmaxes whose sums
// run sequentially in index order, a ratio test p/q against a uniform, and on rejection a draw
// from (p - q)+ by a sequential fp32 prefix sum. Token ids only match the reference if those
// sequential float sums are reproduced bit for bit, so the device recomputes them exactly
// (block_seq_sum and the segmented form below) instead of summing in a tree.
//
// Kernels, on the caller's stream:
//   draft_max_kernel     grid (parts, 2P): per row, partial maxima of l / T (T = 1 when <= 0)
//   draft_exp_kernel     grid (parts, 2P): e = expf(l / T - max) to scratch, NaN flags, and the
//                        double sums of the exact sums' head and segments
//   seg_xfer_kernel, seg_sum_kernel: each softmax's sequential sum
//   seg_ratio_dsum_kernel  the ratio tests, and each rejected position's segment double sums
//   seg_xfer_kernel, seg_residual_kernel: each rejected position's residual sum and draw
//   (seg_residual_kernel's last block: the accept chain over all positions, bonus, result)
// where P is the number of positions with a draft row. The target tokens of the other
// positions, of the fallback and of the bonus row come from the selection code of select.hip,
// run inside two of these launches: draft_max_kernel's extra grid rows write the target rows'
// wave records (wave_records_block) and seg_sum_kernel's extra blocks merge them
// (sample_merge_row), so the selection adds no launch and no stream synchronisation. Target rows
// with shortlists longer than 256 take the selector's own launches (launch_select) on a side
// stream instead, joined before seg_residual_kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "expf_libm.h"
#include "select_core.h"
#include "twd_internal.h"

// Every float expression in this file rounds each operation on its own: hipcc would otherwise
// fuse a * b - c * d into an fma, which the reference's x86-64 build never does.
#pragma clang fp contract(off)

namespace twd {

constexpr int kDraftThreads = 256;   // max / exp kernels
constexpr int kDraftPer = 8;
constexpr uint32_t kDraftChunk = kDraftThreads * kDraftPer;  // entries per block and row
constexpr uint32_t kDraftMaxParts = 128;                     // vocab <= 524288
constexpr int kRejThreads = 1024;    // one block per position
constexpr int kRejWaves = kRejThreads / 64;
constexpr int kRejPer = 16;          // terms per thread per window
constexpr uint32_t kRejWin = kRejThreads * kRejPer;
constexpr uint32_t kNoEvent = 0xFFFFFFFFu;

// Segments of the exact sums (the segmented form below): the first kSegHead terms of a row are
// summed serially, the rest in segments of kSegLen.
constexpr uint32_t kSegHead = 2048;                   // a multiple of kSegLen, <= kDraftChunk
constexpr uint32_t kSegLen = 512;                    // terms per segment after the head
constexpr int kSegPer = kSegLen / 64;                // terms per lane when one wave sums a segment
constexpr uint32_t kSegMax = (1u << 19) / kSegLen;  // segments per row (vocab <= 2048 + 2^19)
static_assert(kSegLen % 256 == 0 && kSegPer % 4 == 0, "whole waves, 16-byte lane loads");
static_assert(kSegMax % 64 == 0, "whole lane strides over the segment double sums");
// draft_exp_kernel's blocks also form the double sums of the head and the segments: a block's
// kDraftChunk entries are kDraftChunk / kSegLen whole parts of kSegLen, the first
// kSegHead / kSegLen parts of the row being the head's
static_assert(kSegHead % kSegLen == 0 && kSegHead <= kDraftChunk && kDraftChunk % kSegLen == 0 &&
                  kSegLen % kDraftThreads == 0,
              "a draft chunk holds whole parts of the head or of segments");

__host__ __device__ inline uint32_t seg_count(uint32_t n) {
    return n > kSegHead ? (n - kSegHead + kSegLen - 1) / kSegLen : 0u;
}

struct DraftPos {
    const float* target;  // row of vocab logits
    const float* draft;
    uint32_t position;    // index i in the draft chain
    float u1, u2;         // the two mt19937_64 draws of step_seed (speculator.cpp:87-89,105)
};

struct DraftArgs {
    uint32_t vocab;
    uint32_t estride;             // row stride of e: vocab rounded up to 16 floats
    uint32_t parts;
    uint32_t npos;
    float temp;                   // compute_softmax's temperature (1 when <= 0)
    const uint32_t* drafts;       // device, draft ids by position
    float* part;                  // [2P][parts] partial maxima
    float* e;                     // [2P][vocab] expf(l / T - max)
    uint32_t* flags;              // [2P] bit 0: a NaN term
    float* sums;                  // [2P] compute_softmax sums
    double* seg_d;                // [2P][segments + 1] double sums of the head and each segment
    uint32_t* xin;                // [2P][kSegMax][2][64] the segments' crossing data
    uint32_t* rej;                // [64][4] {accepted, token, fallback, valid}
    DraftPos pos[TWD_MAX_ROWS];
};


// The target rows' selection inside the draft chain's launches (rows 0 .. nsel - 1 of the
// target logits, all with the parameters `base` and their own uniforms): records by
// draft_max_kernel's grid rows 2P .. 2P + nsel - 1, the merges by seg_sum_kernel's blocks
// 2P .. 2P + nsel - 1. nsel = 0: the selection runs elsewhere.
struct DraftSelect {
    uint32_t nsel;
    twd_row_params base;
    float u[TWD_MAX_ROWS + 1];
    WaveStatsBufs wb;     // the target rows' records
    SampleMergeBufs mb;   // and their merge, tokens into the selector's verify tokens
};

__device__ __forceinline__ const float* draft_row(const DraftArgs& a, uint32_t r) {
    return (r & 1) ? a.pos[r >> 1].draft : a.pos[r >> 1].target;
}

__global__ __launch_bounds__(kDraftThreads) void draft_max_kernel(DraftArgs a, DraftSelect sel) {
    static_assert(kDraftThreads == kWsThreads && kDraftChunk == kWsEntries, "a record block per draft chunk");
    const uint32_t r = blockIdx.y;
    if (r >= 2 * a.npos) {  // the whole block: the target row's records over this chunk
        __shared__ double tbl[64];
        wave_records_block<1>(sel.wb, blockIdx.x, r - 2 * a.npos, tbl);
        return;
    }
    const float* l = draft_row(a, r);
    const uint32_t base = blockIdx.x * kDraftChunk + threadIdx.x;
    // every load issued before any is used (indices past the row clamped to its last entry and
    // their values ignored), so the block waits for memory once
    float xs[kDraftPer];
#pragma unroll
    for (int it = 0; it < kDraftPer; ++it) xs[it] = l[min(base + it * kDraftThreads, a.vocab - 1u)];
    float m = -1e9f;
#pragma unroll
    for (int it = 0; it < kDraftPer; ++it) {
        const uint32_t j = base + it * kDraftThreads;
        if (j < a.vocab) {
            const float x = xs[it] / a.temp;
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
    // (both ignore NaN, start from -1e9f, and equal values are interchangeable). The partial
    // maxima are requested at once, one per thread, then reduced over the block: none is NaN,
    // so the order of the comparisons does not matter.
    __shared__ float red[kDraftThreads / 64];
    const uint32_t base = blockIdx.x * kDraftChunk + threadIdx.x;
    float xs[kDraftPer];  // the row's entries requested first, as in draft_max_kernel
#pragma unroll
    for (int it = 0; it < kDraftPer; ++it) xs[it] = l[min(base + it * kDraftThreads, a.vocab - 1u)];
    float mx = -1e9f;
    for (uint32_t p = threadIdx.x; p < a.parts; p += kDraftThreads) {
        const float y = a.part[r * a.parts + p];
        mx = y > mx ? y : mx;
    }
    mx = wave_reduce(mx, -1e9f, [](float u, float v) { return v > u ? v : u; });
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kDraftThreads / 64; ++w) mx = red[w] > mx ? red[w] : mx;
    bool nan = false;
    float* e = a.e + static_cast<size_t>(r) * a.estride;
    constexpr int kSegsPerChunk = kDraftChunk / kSegLen;
    double ds[kSegsPerChunk] = {};  // this thread's share of each segment's double sum
#pragma unroll
    for (int it = 0; it < kDraftPer; ++it) {
        const uint32_t j = base + it * kDraftThreads;
        if (j < a.vocab) {
            const float x = xs[it] / a.temp;
            const float v = expf_libm<true>(x - mx);  // std::exp(float) of speculator.cpp:23
            nan |= (v != v);
            e[j] = v;
            ds[it * kDraftThreads / kSegLen] += static_cast<double>(v);
        }
    }
    // the segments' double sums, which only predict binades (any order will do)
    __shared__ double dsw[kDraftThreads / 64][kSegsPerChunk];
#pragma unroll
    for (int k = 0; k < kSegsPerChunk; ++k) {
        const double w = wave_reduce(ds[k], 0.0, [](double u, double v) { return u + v; });
        if ((threadIdx.x & 63) == 0) dsw[threadIdx.x >> 6][k] = w;
    }
    if (__syncthreads_or(nan) && threadIdx.x == 0)
        __hip_atomic_fetch_or(a.flags + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x < kSegsPerChunk) {
        constexpr uint32_t kHeadParts = kSegHead / kSegLen;
        const uint32_t k = threadIdx.x, nseg = seg_count(a.vocab);
        const uint32_t g = blockIdx.x * kSegsPerChunk + k;  // the part of the row
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < kDraftThreads / 64; ++w) t += dsw[w][k];
        double* d = a.seg_d + static_cast<size_t>(r) * (nseg + 1);
        if (blockIdx.x == 0 && k == 0) {  // the head: its parts together
            double h = 0.0;
#pragma unroll
            for (uint32_t q = 0; q < kHeadParts; ++q)
#pragma unroll
                for (int w = 0; w < kDraftThreads / 64; ++w) h += dsw[w][q];
            d[0] = h;
        }
        if (g >= kHeadParts && g - kHeadParts < nseg) d[1 + g - kHeadParts] = t;
    }
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
// the scan restarts after it with the new binade's unit. Increments saturate at 2^30: any
// prefix that large has left the binade, and saturating addition stays associative.

constexpr uint32_t kSat = 1u << 30;
constexpr uint32_t kL = 1u << 24;  // S / u at the top of a binade
constexpr int kMarks = 128;         // recorded (k0, S) window starts, for a later search
constexpr uint32_t kSerialUntil = 2048;  // terms summed one by one, in order, at the start

struct Xfer {  // input parity p -> (total increment, output parity)
    uint32_t inc0, inc1;
    uint32_t out;  // bit p: output parity for input parity p
};

__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return min(a + b, kSat); }

__device__ __forceinline__ Xfer xfer_id() { return Xfer{0u, 0u, 2u}; }

// f, then g
__device__ __forceinline__ Xfer xfer_then(const Xfer& f, const Xfer& g) {
    const uint32_t f0 = f.out & 1u, f1 = (f.out >> 1) & 1u;
    Xfer h;
    h.inc0 = sat_add(f.inc0, f0 ? g.inc1 : g.inc0);
    h.inc1 = sat_add(f.inc1, f1 ? g.inc1 : g.inc0);
    h.out = ((g.out >> f0) & 1u) | (((g.out >> f1) & 1u) << 1);
    return h;
}

__device__ __forceinline__ Xfer xfer_shfl_up(const Xfer& x, int d) {
    return Xfer{static_cast<uint32_t>(__shfl_up(x.inc0, d)), static_cast<uint32_t>(__shfl_up(x.inc1, d)),
                static_cast<uint32_t>(__shfl_up(x.out, d))};
}

// The value of a lane CTRL selects (a DPP row shift or row broadcast), or the identity where the
// source lies outside the row or the destination row is masked off: a scan step in a few VALU
// cycles, without the LDS round trip of a permute.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ Xfer xfer_dpp(const Xfer& x) {
    const Xfer id = xfer_id();
    return Xfer{static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(id.inc0), static_cast<int>(x.inc0),
                                                                  CTRL, ROW_MASK, 0xF, false)),
                static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(id.inc1), static_cast<int>(x.inc1),
                                                                  CTRL, ROW_MASK, 0xF, false)),
                static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(id.out), static_cast<int>(x.out),
                                                                  CTRL, ROW_MASK, 0xF, false))};
}
constexpr int kDppRowShr = 0x110;     // + n: row_shr:n
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kDppRowBcast31 = 0x143;  // lane 31 to rows 2 and 3

// Inclusive scan of the 64 lanes' transfer functions, lane order (earlier lanes applied first).
__device__ __forceinline__ Xfer xfer_wave_scan(Xfer v) {
    v = xfer_then(xfer_dpp<kDppRowShr + 1, 0xF>(v), v);
    v = xfer_then(xfer_dpp<kDppRowShr + 2, 0xF>(v), v);
    v = xfer_then(xfer_dpp<kDppRowShr + 4, 0xF>(v), v);
    v = xfer_then(xfer_dpp<kDppRowShr + 8, 0xF>(v), v);
    v = xfer_then(xfer_dpp<kDppRowBcast15, 0xA>(v), v);
    v = xfer_then(xfer_dpp<kDppRowBcast31, 0xC>(v), v);
    return v;
}

// Inclusive scan of the lanes' increments under saturating addition, lane order, by the DPP
// steps of xfer_wave_scan (lanes outside a step's source row take 0).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t inc_dpp(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ uint32_t inc_wave_scan(uint32_t v) {
    v = sat_add(inc_dpp<kDppRowShr + 1, 0xF>(v), v);
    v = sat_add(inc_dpp<kDppRowShr + 2, 0xF>(v), v);
    v = sat_add(inc_dpp<kDppRowShr + 4, 0xF>(v), v);
    v = sat_add(inc_dpp<kDppRowShr + 8, 0xF>(v), v);
    v = sat_add(inc_dpp<kDppRowBcast15, 0xA>(v), v);
    v = sat_add(inc_dpp<kDppRowBcast31, 0xC>(v), v);
    return v;
}

// Lane l's value, for a wave-uniform l: a register read, where a shuffle is an LDS round trip.
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int l) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}
__device__ __forceinline__ float lane_f32(float v, int l) { return __uint_as_float(lane_u32(__float_as_uint(v), l)); }

__device__ __forceinline__ Xfer xfer_shfl(const Xfer& x, int src) {
    return Xfer{static_cast<uint32_t>(__shfl(x.inc0, src)), static_cast<uint32_t>(__shfl(x.inc1, src)),
                static_cast<uint32_t>(__shfl(x.out, src))};
}

// Term a >= 0 in units of u = 2^(E - 23): floor k (saturated), and kind 0 exact or rounds
// down, 1 rounds up, 2 exactly half-way. Branch-free: a zero term, or one below u / 2 (shift
// >= 25), comes out as k = 0, kind 0; one at least u * 2^24 saturates.
__device__ __forceinline__ void split_term(float a, int E, uint32_t& k, uint32_t& kind) {
    const uint32_t b = __float_as_uint(a);
    const uint32_t f = b >> 23;
    const uint32_t m = (b & 0x7FFFFFu) | (f ? 0x800000u : 0u);
    const int sh = E - (max(static_cast<int>(f), 1) - 127);
    const int shc = min(max(sh, 1), 31);
    const uint32_t rem = m & ((1u << shc) - 1u), half = 1u << (shc - 1);
    const uint32_t kr = rem > half ? 1u : (rem == half ? 2u : 0u);
    k = sh > 0 ? (m >> shc) : (sh == 0 ? m : kSat);
    kind = sh > 0 ? kr : 0u;
}

__device__ __forceinline__ Xfer term_xfer(uint32_t k, uint32_t kind) {
    const uint32_t c = k + (kind & 1u), cp = c & 1u;
    const uint32_t kp = k & 1u;
    const bool tie = kind == 2u;  // ties go to the even neighbour
    return Xfer{tie ? k + kp : c, tie ? k + (kp ^ 1u) : c, tie ? 0u : (cp | ((cp ^ 1u) << 1))};
}

__device__ __forceinline__ uint32_t term_inc(uint32_t k, uint32_t kind, uint32_t par) {
    return k + (kind == 2u ? ((par + k) & 1u) : kind);
}

struct SeqShared {
    Xfer wave_total[kRejWaves];
    uint32_t event;
    float S;
    uint32_t k0;
    uint32_t stop;
    uint32_t n_marks;
    uint32_t mark_k0[kMarks];
    float mark_S[kMarks];
    // the first terms, for the serial start: every thread stages four, so the array spans
    // 4 * kRejThreads entries although only [0, kSerialUntil) is read
    float head[4 * kRejThreads];
};
static_assert(kSerialUntil <= 4 * kRejThreads, "the serial start is staged in one pass");

// s + t[0] + t[1] + ... + t[n - 1], added in order (n a multiple of 16, t in LDS): the next
// sixteen terms are read while the current sixteen are added, so the reads' latency hides
// behind the chain of adds.
__device__ __forceinline__ float serial_sum16(const float* t, uint32_t n, float s) {
    float c[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) c[q] = t[q];
    for (uint32_t j = 16; j < n; j += 16) {
        float nx[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) nx[q] = t[j + q];
#pragma unroll
        for (int q = 0; q < 16; ++q) s += c[q];
#pragma unroll
        for (int q = 0; q < 16; ++q) c[q] = nx[q];
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) s += c[q];
    return s;
}

// One window of block_seq_sum: PER terms per thread from the 16-aligned start a0 <= k0; terms
// before k0 or at n and beyond count as zero. load(j0, a) fills a[0..PER) with terms j0.. (j0
// a multiple of PER, in range or not), term(j) gives one term.
template <int PER, typename Load, typename Term>
__device__ __forceinline__ void seq_window(Load load, Term term, uint32_t n, float& S, uint32_t& k0,
                                           float thr, bool want_stop, uint32_t& stop, SeqShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr uint32_t kWin = kRejThreads * PER;
    // the binade of S: S = B * 2^(E - 23) with B < 2^24
    const uint32_t sb = __float_as_uint(S);
    const uint32_t sf = sb >> 23;
    const int E = sf ? static_cast<int>(sf) - 127 : -126;
    const uint32_t B = sf ? ((sb & 0x7FFFFFu) | 0x800000u) : sb;
    const uint32_t p0 = B & 1u;
    // the prefix threshold in units of u: R >= thr / u <=> R >= ceil(thr / u) for integer R
    uint32_t Tu = 0xFFFFFFFFu;
    if (want_stop) {
        const double t = ceil(ldexp(static_cast<double>(thr), 23 - E));
        Tu = t <= 0.0 ? 0u : (t >= 4294967295.0 ? 0xFFFFFFFFu : static_cast<uint32_t>(t));
    }

    const uint32_t a0 = k0 & ~(kRejPer - 1u);
    const uint32_t j0 = a0 + static_cast<uint32_t>(tid) * PER;
    uint32_t kk[PER], kd[PER];
    Xfer t = xfer_id();
    {
        // rows are padded to a multiple of 16 floats: a load starting below that end stays in
        // the row, one starting at or past it is skipped (its terms are all past n)
        float a[PER];
        if (j0 < ((n + 15u) & ~15u)) {
            load(j0, a);
        } else {
#pragma unroll
            for (int q = 0; q < PER; ++q) a[q] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const uint32_t j = j0 + q;
            split_term((j >= k0 && j < n) ? a[q] : 0.0f, E, kk[q], kd[q]);
            t = xfer_then(t, term_xfer(kk[q], kd[q]));
        }
    }
    // wave inclusive scan
    const Xfer inc = xfer_wave_scan(t);
    Xfer ex = xfer_shfl_up(inc, 1);
    if (lane == 0) ex = xfer_id();
    if (lane == 63) sh.wave_total[wave] = inc;
    if (tid == 0) sh.event = kNoEvent;
    __syncthreads();
    // prefix over the waves before this one: a 16-lane scan of the wave totals
    static_assert(kRejWaves == 16, "the wave totals fill one DPP row");
    Xfer wt = lane < kRejWaves ? sh.wave_total[lane] : xfer_id();
    wt = xfer_then(xfer_dpp<kDppRowShr + 1, 0xF>(wt), wt);
    wt = xfer_then(xfer_dpp<kDppRowShr + 2, 0xF>(wt), wt);
    wt = xfer_then(xfer_dpp<kDppRowShr + 4, 0xF>(wt), wt);
    wt = xfer_then(xfer_dpp<kDppRowShr + 8, 0xF>(wt), wt);
    Xfer wp = xfer_shfl(wt, wave > 0 ? wave - 1 : 0);
    if (wave == 0) wp = xfer_id();
    const Xfer in = xfer_then(wp, ex);

    // replay: the first term that leaves the binade (an exact add follows), or whose prefix
    // reaches thr. A thread entering at R >= 2^24 follows an earlier thread's event.
    uint32_t R = sat_add(B, p0 ? in.inc1 : in.inc0);
    uint32_t par = (in.out >> p0) & 1u;
    uint32_t my_event = kNoEvent;
    uint32_t R_before = R;
    bool live = R < kL;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const uint32_t j = j0 + q;
        const uint32_t d = term_inc(kk[q], kd[q], par);
        const bool go = live && j >= k0 && j < n;
        const bool cross = go && (R + d >= kL);
        const bool adv = go && !cross;
        if (cross) {
            my_event = 2 * j;
            R_before = R;
        }
        R = adv ? R + d : R;
        par = adv ? ((par + d) & 1u) : par;
        const bool hit = adv && R >= Tu;
        if (hit) my_event = 2 * j + 1;
        live = live && !cross && !hit;
    }
    if (my_event != kNoEvent) atomicMin(&sh.event, my_event);
    __syncthreads();
    const uint32_t ev = sh.event;
    if (ev == kNoEvent) {
        if (tid == kRejThreads - 1) {
            sh.S = ldexpf(static_cast<float>(R), E - 23);
            sh.k0 = min(n, a0 + kWin);
            sh.stop = n;
        }
    } else if (my_event == ev) {
        const uint32_t j = ev >> 1;
        if (ev & 1) {  // reaches thr, no binade change before it
            sh.S = ldexpf(static_cast<float>(R), E - 23);
            sh.k0 = n;
            sh.stop = j;
        } else {
            const float s_new = ldexpf(static_cast<float>(R_before), E - 23) + term(j);
            const bool hit = want_stop && s_new >= thr;
            sh.S = s_new;
            sh.k0 = hit ? n : j + 1;
            sh.stop = hit ? j : n;
        }
    }
    __syncthreads();
    S = sh.S;
    k0 = sh.k0;
    stop = sh.stop;
    __syncthreads();  // sh is rewritten by the next window
}

// Continues the sequential sum from prefix S (the sum of terms [0, k0)) over terms [k0, n).
// Returns the sum; *stop_at (when non-null) receives the first index whose prefix is >= thr, or
// n when none is. With `record`, the start (k0, S) of every window is kept in sh's marks.
// Windows are short (4 terms per thread) while k0 < kShortUntil, where the sum still changes
// binade often and each change discards the rest of its window, and long (16) after.
constexpr uint32_t kShortUntil = 65536;

template <typename Load, typename Term>
__device__ float block_seq_sum(Load load, Term term, uint32_t n, float S, uint32_t k0, float thr,
                               uint32_t* stop_at, bool record, SeqShared& sh) {
    const bool want_stop = stop_at != nullptr;
    uint32_t stop = n;
    if (record && threadIdx.x == 0) sh.n_marks = 0;
    if (k0 < kSerialUntil) {
        // The head of the sequence, where the sum changes binade at almost every doubling of
        // its length: staged in LDS by the whole block, then added one term at a time, in
        // order, by wave 0 -- the sequential loop itself, with no window restarts.
        if (record && threadIdx.x == 0) {
            sh.mark_k0[0] = k0;
            sh.mark_S[0] = S;
            sh.n_marks = 1;
        }
        const uint32_t end = min(n, kSerialUntil);
        for (uint32_t base = 0; base < kSerialUntil; base += kRejThreads * 4) {
            const uint32_t j0 = base + threadIdx.x * 4;
            float a[4];
            if (j0 < ((n + 15u) & ~15u)) {
                load(j0, a);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) a[q] = 0.0f;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) sh.head[j0 + q] = a[q];
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            float s = S;
            uint32_t hit = n;
            if (want_stop) {
                for (uint32_t j = k0; j < end; ++j) {
                    s += sh.head[j];
                    if (s >= thr) {
                        hit = j;
                        break;
                    }
                }
            } else {
                // no exit: sixteen terms read at a time, then added in order
                uint32_t j = k0;
                for (; j + 16 <= end; j += 16) {
                    float t[16];
#pragma unroll
                    for (int q = 0; q < 16; ++q) t[q] = sh.head[j + q];
#pragma unroll
                    for (int q = 0; q < 16; ++q) s += t[q];
                }
                for (; j < end; ++j) s += sh.head[j];
            }
            if (threadIdx.x == 0) {
                sh.S = s;
                sh.k0 = hit < n ? n : end;
                sh.stop = hit;
            }
        }
        __syncthreads();
        S = sh.S;
        k0 = sh.k0;
        stop = sh.stop;
        __syncthreads();
    }
    while (k0 < n) {
        if (record && threadIdx.x == 0 && sh.n_marks < kMarks) {
            sh.mark_k0[sh.n_marks] = k0;
            sh.mark_S[sh.n_marks] = S;
            ++sh.n_marks;
        }
        if (k0 < kShortUntil)
            seq_window<4>(load, term, n, S, k0, thr, want_stop, stop, sh);
        else
            seq_window<kRejPer>(load, term, n, S, k0, thr, want_stop, stop, sh);
    }
    if (want_stop) *stop_at = stop;
    return S;
}

// PER consecutive floats from a 16 B aligned row position (row stride padded to 16 floats, so
// reads past n stay inside the row's allocation)
template <int PER>
__device__ __forceinline__ void load_row(const float* row, uint32_t j0, float (&a)[PER]) {
    const float4* p = reinterpret_cast<const float4*>(row + j0);
#pragma unroll
    for (int v = 0; v < PER / 4; ++v) {
        const float4 x = p[v];
        a[4 * v] = x.x;
        a[4 * v + 1] = x.y;
        a[4 * v + 2] = x.z;
        a[4 * v + 3] = x.w;
    }
}

// ---- the segmented form: the same exact sums, spread over the GPU ---------------------------------
//
// block_seq_sum runs one row on one CU. Here a row's terms after the serial head are cut into
// segments of kSegLen, and three launches sum them exactly:
//   double sums      (a wave per segment): each segment's sum in double, and the head's
//                    (seg_dsum_kernel; for the softmax rows draft_exp_kernel forms them, for
//                    the residual seg_ratio_dsum_kernel);
//   seg_xfer_kernel  (a wave per segment): the double prefix D before the segment predicts the
//                    binade of the fp32 running sum there. For that binade and its nearer
//                    neighbour the segment's terms become transfer functions (as in a window of
//                    block_seq_sum) and their ordered composition is the segment's record.
//                    Block 0 of each row adds the head serially;
//   a chain kernel   (one block per row): from the head's sum, wave 0 walks the records 64 at
//                    a time: when the exact sum S at a segment start lies in one of the record's
//                    two binades, and the composed increment keeps it there (and below a stop
//                    threshold), S jumps to the segment's end; otherwise (a binade change, a
//                    wrong prediction, the stop) the wave sums that one segment exactly with
//                    wave_seg_sum, and the walk resumes.
// A prediction only decides which transfer functions are ready; the walk checks every record
// against the exact S, so a wrong prediction costs one exact segment, never a wrong sum. No
// block waits on another: the launches are ordered on the stream.
static_assert(kSegHead <= kSerialUntil, "block_seq_sum adds a head in order");

struct SegRec {
    int E[2];   // the two candidate binades (exponents of S's leading bit; -126: below 2^-125)
    Xfer f[2];  // the segment's composed transfer functions in units of 2^(E - 23)
    // crossing data, written where the double sums predict a binade change inside the segment:
    // bit 0 present; bit 1 + c: candidate c's terms hold no exact half-way case. The data itself
    // (kXinWords per segment): per candidate c and lane l, the increments of lanes 0 .. l in c's
    // units (the lanes' inclusive scan, saturating)
    uint32_t xl;
};
constexpr uint32_t kXinWords = 2 * 64;

struct SegHead {  // the serial head's sum; with a stop, the first index whose prefix reaches thr
    float S;
    uint32_t stop;   // n when none in the head does
};

// Term sources: active(row) and term(row, j) for j < n (the kernels give zero past n).
struct SegSrcArray {  // one plain array (twd_sequential_sum)
    const float* x;
    __device__ bool active(uint32_t) const { return true; }
    __device__ float term(uint32_t, uint32_t j) const { return x[j]; }
};
struct SegSrcSoftmax {  // the e rows of compute_softmax, NaN rows skipped
    const float* e;
    uint32_t estride;
    const uint32_t* flags;
    __device__ bool active(uint32_t r) const { return !(flags[r] & 1u); }
    __device__ float term(uint32_t r, uint32_t j) const { return e[static_cast<size_t>(r) * estride + j]; }
};
struct SegSrcResidual {  // (p - q)+ of a rejected position (draft_reject_kernel's diff)
    const float* e;
    uint32_t estride;
    const float* sums;
    const uint32_t* live;  // [P] 1: the position was rejected
    __device__ bool active(uint32_t pi) const { return live[pi] != 0u; }
    __device__ float term(uint32_t pi, uint32_t j) const {
        const float sp = sums[2 * pi], sq = sums[2 * pi + 1];
        const float inv_p = 1.0f / (sp > 1e-12f ? sp : 1.0f);
        const float inv_q = 1.0f / (sq > 1e-12f ? sq : 1.0f);
        const float pt = e[static_cast<size_t>(2 * pi) * estride + j];
        const float qd = e[static_cast<size_t>(2 * pi + 1) * estride + j];
        const float x = pt * inv_p - qd * inv_q;
        return (0.0f < x) ? x : 0.0f;
    }
};

// The segment kernels' shape: one wave per segment, kXferSegs segments per block, no barrier
// (block 0 of a row takes the head)
constexpr int kXferThreads = 256;
constexpr uint32_t kXferSegs = kXferThreads / 64;
__host__ __device__ inline uint32_t xfer_blocks(uint32_t n) { return 1u + (seg_count(n) + kXferSegs - 1u) / kXferSegs; }
static_assert(kSegLen == 64 * kSegPer && kSegHead % kXferThreads == 0, "a wave per segment, whole head strides");

// Block b of row `row` (kXferThreads threads): b = 0 the head's double sum into d[row][0]; in
// block b >= 1, wave w segment s = (b - 1) kXferSegs + w into d[row][1 + s]. Every term is
// requested before any is added (indices clamped into the row, values past its end dropped).
template <class Src>
__device__ __forceinline__ void seg_dsum_block(const Src& src, uint32_t row, uint32_t b, uint32_t n, double* d,
                                               double* red) {
    const uint32_t nseg = seg_count(n);
    const int lane = threadIdx.x & 63;
    double* dr = d + static_cast<size_t>(row) * (nseg + 1);
    if (b == 0) {
        const uint32_t nh = min(n, kSegHead);
        constexpr int kPer = kSegHead / kXferThreads;
        float v[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) v[q] = src.term(row, min(threadIdx.x + q * kXferThreads, n - 1u));
        double t = 0.0;
#pragma unroll
        for (int q = 0; q < kPer; ++q) t += threadIdx.x + q * kXferThreads < nh ? static_cast<double>(v[q]) : 0.0;
        t = wave_reduce(t, 0.0, [](double x, double y) { return x + y; });
        if (lane == 0) red[threadIdx.x >> 6] = t;
        __syncthreads();
        if (threadIdx.x == 0) {
            double h = red[0];
            for (uint32_t w = 1; w < kXferSegs; ++w) h += red[w];
            dr[0] = h;
        }
        return;
    }
    const uint32_t s = (b - 1) * kXferSegs + (threadIdx.x >> 6);
    if (s >= nseg) return;  // the whole wave
    const uint32_t j0 = kSegHead + s * kSegLen + static_cast<uint32_t>(lane) * kSegPer;
    float v[kSegPer];
#pragma unroll
    for (int q = 0; q < kSegPer; ++q) v[q] = src.term(row, min(j0 + q, n - 1u));
    double t = 0.0;
#pragma unroll
    for (int q = 0; q < kSegPer; ++q) t += j0 + q < n ? static_cast<double>(v[q]) : 0.0;
    t = wave_reduce(t, 0.0, [](double x, double y) { return x + y; });
    if (lane == 0) dr[1 + s] = t;
}

// grid (xfer_blocks(n), rows): the head's and the segments' double sums
template <class Src>
__global__ __launch_bounds__(kXferThreads) void seg_dsum_kernel(Src src, uint32_t n, double* d) {
    __shared__ double red[kXferSegs];
    const uint32_t row = blockIdx.y;
    if (!src.active(row)) return;  // the whole block
    seg_dsum_block(src, row, blockIdx.x, n, d, red);
}

// grid (xfer_blocks(n), rows): block 0 the serial head's sum (and its stop, with want_stop) into
// head[row]; in block b >= 1, wave w the record of segment (b - 1) kXferSegs + w. The head runs
// here, beside the records, so that the chain kernel starts at the walk.
template <class Src>
__global__ __launch_bounds__(kXferThreads) void seg_xfer_kernel(Src src, uint32_t n, const double* d, SegRec* rec,
                                                                float thr, uint32_t want_stop, SegHead* head,
                                                                uint32_t* xin) {
    __shared__ float hterm[kSegHead];
    const uint32_t row = blockIdx.y;
    if (!src.active(row)) return;  // the whole block
    if (blockIdx.x == 0) {
        const uint32_t nh = min(n, kSegHead);
        constexpr int kPer = kSegHead / kXferThreads;
        float v[kPer];  // all loads first
#pragma unroll
        for (int q = 0; q < kPer; ++q) v[q] = src.term(row, min(threadIdx.x + q * kXferThreads, n - 1u));
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const uint32_t j = threadIdx.x + q * kXferThreads;
            hterm[j] = j < nh ? v[q] : 0.0f;
        }
        __syncthreads();
        if (threadIdx.x < 64) {  // wave 0, every lane the same: the in-order loop itself
            float S = 0.0f;
            uint32_t stop = n;
            if (want_stop) {
                for (uint32_t j = 0; j < nh; ++j) {
                    S += hterm[j];
                    if (S >= thr) {
                        stop = j;
                        break;
                    }
                }
            } else {
                S = serial_sum16(hterm, kSegHead, S);  // the zeros past nh leave S as it is
            }
            if (threadIdx.x == 0) head[row] = SegHead{S, stop};
        }
        return;
    }
    const int lane = threadIdx.x & 63;
    const uint32_t nseg = seg_count(n);
    const uint32_t s = (blockIdx.x - 1) * kXferSegs + (threadIdx.x >> 6);
    if (s >= nseg) return;  // the whole wave; nothing below waits on another wave
    const double* dr = d + static_cast<size_t>(row) * (nseg + 1);
    // D: the head's and the earlier segments' double sums (entries past s read dr[s], dropped)
    constexpr int kDq = kSegMax / 64;
    double dv[kDq];
#pragma unroll
    for (int q = 0; q < kDq; ++q) dv[q] = dr[min(static_cast<uint32_t>(lane + q * 64), s)];
    const double dseg = dr[1 + s];  // this segment's own double sum
    double t = 0.0;
#pragma unroll
    for (int q = 0; q < kDq; ++q) t += static_cast<uint32_t>(lane + q * 64) <= s ? dv[q] : 0.0;
    const double D = wave_reduce(t, 0.0, [](double x, double y) { return x + y; });
    int ex = 0;
    const double m = frexp(D, &ex);  // D = m * 2^ex, m in [0.5, 1)
    const bool low = D < 0x1p-125;
    const int E0 = low ? -126 : ex - 1;
    const int E1 = low ? -125 : max(-126, m < 0.75 ? ex - 2 : ex);
    // this lane's kSegPer terms, in order, for both candidates; then the ordered composition
    // over the lanes
    const uint32_t j0 = kSegHead + s * kSegLen + static_cast<uint32_t>(lane) * kSegPer;
    float av[kSegPer];  // all loads first
#pragma unroll
    for (int q = 0; q < kSegPer; ++q) av[q] = src.term(row, min(j0 + q, n - 1u));
    Xfer f0 = xfer_id(), f1 = xfer_id();
    bool tie0 = false, tie1 = false;
#pragma unroll
    for (int q = 0; q < kSegPer; ++q) {
        const float a = j0 + q < n ? av[q] : 0.0f;
        uint32_t kk, kd;
        split_term(a, E0, kk, kd);
        f0 = xfer_then(f0, term_xfer(kk, kd));
        tie0 = tie0 || kd == 2u;
        split_term(a, E1, kk, kd);
        f1 = xfer_then(f1, term_xfer(kk, kd));
        tie1 = tie1 || kd == 2u;
    }
    f0 = xfer_wave_scan(f0);
    f1 = xfer_wave_scan(f1);
    // the crossing data, where the double sums before and after the segment (widened by 2^-10)
    // lie in different binades: the walk finds the lane that leaves S's binade from it
    int e_lo = 0, e_hi = 0;
    (void)frexp(D * (1.0 - 0x1p-10), &e_lo);
    (void)frexp((D + dseg) * (1.0 + 0x1p-10), &e_hi);
    uint32_t xl = 0u;
    if (xin && e_lo != e_hi) {
        xl = 1u | (__ballot(tie0) == 0 ? 2u : 0u) | (__ballot(tie1) == 0 ? 4u : 0u);
        uint32_t* x = xin + (static_cast<size_t>(row) * kSegMax + s) * kXinWords;
        x[lane] = f0.inc0;
        x[64 + lane] = f1.inc0;
    }
    if (lane == 63) {
        SegRec r;
        r.E[0] = E0;
        r.E[1] = E1;
        r.f[0] = f0;
        r.f[1] = f1;
        r.xl = xl;
        rec[static_cast<size_t>(row) * kSegMax + s] = r;
    }
}

// One segment summed exactly by one wave, with no block barrier and one load per term: terms
// [k0, k1) of a row of n (k1 - k0 <= kSegLen, k0 a multiple of kSegPer) from prefix S; lane l
// holds terms k0 + kSegPer l .. + kSegPer - 1 in registers. Each pass does what a window of block_seq_sum does --
// the terms in units of the binade of S, their transfer functions scanned across the wave, a
// replay to the first term that leaves the binade or reaches thr -- and an exact add of that
// term; the next pass continues after it from the same registers. Returns the sum; *stop_at
// receives the first index whose prefix reaches thr (want_stop), else k1. Every lane returns
// the same values.
template <typename Load>
__device__ float wave_seg_sum(Load load, uint32_t n, uint32_t k0, uint32_t k1, float S, float thr,
                              bool want_stop, uint32_t* stop_at) {
    const int lane = threadIdx.x & 63;
    const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
    float a[kSegPer];
    if (j0 < ((n + 15u) & ~15u)) {  // rows are padded to 16 floats: the whole load is inside
        load(j0, a);
    } else {
#pragma unroll
        for (int q = 0; q < kSegPer; ++q) a[q] = 0.0f;
    }
#pragma unroll
    for (int q = 0; q < kSegPer; ++q)
        if (j0 + q >= k1) a[q] = 0.0f;
    uint32_t kc = k0;  // the first term not yet added
    uint32_t stop = k1;
    for (uint32_t pass = 0; pass <= kSegLen; ++pass) {  // each pass adds at least one term
        const uint32_t sb = __float_as_uint(S), sf = sb >> 23;
        const int E = sf ? static_cast<int>(sf) - 127 : -126;
        const uint32_t B = sf ? ((sb & 0x7FFFFFu) | 0x800000u) : sb;
        const uint32_t p0 = B & 1u;
        uint32_t Tu = 0xFFFFFFFFu;
        if (want_stop) {
            const double t = ceil(ldexp(static_cast<double>(thr), 23 - E));
            Tu = t <= 0.0 ? 0u : (t >= 4294967295.0 ? 0xFFFFFFFFu : static_cast<uint32_t>(t));
        }
        // Each term in units of u = 2^(E - 23): x = a / u is exact (a power-of-two scaling of a
        // value with at most 24 significant bits; an x that underflows is far below 1/2 and
        // one that overflows saturates), and so is x - floor(x). The pass is tie-free when no
        // x lies exactly half-way between integers; then every increment is rint(x), whatever
        // the parity of S / u.
        // The same for the next binade up (units 2u), where the sum goes at a crossing: k2 and
        // its prefix sums let the pass finish the segment after the crossing term itself.
        uint32_t kk[kSegPer], kd[kSegPer], k2[kSegPer];
        bool tie = false, tie2 = false;
#pragma unroll
        for (int q = 0; q < kSegPer; ++q) {
            const float aq = j0 + q >= kc ? a[q] : 0.0f;
            const float x = ldexpf(aq, 23 - E), x2 = ldexpf(aq, 22 - E);
            tie = tie || (x - floorf(x) == 0.5f);
            tie2 = tie2 || (x2 - floorf(x2) == 0.5f);
            kk[q] = static_cast<uint32_t>(fminf(rintf(x), 0x1p30f));  // saturated at kSat
            k2[q] = static_cast<uint32_t>(fminf(rintf(x2), 0x1p30f));
            kd[q] = 0u;
        }
        uint32_t R, Rend, par = 0;  // R: this lane's start; Rend: its end (lane 63: the wave's)
        uint32_t incl2 = 0u, total2 = kSat;
        const bool fast = __ballot(tie) == 0;
        if (fast) {
            // no exact half-way case in this pass: a saturating prefix sum of the increments
            // stands in for the scan of transfer functions, at about half its cost
            uint32_t tot = 0, tot2 = 0;
#pragma unroll
            for (int q = 0; q < kSegPer; ++q) {
                tot = sat_add(tot, kk[q]);
                tot2 = sat_add(tot2, k2[q]);
            }
            if (__ballot(tie2) == 0) {
                incl2 = inc_wave_scan(tot2);
                total2 = lane_u32(incl2, 63);  // below kSat: every prefix of it is exact
            }
            const uint32_t incl = inc_wave_scan(tot);
            uint32_t ex = static_cast<uint32_t>(__shfl_up(incl, 1));
            if (lane == 0) ex = 0u;
            R = sat_add(B, ex);
            Rend = sat_add(B, incl);
        } else {
#pragma unroll
            for (int q = 0; q < kSegPer; ++q) split_term(j0 + q >= kc ? a[q] : 0.0f, E, kk[q], kd[q]);
            Xfer t = xfer_id();
#pragma unroll
            for (int q = 0; q < kSegPer; ++q) t = xfer_then(t, term_xfer(kk[q], kd[q]));
            const Xfer incl = xfer_wave_scan(t);
            Xfer ex = xfer_shfl_up(incl, 1);
            if (lane == 0) ex = xfer_id();
            R = sat_add(B, p0 ? ex.inc1 : ex.inc0);
            par = (ex.out >> p0) & 1u;
            Rend = sat_add(B, p0 ? incl.inc1 : incl.inc0);
        }
        uint32_t ev = kNoEvent, R_before = R;
        bool live = R < kL;
        if (fast) {
            // the replay with parity-free increments. The terms outside [kc, k1) are zeros: one
            // can neither leave the binade nor be the first to reach thr (S < thr at a pass's
            // start), so they need no range test here.
#pragma unroll
            for (int q = 0; q < kSegPer; ++q) {
                const uint32_t j = j0 + q, d = kk[q];
                const bool cross = live && (R + d >= kL);
                if (cross) {
                    ev = 2 * j;
                    R_before = R;
                }
                const bool adv = live && !cross;
                R = adv ? R + d : R;
                const bool hit = adv && R >= Tu;
                if (hit) ev = 2 * j + 1;
                live = adv && !hit;
            }
        } else {
#pragma unroll
            for (int q = 0; q < kSegPer; ++q) {
                const uint32_t j = j0 + q;
                const uint32_t d = term_inc(kk[q], kd[q], par);
                const bool go = live && j >= kc && j < k1;
                const bool cross = go && (R + d >= kL);
                const bool adv = go && !cross;
                if (cross) {
                    ev = 2 * j;
                    R_before = R;
                }
                R = adv ? R + d : R;
                par = adv ? ((par + d) & 1u) : par;
                const bool hit = adv && R >= Tu;
                if (hit) ev = 2 * j + 1;
                live = live && !cross && !hit;
            }
        }
        // the earliest event is the lowest lane's (lanes hold increasing indices)
        const uint64_t m = __ballot(ev != kNoEvent);
        if (m == 0) {  // no event: lane 63's end is the segment's
            S = ldexpf(static_cast<float>(lane_u32(Rend, 63)), E - 23);
            break;
        }
        const int owner = __ffsll(static_cast<long long>(m)) - 1;
        const uint32_t e = lane_u32(ev, owner);
        const uint32_t j = e >> 1;
        if (e & 1u) {  // reaches thr, no binade change before it
            S = ldexpf(static_cast<float>(lane_u32(R, owner)), E - 23);
            stop = j;
            break;
        }
        // the term that leaves the binade, added exactly
        float aj = 0.0f;
#pragma unroll
        for (int q = 0; q < kSegPer; ++q) aj = (j0 + q == j) ? a[q] : aj;
        aj = lane_f32(aj, owner);
        const float s_new = ldexpf(static_cast<float>(lane_u32(R_before, owner)), E - 23) + aj;
        S = s_new;
        if (want_stop && s_new >= thr) {
            stop = j;
            break;
        }
        kc = j + 1;
        if (kc >= k1) break;
        if (total2 < kSat) {
            // S is now in binade E + 1 (checked): with no exact half-way term there and no
            // saturation, the terms after j add sum2 = (the owner lane's terms after j) + (the
            // lanes after it) units of 2u. If that stays in the binade and below thr, the
            // segment ends here; otherwise the next pass takes it from kc.
            const uint32_t sb2 = __float_as_uint(S), sf2 = sb2 >> 23;
            const int E2 = sf2 ? static_cast<int>(sf2) - 127 : -126;
            if (E2 == E + 1) {
                const uint32_t B2 = sf2 ? ((sb2 & 0x7FFFFFu) | 0x800000u) : sb2;
                uint32_t mine = 0u;
#pragma unroll
                for (int q = 0; q < kSegPer; ++q) mine += j0 + q > j ? k2[q] : 0u;
                const uint32_t sum2 = lane_u32(mine, owner) + (total2 - lane_u32(incl2, owner));
                const uint32_t Rend2 = B2 + sum2;  // B2 < 2^24, sum2 < 2^30
                uint32_t Tu2 = 0xFFFFFFFFu;
                if (want_stop) {
                    const double t2 = ceil(ldexp(static_cast<double>(thr), 23 - E2));
                    Tu2 = t2 <= 0.0 ? 0u : (t2 >= 4294967295.0 ? 0xFFFFFFFFu : static_cast<uint32_t>(t2));
                }
                if (Rend2 < kL && Rend2 < Tu2) {
                    S = ldexpf(static_cast<float>(Rend2), E2 - 23);
                    break;
                }
            }
        }
    }
    if (want_stop) *stop_at = stop;
    return S;
}

// The walk's crossing shortcut for segment [k0, k1) (one wave, no stop threshold). When the
// segment carries crossing data for S's binade E and for E + 1, both free of exact half-way
// terms, each lane's increments in units of E locate the lane c where S leaves E: the sum
// before lane c is exact (integer increments inside one binade); lane c's terms are added one
// by one with fp32 adds, the reference's own operations; and when S has then reached E + 1, the
// later lanes' increments in units of E + 1 give the segment's end unless it leaves E + 1 too.
// Where the shortcut stops short, wave_seg_sum sums the rest of the segment exactly. Returns
// false, with S untouched, when the data does not apply; otherwise S is the sum after the
// segment. x: the segment's kXinWords crossing words; xw and xt, when not null, the same words
// and the segment's terms (zeros past its end) staged in LDS. Every lane returns the same values.
template <typename Load>
__device__ bool seg_crossing(Load load, uint32_t n, const SegRec& R, const uint32_t* x, const uint32_t* xw,
                             const float* xt, uint32_t k0, uint32_t k1, float& S) {
    if (!(R.xl & 1u)) return false;
    const int lane = threadIdx.x & 63;
    const uint32_t sb = __float_as_uint(S), sf = sb >> 23;
    const int E = sf ? static_cast<int>(sf) - 127 : -126;
    const uint32_t B = sf ? ((sb & 0x7FFFFFu) | 0x800000u) : sb;
    const int ce = R.E[0] == E ? 0 : (R.E[1] == E ? 1 : -1);
    if (ce < 0 || R.E[1 - ce] != E + 1 || !((R.xl >> (1 + ce)) & 1u) || !((R.xl >> (2 - ce)) & 1u)) return false;
    // the lanes' increments in both binades and the lane's terms: from LDS when staged, else
    // one round trip
    const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
    uint32_t incE, incE1;
    float a[kSegPer];
    if (xw) {
        incE = xw[ce * 64 + lane];
        incE1 = xw[(1 - ce) * 64 + lane];
#pragma unroll
        for (int q = 0; q < kSegPer; ++q) a[q] = xt[lane * kSegPer + q];
    } else {
        incE = x[ce * 64 + lane];
        incE1 = x[(1 - ce) * 64 + lane];
        if (j0 < ((n + 15u) & ~15u)) {  // rows are padded to 16 floats: the whole load is inside
            load(j0, a);
        } else {
#pragma unroll
            for (int q = 0; q < kSegPer; ++q) a[q] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < kSegPer; ++q)
            if (j0 + q >= k1) a[q] = 0.0f;
    }
    const uint64_t over = __ballot(B + incE >= kL);  // B < 2^24, incE <= 2^30: no wrap
    if (over == 0) return false;  // no lane leaves E: the walk stopped here for another reason
    const int c = __ffsll(static_cast<long long>(over)) - 1;
    const uint32_t ex = c > 0 ? lane_u32(incE, c - 1) : 0u;  // < 2^24 - B: S stays in E
    float sc = ldexpf(static_cast<float>(B + ex), E - 23);
#pragma unroll
    for (int q = 0; q < kSegPer; ++q) sc = sc + lane_f32(a[q], c);
    const uint32_t sb2 = __float_as_uint(sc), sf2 = sb2 >> 23;
    const int E2 = sf2 ? static_cast<int>(sf2) - 127 : -126;
    const uint32_t B2 = sf2 ? ((sb2 & 0x7FFFFFu) | 0x800000u) : sb2;
    const uint32_t tot1 = lane_u32(incE1, 63), pre1 = lane_u32(incE1, c);
    if (E2 == E + 1 && tot1 < kSat && B2 + (tot1 - pre1) < kL) {
        S = ldexpf(static_cast<float>(B2 + (tot1 - pre1)), E2 - 23);
        return true;
    }
    S = sc;
    const uint32_t jn = k0 + static_cast<uint32_t>(c + 1) * kSegPer;
    if (jn < k1) {
        uint32_t at = k1;
        S = wave_seg_sum(load, n, jn, k1, S, 0.0f, false, &at);
    }
    return true;
}

constexpr uint32_t kXSlots = 16;         // crossing segments staged in LDS per row
constexpr uint32_t kNoSlot = 0xFFFFFFFFu;
struct ChainShared {
    SegRec rec[kSegMax];
    float start[kSegMax + 1];  // the exact sum at each segment start, then the row's sum
    float S;
    uint32_t s;
    // the first kXSlots segments with crossing data, staged while wave 0 walks: xslot[t] is the
    // slot of segment t, stored (release) once the slot holds its words and terms
    uint32_t xslot[kSegMax];
    uint32_t xw[kXSlots][kXinWords];
    float xt[kXSlots][kSegLen];
};

// The walk and the exact segments after the head: S is the sum of terms [0, kSegHead) on entry.
// Returns the row's sum (or, with stop_at, the prefix at the first index reaching thr, whose
// index goes to *stop_at; n when none does). ch.start[t] receives the sum before segment t for
// every t the chain passes.
template <typename Load, typename Term>
__device__ float seg_chain(Load load, Term term, uint32_t n, float S, float thr, uint32_t* stop_at,
                           const uint32_t* xr, SeqShared& sh, ChainShared& ch) {
    (void)term;
    (void)sh;
    const uint32_t nseg = seg_count(n);
    const bool want_stop = stop_at != nullptr;
    if (threadIdx.x < 64) {
        // wave 0: walks 64 records at a time (the composed increments of the lanes' records, an
        // ordered scan of transfer functions, give every lane its segment's start and end at
        // once), advancing to the first lane whose record does not apply; that segment it sums
        // exactly with wave_seg_sum, then walks on
        const int lane = threadIdx.x;
        uint32_t stop = n;
        uint32_t t = 0;
        while (t < nseg) {
            for (;;) {
                const uint32_t sb = __float_as_uint(S), sf = sb >> 23;
                const int E = sf ? static_cast<int>(sf) - 127 : -126;
                const uint32_t B = sf ? ((sb & 0x7FFFFFu) | 0x800000u) : sb;
                const uint32_t p0 = B & 1u;
                const uint32_t idx = t + static_cast<uint32_t>(lane);
                int c = -1;
                Xfer f = xfer_id();
                if (idx < nseg) {
                    const SegRec& R = ch.rec[idx];
                    c = R.E[0] == E ? 0 : (R.E[1] == E ? 1 : -1);
                    if (c >= 0) f = R.f[c];
                }
                // b0, b1: S / u at the lane's segment start and end (< 2^24 up to the first bad
                // lane). A record is parity-free when its segment holds no exact half-way
                // term: the same increment for either parity of S / u. With every record
                // parity-free a saturating prefix sum of the increments stands in for the scan
                // of transfer functions.
                const bool pfree = f.inc0 == f.inc1 && f.out == ((f.inc0 & 1u) ? 1u : 2u);
                uint32_t b0, b1;
                if (__ballot(!pfree) == 0) {
                    const uint32_t incl = inc_wave_scan(f.inc0);
                    uint32_t excl = static_cast<uint32_t>(__shfl_up(incl, 1));
                    if (lane == 0) excl = 0u;
                    b0 = B + excl;
                    b1 = B + incl;
                } else {
                    const Xfer incl = xfer_wave_scan(f);
                    Xfer excl = xfer_shfl_up(incl, 1);
                    if (lane == 0) excl = xfer_id();
                    b0 = B + (p0 ? excl.inc1 : excl.inc0);
                    b1 = B + (p0 ? incl.inc1 : incl.inc0);
                }
                const float Se = ldexpf(static_cast<float>(b1), E - 23);
                const bool good = c >= 0 && b1 < kL && !(want_stop && Se >= thr);
                const uint64_t bad = __ballot(!good);
                const uint32_t first = bad ? static_cast<uint32_t>(__ffsll(static_cast<long long>(bad)) - 1) : 64u;
                // every lane up to the first bad one starts where the records before it end
                if (static_cast<uint32_t>(lane) <= first && idx < nseg) ch.start[idx] = ldexpf(static_cast<float>(b0), E - 23);
                if (first > 0) S = lane_f32(Se, static_cast<int>(first) - 1);
                t += first;
                if (first < 64 || t >= nseg) break;
            }
            if (t >= nseg) break;
            // segment t exactly, from S: by its crossing data where that applies
            const uint32_t k0 = kSegHead + t * kSegLen, k1 = min(n, k0 + kSegLen);
            if (!want_stop && xr) {
                const uint32_t sl = __hip_atomic_load(&ch.xslot[t], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
                const bool staged = sl < kXSlots;
                if (seg_crossing(load, n, ch.rec[t], xr + static_cast<size_t>(t) * kXinWords,
                                 staged ? ch.xw[sl] : nullptr, staged ? ch.xt[sl] : nullptr, k0, k1, S)) {
                    ++t;
                    continue;
                }
            }
            uint32_t at = k1;
            S = wave_seg_sum(load, n, k0, k1, S, thr, want_stop, &at);
            if (want_stop && at < k1) {
                stop = at;
                break;
            }
            ++t;
        }
        if (lane == 0) {
            ch.S = S;
            ch.s = stop;
            ch.start[nseg] = S;
        }
    }
    __syncthreads();
    S = ch.S;
    if (want_stop) *stop_at = ch.s;
    __syncthreads();  // ch is read before any later write
    return S;
}

// The chain of one row: its records into LDS, the head's sum from seg_xfer_kernel, the walk.
template <typename Load, typename Term>
__device__ float seg_row_sum(Load load, Term term, uint32_t n, const SegRec* rec, const SegHead* hd, float thr,
                             uint32_t* stop_at, const uint32_t* xr, SeqShared& sh, ChainShared& ch) {
    const uint32_t nseg = seg_count(n);
    const SegHead h = *hd;  // the same value in every thread; requested with the records
    for (uint32_t i = threadIdx.x; i < nseg; i += blockDim.x) {
        ch.rec[i] = rec[i];
        ch.xslot[i] = kNoSlot;
    }
    __syncthreads();
    if (stop_at && h.stop < min(n, kSegHead)) {
        *stop_at = h.stop;
        return h.S;
    }
    if (!stop_at && xr && threadIdx.x >= 64) {
        // waves 1 .. stage the first kXSlots segments with crossing data, in segment order, slot
        // q by wave 1 + q % (waves - 1): the words and the terms into LDS, then (release) the
        // slot number into xslot, which the walk reads (acquire) at a crossing. Nothing waits:
        // a crossing the walk reaches before its slot is published goes to memory instead.
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const uint32_t stagers = blockDim.x / 64 - 1;
        uint32_t q = 0;
        for (uint32_t base = 0; base < nseg && q < kXSlots; base += 64) {
            const uint32_t i = base + static_cast<uint32_t>(lane);
            const uint64_t cm = __ballot(i < nseg && (ch.rec[i].xl & 1u));
            uint64_t m = cm;
            while (m != 0 && q < kXSlots) {
                const int b = __ffsll(static_cast<long long>(m)) - 1;
                m &= m - 1;
                const uint32_t t = base + static_cast<uint32_t>(b);
                if (q % stagers == static_cast<uint32_t>(wave - 1)) {
                    const uint32_t* x = xr + static_cast<size_t>(t) * kXinWords;
                    const uint32_t k0 = kSegHead + t * kSegLen, k1 = min(n, k0 + kSegLen);
                    const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
                    const uint32_t w0 = x[lane], w1 = x[64 + lane];
                    float a[kSegPer];
                    if (j0 < ((n + 15u) & ~15u)) {
                        load(j0, a);
                    } else {
#pragma unroll
                        for (int r = 0; r < kSegPer; ++r) a[r] = 0.0f;
                    }
                    ch.xw[q][lane] = w0;
                    ch.xw[q][64 + lane] = w1;
#pragma unroll
                    for (int r = 0; r < kSegPer; ++r) ch.xt[q][lane * kSegPer + r] = j0 + r < k1 ? a[r] : 0.0f;
                    __builtin_amdgcn_wave_barrier();
                    if (lane == 0)
                        __hip_atomic_store(&ch.xslot[t], q, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
                ++q;
            }
        }
    }
    return seg_chain(load, term, n, h.S, thr, stop_at, xr, sh, ch);
}

// The softmax sums of the e rows: one block per row.
// LDS of seg_sum_kernel: a softmax row's chain, or a target row's merge
union SumOrMergeShared {
    struct {
        SeqShared sh;
        ChainShared ch;
    } seg;
    SampleMergeShared sm;
};

__global__ __launch_bounds__(kRejThreads) void seg_sum_kernel(DraftArgs a, const SegRec* rec, const SegHead* heads,
                                                              DraftSelect sel) {
    static_assert(kRejThreads == kSmThreads, "a merge block is a chain block");
    __shared__ SumOrMergeShared u;
    const uint32_t r = blockIdx.x;
    if (r >= 2 * a.npos) {  // the whole block: sample_token of target row r - 2P from its records
        const uint32_t row = r - 2 * a.npos;
        twd_row_params p = sel.base;
        p.uniform = sel.u[row];
        sample_merge_row(p, row, sel.mb, u.sm);
        return;
    }
    SeqShared& sh = u.seg.sh;
    ChainShared& ch = u.seg.ch;
    const float* e = a.e + static_cast<size_t>(r) * a.estride;
    float s = __uint_as_float(0x7FC00000u);
    if (!(a.flags[r] & 1u))
        s = seg_row_sum([&](uint32_t j0, auto& v) { load_row(e, j0, v); }, [&](uint32_t j) { return e[j]; },
                        a.vocab, rec + static_cast<size_t>(r) * kSegMax, heads + r, 0.0f, nullptr,
                        a.xin + static_cast<size_t>(r) * kSegMax * kXinWords, sh, ch);
    if (threadIdx.x == 0) a.sums[r] = s;
}

// The ratio test of position pi (speculator.cpp:83-92); *dt_out receives the draft token.
__device__ __forceinline__ bool draft_accepts(const DraftArgs& a, uint32_t pi, uint32_t* dt_out) {
    const DraftPos& P = a.pos[pi];
    const uint32_t V = a.vocab;
    const float* et = a.e + static_cast<size_t>(2 * pi) * a.estride;
    const float* ed = a.e + static_cast<size_t>(2 * pi + 1) * a.estride;
    const float sp = a.sums[2 * pi], sq = a.sums[2 * pi + 1];
    const float inv_p = 1.0f / (sp > 1e-12f ? sp : 1.0f);
    const float inv_q = 1.0f / (sq > 1e-12f ? sq : 1.0f);
    const uint32_t dt = a.drafts[P.position];
    const float p_val = dt < V ? et[dt] * inv_p : 0.0f;
    const float q_val = dt < V ? ed[dt] * inv_q : 0.0f;
    const float r = (q_val > 1e-12f) ? (p_val / q_val) : 1.0f;
    *dt_out = dt;
    return P.u1 <= r;
}

// The residual's double segment sums, grid (xfer_blocks(V), P), each block first repeating its
// position's ratio test (every block gets the same answer): an accepted draft is final (block 0
// records it) and the position's blocks stop; a rejected one is marked live for the residual
// draw (speculator.cpp:94-116).
__global__ __launch_bounds__(kXferThreads) void seg_ratio_dsum_kernel(DraftArgs a, uint32_t* live, double* d) {
    __shared__ double red[kXferSegs];
    const uint32_t pi = blockIdx.y;
    uint32_t dt = 0;
    const bool accepted = draft_accepts(a, pi, &dt);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (accepted) {
            uint32_t* out = a.rej + a.pos[pi].position * 4;
            out[0] = 1u;
            out[1] = dt;
            out[2] = 0u;
            out[3] = 1u;
        }
        live[pi] = accepted ? 0u : 1u;
    }
    if (accepted) return;  // the whole block
    const SegSrcResidual src{a.e, a.estride, a.sums, live};  // terms only: live is not read here
    seg_dsum_block(src, pi, blockIdx.x, a.vocab, d, red);
}

// The residual (p - q)+ of a rejected position (speculator.cpp:94-116): its sum, then the first
// index whose prefix reaches u2 * sum, found in the segment where the recorded starts straddle
// it. One block per position; accepted positions return at once.
__device__ void draft_finish_body(const uint32_t* row_tokens, uint32_t rows, const uint32_t* drafts, uint32_t nd,
                                  uint64_t has_draft, const uint32_t* rej, twd_verify_result* v);

__device__ __forceinline__ void seg_residual_block(const DraftArgs& a, uint32_t pi, const SegRec* rec,
                                                   const SegHead* heads, SeqShared& sh, ChainShared& ch);

struct DraftFinish {  // the accept chain's inputs: the residual launch's last block runs it
    const uint32_t* row_tokens;  // the selector's tokens (joined before the launch)
    uint32_t rows;
    const uint32_t* drafts;
    uint32_t nd;
    uint64_t has_draft;
    twd_verify_result* v;
    unsigned long long* ctr;     // [kArriveWords] grid_arrive's arrival counter
    uint32_t epoch, next_epoch;  // this call's epoch (never 0) and the next call's
};

__global__ __launch_bounds__(kRejThreads) void seg_residual_kernel(DraftArgs a, const uint32_t* live,
                                                                   const SegRec* rec, const SegHead* heads,
                                                                   DraftFinish f) {
    __shared__ SeqShared sh;
    __shared__ ChainShared ch;
    const uint32_t pi = blockIdx.x;
    if (live[pi]) seg_residual_block(a, pi, rec, heads, sh, ch);  // block-uniform
    // count in, the position's outcome (written above, or by seg_ratio_dsum_kernel) published
    // first; the last block reads every outcome after an acquiring fence
    if (threadIdx.x == 0) {
        __threadfence();
        if (grid_arrive(f.ctr, gridDim.x, f.epoch, f.next_epoch)) {
            __threadfence();
            draft_finish_body(f.row_tokens, f.rows, f.drafts, f.nd, f.has_draft, a.rej, f.v);
        }
    }
}

// A rejected position's residual sum and draw (the body of seg_residual_kernel).
__device__ __forceinline__ void seg_residual_block(const DraftArgs& a, uint32_t pi, const SegRec* rec,
                                                   const SegHead* heads, SeqShared& sh, ChainShared& ch) {
    const DraftPos& P = a.pos[pi];
    const uint32_t V = a.vocab;
    const float* et = a.e + static_cast<size_t>(2 * pi) * a.estride;
    const float* ed = a.e + static_cast<size_t>(2 * pi + 1) * a.estride;
    const float sp = a.sums[2 * pi], sq = a.sums[2 * pi + 1];
    const float inv_p = 1.0f / (sp > 1e-12f ? sp : 1.0f);
    const float inv_q = 1.0f / (sq > 1e-12f ? sq : 1.0f);
    // std::max(0.0f, x) keeps 0 for x <= 0 and for NaN; each product rounded on its own
    auto diff1 = [&](float pt, float qd) {
        const float x = pt * inv_p - qd * inv_q;
        return (0.0f < x) ? x : 0.0f;
    };
    auto diff = [&](uint32_t j) { return diff1(et[j], ed[j]); };
    auto load_diff = [&](uint32_t j0, auto& v) {
        constexpr int PER = sizeof(v) / sizeof(float);
        float w[PER];
        load_row(et, j0, v);
        load_row(ed, j0, w);
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = diff1(v[q], w[q]);
    };
    const SegRec* rr = rec + static_cast<size_t>(pi) * kSegMax;
    const float sum_diff = seg_row_sum(load_diff, diff, V, rr, heads + pi, 0.0f, nullptr,
                                       a.xin + static_cast<size_t>(pi) * kSegMax * kXinWords, sh, ch);
    uint32_t corr = 0, fallback = 0;
    if (sum_diff > 1e-9f) {
        const float r_val = P.u2 * sum_diff;
        uint32_t at = V;
        const uint32_t nh = min(V, kSegHead);
        const uint32_t nseg = seg_count(V);
        // the head holds the stop when its sum reaches r_val; otherwise the last segment whose
        // recorded start lies below r_val does (prefixes never decrease)
        const bool in_head = nseg == 0 || ch.start[0] >= r_val;
        if (in_head) {
            block_seq_sum(load_diff, diff, nh, 0.0f, 0u, r_val, &at, false, sh);
        } else {
            // the starts never decrease, so the last one below r_val is at the count of those
            // below it among starts 1 .. nseg - 1
            int below = 0;
            for (uint32_t i = 1 + threadIdx.x; i < nseg; i += kRejThreads) below += ch.start[i] < r_val;
            const uint32_t t = static_cast<uint32_t>(__syncthreads_count(below));
            const float S0 = ch.start[t];
            const uint32_t k0 = kSegHead + t * kSegLen, k1 = min(V, k0 + kSegLen);
            if (threadIdx.x < 64) {
                wave_seg_sum(load_diff, V, k0, k1, S0, r_val, true, &at);
                if (threadIdx.x == 0) ch.s = at;
            }
            __syncthreads();
            at = ch.s;
            if (at >= k1) at = V;
        }
        corr = at < V ? at : 0u;  // corr_tok starts at 0 (:101)
    } else {
        fallback = 1;  // sample_token on the target row (:114): the selector's token
    }
    if (threadIdx.x == 0) {
        uint32_t* out = a.rej + P.position * 4;
        out[0] = 0u;
        out[1] = corr;
        out[2] = fallback;
        out[3] = 1u;
    }
}

// twd_sequential_sum through the segmented form: one row of n terms.
template <bool STOP>
__global__ __launch_bounds__(kRejThreads) void seg_array_kernel(const float* x, uint32_t n, float thr,
                                                                const SegRec* rec, const SegHead* hd,
                                                                const uint32_t* xin, float* sum_out,
                                                                uint32_t* stop_out) {
    __shared__ SeqShared sh;
    __shared__ ChainShared ch;
    uint32_t stop = n;
    const float s = seg_row_sum([&](uint32_t j0, auto& v) { load_row(x, j0, v); }, [&](uint32_t j) { return x[j]; },
                                n, rec, hd, thr, STOP ? &stop : nullptr, xin, sh, ch);
    if (threadIdx.x == 0) {
        *sum_out = s;
        if (STOP) *stop_out = stop;
    }
}

// The accept chain of speculator.cpp:53-146 over per-position outcomes: rej[i] for positions
// with draft rows (has_draft bit i), the selector's sampled token row_tok[i] otherwise, for the
// fallback, and for the bonus row k.
__device__ void draft_finish_body(const uint32_t* row_tokens, uint32_t rows, const uint32_t* drafts, uint32_t nd,
                                  uint64_t has_draft, const uint32_t* rej, twd_verify_result* v) {
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
    const size_t need_e = static_cast<size_t>(2) * npos * ((vocab + 15u) & ~15u);
    const size_t need_part = static_cast<size_t>(2) * npos * parts;
    const size_t need_x = static_cast<size_t>(2) * npos * kSegMax * kXinWords;
    // the capacities are set only once every buffer exists, so a call after a failed one never
    // finds a partial set
    if (d->e_capacity >= need_e && d->part_capacity >= need_part && d->x_capacity >= need_x && d->side)
        return TWD_OK;
    draft_scratch_free(d);  // grows: later calls with as many positions reuse it
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = hipMalloc(&d->e, need_e * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d->part, need_part * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d->xin, need_x * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d->flags, 2 * TWD_MAX_ROWS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d->rej, 4 * TWD_MAX_ROWS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d->sums, 2 * TWD_MAX_ROWS * sizeof(float));
    if (e == hipSuccess)
        e = hipMalloc(&d->seg_d, static_cast<size_t>(2) * TWD_MAX_ROWS * (kSegMax + 1) * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&d->seg_rec, static_cast<size_t>(2) * TWD_MAX_ROWS * kSegMax * sizeof(SegRec));
    if (e == hipSuccess) e = hipMalloc(&d->seg_head, static_cast<size_t>(2) * TWD_MAX_ROWS * sizeof(SegHead));
    if (e == hipSuccess) e = hipMalloc(&d->live, TWD_MAX_ROWS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d->fin_ctr, kArriveWords * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(d->fin_ctr, 0, kArriveWords * sizeof(uint64_t));
    const uint64_t armed = kFirstEpoch;  // the counter starts armed for the first call
    if (e == hipSuccess) e = hipMemcpy(d->fin_ctr, &armed, sizeof(armed), hipMemcpyHostToDevice);
    if (e == hipSuccess && !d->side) {  // kept across growth: freed with the selector
        e = hipStreamCreateWithFlags(&d->side, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&d->fork, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&d->join, hipEventDisableTiming);
        if (e != hipSuccess) draft_side_free(d);
    }
    if (e != hipSuccess) {
        draft_scratch_free(d);
        return hip_fail(e, "allocating the draft verify's scratch");
    }
    d->fin_epoch = kFirstEpoch - 1;
    d->e_capacity = need_e;
    d->part_capacity = need_part;
    d->x_capacity = need_x;
    return TWD_OK;
}

void draft_scratch_free(DraftScratch* d) {
    if (d->e) (void)hipFree(d->e);
    if (d->part) (void)hipFree(d->part);
    if (d->xin) (void)hipFree(d->xin);
    if (d->flags) (void)hipFree(d->flags);
    if (d->rej) (void)hipFree(d->rej);
    if (d->sums) (void)hipFree(d->sums);
    if (d->seg_d) (void)hipFree(d->seg_d);
    if (d->seg_rec) (void)hipFree(d->seg_rec);
    if (d->seg_head) (void)hipFree(d->seg_head);
    if (d->live) (void)hipFree(d->live);
    if (d->fin_ctr) (void)hipFree(d->fin_ctr);
    const DraftScratch keep = *d;
    *d = DraftScratch{};
    d->side = keep.side;
    d->fork = keep.fork;
    d->join = keep.join;
}

void draft_side_free(DraftScratch* d) {
    if (d->side) {
        (void)hipStreamSynchronize(d->side);
        (void)hipStreamDestroy(d->side);
    }
    if (d->fork) (void)hipEventDestroy(d->fork);
    if (d->join) (void)hipEventDestroy(d->join);
    d->side = nullptr;
    d->fork = d->join = nullptr;
}

}  // namespace twd

using namespace twd;

extern "C" {

TWD_API void* twd_selector_verify_state(const twd_selector* sel) {
    return sel ? static_cast<void*>(sel->draft.fin_ctr) : nullptr;
}

TWD_API int twd_verify_draft_sums(const twd_selector* sel, float* sums, uint32_t* positions,
                                  uint32_t capacity, uint32_t* n) {
    clear_error();
    if (!sel || !n) return fail(TWD_E_INVALID, "null selector or n");
    const uint32_t np = sel->draft.last_npos;
    *n = np;
    if (np == 0) return TWD_OK;
    if (capacity < np || !sums || !positions) return fail(TWD_E_INVALID, "capacity below the positions of the last call");
    TWD_HIP(hipDeviceSynchronize());
    TWD_HIP(hipMemcpy(sums, sel->draft.sums, 2 * np * sizeof(float), hipMemcpyDeviceToHost));
    for (uint32_t i = 0; i < np; ++i) positions[i] = sel->draft.last_pos[i];
    return TWD_OK;
}

TWD_API int twd_sequential_sum(const float* terms, uint32_t n, float thr, float* sum_out,
                               uint32_t* stop_out, void* stream) {
    clear_error();
    if (!terms || !sum_out) return fail(TWD_E_INVALID, "null terms or sum_out");
    if (n == 0) return fail(TWD_E_INVALID, "n must be > 0");
    if ((reinterpret_cast<uintptr_t>(terms) & 15u) != 0) return fail(TWD_E_INVALID, "terms must be 16-byte aligned");
    if (seg_count(n) > kSegMax) return fail(TWD_E_INVALID, "n above the segmented sums' limit (2^19 after the head)");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // one row's segment scratch, allocated on the first call and kept for the process
    static std::mutex mu;
    static double* seg_d = nullptr;
    static SegRec* seg_rec = nullptr;
    static SegHead* seg_head = nullptr;
    static uint32_t* xin = nullptr;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!xin) {
            if (!seg_d) TWD_HIP(hipMalloc(&seg_d, (kSegMax + 1) * sizeof(double)));
            if (!seg_rec) TWD_HIP(hipMalloc(&seg_rec, kSegMax * sizeof(SegRec)));
            if (!seg_head) TWD_HIP(hipMalloc(&seg_head, sizeof(SegHead)));
            TWD_HIP(hipMalloc(&xin, static_cast<size_t>(kSegMax) * kXinWords * sizeof(uint32_t)));
        }
    }
    const uint32_t nseg = seg_count(n);
    const SegSrcArray src{terms};
    seg_dsum_kernel<<<dim3(xfer_blocks(n), 1), kXferThreads, 0, s>>>(src, n, seg_d);
    seg_xfer_kernel<<<dim3(xfer_blocks(n), 1), kXferThreads, 0, s>>>(src, n, seg_d, seg_rec, thr,
                                                                     stop_out ? 1u : 0u, seg_head, xin);
    if (stop_out)
        seg_array_kernel<true><<<1, kRejThreads, 0, s>>>(terms, n, thr, seg_rec, seg_head, xin, sum_out, stop_out);
    else
        seg_array_kernel<false><<<1, kRejThreads, 0, s>>>(terms, n, thr, seg_rec, seg_head, xin, sum_out, stop_out);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

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
    int rc = order_before(sel->order, s);
    if (rc) return rc;
    rc = verify_draft_launches(sel, logits, vocab, rows, row_stride, draft_rows, n_draft_rows, params,
                               base_seed, drafts, n_drafts, result, s);
    const int rc2 = order_after(sel->order, s);
    return rc ? rc : rc2;
}

}  // extern "C"

namespace twd {

int verify_draft_launches(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                          uint64_t row_stride, const float* const* draft_rows, uint32_t n_draft_rows,
                          const twd_row_params* params, uint64_t base_seed, const uint32_t* drafts,
                          uint32_t n_drafts, twd_verify_result* result, hipStream_t s) {
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
        return verify_launches(sel, logits, vocab, rows, row_stride, params, base_seed, drafts,
                               n_drafts, result, s);
    if (vocab == 0) return fail(TWD_E_INVALID, "vocab must be > 0");

    int rc = draft_scratch_reserve(&sel->draft, vocab, a.npos);
    if (rc) return rc;
    DraftScratch& ds = sel->draft;

    // target tokens for the positions without draft rows, the fallback and the bonus row, read
    // by seg_residual_kernel's last block: sample_token of the target rows 0 .. used - 1
    const uint32_t used = (rows > k) ? k + 1 : k;
    twd_row_params rp[TWD_MAX_ROWS + 1];
    for (uint32_t i = 0; i < used; ++i) {
        rp[i] = *params;
        rp[i].repetition_penalty = 1.0f;
        rp[i].history_len = 0;
        rp[i].uniform = twd_uniform_from_seed(twd_splitmix64(base_seed + i));
    }
    // Inside the draft chain's launches (records in draft_max_kernel's grid, merges in
    // seg_sum_kernel's) when the selector holds the rows' records and no shortlist is longer
    // than 256; otherwise the selector's launches run on the side stream beside the chain and
    // join it before seg_residual_kernel. (A fork and a join cost more host time per call than
    // the merges take on the GPU.)
    const SelectScratch& ss = sel->scratch;
    const uint32_t waves = (vocab + kSampleWaveRows - 1) / kSampleWaveRows;
    bool fused = ss.wkey != nullptr && waves <= ss.wave_cap && waves <= kSampleMaxWaves;
    for (uint32_t i = 0; i < used; ++i) fused = fused && !long_row(rp[i], vocab);
    DraftSelect dsel{};
    if (fused) {
        const SampleStats st{ss.wkey, ss.wsum, ss.wmax, ss.waux, __builtin_nanf("")};
        dsel.nsel = used;
        dsel.base = rp[0];
        for (uint32_t i = 0; i < used; ++i) dsel.u[i] = rp[i].uniform;
        dsel.wb = WaveStatsBufs{logits, row_stride, vocab, waves,
                                (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (row_stride & 3) == 0 ? 1u : 0u,
                                st};
        dsel.mb = SampleMergeBufs{logits, row_stride, vocab, waves, st, ss.verify_tokens};
    } else {
        TWD_HIP(hipEventRecord(ds.fork, s));
        TWD_HIP(hipStreamWaitEvent(ds.side, ds.fork, 0));
        rc = launch_select(sel->scratch, const_cast<float*>(logits), vocab, used, row_stride, rp, nullptr,
                           sel->scratch.verify_tokens, ds.side);
        TWD_HIP(hipEventRecord(ds.join, ds.side));
        if (rc) {
            (void)hipStreamWaitEvent(s, ds.join, 0);
            return rc;
        }
    }

    a.vocab = vocab;
    a.estride = (vocab + 15u) & ~15u;
    a.parts = (vocab + kDraftChunk - 1) / kDraftChunk;
    a.temp = params->temperature <= 0.0f ? 1.0f : params->temperature;
    a.drafts = drafts;
    a.part = sel->draft.part;
    a.e = sel->draft.e;
    a.flags = sel->draft.flags;
    a.rej = sel->draft.rej;
    a.sums = sel->draft.sums;
    a.seg_d = sel->draft.seg_d;
    a.xin = sel->draft.xin;
    sel->draft.last_npos = a.npos;
    for (uint32_t i = 0; i < a.npos; ++i) sel->draft.last_pos[i] = a.pos[i].position;
    const dim3 grid(a.parts, 2 * a.npos);
    draft_max_kernel<<<dim3(a.parts, 2 * a.npos + dsel.nsel), kDraftThreads, 0, s>>>(a, dsel);
    draft_exp_kernel<<<grid, kDraftThreads, 0, s>>>(a);
    // the softmax sums, then the ratio tests, then the residual draws of rejected positions,
    // each exact sum through the segmented pipeline
    const uint32_t nseg = seg_count(vocab);
    double* seg_d = sel->draft.seg_d;
    SegRec* seg_rec = static_cast<SegRec*>(sel->draft.seg_rec);
    const SegSrcSoftmax src_e{a.e, a.estride, a.flags};
    SegHead* seg_head = static_cast<SegHead*>(ds.seg_head);
    seg_xfer_kernel<<<dim3(xfer_blocks(vocab), 2 * a.npos), kXferThreads, 0, s>>>(src_e, vocab, seg_d, seg_rec,
                                                                                 0.0f, 0u, seg_head, a.xin);
    seg_sum_kernel<<<2 * a.npos + dsel.nsel, kRejThreads, 0, s>>>(a, seg_rec, seg_head, dsel);
    seg_ratio_dsum_kernel<<<dim3(xfer_blocks(vocab), a.npos), kXferThreads, 0, s>>>(a, ds.live, seg_d);
    const SegSrcResidual src_r{a.e, a.estride, a.sums, ds.live};
    seg_xfer_kernel<<<dim3(xfer_blocks(vocab), a.npos), kXferThreads, 0, s>>>(src_r, vocab, seg_d, seg_rec, 0.0f, 0u,
                                                                             seg_head, a.xin);
    if (!fused) TWD_HIP(hipStreamWaitEvent(s, ds.join, 0));  // the selector's tokens, read by the finish
    ds.fin_epoch = epoch_after(ds.fin_epoch);
    const DraftFinish fin{sel->scratch.verify_tokens, used, drafts, n_drafts, has, result,
                          reinterpret_cast<unsigned long long*>(ds.fin_ctr), ds.fin_epoch,
                          epoch_after(ds.fin_epoch)};
    seg_residual_kernel<<<a.npos, kRejThreads, 0, s>>>(a, ds.live, seg_rec, seg_head, fin);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

}  // namespace twd
