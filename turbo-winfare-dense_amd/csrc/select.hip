// Token selection over device logit rows on gfx950: repetition penalty, greedy argmax and the
// sampled chain of sample_token (src/sampling.cpp:74-169), plus verify bookkeeping.
//
// select_slice_kernel covers all rows: grid (parts, rows), each 512-thread block owns an
// 8192-entry slice of one row, 16 values per thread held in registers. Per block: penalty on
// the slice's history ids (occurrence counts in LDS, each applied one occurrence at a time like
// the reference loop), then either the greedy rank maximum or {slice max, sum exp(l - slice max)
// in double, the slice's top-`want` ranks}. A row held by one slice finishes in the same
// block; otherwise select_merge_kernel (one block per row, second launch) merges the slices,
// ranks the global top-`want`, and runs top-p, top-k and the draw in reference order.
//
// The top-`want` of a block (block_top) is found by distance from the block's maximum: a
// 256-bin histogram of (max - v) locates the bin holding the want-th rank, every entry of a
// nearer bin is taken, and the boundary bin's entries are ranked exactly among themselves by
// the 64-bit (value desc, index asc) rank. Only the boundary bin needs exact work, and the
// histogram's atomics spread over 8 replicas. Blocks whose values do not bin usefully (all
// equal, non-finite extremes, an overfull boundary bin) fall back to a radix select on ranks.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "select_core.h"

namespace twd {


constexpr int kSliceThreads = 512;     // two slice blocks share a CU
constexpr int kSelPerThread = 16;
constexpr uint32_t kSlice = kSliceThreads * kSelPerThread;  // vocabulary entries per slice block
constexpr uint32_t kMaxParts = 64;    // vocab <= 64 * 8192 = 524288
constexpr int kMergeThreads = 256;
constexpr int kMergePerThread = kMaxParts * kMaxWant / kMergeThreads;  // 64

struct SelectArgs {
    uint32_t rows;
    uint32_t parts;
    uint32_t penalty_only;  // stop after the repetition penalty
    uint32_t one_pass;      // every row greedy: the slice blocks finish the rows themselves
    uint32_t epoch, next_epoch;
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
    uint64_t* gbest;  // one-pass greedy: per-row best ranks, zero between launches
    uint64_t* gctr;   // its arrival counter, kArriveWords words (grid_arrive)
};

// ... and per kernel: the slice kernel's penalty counts, then a copy of its values for the
// radix fallback, one entry per thread and slot so neither needs a barrier to hand over (two
// slice blocks fit on a CU); the merge kernel keeps every slice's ranks.
struct SliceShared {
    union {
        uint32_t cnt[kSlice];
        float vals[kSlice];
    } u;
    TopScratch t;
    SelCommon c;
};

struct MergeShared {
    uint64_t cand[kMaxParts * kMaxWant];  // every slice's ranks, packed
    uint32_t offs[kMaxParts + 1];         // where each slice's ranks start in cand
    TopScratch t;
    SelCommon c;
};

// After c.top[0..want) holds the row's shortlist and c.gmax/total/flag its statistics:
// the degenerate check of sampling.cpp:116-118, the shortlist sort, and steps 5-7.
__device__ __forceinline__ void finish_row(SelCommon& c, uint32_t want, const twd_row_params& p,
                           uint32_t* token_out, const float* row_logits, uint32_t vocab) {
    const int tid = threadIdx.x;
    if (c.flag != 0 || !(c.total > 0.0)) {
        if (tid == 0) *token_out = TWD_TOKEN_DEGENERATE;
        return;
    }
    block_sort_desc(c, want);
    const uint32_t tok = finish_sampled(c, want, p, c.total, RowSrc{row_logits, vocab, c.gmax, want});
    if (tid == 0) *token_out = tok;
}

// One-pass greedy finish (every row of the launch greedy, more than one slice): each slice block
// folds its best rank into its row's gbest slot with a returning atomic max and then counts
// itself in; the block that completes the count reads and clears every row's slot and writes
// the tokens. The protocol is the head's grid finish (device-scope atomics only, no fence):
// a returning atomic is performed at the memory-side coherence point before it returns, and
// the block waits for that return before it counts in, so every maximum precedes its
// block's arrival. The count is grid_arrive's (an epoch per launch, replay slots for captured
// launches).
__device__ __forceinline__ void select_greedy_finish(const SelectArgs& args, const SelectBufs& b, uint32_t row,
                                                     uint64_t k, SelCommon& c) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        const unsigned long long seen = __hip_atomic_fetch_max(reinterpret_cast<unsigned long long*>(b.gbest + row),
                                                               static_cast<unsigned long long>(k), __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT);
        c.red64[0] = seen;  // waits for the return: the maximum is performed before the count
        const uint32_t nb = gridDim.x * gridDim.y;
        const bool last = grid_arrive(reinterpret_cast<unsigned long long*>(b.gctr), nb, args.epoch, args.next_epoch);
        c.misc[7] = last ? 1u : 0u;
    }
    __syncthreads();
    if (!c.misc[7]) return;
    for (uint32_t r = tid; r < args.rows; r += blockDim.x) {
        const uint64_t kk = __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(b.gbest + r), 0ull,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        b.tokens[r] = rank_index(kk);
    }
}

// SelectArgs is the first kernel argument, so it sits at offset 0 of the kernarg segment. The
// row's parameters are read through that pointer: indexing the by-value argument with
// blockIdx.y would make the compiler copy all of it into per-lane scratch memory.
__global__ __launch_bounds__(kSliceThreads) __attribute__((amdgpu_waves_per_eu(4)))
void select_slice_kernel(SelectArgs args_by_value, SelectBufs b) {
    constexpr int NT = kSliceThreads;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    SliceShared& sh = *reinterpret_cast<SliceShared*>(smem_raw);
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
        const uint32_t i = lo + tid + NT * e;
        v[e] = i < hi ? lg[i] : 0.0f;
    }
    for (uint32_t i = tid; i < kReps * kBins; i += NT) sh.t.hist[i] = 0;  // for block_top

    // ---- repetition penalty, sampling.cpp:74-90 ----
    if (p.repetition_penalty != 1.0f && p.history_len > 0) {
        // history ids in batches of kHistBatch per thread, each batch requested at once (one
        // round trip, not one per id); the first batch before the counts are cleared
        constexpr int kHistBatch = 8;
        const uint32_t* hist = b.history + p.history_offset;
        const uint32_t hlen = p.history_len;
        uint32_t ids[kHistBatch];
        auto fetch = [&](uint32_t j0) {
#pragma unroll
            for (int q = 0; q < kHistBatch; ++q) {
                const uint32_t j = j0 + tid + NT * q;
                ids[q] = j < hlen ? hist[j] : 0xFFFFFFFFu;  // never inside a slice
            }
        };
        auto count = [&]() {
#pragma unroll
            for (int q = 0; q < kHistBatch; ++q)
                if (ids[q] >= lo && ids[q] < hi) atomicAdd(&sh.u.cnt[ids[q] - lo], 1u);
        };
        fetch(0);
#pragma unroll
        for (int e = 0; e < kSelPerThread; ++e) sh.u.cnt[tid + NT * e] = 0;
        __syncthreads();
        count();
        for (uint32_t j0 = NT * kHistBatch; j0 < hlen; j0 += NT * kHistBatch) {
            fetch(j0);
            count();
        }
        __syncthreads();
        const float rp = p.repetition_penalty;
        const float limit = (p.softcap > 0.0f) ? p.softcap * 0.9999f : 0.0f;
#pragma unroll
        for (int e = 0; e < kSelPerThread; ++e) {
            const uint32_t n = sh.u.cnt[tid + NT * e];
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
            lg[lo + tid + NT * e] = x;
        }
    }
    if (args.penalty_only) return;

    auto key_at = [&](int e) -> uint64_t {
        const uint32_t i = lo + tid + NT * e;
        return i < hi ? rank_key(v[e], i) : 0ull;
    };
    const bool greedy = p.temperature <= 0.0f;  // sampling.cpp:97: a NaN temperature samples
    if (greedy) {
        // ---- sampling.cpp:97-104 ----
        uint64_t k = 0;
#pragma unroll
        for (int e = 0; e < kSelPerThread; ++e) {
            const uint64_t r = key_at(e);
            k = r > k ? r : k;
        }
        k = block_max_u64<NT>(k, sh.c);
        if (parts == 1) {
            if (tid == 0) b.tokens[row] = rank_index(k);
            return;
        }
        if (args.one_pass) {
            select_greedy_finish(args, b, row, k, sh.c);
            return;
        }
        if (tid == 0) b.part_key[static_cast<size_t>(row) * parts + part] = k;
        return;
    }

    // a shortlist longer than kMaxWant: the long path finishes the row from its wave records
    if (p.top_k > static_cast<int32_t>(kMaxWant) && b.vocab > kMaxWant) return;
    // ---- sampled: slice statistics, sampling.cpp:109-118 ----
    // Any NaN makes the row degenerate, so the max only has to be right for NaN-free rows.
    uint32_t nan_seen = 0;
    float mx = -INFINITY, mn = INFINITY;
#pragma unroll
    for (int e = 0; e < kSelPerThread; ++e) {
        sh.u.vals[tid + NT * e] = v[e];  // the slot's count was read by this same thread
        if (lo + tid + NT * e < hi) {
            if (v[e] != v[e]) nan_seen = 1;
            mx = fmaxf(mx, v[e]);
            if (__builtin_isfinite(v[e])) mn = fminf(mn, v[e]);
        }
    }
    if (tid < 64) sh.c.exp2_tbl[tid] = kExp2Table[tid];
    block_stats<NT>(nan_seen, mx, mn, sh.c);  // its barriers also retire the penalty's counts
    const double dmx = static_cast<double>(mx);
    double s = 0.0;
#pragma unroll
    for (int e = 0; e < kSelPerThread; ++e)
        if (lo + tid + NT * e < hi) s += exp_for_sum(static_cast<double>(v[e]) - dmx, sh.c.exp2_tbl);
    s = block_sum_f64<NT>(s, sh.c);
    // A slice of -inf entries only adds exp(-inf - row max) = 0 to the row's sum whenever the
    // row has a finite maximum elsewhere (its own exp(-inf - -inf) would be NaN). If the whole
    // row is -inf every slice reports 0, the row total is 0 and the row is degenerate, as the
    // reference's NaN total makes it.
    if (mx == -INFINITY) s = 0.0;

    // ---- shortlist of this slice, sampling.cpp:120-137 ----
    const uint32_t want_row = (p.top_k > 0) ? min(static_cast<uint32_t>(p.top_k), b.vocab)
                                            : min(kMaxWant, b.vocab);
    const uint32_t n_here = hi - lo;
    const uint32_t want = min(want_row, n_here);
    auto val_at = [&](int e) -> float { return v[e]; };
    auto slow_val = [&](int e) -> float { return sh.u.vals[tid + NT * e]; };
    auto slow_key = [&](int e) -> uint64_t {
        const uint32_t i = lo + tid + NT * e;
        return i < hi ? rank_key(sh.u.vals[tid + NT * e], i) : 0ull;
    };
    uint64_t* out = (parts == 1) ? sh.c.top : b.cand + (static_cast<size_t>(row) * parts + part) * kMaxWant;
    block_top<NT, kSelPerThread>(val_at, key_at, slow_val, slow_key, kSelPerThread, mx, mn, want, out,
                                 sh.t, sh.c);

    if (parts > 1) {
        if (tid == 0) {
            const size_t o = static_cast<size_t>(row) * parts + part;
            b.part_max[o] = mx;
            b.part_sum[o] = s;
            b.part_flag[o] = nan_seen;
            b.part_count[o] = min(sh.c.misc[4], want);  // fewer only when NaNs hold no rank
        }
        return;  // select_merge_kernel finishes the row
    }
    if (tid == 0) {
        sh.c.gmax = mx;
        sh.c.total = s;
        sh.c.flag = nan_seen;
    }
    __syncthreads();
    finish_row(sh.c, want_row, p, b.tokens + row, b.logits + static_cast<size_t>(row) * b.stride, b.vocab);
}

// Second launch when a row spans several slices: global max, the rescaled sum of exponentials,
// the global shortlist from every slice's candidates, then the draw. One block per row.
__global__ __launch_bounds__(kMergeThreads) void select_merge_kernel(SelectArgs args_by_value, SelectBufs b) {
    constexpr int NT = kMergeThreads;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    MergeShared& sh = *reinterpret_cast<MergeShared*>(smem_raw);
#if __HIP_DEVICE_COMPILE__
    const SelectArgs& args =
        *reinterpret_cast<const SelectArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
#else
    const SelectArgs& args = args_by_value;
#endif
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t row = blockIdx.x;
    const uint32_t parts = args.parts;  // <= kMaxParts = 64: one lane of wave 0 per slice
    const twd_row_params p = args.p[row];
    const size_t o = static_cast<size_t>(row) * parts;

    if (p.temperature <= 0.0f) {  // greedy: the best rank over the slices
        if (tid < 64) {
            const uint64_t m = wave_max_u64(static_cast<uint32_t>(lane) < parts ? b.part_key[o + lane] : 0ull);
            if (tid == 0) b.tokens[row] = rank_index(m);
        }
        return;
    }
    const uint32_t want_row = (p.top_k > 0) ? min(static_cast<uint32_t>(p.top_k), b.vocab)
                                            : min(kMaxWant, b.vocab);
    if (want_row > kMaxWant) return;  // the long path finishes the row
    for (uint32_t i = tid; i < kReps * kBins; i += NT) sh.t.hist[i] = 0;  // for block_top
    // Wave 0: global max and NaN flag over the slices, the row sum
    // sum_q part_sum[q] * exp(part_max[q] - max), and where each slice's ranks go.
    if (tid < 64) {
        const bool live = static_cast<uint32_t>(lane) < parts;
        const float pm = live ? b.part_max[o + lane] : -INFINITY;
        const double ps = live ? b.part_sum[o + lane] : 0.0;
        uint32_t fl = live ? b.part_flag[o + lane] : 0u;
        const uint32_t cnt = live ? b.part_count[o + lane] : 0u;
        float gm = pm;
        uint32_t x = cnt;  // inclusive prefix sum of the counts
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            gm = fmaxf(gm, __shfl_xor(gm, m));
            fl |= __shfl_xor(fl, m);
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        double contrib = live ? ps * exp(static_cast<double>(pm) - static_cast<double>(gm)) : 0.0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) contrib += __shfl_xor(contrib, m);
        sh.offs[lane] = x - cnt;
        if (lane == 63) sh.offs[kMaxParts] = x;
        if (lane == 0) {
            sh.c.gmax = gm;
            sh.c.total = contrib;
            sh.c.flag = fl;
        }
    }
    __syncthreads();
    const uint32_t n_cand = sh.offs[kMaxParts];
    const float gm = sh.c.gmax;
    // every slice's ranks, packed into cand[0 .. n_cand)
    float cmn = INFINITY;
    const uint32_t nf = parts * want_row;
    constexpr int kGatherBatch = 4;  // loads requested together, then stored
    for (uint32_t f0 = 0; f0 < nf; f0 += NT * kGatherBatch) {
        uint64_t kk[kGatherBatch];
        uint32_t at[kGatherBatch];
#pragma unroll
        for (int u = 0; u < kGatherBatch; ++u) {
            const uint32_t f = f0 + tid + NT * u;
            at[u] = 0xFFFFFFFFu;
            kk[u] = 0;
            if (f < nf) {
                const uint32_t q = f / want_row, slot = f % want_row;
                const uint32_t a = sh.offs[q] + slot;
                if (a < sh.offs[q + 1]) {
                    at[u] = a;
                    kk[u] = b.cand[(o + q) * kMaxWant + slot];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kGatherBatch; ++u) {
            if (at[u] == 0xFFFFFFFFu) continue;
            sh.cand[at[u]] = kk[u];
            const float x = rank_value(kk[u]);
            if (kk[u] != 0 && __builtin_isfinite(x)) cmn = fminf(cmn, x);
        }
    }
    uint32_t no_flag = 0;
    float no_max = -INFINITY;
    block_stats<NT>(no_flag, no_max, cmn, sh.c);  // its barriers also publish sh.cand
    auto merge_key = [&](int e) -> uint64_t {
        const uint32_t f = tid + NT * e;
        return f < n_cand ? sh.cand[f] : 0ull;
    };
    auto merge_val = [&](int e) -> float { return rank_value(merge_key(e)); };
    const int per = static_cast<int>((n_cand + NT - 1) / NT);
    block_top<NT, kMergePerThread>(merge_val, merge_key, merge_val, merge_key, per, gm, cmn, want_row,
                                   sh.c.top, sh.t, sh.c);
    finish_row(sh.c, want_row, p, b.tokens + row, b.logits + static_cast<size_t>(row) * b.stride, b.vocab);
}

// ---- after the head's sample mode (or the wave-record pass): one block per row --------------------
// sample_merge_row (select_core.h) finishes each row from its per-64-entry records.
__global__ __launch_bounds__(kSmThreads) void select_sample_merge_kernel(SelectArgs args_by_value,
                                                                         SampleMergeBufs b) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    SampleMergeShared& sh = *reinterpret_cast<SampleMergeShared*>(smem_raw);
#if __HIP_DEVICE_COMPILE__
    const SelectArgs& args =
        *reinterpret_cast<const SelectArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
#else
    const SelectArgs& args = args_by_value;
#endif
    const uint32_t row = blockIdx.x;
    sample_merge_row(args.p[row], row, b, sh);
}

// ---- shortlists longer than 256: top_k > 256 -------------------------------------------------------
//
// sample_token takes any top_k: its shortlist is the top want = min(top_k, V) entries in the
// order (value desc, index asc), and steps 5-7 run over all of them (sampling.cpp:120-168).
// Rows with temperature > 0 and want > 256 are finished here, from the penalised logits and the
// same wave records as the shorter rows (so the same row max and total):
//   * long_gather_kernel, one block per row: records_stats, then every entry of a candidate wave
//     (maximum in a bin <= b*) that lies in a bin <= b*, into the row's sort buffer in any
//     order. Every top-`want` entry is among them. The buffer is padded with zero ranks (below
//     every real rank) to a power of two, its sort length;
//   * a bitonic sort of each buffer into descending order: long_sort_tile_kernel sorts tiles of
//     kSortTile ranks in LDS (alternating directions); each longer stage k runs its cross-tile
//     steps (long_sort_step_kernel, one launch per step) and then its in-tile steps
//     (long_sort_merge_kernel). The launches cover the longest possible buffer; a block past its
//     row's sort length, or of a stage longer than it, returns at once;
//   * long_finish_kernel, one block per row: steps 5-7 over the sorted ranks, kFinTile at a
//     time. The block forms the terms exp(l - max) / total and exp((l - max) / T) in LDS with the
//     reference's expressions; the two running sums then go in reference order on two lanes of
//     wave 0 (finish_sampled's loop), and the running sums of the temperature weights are kept in
//     memory. After the cut (top-p, then top-k), r = u * denom and the draw is the first running
//     sum >= r: the running sums never decrease, so a search over the tiles' last sums, then
//     over one tile, finds it.
constexpr int kLongThreads = 1024;
constexpr uint32_t kSortTile = 8192;  // ranks sorted in LDS by one block (64 KB)
constexpr int kStepThreads = 256;
constexpr uint32_t kFinTile = 2048;   // shortlist entries per tile of the finish

struct LongArgs {
    uint32_t n;                          // long rows in the launch
    uint32_t row[TWD_MAX_ROWS + 1];      // each one's row in the call
    twd_row_params p[TWD_MAX_ROWS + 1];  // and its parameters
};

struct LongBufs {
    const float* logits;  // [rows][stride], penalised
    uint64_t stride;
    uint32_t vocab;
    uint32_t waves;       // records per row
    SampleStats st;       // [row][waves]
    uint64_t npad;        // sort buffer per long row: a power of two >= vocab
    uint64_t* keys;       // [n][npad]
    double* pre;          // [n][npad] running sums of the temperature weights
    uint32_t* len;        // [n] sort length (0: the row is already finished)
    float* gmax;          // [n]
    double* total;        // [n]
    uint32_t* tokens;
};

struct LongGatherShared {
    uint32_t cwave[kSampleMaxWaves];
    TopScratch t;
    SelCommon c;
};

// The long-path kernels read LongArgs (the first kernel argument) through the kernarg segment
// pointer: indexing the by-value argument with blockIdx would copy it to scratch memory.
#if __HIP_DEVICE_COMPILE__
#define TWD_LONG_ARGS(byval) \
    (*reinterpret_cast<const LongArgs*>(__builtin_amdgcn_kernarg_segment_ptr()))
#else
#define TWD_LONG_ARGS(byval) (byval)
#endif

__global__ __launch_bounds__(kLongThreads) void long_gather_kernel(LongArgs args_by_value, LongBufs b) {
    constexpr int NT = kLongThreads;
    static_assert(NT == kSmThreads, "records_stats' block");
    extern __shared__ __align__(16) unsigned char smem_raw[];
    LongGatherShared& sh = *reinterpret_cast<LongGatherShared*>(smem_raw);
    const LongArgs& args = TWD_LONG_ARGS(args_by_value);
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t j = blockIdx.x;
    const uint32_t row = args.row[j];
    const twd_row_params p = args.p[j];
    const uint32_t W = b.waves;
    const size_t o = static_cast<size_t>(row) * W;
    const float* lg = b.logits + static_cast<size_t>(row) * b.stride;
    uint64_t* keys = b.keys + static_cast<size_t>(j) * b.npad;

    if (tid < 64) sh.c.exp2_tbl[tid] = kExp2Table[tid];
    uint64_t key[kSmPer];
    double wsum[kSmPer];
#pragma unroll
    for (uint32_t q = 0; q < kSmPer; ++q) {
        const uint32_t i = tid + NT * q;
        key[q] = i < W ? b.st.key[o + i] : 0ull;
        wsum[q] = i < W ? b.st.sum[o + i] : 0.0;
    }
    for (uint32_t i = tid; i < kReps * kBins; i += NT) sh.t.hist[i] = 0;
    const uint32_t want = min(static_cast<uint32_t>(p.top_k), b.vocab);
    float wm[kSmPer];
    bool live[kSmPer];
    uint32_t nan = 0;
#pragma unroll
    for (uint32_t q = 0; q < kSmPer; ++q) {
        live[q] = key[q] != 0;
        wm[q] = live[q] ? rank_value(key[q]) : -INFINITY;
        nan |= wsum[q] != wsum[q] ? 1u : 0u;
    }
    const RecStats rs = records_stats(live, wm, nan, wsum, fixed_ref(b.st.cap, p), want, sh.t, sh.c);
    if (rs.degenerate) {  // sampling.cpp:116-118
        if (tid == 0) {
            b.tokens[row] = TWD_TOKEN_DEGENERATE;
            b.len[j] = 0;
        }
        return;
    }
    // the candidate waves, in any order (at most W <= kSampleMaxWaves)
#pragma unroll
    for (uint32_t q = 0; q < kSmPer; ++q) {
        const uint32_t i = tid + NT * q;
        const bool is_cand = key[q] != 0 && rec_bin(rs, wm[q]) <= rs.bstar;
        const uint64_t mask = __ballot(is_cand);
        if (mask != 0) {
            const int leader = __ffsll(static_cast<long long>(mask)) - 1;
            uint32_t base = 0;
            if (lane == leader) base = atomicAdd(&sh.c.misc[3], static_cast<uint32_t>(__popcll(mask)));
            base = __builtin_amdgcn_readlane(base, leader);
            if (is_cand) {
                const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
                sh.cwave[base + below] = i;
            }
        }
    }
    __syncthreads();
    const uint32_t nent = sh.c.misc[3] * kSampleWaveRows;
    // the survivors into the sort buffer, eight loads requested at a time
    constexpr uint32_t kBatch = 8;
    const uint32_t per = (nent + NT - 1) / NT;
    for (uint32_t i0 = 0; i0 < per; i0 += kBatch) {
        float v[kBatch];
        uint32_t r[kBatch];
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) {
            const uint32_t f = (i0 + q) * NT + static_cast<uint32_t>(tid);
            r[q] = 0xFFFFFFFFu;
            v[q] = 0.0f;
            if (i0 + q < per && f < nent) {
                const uint32_t rr = sh.cwave[f / kSampleWaveRows] * kSampleWaveRows + f % kSampleWaveRows;
                if (rr < b.vocab) {
                    r[q] = rr;
                    v[q] = lg[rr];
                }
            }
        }
#pragma unroll
        for (uint32_t q = 0; q < kBatch; ++q) {
            const bool keep = r[q] != 0xFFFFFFFFu && rec_bin(rs, v[q]) <= rs.bstar;
            wave_put(keep, keep ? rank_key(v[q], r[q]) : 0ull, &sh.c.misc[4], keys, static_cast<uint32_t>(b.npad));
        }
    }
    __syncthreads();
    const uint32_t n = sh.c.misc[4];
    uint32_t len = 1;
    while (len < n) len <<= 1;
    for (uint32_t i = n + tid; i < len; i += NT) keys[i] = 0ull;
    if (tid == 0) {
        b.len[j] = len;
        b.gmax[j] = rs.gm;
        b.total[j] = rs.total;
    }
}

// One compare-exchange of the bitonic network over a row's buffer (global positions): the pair
// (i, i | jj) in stage k is put in descending order when bit k of i is clear, ascending when it
// is set, so the last stage (k = length) leaves the whole buffer descending.
__device__ __forceinline__ void bitonic_pair(uint64_t& a, uint64_t& c, uint64_t gi, uint64_t k) {
    const bool desc = (gi & k) == 0;
    if (desc ? a < c : a > c) {
        const uint64_t t = a;
        a = c;
        c = t;
    }
}

// steps jj = j0, j0 / 2, .., 1 of stage k on the LDS tile s of `t` ranks starting at global base
__device__ __forceinline__ void bitonic_tile_steps(uint64_t* s, uint32_t t, uint64_t base, uint64_t k, uint32_t j0) {
    for (uint32_t jj = j0; jj > 0; jj >>= 1) {
        for (uint32_t q = threadIdx.x; q < t / 2; q += blockDim.x) {
            const uint32_t i = ((q & ~(jj - 1)) << 1) | (q & (jj - 1));
            uint64_t a = s[i], c = s[i | jj];
            bitonic_pair(a, c, base + i, k);
            s[i] = a;
            s[i | jj] = c;
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(kLongThreads) void long_sort_tile_kernel(LongBufs b, uint32_t tile) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    uint64_t* s = reinterpret_cast<uint64_t*>(smem_raw);
    const uint32_t j = blockIdx.y;
    const uint32_t len = b.len[j];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile;
    if (base >= len) return;  // the whole block
    const uint32_t t = min(tile, len);  // both powers of two
    uint64_t* keys = b.keys + static_cast<size_t>(j) * b.npad + base;
    for (uint32_t i = threadIdx.x; i < t; i += blockDim.x) s[i] = keys[i];
    __syncthreads();
    for (uint32_t k = 2; k <= t; k <<= 1) bitonic_tile_steps(s, t, base, k, k >> 1);
    for (uint32_t i = threadIdx.x; i < t; i += blockDim.x) keys[i] = s[i];
}

__global__ __launch_bounds__(kStepThreads) void long_sort_step_kernel(LongBufs b, uint32_t k, uint32_t jj) {
    const uint32_t j = blockIdx.y;
    const uint32_t len = b.len[j];
    const uint64_t q = static_cast<uint64_t>(blockIdx.x) * kStepThreads + threadIdx.x;
    if (k > len || 2 * q >= len) return;
    const uint64_t i = ((q & ~static_cast<uint64_t>(jj - 1)) << 1) | (q & (jj - 1));
    uint64_t* keys = b.keys + static_cast<size_t>(j) * b.npad;
    uint64_t a = keys[i], c = keys[i | jj];
    bitonic_pair(a, c, i, k);
    keys[i] = a;
    keys[i | jj] = c;
}

__global__ __launch_bounds__(kLongThreads) void long_sort_merge_kernel(LongBufs b, uint32_t tile, uint32_t k) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    uint64_t* s = reinterpret_cast<uint64_t*>(smem_raw);
    const uint32_t j = blockIdx.y;
    const uint32_t len = b.len[j];
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * tile;
    if (k > len || base >= len) return;  // the whole block; here len >= k > tile
    uint64_t* keys = b.keys + static_cast<size_t>(j) * b.npad + base;
    for (uint32_t i = threadIdx.x; i < tile; i += blockDim.x) s[i] = keys[i];
    __syncthreads();
    bitonic_tile_steps(s, tile, base, k, tile >> 1);
    for (uint32_t i = threadIdx.x; i < tile; i += blockDim.x) keys[i] = s[i];
}

struct LongFinishShared {
    double e[kFinTile];  // exp(l - max) / total, then lane 1's running sums
    double q[kFinTile];  // exp((l - max) / T), then lane 0's running sums
    double base;         // lane 1's running sum before the tile
    double total;        // the reference's row total, when the cut takes it
    uint32_t misc[4];
    uint32_t best;
};

__global__ __launch_bounds__(kLongThreads) void long_finish_kernel(LongArgs args_by_value, LongBufs b) {
    constexpr int NT = kLongThreads;
    __shared__ LongFinishShared sh;
    const LongArgs& args = TWD_LONG_ARGS(args_by_value);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t j = blockIdx.x;
    if (b.len[j] == 0) return;  // degenerate: long_gather_kernel wrote its token
    const uint32_t row = args.row[j];
    const twd_row_params p = args.p[j];
    const uint64_t* keys = b.keys + static_cast<size_t>(j) * b.npad;
    double* pre = b.pre + static_cast<size_t>(j) * b.npad;
    const uint32_t want = min(static_cast<uint32_t>(p.top_k), b.vocab);
    const double mx = static_cast<double>(b.gmax[j]);
    double total = b.total[j];
    const double td = static_cast<double>(p.temperature);
    const bool topp = p.top_p < 1.0f;
    const double pp = static_cast<double>(p.top_p);
    constexpr uint32_t kChunk = 16;
    uint32_t cut = want;
    // a second pass with the reference's own row total when the first pass's cut lies within
    // total_tol of p (see finish_sums_exact)
    for (int pass = 0;; ++pass) {
        double run = 0.0;  // wave 0: lane 0's sum of the weights, lane 1's top-p sum
        uint32_t tl = 0;   // the last tile's first entry
        cut = want;
        if (tid == 0) sh.misc[0] = 0;
        for (uint32_t t0 = 0; t0 < want; t0 += kFinTile) {
            tl = t0;
            const uint32_t cnt = min(kFinTile, want - t0);
            // steps 5 and 7's terms, as sampling.cpp:145 and :157 form them
            for (uint32_t i = tid; i < cnt; i += NT) {
                const double l = static_cast<double>(rank_value(keys[t0 + i]));
                sh.q[i] = exp_libm((l - mx) / td);
                if (topp) sh.e[i] = exp_libm(l - mx) / total;
            }
            __syncthreads();
            if (wave == 0 && lane < 2) {
                // lane 0 reads q and stores its running sums over q; lane 1 does the same over e
                // (over q when top-p is off: its sums are then never used)
                double* src = (lane == 0 || !topp) ? sh.q : sh.e;
                if (lane == 1) sh.base = run;  // the top-p sum before the tile
                double x[kChunk];
#pragma unroll
                for (uint32_t jj = 0; jj < kChunk; ++jj) x[jj] = src[min(jj, cnt - 1)];
                for (uint32_t i0 = 0; i0 < cnt; i0 += kChunk) {
                    double xn[kChunk], pr[kChunk];
                    if (i0 + kChunk < cnt) {
#pragma unroll
                        for (uint32_t jj = 0; jj < kChunk; ++jj) xn[jj] = src[min(i0 + kChunk + jj, cnt - 1)];
                    }
#pragma unroll
                    for (uint32_t jj = 0; jj < kChunk; ++jj) {
                        run += x[jj];
                        pr[jj] = run;
                    }
                    uint32_t hit = 0;
#pragma unroll
                    for (uint32_t jj = 0; jj < kChunk; ++jj) {
                        src[i0 + jj] = pr[jj];  // i0 + jj < cnt rounded up to kChunk <= kFinTile
                        hit |= (pr[jj] >= pp ? 1u : 0u) << jj;
                    }
                    uint32_t h1 = __builtin_amdgcn_readlane(hit, 1);
                    h1 &= cnt - i0 >= kChunk ? 0xFFFFu : ((1u << (cnt - i0)) - 1u);
                    if (topp && h1 != 0) {  // lane 0's sums cover the cut
                        if (lane == 0) sh.misc[0] = t0 + i0 + static_cast<uint32_t>(__builtin_ctz(h1)) + 1;
                        break;
                    }
#pragma unroll
                    for (uint32_t jj = 0; jj < kChunk; ++jj) x[jj] = xn[jj];
                }
            }
            __syncthreads();
            const uint32_t c = sh.misc[0];  // the cut, once the top-p sum has reached p
            const uint32_t keep = c != 0 ? c - t0 : cnt;
            for (uint32_t i = tid; i < keep; i += NT) pre[t0 + i] = sh.q[i];
            if (c != 0) {
                cut = c;
                break;
            }
            __syncthreads();  // the next tile's terms overwrite sh
        }
        if (!topp || pass > 0) break;
        // the last tile's top-p sums are in sh.e: the one at the cut (when it reached p) and the
        // one before it decide (as in finish_sums_exact)
        if (tid == 0) {
            const double tc = total_tol(b.vocab);
            const double hi = sh.e[cut - 1 - tl];
            const double lo = cut >= 2 ? (cut - 2 >= tl ? sh.e[cut - 2 - tl] : sh.base) : 0.0;
            const bool near = (hi >= pp && hi <= pp * (1.0 + tc)) ||
                              (cut >= 2 && lo >= pp * (1.0 - tc) && lo <= pp * (1.0 + tc));
            sh.misc[2] = near ? 1u : 0u;
        }
        __syncthreads();
        if (sh.misc[2] == 0) break;
        if (wave == 0) {
            const double t = exact_row_total(RowSrc{b.logits + static_cast<size_t>(row) * b.stride, b.vocab,
                                                    b.gmax[j], 0u}, sh.e);
            if (lane == 0) sh.total = t;
        }
        __syncthreads();
        total = sh.total;
    }
    if (p.top_k > 0 && cut > static_cast<uint32_t>(p.top_k)) cut = static_cast<uint32_t>(p.top_k);
    if (cut < 1) cut = 1;
    if (tid == 0) sh.best = cut - 1;  // the reference's fallback: the last survivor
    __syncthreads();                  // also publishes pre (block scope)
    const double r = static_cast<double>(p.uniform) * pre[cut - 1];  // r = u * denom
    // the first tile whose last running sum (within the cut) reaches r, then its first entry
    const uint32_t ntiles = (cut + kFinTile - 1) / kFinTile;
    if (tid == 0) sh.misc[1] = ntiles - 1;
    __syncthreads();
    for (uint32_t t = tid; t < ntiles; t += NT)
        if (pre[min((t + 1) * kFinTile, cut) - 1] >= r) atomicMin(&sh.misc[1], t);
    __syncthreads();
    const uint32_t t0 = sh.misc[1] * kFinTile, t1 = min(t0 + kFinTile, cut);
    for (uint32_t i = t0 + tid; i < t1; i += NT)
        if (pre[i] >= r) atomicMin(&sh.best, i);
    __syncthreads();
    if (tid == 0) b.tokens[row] = rank_index(keys[sh.best]);
}

// ---- the wave-record path for logits that are already in memory ---------------------------------
//
// Rows whose logits the caller holds (twd_select, the head for rows > 4) reach
// select_sample_merge_kernel through two short passes instead of the slice kernels:
//   * penalty_hash_kernel, one block per row: the row's history ids into an LDS hash table of
//     (id, occurrences) while each id's logit is requested, then each distinct id's logit gets
//     the penalty once per occurrence, one after another as the reference loop applies them
//     (sampling.cpp:74-90), from the thread that entered the id; only those entries are read
//     and written;
//   * wave_stats_kernel: per 64 entries of a row, the record the head's sample mode publishes
//     -- the best rank (value desc, index asc) and the sum of exp(v - that value) in double,
//     NaN when a NaN was seen. Eight lanes hold one record's 64 entries, eight each.
constexpr int kPhThreads = 1024;
constexpr uint32_t kHashSlots = 8192;    // LDS hash table of one row's history
constexpr uint32_t kHashMaxIds = 4096;   // history ids per row the table takes (load <= 1/2)
constexpr uint32_t kHashEmpty = 0xFFFFFFFFu;  // never an id below vocab <= 2^30

struct PenaltyBufs {
    float* logits;
    uint64_t stride;
    uint32_t vocab;
    const uint32_t* history;
};

__global__ __launch_bounds__(kPhThreads) void penalty_hash_kernel(SelectArgs args_by_value, PenaltyBufs b) {
    constexpr int NT = kPhThreads;
    constexpr uint32_t kIdsPer = kHashMaxIds / NT;     // history ids per thread
    constexpr uint32_t kSlotsPer = kHashSlots / NT;    // table slots per thread
    __shared__ uint32_t keys[kHashSlots];
    __shared__ uint32_t cnt[kHashSlots];
#if __HIP_DEVICE_COMPILE__
    const SelectArgs& args =
        *reinterpret_cast<const SelectArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
#else
    const SelectArgs& args = args_by_value;
#endif
    const int tid = threadIdx.x;
    const uint32_t row = blockIdx.x;
    const twd_row_params p = args.p[row];
    if (p.repetition_penalty == 1.0f || p.history_len == 0) return;  // the whole block
    // every id requested at once (history_len <= kHashMaxIds, checked by the launch)
    const uint32_t* hist = b.history + p.history_offset;
    uint32_t ids[kIdsPer];
#pragma unroll
    for (uint32_t q = 0; q < kIdsPer; ++q) {
        const uint32_t j = tid + NT * q;
        const uint32_t id = hist[min(j, p.history_len - 1)];  // unconditional: no branch per load
        ids[q] = j < p.history_len ? id : kHashEmpty;
    }
#pragma unroll
    for (uint32_t q = 0; q < kSlotsPer; ++q) {
        keys[tid + NT * q] = kHashEmpty;
        cnt[tid + NT * q] = 0;
    }
    // each id's logit, requested now so that its round trip overlaps the table's construction
    // (only the thread that enters an id into the table uses it)
    float* lg = b.logits + static_cast<size_t>(row) * b.stride;
    float x[kIdsPer];
#pragma unroll
    for (uint32_t q = 0; q < kIdsPer; ++q) x[q] = lg[ids[q] < b.vocab ? ids[q] : 0u];  // no branch per load
    __syncthreads();
    uint32_t slot[kIdsPer];  // the slot this thread entered id q into, or kHashEmpty
#pragma unroll
    for (uint32_t q = 0; q < kIdsPer; ++q) {
        const uint32_t id = ids[q];
        slot[q] = kHashEmpty;
        if (id >= b.vocab) continue;  // out-of-range ids are ignored (sampling.cpp:82)
        // linear probing from a multiplicative hash; the table is at most half full, so a free
        // or matching slot is always found
        uint32_t h = (id * 0x9E3779B1u) >> (32 - 13);
        for (;;) {
            const uint32_t prev = atomicCAS(&keys[h], kHashEmpty, id);
            if (prev == kHashEmpty || prev == id) {
                atomicAdd(&cnt[h], 1u);
                if (prev == kHashEmpty) slot[q] = h;
                break;
            }
            h = (h + 1) & (kHashSlots - 1);
        }
    }
    __syncthreads();
    const float rp = p.repetition_penalty;
    const float limit = (p.softcap > 0.0f) ? p.softcap * 0.9999f : 0.0f;
    // each distinct id, by the thread that entered it: the penalty once per occurrence, the store
#pragma unroll
    for (uint32_t q = 0; q < kIdsPer; ++q) {
        if (slot[q] == kHashEmpty) continue;
        const uint32_t n = cnt[slot[q]];
        float v = x[q];
        for (uint32_t t = 0; t < n; ++t) {
            v = (v > 0.0f) ? (v / rp) : (v * rp);
            if (limit > 0.0f) v = (v < -limit) ? -limit : ((limit < v) ? limit : v);
        }
        lg[ids[q]] = v;
    }
}

// NB 8-entry batches per lane. One: many short blocks, so that later blocks' loads overlap
// earlier blocks' arithmetic (with four, every wave requested all its loads first, and the pass
// ran as a load phase, then an arithmetic phase).
template <uint32_t NB, bool AUX>
__global__ __launch_bounds__(kWsThreads) __attribute__((amdgpu_waves_per_eu(8)))
void wave_stats_kernel(WaveStatsBufs b) {
    __shared__ double tbl[64];
    wave_records_block<NB, AUX>(b, blockIdx.x, blockIdx.y, tbl);
}

// Rows up to which the record pass also forms the record words: its blocks are then few and
// short of work, and the words spare most merges their gather; past it the words cost the
// pass more than the merges save (64 rows: 25.0 against 20.9 us for the pass).
constexpr uint32_t kAuxMaxRows = 8;

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

// ---- the no-allocation selection: scratch in a device array of fixed size ------------------------
// The selection scratch of at most kStaticRows rows of at most kStaticVocab entries, carved the
// way scratch_alloc lays it out. Each GPU holds its own copy for the life of the process; every
// twd_select_noalloc call on a GPU shares it.
constexpr uint32_t kStaticRows = TWD_MAX_ROWS;
constexpr uint32_t kStaticVocab = 262144;
constexpr uint32_t kStaticParts = kStaticVocab / kSlice;  // 32
constexpr size_t kStaticSlots = static_cast<size_t>(kStaticRows) * kStaticParts;
constexpr size_t kStaticOffSum = 0;                                   // double [slots]
constexpr size_t kStaticOffKey = kStaticOffSum + 8 * kStaticSlots;    // uint64 [slots]
constexpr size_t kStaticOffMax = kStaticOffKey + 8 * kStaticSlots;    // float [slots]
constexpr size_t kStaticOffFlag = kStaticOffMax + 4 * kStaticSlots;   // uint32 [slots]
constexpr size_t kStaticOffCount = kStaticOffFlag + 4 * kStaticSlots; // uint32 [slots]
constexpr size_t kStaticOffCand = kStaticOffCount + 4 * kStaticSlots; // uint64 [slots][kMaxWant]
constexpr size_t kStaticOffGbest = kStaticOffCand + 8 * kStaticSlots * kMaxWant;  // uint64 [rows + kArriveWords]
constexpr size_t kStaticBytes = kStaticOffGbest + 8 * (kStaticRows + kArriveWords);  // 4,252,208 B
static_assert(kStaticBytes == 4252208, "the size twd_head.h states");
static_assert(kStaticOffCand % 256 == 0, "candidate array alignment");

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

namespace {

// The device address of `scratch` on each GPU (its own copy there), found once per device with
// that device current. Host code uses these addresses, never the array's name: on the host the
// name is a stand-in that no kernel may dereference.
constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
void* g_static_ptr[kMaxDevices] = {};
uint32_t g_static_epoch[kMaxDevices] = {};  // of each GPU's last one-pass greedy launch

int static_scratch(SelectScratch* out) {
    int dev = 0;
    TWD_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(TWD_E_UNSUPPORTED, "device index above 63");
    void* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_static_mu);
        if (!g_static_ptr[dev]) {
            void* p = nullptr;
            TWD_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
            if (!p) return fail(TWD_E_HIP, "hipGetSymbolAddress returned no address for the scratch array");
            g_static_ptr[dev] = p;
        }
        base = g_static_ptr[dev];
    }
    unsigned char* b = static_cast<unsigned char*>(base);
    SelectScratch s{};
    s.max_rows = kStaticRows;
    s.max_parts = kStaticParts;
    s.part_sum = reinterpret_cast<double*>(b + kStaticOffSum);
    s.part_key = reinterpret_cast<uint64_t*>(b + kStaticOffKey);
    s.part_max = reinterpret_cast<float*>(b + kStaticOffMax);
    s.part_flag = reinterpret_cast<uint32_t*>(b + kStaticOffFlag);
    s.part_count = reinterpret_cast<uint32_t*>(b + kStaticOffCount);
    s.cand = reinterpret_cast<uint64_t*>(b + kStaticOffCand);
    // zero at load: the first one-pass greedy launch on a GPU finds the counter unarmed and
    // counts in on the fallback word, then arms it for the next
    s.gbest = reinterpret_cast<uint64_t*>(b + kStaticOffGbest);
    s.gctr = s.gbest + kStaticRows;
    s.epoch = &g_static_epoch[dev];
    s.verify_tokens = nullptr;  // twd_select does not use it
    *out = s;
    return TWD_OK;
}

}  // namespace

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
    // the wave records of the wave-record path, ceil(max_vocab / 64) per row
    s->wave_cap = (max_vocab + kSampleWaveRows - 1) / kSampleWaveRows;
    const size_t nw = static_cast<size_t>(max_rows) * s->wave_cap;
    if (e == hipSuccess) e = hipMalloc(&s->wkey, nw * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc(&s->wsum, nw * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&s->wmax, nw * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&s->waux, nw * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&s->gbest, (max_rows + kArriveWords) * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(s->gbest, 0, (max_rows + kArriveWords) * sizeof(uint64_t));
    const uint64_t armed = kFirstEpoch;  // the counter starts armed for the first launch
    if (e == hipSuccess) e = hipMemcpy(s->gbest + max_rows, &armed, sizeof(armed), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        s->gctr = s->gbest + max_rows;
        s->epoch = new uint32_t(kFirstEpoch - 1);
        s->lng = new LongScratch();
    }
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
    (void)hipFree(s->wkey);
    (void)hipFree(s->wsum);
    (void)hipFree(s->wmax);
    (void)hipFree(s->waux);
    (void)hipFree(s->gbest);
    delete s->epoch;
    if (s->lng) {
        long_free(s->lng);
        delete s->lng;
    }
    *s = SelectScratch{};
}

void long_free(LongScratch* l) {
    (void)hipFree(l->keys);
    (void)hipFree(l->pre);
    (void)hipFree(l->len);
    (void)hipFree(l->gmax);
    (void)hipFree(l->total);
    *l = LongScratch{};
}

namespace {
int long_reserve(LongScratch* l, uint32_t rows, uint64_t npad) {
    if (l->keys && l->rows_cap >= rows && l->npad_cap >= npad) return TWD_OK;
    const uint32_t r = std::max(rows, l->rows_cap);
    const uint64_t n = std::max(npad, l->npad_cap);
    long_free(l);  // waits for the device (hipFree) before the old buffers go
    const size_t m = static_cast<size_t>(r) * n;
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = hipMalloc(&l->keys, m * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMalloc(&l->pre, m * sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&l->len, r * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&l->gmax, r * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&l->total, r * sizeof(double));
    if (e != hipSuccess) {
        long_free(l);
        return hip_fail(e, "allocating the long-shortlist scratch");
    }
    l->rows_cap = r;
    l->npad_cap = n;
    return TWD_OK;
}
}  // namespace

int launch_long(LongScratch* lng, const SampleStats& st, uint32_t waves, const float* logits, uint64_t stride,
                uint32_t vocab, uint32_t rows, const twd_row_params* params, uint32_t* tokens,
                hipStream_t stream) {
    LongArgs a{};
    for (uint32_t r = 0; r < rows; ++r) {
        if (!long_row(params[r], vocab)) continue;
        a.row[a.n] = r;
        a.p[a.n] = params[r];
        ++a.n;
    }
    if (a.n == 0) return TWD_OK;
    if (!lng) return fail(TWD_E_INVALID, "top_k > 256 needs a selector's scratch (twd_select)");
    if (waves == 0 || waves > kSampleMaxWaves) return fail(TWD_E_INVALID, "long shortlist: wave records out of range");
    uint64_t npad = 1;
    while (npad < vocab) npad <<= 1;
    int rc = long_reserve(lng, a.n, npad);
    if (rc) return rc;
    LongBufs b{};
    b.logits = logits;
    b.stride = stride;
    b.vocab = vocab;
    b.waves = waves;
    b.st = st;
    b.npad = npad;
    b.keys = lng->keys;
    b.pre = lng->pre;
    b.len = lng->len;
    b.gmax = lng->gmax;
    b.total = lng->total;
    b.tokens = tokens;
    long_gather_kernel<<<a.n, kLongThreads, sizeof(LongGatherShared), stream>>>(a, b);
    TWD_HIP(hipGetLastError());
    const uint32_t tile = static_cast<uint32_t>(std::min<uint64_t>(npad, kSortTile));
    const size_t tile_bytes = static_cast<size_t>(tile) * sizeof(uint64_t);
    const uint32_t ntile = static_cast<uint32_t>(npad / tile);
    long_sort_tile_kernel<<<dim3(ntile, a.n), kLongThreads, tile_bytes, stream>>>(b, tile);
    TWD_HIP(hipGetLastError());
    for (uint64_t k = 2ull * tile; k <= npad; k <<= 1) {
        for (uint64_t jj = k >> 1; jj >= tile; jj >>= 1) {
            long_sort_step_kernel<<<dim3(static_cast<uint32_t>(npad / 2 / kStepThreads), a.n), kStepThreads, 0,
                                    stream>>>(b, static_cast<uint32_t>(k), static_cast<uint32_t>(jj));
            TWD_HIP(hipGetLastError());
        }
        long_sort_merge_kernel<<<dim3(ntile, a.n), kLongThreads, tile_bytes, stream>>>(b, tile,
                                                                                       static_cast<uint32_t>(k));
        TWD_HIP(hipGetLastError());
    }
    long_finish_kernel<<<a.n, kLongThreads, 0, stream>>>(a, b);
    TWD_HIP(hipGetLastError());
    return TWD_OK;
}

// Lets the selection kernels use the LDS they need (no memory is allocated).
int enable_select_kernels() {
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        err = hipFuncSetAttribute(reinterpret_cast<const void*>(select_slice_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(sizeof(SliceShared)));
        if (err == hipSuccess)
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(select_merge_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(sizeof(MergeShared)));
        if (err == hipSuccess)
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(select_sample_merge_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(sizeof(SampleMergeShared)));
        if (err == hipSuccess)
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(long_gather_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(sizeof(LongGatherShared)));
        if (err == hipSuccess)
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(long_sort_tile_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kSortTile * sizeof(uint64_t)));
        if (err == hipSuccess)
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(long_sort_merge_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kSortTile * sizeof(uint64_t)));
    });
    if (err != hipSuccess) return hip_fail(err, "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    return TWD_OK;
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
    bool any_long = false;
    for (uint32_t r = 0; r < rows; ++r) {
        const twd_row_params& p = params[r];
        if (p.repetition_penalty != 1.0f && p.history_len > 0 && !history)
            return fail(TWD_E_INVALID, "null history with a non-empty history_len");
        a.p[r] = p;
        any_long |= !penalty_only && long_row(p, vocab);
    }
    const uint32_t waves = (vocab + kSampleWaveRows - 1) / kSampleWaveRows;
    const bool have_records = s.wkey != nullptr && waves <= s.wave_cap && waves <= kSampleMaxWaves;
    if (any_long && (!s.lng || !have_records))
        return fail(TWD_E_INVALID, "top_k > 256 needs a selector's scratch (twd_select, not twd_select_noalloc)");
    // sampled rows with short histories: the wave-record path (penalty pass, per-64-entry
    // statistics, then the one-block-per-row merge that reads only the candidate waves)
    bool records = !penalty_only && have_records;
    bool any_sampled = false, any_penalty = false;
    for (uint32_t r = 0; r < rows; ++r) {
        const twd_row_params& p = params[r];
        any_sampled |= !(p.temperature <= 0.0f);
        if (p.repetition_penalty != 1.0f && p.history_len > 0) {
            any_penalty = true;
            records &= p.history_len <= kHashMaxIds;
        }
    }
    if (records && any_sampled) {
        int rc = enable_select_kernels();
        if (rc) return rc;
        if (any_penalty) {
            PenaltyBufs pb{logits, stride, vocab, history};
            penalty_hash_kernel<<<rows, kPhThreads, 0, stream>>>(a, pb);
            TWD_HIP(hipGetLastError());
        }
        const bool aux = rows <= kAuxMaxRows;
        const SampleStats st{s.wkey, s.wsum, s.wmax, aux ? s.waux : nullptr, __builtin_nanf("")};  // no cap
        WaveStatsBufs wb{logits, stride, vocab, waves,
                         (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (stride & 3) == 0 ? 1u : 0u, st};
        const dim3 grid((vocab + kWsEntries - 1) / kWsEntries, rows);
        if (aux)
            wave_stats_kernel<1, true><<<grid, kWsThreads, 0, stream>>>(wb);
        else
            wave_stats_kernel<1, false><<<grid, kWsThreads, 0, stream>>>(wb);
        TWD_HIP(hipGetLastError());
        SampleMergeBufs mb{};
        mb.logits = logits;
        mb.stride = stride;
        mb.vocab = vocab;
        mb.waves = waves;
        mb.st = st;
        mb.tokens = tokens;
        select_sample_merge_kernel<<<rows, kSmThreads, sizeof(SampleMergeShared), stream>>>(a, mb);
        TWD_HIP(hipGetLastError());
        return launch_long(s.lng, st, waves, logits, stride, vocab, rows, params, tokens, stream);
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
    // every row greedy: the slice blocks finish the rows (one launch instead of two)
    if (!penalty_only && !any_sampled && parts > 1 && s.gbest && s.gctr && s.epoch) {
        *s.epoch = epoch_after(*s.epoch);  // 1 .. 2^31 - 1, never 0
        a.one_pass = 1;
        a.epoch = *s.epoch;
        a.next_epoch = epoch_after(*s.epoch);
        b.gbest = s.gbest;
        b.gctr = s.gctr;
    }
    select_slice_kernel<<<dim3(parts, rows), kSliceThreads, sizeof(SliceShared), stream>>>(a, b);
    TWD_HIP(hipGetLastError());
    if (parts > 1 && !penalty_only && !a.one_pass) {
        select_merge_kernel<<<rows, kMergeThreads, sizeof(MergeShared), stream>>>(a, b);
        TWD_HIP(hipGetLastError());
    }
    if (any_long) {  // their wave records from the penalised logits, then the long path
        const SampleStats st{s.wkey, s.wsum, s.wmax, nullptr, __builtin_nanf("")};  // no merge reads words
        WaveStatsBufs wb{logits, stride, vocab, waves,
                         (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (stride & 3) == 0 ? 1u : 0u, st};
        wave_stats_kernel<1, false><<<dim3((vocab + kWsEntries - 1) / kWsEntries, rows), kWsThreads, 0, stream>>>(wb);
        TWD_HIP(hipGetLastError());
        return launch_long(s.lng, st, waves, logits, stride, vocab, rows, params, tokens, stream);
    }
    return TWD_OK;
}

int launch_sample_merge(const SampleStats& st, uint32_t waves, const float* logits, uint32_t vocab,
                        uint32_t rows, const twd_row_params* params, uint32_t* tokens,
                        LongScratch* lng, hipStream_t stream) {
    if (waves == 0 || waves > kSampleMaxWaves) return fail(TWD_E_INVALID, "sample merge: head waves out of range");
    if (rows == 0 || rows > TWD_MAX_ROWS) return fail(TWD_E_INVALID, "sample merge: rows out of range");
    int rc = enable_select_kernels();
    if (rc) return rc;
    SelectArgs a{};
    a.rows = rows;
    a.parts = waves;
    for (uint32_t r = 0; r < rows; ++r) a.p[r] = params[r];
    SampleMergeBufs b{};
    b.logits = logits;
    b.stride = vocab;
    b.vocab = vocab;
    b.waves = waves;
    b.st = st;
    b.tokens = tokens;
    select_sample_merge_kernel<<<rows, kSmThreads, sizeof(SampleMergeShared), stream>>>(a, b);
    TWD_HIP(hipGetLastError());
    return launch_long(lng, st, waves, logits, vocab, vocab, rows, params, tokens, stream);
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
    if (parts_for(max_vocab) > kMaxParts) return fail(TWD_E_UNSUPPORTED, "max_vocab above 524288");
    int rc0 = enable_select_kernels();
    if (rc0) return rc0;
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
    order_release(s->order);
    draft_side_free(&s->draft);  // waits for the side stream's work
    scratch_free(&s->scratch);
    draft_scratch_free(&s->draft);
    delete s;
}

TWD_API int twd_select(twd_selector* sel, float* logits, uint32_t vocab, uint32_t rows,
                       uint64_t row_stride, const twd_row_params* params,
                       const uint32_t* history, uint32_t* tokens, void* stream) {
    clear_error();
    if (!sel) return fail(TWD_E_INVALID, "null selector");
    if (vocab > sel->max_vocab) return fail(TWD_E_INVALID, "vocab larger than this selector's max_vocab");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = order_before(sel->order, s);
    if (rc) return rc;
    rc = launch_select(sel->scratch, logits, vocab, rows, row_stride, params, history, tokens, s);
    const int rc2 = order_after(sel->order, s);
    return rc ? rc : rc2;
}

TWD_API int twd_select_noalloc(float* logits, uint32_t vocab, uint32_t rows, uint64_t row_stride,
                               const twd_row_params* params, const uint32_t* history,
                               uint32_t* tokens, void* stream) {
    clear_error();
    if (vocab > kStaticVocab)
        return fail(TWD_E_INVALID, "twd_select_noalloc: vocab above its fixed scratch's 262144 entries");
    if (rows > kStaticRows) return fail(TWD_E_INVALID, "twd_select_noalloc: rows above 64");
    int rc = enable_select_kernels();
    if (rc) return rc;
    SelectScratch s{};
    if ((rc = static_scratch(&s))) return rc;
    return launch_select(s, logits, vocab, rows, row_stride, params, history, tokens,
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
    int rc = order_before(sel->order, s);
    if (rc) return rc;
    rc = verify_launches(sel, logits, vocab, rows, row_stride, params, base_seed, drafts, n_drafts,
                         result, s);
    const int rc2 = order_after(sel->order, s);
    return rc ? rc : rc2;
}

}  // extern "C"

namespace twd {

int verify_launches(twd_selector* sel, const float* logits, uint32_t vocab, uint32_t rows,
                    uint64_t row_stride, const twd_row_params* params, uint64_t base_seed,
                    const uint32_t* drafts, uint32_t n_drafts, twd_verify_result* result,
                    hipStream_t s) {
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

}  // namespace twd
