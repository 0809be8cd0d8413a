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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint64_t o = shfl_xor_u64(v, m);
        v = o > v ? o : v;
    }
    return v;
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
    size_t e_capacity = 0;
    size_t part_capacity = 0;
};

int draft_scratch_reserve(DraftScratch* d, uint32_t vocab, uint32_t npos);
// Gives the head a device copy of the final RMSNorm weight (bf16 [d]), freed with the head.
int head_set_norm_weight(twd_head* h, const uint16_t* host_w, uint32_t d);
void draft_scratch_free(DraftScratch* d);

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
