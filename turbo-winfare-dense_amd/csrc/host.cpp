// Host side of the C-ABI: thread-local errors (the convention of src/c_api.cpp:82-93) and the
// reference's seeding and validation, which are parameter logic rather than per-token compute
// (src/sampling.cpp:15-72).
#include <hip/hip_runtime.h>

#include <cmath>
#include <random>
#include <string>

#include "twd_internal.h"

namespace twd {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return TWD_E_HIP;
}

// Under stream capture nothing runs: the calls become graph nodes, replayed later in an order
// only the caller knows, so the caller orders the replays against the object's other calls. A
// captured call waits for nothing (a device-wide wait, or a wait on an event recorded outside
// the capture, would invalidate the capture), records nothing, and leaves the object's stream
// where it was.
int order_before(StreamOrder& o, hipStream_t s) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    TWD_HIP(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone) return TWD_OK;
    if (!o.used) {
        o.used = true;
        o.last = s;
        return TWD_OK;
    }
    if (s == o.last) return TWD_OK;
    if (!o.multi) {
        // the first change of stream: nothing recorded the old stream's last call, so wait for
        // the device once, then track every call with the event
        TWD_HIP(hipDeviceSynchronize());
        TWD_HIP(hipEventCreateWithFlags(&o.ev, hipEventDisableTiming));
        o.multi = true;
    } else {
        TWD_HIP(hipStreamWaitEvent(s, o.ev, 0));
    }
    o.last = s;
    return TWD_OK;
}

int order_after(StreamOrder& o, hipStream_t s) {
    if (!o.multi) return TWD_OK;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    TWD_HIP(hipStreamIsCapturing(s, &cap));
    if (cap == hipStreamCaptureStatusNone) TWD_HIP(hipEventRecord(o.ev, s));
    return TWD_OK;
}

void order_release(StreamOrder& o) {
    if (o.ev) (void)hipEventDestroy(o.ev);
    o = StreamOrder{};
}

}  // namespace twd

using namespace twd;

extern "C" {

TWD_API const char* twd_last_error(void) { return g_last_error.c_str(); }

TWD_API uint64_t twd_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

TWD_API uint64_t twd_seed_for(int has_seed, uint64_t seed, int position) {
    const uint64_t pos = static_cast<uint64_t>(static_cast<int64_t>(position));
    const uint64_t base = has_seed ? seed + pos
                                   : (0x9E3779B97F4A7C15ULL ^ (pos * 0xD1B54A32D192ED03ULL));
    const uint64_t s = twd_splitmix64(base);
    return s ? s : 0x9E3779B97F4A7C15ULL;  // a zero xorshift state would stay zero
}

TWD_API float twd_uniform_from_seed(uint64_t seed) {
    uint64_t s = seed;  // one xorshift64* step, top 24 bits as an exact fraction of 2^24
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    const uint64_t r = s * 0x2545F4914F6CDD1DULL;
    return static_cast<float>((r >> 40) & 0xFFFFFFu) / 16777216.0f;
}

TWD_API void twd_rejection_uniforms(uint64_t step_seed, float* u1, float* u2) {
    std::mt19937_64 rng(step_seed);
    std::uniform_real_distribution<float> udist(0.0f, 1.0f);
    const float a = udist(rng);  // ratio test
    const float b = udist(rng);  // residual draw
    if (u1) *u1 = a;
    if (u2) *u2 = b;
}

TWD_API int twd_validate_sampling(float t, float p, int32_t k, float rp) {
    clear_error();
    if (!std::isfinite(t) || t < 0.0f)
        return fail(TWD_E_INVALID, "temperature must be finite and >= 0 (0 = greedy)");
    if (!std::isfinite(p) || p <= 0.0f || p > 1.0f) return fail(TWD_E_INVALID, "top_p must be in (0, 1]");
    if (k < 0 || k > static_cast<int32_t>(TWD_MAX_WANT))
        return fail(TWD_E_INVALID, "top_k must be in 0..256 (0 disables it)");
    if (!std::isfinite(rp) || rp <= 0.0f)
        return fail(TWD_E_INVALID, "repetition_penalty must be finite and > 0 (1 = disabled)");
    if (t > 0.0f && p < 1.0f && k == 0)
        return fail(TWD_E_INVALID,
                    "top_p < 1 with temperature > 0 requires top_k in 1..256; full-vocabulary "
                    "nucleus sampling is not implemented");
    return TWD_OK;
}

}  // extern "C"
