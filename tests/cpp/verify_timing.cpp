// Times twd_verify_draft (evaluate_verification with draft logits, src/speculator.cpp:71-122)
// from C++, on the config-4 shape: 5 target rows and 4 draft rows of V = 262144 logits, T = 0.8,
// top_k = 40, top_p = 0.9. It reports the GPU time per verify (HIP events around N back-to-back
// calls), the GPU time of one verify alone, and the host time to issue one call (the same N
// calls, timed on the host clock without waiting), with no Python wrapper in between, for two
// sets of draft ids: the target rows' argmax at 6 positions in 10 (most positions accepted) and
// random ids (most positions rejected, each then summing its residual exactly). Prints one JSON
// line.
//
//   verify_timing [calls]
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "twd_head.h"

#define CHECK_HIP(x)                                                              \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));          \
            std::exit(1);                                                         \
        }                                                                         \
    } while (0)
#define CHECK_TWD(x)                                                              \
    do {                                                                          \
        if ((x) != TWD_OK) {                                                      \
            std::fprintf(stderr, "%s: %s\n", #x, twd_last_error());               \
            std::exit(1);                                                         \
        }                                                                         \
    } while (0)

int main(int argc, char** argv) {
    const int calls = argc > 1 ? std::atoi(argv[1]) : 200;
    const uint32_t V = 262144, rows = 5, nd = 4;
    std::mt19937 gen(20261202);
    std::normal_distribution<float> nd2(0.0f, 2.0f), nd15(0.0f, 1.5f);
    std::vector<float> target(static_cast<size_t>(rows) * V), draft(static_cast<size_t>(nd) * V);
    for (auto& x : target) x = nd2(gen);
    for (uint32_t i = 0; i < nd; ++i)
        for (uint32_t j = 0; j < V; ++j)
            draft[static_cast<size_t>(i) * V + j] = 0.8f * target[static_cast<size_t>(i) * V + j] + nd15(gen);
    float *d_target = nullptr, *d_draft = nullptr;
    uint32_t* d_drafts = nullptr;
    twd_verify_result* d_res = nullptr;
    CHECK_HIP(hipMalloc(&d_target, target.size() * sizeof(float)));
    CHECK_HIP(hipMalloc(&d_draft, draft.size() * sizeof(float)));
    CHECK_HIP(hipMalloc(&d_drafts, 64 * nd * sizeof(uint32_t)));
    CHECK_HIP(hipMalloc(&d_res, sizeof(twd_verify_result)));
    CHECK_HIP(hipMemcpy(d_target, target.data(), target.size() * sizeof(float), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_draft, draft.data(), draft.size() * sizeof(float), hipMemcpyHostToDevice));
    // 64 draft sets of each kind: [0, 64) the rows' argmax at 6 positions in 10, else random
    // (accepted often); [64, 128) random ids (rejected often)
    std::vector<uint32_t> drafts(128 * nd);
    for (uint32_t c = 0; c < 128; ++c)
        for (uint32_t i = 0; i < nd; ++i) {
            uint32_t best = 0;
            const float* r = target.data() + static_cast<size_t>(i) * V;
            for (uint32_t j = 1; j < V; ++j) best = r[j] > r[best] ? j : best;
            drafts[c * nd + i] = (c < 64 && gen() % 10 < 6) ? best : static_cast<uint32_t>(gen() % V);
        }
    CHECK_HIP(hipFree(d_drafts));
    CHECK_HIP(hipMalloc(&d_drafts, drafts.size() * sizeof(uint32_t)));
    CHECK_HIP(hipMemcpy(d_drafts, drafts.data(), drafts.size() * sizeof(uint32_t), hipMemcpyHostToDevice));

    twd_selector* sel = nullptr;
    CHECK_TWD(twd_selector_create(V, rows, &sel));
    hipStream_t s;
    CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    const float* rows_ptr[nd];
    for (uint32_t i = 0; i < nd; ++i) rows_ptr[i] = d_draft + static_cast<size_t>(i) * V;
    twd_row_params p{0.8f, 0.9f, 40, 1.0f, 0.0f, 30.0f, 0, 0};
    hipEvent_t e0, e1;
    CHECK_HIP(hipEventCreate(&e0));
    CHECK_HIP(hipEventCreate(&e1));
    std::printf("{\"calls\": %d", calls);
    for (int set = 0; set < 2; ++set) {
        uint32_t accepted = 0;
        auto call = [&](int i) {
            CHECK_TWD(twd_verify_draft(sel, d_target, V, rows, V, rows_ptr, nd, &p, 1000u + static_cast<uint64_t>(i),
                                       d_drafts + (64 * set + i % 64) * nd, nd, d_res, s));
        };
        for (int i = 0; i < 64; ++i) {  // warm-up, and the mean accepted count of the 64 sets
            call(i);
            twd_verify_result r{};
            CHECK_HIP(hipMemcpyAsync(&r, d_res, sizeof(r), hipMemcpyDeviceToHost, s));
            CHECK_HIP(hipStreamSynchronize(s));
            accepted += r.num_accepted;
        }
        CHECK_HIP(hipEventRecord(e0, s));
        const auto h0 = std::chrono::steady_clock::now();
        for (int i = 0; i < calls; ++i) call(i);
        const auto h1 = std::chrono::steady_clock::now();
        CHECK_HIP(hipEventRecord(e1, s));
        CHECK_HIP(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));
        const double host_us = std::chrono::duration<double, std::micro>(h1 - h0).count() / calls;
        // each call spaced by a host wait: the GPU time of one verify alone
        double alone = 0.0;
        const int spaced = 50;
        for (int i = 0; i < spaced; ++i) {
            CHECK_HIP(hipEventRecord(e0, s));
            call(i);
            CHECK_HIP(hipEventRecord(e1, s));
            CHECK_HIP(hipEventSynchronize(e1));
            float m = 0.0f;
            CHECK_HIP(hipEventElapsedTime(&m, e0, e1));
            alone += m * 1e3 / spaced;
        }
        std::printf(", \"%s\": {\"mean_accepted\": %.3f, \"gpu_us_per_verify_back_to_back\": %.2f, "
                    "\"host_issue_us_per_call\": %.2f, \"gpu_us_per_verify_alone\": %.2f}",
                    set == 0 ? "argmax_drafts" : "random_drafts", accepted / 64.0, ms * 1e3 / calls, host_us, alone);
    }
    std::printf("}\n");
    twd_selector_destroy(sel);
    CHECK_HIP(hipStreamDestroy(s));
    return 0;
}
