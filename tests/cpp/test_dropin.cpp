// Drives the drop-in C++ API (include/g4dense/sampling.hpp, speculator.hpp) through
// libtwd_head.so on the GPU, with the assertions of the reference's own tests:
// tests/test_sampling.cpp:92-265 and tests/test_speculative.cpp:29-77.
// Prints one line per block and exits nonzero on the first failure.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <thread>
#include <vector>

#include "g4dense/sampling.hpp"
#include "g4dense/speculator.hpp"

using namespace g4dense;

#define CHECK(cond)                                                          \
    do {                                                                     \
        if (!(cond)) {                                                       \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                    \
        }                                                                    \
    } while (0)

// sample_token restated with a full sort of the row (the shortlist is its first want entries),
// sequential double sums and the host's exp: the expectation for top_k above 256.
static uint32_t full_sort_sample(const std::vector<float>& lg, const SamplingParams& p, uint64_t seed) {
    const uint32_t V = static_cast<uint32_t>(lg.size());
    std::vector<uint32_t> order(V);
    for (uint32_t i = 0; i < V; ++i) order[i] = i;
    std::sort(order.begin(), order.end(),
              [&](uint32_t a, uint32_t b) { return lg[a] != lg[b] ? lg[a] > lg[b] : a < b; });
    float mx = lg[0];
    for (float x : lg) mx = x > mx ? x : mx;
    double total = 0.0;
    for (float x : lg) total += std::exp(static_cast<double>(x) - mx);
    const size_t want = p.top_k > 0 ? std::min<size_t>(static_cast<size_t>(p.top_k), V) : std::min<size_t>(256, V);
    size_t cut = want;
    if (p.top_p < 1.0f) {
        double run = 0.0;
        for (size_t i = 0; i < want; ++i) {
            run += std::exp(static_cast<double>(lg[order[i]]) - mx) / total;
            if (run >= static_cast<double>(p.top_p)) {
                cut = i + 1;
                break;
            }
        }
    }
    if (p.top_k > 0) cut = std::min(cut, static_cast<size_t>(p.top_k));
    cut = std::max<size_t>(cut, 1);
    std::vector<double> q(cut);
    double denom = 0.0;
    for (size_t i = 0; i < cut; ++i) {
        q[i] = std::exp((static_cast<double>(lg[order[i]]) - mx) / p.temperature);
        denom += q[i];
    }
    uint64_t s = seed;  // one xorshift64* step, the top 24 bits as a fraction of 2^24
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    const float u = static_cast<float>(((s * 0x2545F4914F6CDD1DULL) >> 40) & 0xFFFFFFu) / 16777216.0f;
    const double r = static_cast<double>(u) * denom;
    double acc = 0.0;
    for (size_t i = 0; i < cut; ++i) {
        acc += q[i];
        if (acc >= r) return order[i];
    }
    return order[cut - 1];
}

static bool rejects(const SamplingParams& p) {
    try {
        validate_sampling(p);
        return false;
    } catch (const G4DenseFormatError&) {
        return true;
    }
}

int main() {
    // validation matrix
    CHECK(!rejects(SamplingParams{0.2f, 0.95f, 64, 1.0f, false, 0}));
    CHECK(!rejects(SamplingParams{0.0f, 1.0f, 0, 1.0f, false, 0}));
    CHECK(rejects(SamplingParams{-0.1f, 1.0f, 0, 1.0f, false, 0}));
    CHECK(rejects(SamplingParams{0.2f, 0.0f, 64, 1.0f, false, 0}));
    CHECK(rejects(SamplingParams{0.2f, 1.5f, 64, 1.0f, false, 0}));
    CHECK(rejects(SamplingParams{0.2f, 0.95f, 257, 1.0f, false, 0}));
    CHECK(rejects(SamplingParams{0.2f, 0.95f, -1, 1.0f, false, 0}));
    CHECK(rejects(SamplingParams{0.2f, 0.95f, 64, 0.0f, false, 0}));
    CHECK(rejects(SamplingParams{0.7f, 0.9f, 0, 1.0f, false, 0}));
    CHECK(!rejects(SamplingParams{0.7f, 1.0f, 0, 1.0f, false, 0}));
    CHECK(!rejects(SamplingParams{0.0f, 0.9f, 0, 1.0f, false, 0}));
    std::puts("validation ok");

    CHECK(splitmix64(0) == 0xE220A8397B1DCDAFULL);
    CHECK(splitmix64(3) == 0x1D0B14E4DB018FEDULL);
    SamplingParams seeded{0.7f, 1.0f, 0, 1.0f, true, 12345};
    for (int pos = 0; pos < 1000; ++pos) CHECK(seed_for(seeded, pos) != 0);
    std::puts("seeding ok");

    {
        std::vector<float> lg{1.0f, 5.0f, 3.0f, 5.0f, 2.0f};
        SamplingParams greedy{0.0f, 1.0f, 0, 1.0f, false, 0};
        CHECK(sample_token(lg.data(), 5, greedy, 1) == 1);
        std::vector<float> one{7.0f};
        CHECK(sample_token(one.data(), 1, greedy, 1) == 0);
    }
    std::puts("greedy ok");

    {
        std::vector<float> lg{3.0f, 2.5f, 2.0f, 1.5f, -1.0f, -2.0f, -3.0f, -4.0f};
        SamplingParams p{1.0f, 0.9f, 2, 1.0f, true, 7};
        std::set<uint32_t> seen;
        for (int i = 0; i < 300; ++i) seen.insert(sample_token(lg.data(), 8, p, seed_for(p, i)));
        CHECK(seen.size() == 2 && seen.count(0) && seen.count(1));
    }
    std::puts("truncation order ok");

    {
        std::vector<float> lg{10.0f, -10.0f, 0.0f, 29.999f};
        std::vector<uint32_t> hist{0, 1, 3, 99999};
        auto v = lg;
        apply_repetition_penalty(v.data(), 4, hist, 2.0f, 30.0f);
        CHECK(std::fabs(v[0] - 5.0f) < 1e-5f && std::fabs(v[1] + 20.0f) < 1e-5f && v[2] == 0.0f);
        CHECK(v[3] < 15.1f && v[3] > 14.9f);
        auto w = lg;
        apply_repetition_penalty(w.data(), 4, hist, 1.0f, 30.0f);
        CHECK(w == lg);
        std::vector<float> g{9.0f, 8.0f};
        SamplingParams greedy{0.0f, 1.0f, 0, 1.0f, false, 0};
        apply_repetition_penalty(g.data(), 2, {0}, 2.0f, 30.0f);
        CHECK(sample_token(g.data(), 2, greedy, 1) == 1);
    }
    std::puts("penalty ok");

    {
        std::vector<float> bad(16, -INFINITY);
        SamplingParams p{0.7f, 1.0f, 0, 1.0f, false, 0};
        bool threw = false;
        try {
            sample_token(bad.data(), 16, p, 1);
        } catch (const G4DenseFormatError&) {
            threw = true;
        }
        CHECK(threw);
    }
    std::puts("degenerate ok");

    {
        std::mt19937 rng(4242);
        std::normal_distribution<float> nd(0.0f, 4.0f);
        std::vector<float> lg(4096);
        for (auto& x : lg) x = nd(rng);
        SamplingParams p{0.8f, 0.95f, 64, 1.0f, true, 20260721};
        std::vector<uint32_t> a, b;
        for (int i = 0; i < 32; ++i) a.push_back(sample_token(lg.data(), 4096, p, seed_for(p, i)));
        for (int i = 0; i < 32; ++i) b.push_back(sample_token(lg.data(), 4096, p, seed_for(p, i)));
        CHECK(a == b);
    }
    std::puts("determinism ok");

    // top_k above 256: sample_token takes any top_k (want = min(top_k, V), sampling.cpp:122-124);
    // only validate_sampling bounds it. Ids at V = 262144 against the full-sort restatement.
    {
        const uint32_t V = 262144;
        std::mt19937 rng(20261202);
        std::normal_distribution<float> nd(0.0f, 4.0f);
        std::vector<float> lg(V);
        for (auto& x : lg) x = nd(rng);
        const SamplingParams cases[] = {{0.8f, 0.95f, 1000, 1.0f, true, 11},
                                        {1.2f, 1.0f, 1000, 1.0f, true, 12},
                                        {0.7f, 0.99f, 4096, 1.0f, true, 13},
                                        {1.0f, 1.0f, 300000, 1.0f, true, 14}};
        for (const auto& p : cases) {
            CHECK(rejects(p));
            for (int i = 0; i < 4; ++i) {
                const uint64_t seed = seed_for(p, i);
                CHECK(sample_token(lg.data(), V, p, seed) == full_sort_sample(lg, p, seed));
            }
        }
    }
    std::puts("top_k above 256 ok");

    {
        SpeculativeCoordinator spec;
        const uint32_t V = 1024;
        SamplingParams greedy;
        std::vector<std::vector<float>> rows(5, std::vector<float>(V, 0.0f));
        rows[0][42] = rows[1][100] = rows[2][200] = rows[3][300] = rows[4][400] = 10.0f;
        std::vector<const float*> ptrs;
        for (auto& r : rows) ptrs.push_back(r.data());
        auto e1 = spec.evaluate_verification({42, 100, 200, 300}, ptrs, V, greedy, 12345);
        CHECK(e1.num_accepted == 4 && e1.bonus_token_sampled && e1.bonus_token == 400);
        CHECK((e1.accepted_tokens == std::vector<uint32_t>{42, 100, 200, 300, 400}));
        auto e2 = spec.evaluate_verification({42, 100, 999, 300}, ptrs, V, greedy, 12345);
        CHECK(e2.num_accepted == 2 && e2.bonus_token == 200);
        CHECK((e2.accepted_tokens == std::vector<uint32_t>{42, 100, 200}));
        auto e3 = spec.evaluate_verification({999, 100}, ptrs, V, greedy, 12345);
        CHECK(e3.num_accepted == 0 && e3.accepted_tokens.size() == 1 && e3.accepted_tokens[0] == 42);
        CHECK(spec.total_draft_tokens() == 10 && spec.total_accepted_tokens() == 6);
    }
    std::puts("speculative verify ok");

    {
        // draft logits (speculator.cpp:71-122). Identical draft and target rows: p == q, so
        // r == 1 and every position is accepted; the bonus is sample_token of the last row.
        SpeculativeCoordinator spec;
        const uint32_t V = 1024;
        std::mt19937 rng(99);
        std::normal_distribution<float> nd(0.0f, 3.0f);
        std::vector<std::vector<float>> rows(4, std::vector<float>(V));
        for (auto& r : rows)
            for (auto& x : r) x = nd(rng);
        std::vector<const float*> ptrs;
        for (auto& r : rows) ptrs.push_back(r.data());
        SamplingParams sp{0.9f, 1.0f, 0, 1.0f, false, 0};
        std::vector<std::vector<float>> drafts_l(rows.begin(), rows.begin() + 3);
        auto e = spec.evaluate_verification({5, 6, 7}, ptrs, V, sp, 321, drafts_l);
        CHECK(e.num_accepted == 3 && e.bonus_token_sampled);
        CHECK(e.bonus_token == sample_token(ptrs[3], V, sp, splitmix64(321 + 3)));

        // Flat target logits (p = 1/1024 everywhere) against a draft row of zeros with one NaN:
        // the draft's softmax sum is NaN, so q stays unnormalised (q = 1), r = 2^-10, and a
        // rejection finds (p - q)+ summing to 0: the fallback sample_token of the target row.
        std::vector<float> flat(V, 0.0f);
        std::vector<std::vector<float>> nan_row(1, std::vector<float>(V, 0.0f));
        nan_row[0][500] = std::nanf("");
        std::vector<const float*> one{flat.data()};
        const uint64_t base = 777;
        std::mt19937_64 g(splitmix64(base));
        std::uniform_real_distribution<float> ud(0.0f, 1.0f);
        const float u1 = ud(g);
        auto f = spec.evaluate_verification({9}, one, V, sp, base, nan_row);
        if (u1 <= 1.0f / 1024.0f) {
            CHECK(f.num_accepted == 1 && f.accepted_tokens[0] == 9);
        } else {
            CHECK(f.num_accepted == 0 && f.accepted_tokens.size() == 1);
            CHECK(f.accepted_tokens[0] == sample_token(flat.data(), V, sp, splitmix64(base)));
        }
    }
    std::puts("draft-logits verify ok");

    // evaluate_verification has no bound on the number of drafts (speculator.cpp:50): 100
    // drafts against 101 rows, greedy and sampled, each row's expected id from sample_token
    // with the step seed splitmix64(base + i) (:56)
    {
        const uint32_t V = 1536, K = 100;
        std::mt19937 gen(4242);
        std::normal_distribution<float> nd(0.0f, 2.0f);
        std::vector<std::vector<float>> rows(K + 1, std::vector<float>(V));
        for (auto& r : rows)
            for (auto& x : r) x = nd(gen);
        std::vector<const float*> ptrs;
        for (auto& r : rows) ptrs.push_back(r.data());
        const uint64_t base = 31337;
        for (int sampled = 0; sampled < 2; ++sampled) {
            SamplingParams sp = sampled ? SamplingParams{0.8f, 0.9f, 40, 1.0f, false, 0}
                                        : SamplingParams{};
            std::vector<uint32_t> want;
            for (uint32_t i = 0; i <= K; ++i) want.push_back(sample_token(ptrs[i], V, sp, splitmix64(base + i)));
            // all accepted: 100 drafts, then the bonus row's id
            std::vector<uint32_t> drafts(want.begin(), want.begin() + K);
            SpeculativeCoordinator spec;
            auto all = spec.evaluate_verification(drafts, ptrs, V, sp, base);
            CHECK(all.num_accepted == K && all.bonus_token_sampled && all.bonus_token == want[K]);
            CHECK(all.accepted_tokens.size() == K + 1 && all.accepted_tokens == want);
            CHECK(all.total_drafted == K);
            // a mismatch at position 77, in the second batch of 64: 77 accepted + the correction
            drafts[77] = (drafts[77] + 1) % V;
            auto miss = spec.evaluate_verification(drafts, ptrs, V, sp, base);
            CHECK(miss.num_accepted == 77 && miss.bonus_token_sampled && miss.bonus_token == want[77]);
            CHECK(miss.accepted_tokens.size() == 78 && miss.accepted_tokens[77] == want[77]);
            CHECK(spec.total_draft_tokens() == 2 * K && spec.total_accepted_tokens() == K + 77);
        }
    }
    std::puts("100-draft verify ok");

    // calls from several threads at once (each leases its own staging area and stream) give
    // the ids of the same calls made one after another
    {
        const uint32_t V = 50000;
        std::mt19937 gen(777);
        std::normal_distribution<float> nd(0.0f, 3.0f);
        constexpr int kThreads = 6, kCalls = 20;
        std::vector<std::vector<float>> rows(kThreads * kCalls, std::vector<float>(V));
        for (auto& r : rows)
            for (auto& x : r) x = nd(gen);
        const SamplingParams sp{0.8f, 0.95f, 64, 1.0f, false, 0};
        std::vector<uint32_t> want(rows.size()), got(rows.size());
        for (size_t i = 0; i < rows.size(); ++i) want[i] = sample_token(rows[i].data(), V, sp, splitmix64(i));
        std::vector<std::thread> th;
        for (int t = 0; t < kThreads; ++t)
            th.emplace_back([&, t] {
                for (int c = 0; c < kCalls; ++c) {
                    const size_t i = static_cast<size_t>(t) * kCalls + c;
                    got[i] = sample_token(rows[i].data(), V, sp, splitmix64(i));
                }
            });
        for (auto& x : th) x.join();
        CHECK(got == want);
    }
    std::puts("concurrent callers ok");
    std::puts("ALL OK");
    return 0;
}
