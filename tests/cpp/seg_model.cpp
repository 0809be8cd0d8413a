// A CPU model of the draft verify's exact sequential-sum engine (turbo-winfare-dense_amd/csrc/
// verify.hip: seg_xfer_kernel with its crossing data, seg_chain with seg_crossing, wave_seg_sum,
// seg_residual_block's search), over a
// simulated 64-lane wave, statement for statement with the device code. The engine reproduces
// `float s = 0; for (j = 0; j < n; ++j) s += t[j];` bit for bit (the sums of compute_softmax and
// of the residual draw, src/speculator.cpp:22-26,104-116); this program checks it against that
// loop and asserts what the device code relies on:
//   * every LDS index: the record array (kSegMax), the segment starts (kSegMax + 1), the head's
//     staging (kSegHead), each lane's terms inside its segment;
//   * every value the device code treats as wave- or block-uniform (the sum S and its binade,
//     the walk's first failing lane and position, a pass's tie-free choice, the owner lane of an
//     event and the event) is computed in every simulated lane and compared across lanes;
//   * every loop ends: the walk advances by at least one segment per outer step, a pass of
//     wave_seg_sum adds at least one term, and no segment takes more than kSegLen + 1 passes.
// Cross-lane operations are modelled by their definitions: the device's DPP scans compute
// inclusive scans under saturating addition or composition of transfer functions, which are
// associative, so any grouping of the lanes (here: in lane order) gives the same result.
//
//   seg_model [rows] [seed]     prints one line per row kind and "MODEL OK" at the end
#include <array>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr uint32_t kSegHead = 2048;
constexpr uint32_t kSegLen = 512;
constexpr int kSegPer = kSegLen / 64;
constexpr uint32_t kSegMax = (1u << 19) / kSegLen;
constexpr uint32_t kSat = 1u << 30;
constexpr uint32_t kL = 1u << 24;
constexpr uint32_t kNoEvent = 0xFFFFFFFFu;
constexpr int W = 64;

#define MODEL_ASSERT(c, what)                                                                      \
    do {                                                                                           \
        if (!(c)) throw std::runtime_error(std::string("model assertion failed: ") + (what) + " (" #c ")"); \
    } while (0)

template <typename T>
using Lanes = std::array<T, W>;

template <typename T>
void uniform(const Lanes<T>& v, const char* what) {
    for (int l = 1; l < W; ++l) MODEL_ASSERT(std::memcmp(&v[l], &v[0], sizeof(T)) == 0, what);
}

uint32_t f2u(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

uint32_t seg_count(uint32_t n) { return n > kSegHead ? (n - kSegHead + kSegLen - 1) / kSegLen : 0u; }

struct Xfer {
    uint32_t inc0, inc1, out;
};
uint32_t sat_add(uint32_t a, uint32_t b) { return std::min(a + b, kSat); }
Xfer xfer_id() { return Xfer{0u, 0u, 2u}; }
Xfer xfer_then(const Xfer& f, const Xfer& g) {
    const uint32_t f0 = f.out & 1u, f1 = (f.out >> 1) & 1u;
    Xfer h;
    h.inc0 = sat_add(f.inc0, f0 ? g.inc1 : g.inc0);
    h.inc1 = sat_add(f.inc1, f1 ? g.inc1 : g.inc0);
    h.out = ((g.out >> f0) & 1u) | (((g.out >> f1) & 1u) << 1);
    return h;
}

void split_term(float a, int E, uint32_t& k, uint32_t& kind) {
    const uint32_t b = f2u(a);
    const uint32_t f = b >> 23;
    const uint32_t m = (b & 0x7FFFFFu) | (f ? 0x800000u : 0u);
    const int sh = E - (std::max(static_cast<int>(f), 1) - 127);
    const int shc = std::min(std::max(sh, 1), 31);
    const uint32_t rem = m & ((1u << shc) - 1u), half = 1u << (shc - 1);
    const uint32_t kr = rem > half ? 1u : (rem == half ? 2u : 0u);
    k = sh > 0 ? (m >> shc) : (sh == 0 ? m : kSat);
    kind = sh > 0 ? kr : 0u;
}
Xfer term_xfer(uint32_t k, uint32_t kind) {
    const uint32_t c = k + (kind & 1u), cp = c & 1u, kp = k & 1u;
    const bool tie = kind == 2u;
    return Xfer{tie ? k + kp : c, tie ? k + (kp ^ 1u) : c, tie ? 0u : (cp | ((cp ^ 1u) << 1))};
}
uint32_t term_inc(uint32_t k, uint32_t kind, uint32_t par) { return k + (kind == 2u ? ((par + k) & 1u) : kind); }

// the wave operations
Lanes<uint32_t> inc_scan(const Lanes<uint32_t>& v) {
    Lanes<uint32_t> o;
    uint32_t run = 0;
    for (int l = 0; l < W; ++l) o[l] = run = sat_add(run, v[l]);
    return o;
}
Lanes<Xfer> xfer_scan(const Lanes<Xfer>& v) {
    Lanes<Xfer> o;
    Xfer run = xfer_id();
    for (int l = 0; l < W; ++l) o[l] = run = xfer_then(run, v[l]);
    return o;
}
template <typename T>
Lanes<T> shfl_up1(const Lanes<T>& v, T fill) {
    Lanes<T> o;
    o[0] = fill;
    for (int l = 1; l < W; ++l) o[l] = v[l - 1];
    return o;
}
uint64_t ballot(const Lanes<bool>& p) {
    uint64_t m = 0;
    for (int l = 0; l < W; ++l) m |= static_cast<uint64_t>(p[l]) << l;
    return m;
}
int ffs64(uint64_t m) { return m ? __builtin_ctzll(m) : -1; }

int binade(float S, uint32_t& B) {
    const uint32_t sb = f2u(S), sf = sb >> 23;
    B = sf ? ((sb & 0x7FFFFFu) | 0x800000u) : sb;
    return sf ? static_cast<int>(sf) - 127 : -126;
}
uint32_t thr_units(float thr, int E) {
    const double t = std::ceil(std::ldexp(static_cast<double>(thr), 23 - E));
    return t <= 0.0 ? 0u : (t >= 4294967295.0 ? 0xFFFFFFFFu : static_cast<uint32_t>(t));
}

struct SegRec {
    int E[2];
    Xfer f[2];
    // crossing data (seg_xfer_kernel writes it where the double sums predict a binade change in
    // the segment): bit 0 present, bit 1 + c: candidate c's terms hold no exact half-way case;
    // lane_inc[c][l] the increments of lanes 0..l in candidate c's units (inclusive, saturating)
    uint32_t xl = 0;
    uint32_t lane_inc[2][W] = {};
};

struct Stats {
    long exact_segments = 0, passes = 0, tie_passes = 0, walk_steps = 0, mispredicted = 0;
    long crossings = 0, crossings_finished = 0;
};

// seg_xfer_kernel, wave w's segment s: the double prefix D predicts the binade of the running
// sum at the segment start; the segment's transfer functions for that binade and its nearer
// neighbour, composed in order
SegRec make_record(const std::vector<float>& t, uint32_t n, uint32_t s, double D, double Dend) {
    int ex = 0;
    const double m = std::frexp(D, &ex);
    const bool low = D < 0x1p-125;
    const int E0 = low ? -126 : ex - 1;
    const int E1 = low ? -125 : std::max(-126, m < 0.75 ? ex - 2 : ex);
    Lanes<Xfer> f0, f1;
    Lanes<bool> tie0, tie1;
    for (int lane = 0; lane < W; ++lane) {
        const uint32_t j0 = kSegHead + s * kSegLen + static_cast<uint32_t>(lane) * kSegPer;
        Xfer a0 = xfer_id(), a1 = xfer_id();
        tie0[lane] = tie1[lane] = false;
        for (int q = 0; q < kSegPer; ++q) {
            const float a = j0 + q < n ? t[j0 + q] : 0.0f;
            uint32_t kk, kd;
            split_term(a, E0, kk, kd);
            a0 = xfer_then(a0, term_xfer(kk, kd));
            tie0[lane] = tie0[lane] || kd == 2u;
            split_term(a, E1, kk, kd);
            a1 = xfer_then(a1, term_xfer(kk, kd));
            tie1[lane] = tie1[lane] || kd == 2u;
        }
        f0[lane] = a0;
        f1[lane] = a1;
    }
    const Lanes<Xfer> s0 = xfer_scan(f0), s1 = xfer_scan(f1);
    SegRec r;
    r.E[0] = E0;
    r.E[1] = E1;
    r.f[0] = s0[W - 1];  // lane 63's inclusive scan
    r.f[1] = s1[W - 1];
    // a predicted crossing: the double sums before and after the segment, widened by 2^-10,
    // lie in different binades
    int e_lo = 0, e_hi = 0;
    (void)std::frexp(D * (1.0 - 0x1p-10), &e_lo);
    (void)std::frexp(Dend * (1.0 + 0x1p-10), &e_hi);
    if (e_lo != e_hi) {
        r.xl = 1u | (ballot(tie0) == 0 ? 2u : 0u) | (ballot(tie1) == 0 ? 4u : 0u);
        for (int lane = 0; lane < W; ++lane) {
            r.lane_inc[0][lane] = s0[lane].inc0;
            r.lane_inc[1][lane] = s1[lane].inc0;
        }
    }
    return r;
}

// wave_seg_sum: terms [k0, k1) from prefix S, one wave, lane l holding k0 + kSegPer l ..
float wave_seg_sum(const std::vector<float>& t, uint32_t n, uint32_t k0, uint32_t k1, float S, float thr,
                   bool want_stop, uint32_t* stop_at, Stats& st) {
    MODEL_ASSERT(k1 > k0 && k1 - k0 <= kSegLen && k0 % kSegPer == 0, "segment bounds");
    ++st.exact_segments;
    Lanes<std::array<float, kSegPer>> a;
    for (int lane = 0; lane < W; ++lane) {
        const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
        for (int q = 0; q < kSegPer; ++q) {
            // the device loads j0 .. j0 + kSegPer - 1 from a row padded to 16 floats
            const uint32_t j = j0 + q;
            a[lane][q] = (j < n && j < k1) ? t[j] : 0.0f;
        }
    }
    uint32_t kc = k0;
    uint32_t stop = k1;
    Lanes<float> S_l;  // every lane's copy of S: the device keeps S in a per-lane register
    S_l.fill(S);
    for (uint32_t pass = 0;; ++pass) {
        MODEL_ASSERT(pass <= kSegLen, "a segment takes at most kSegLen + 1 passes");
        ++st.passes;
        Lanes<int> E_l;
        Lanes<uint32_t> B_l, Tu_l;
        for (int lane = 0; lane < W; ++lane) {
            E_l[lane] = binade(S_l[lane], B_l[lane]);
            Tu_l[lane] = want_stop ? thr_units(thr, E_l[lane]) : 0xFFFFFFFFu;
        }
        uniform(S_l, "S at a pass start");
        uniform(E_l, "the binade of S");
        uniform(B_l, "S in units of its binade");
        uniform(Tu_l, "the stop threshold in units");
        S = S_l[0];
        const int E = E_l[0];
        const uint32_t B = B_l[0];
        const uint32_t p0 = B & 1u;
        const uint32_t Tu = Tu_l[0];
        Lanes<std::array<uint32_t, kSegPer>> kk, kd, k2;
        Lanes<bool> tie, tie2;
        for (int lane = 0; lane < W; ++lane) {
            const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
            tie[lane] = tie2[lane] = false;
            for (int q = 0; q < kSegPer; ++q) {
                const float aq = j0 + q >= kc ? a[lane][q] : 0.0f;
                const float x = std::ldexp(aq, 23 - E), x2 = std::ldexp(aq, 22 - E);
                tie[lane] = tie[lane] || (x - std::floor(x) == 0.5f);
                tie2[lane] = tie2[lane] || (x2 - std::floor(x2) == 0.5f);
                kk[lane][q] = static_cast<uint32_t>(std::fmin(std::rint(x), 0x1p30f));
                k2[lane][q] = static_cast<uint32_t>(std::fmin(std::rint(x2), 0x1p30f));
                kd[lane][q] = 0u;
            }
        }
        const bool fast = ballot(tie) == 0;  // wave-uniform by construction (a ballot)
        if (!fast) ++st.tie_passes;
        Lanes<uint32_t> R, Rend, par, incl2;
        uint32_t total2 = kSat;
        if (fast) {
            Lanes<uint32_t> tot, tot2;
            for (int lane = 0; lane < W; ++lane) {
                tot[lane] = tot2[lane] = 0;
                for (int q = 0; q < kSegPer; ++q) {
                    tot[lane] = sat_add(tot[lane], kk[lane][q]);
                    tot2[lane] = sat_add(tot2[lane], k2[lane][q]);
                }
            }
            incl2.fill(0u);
            if (ballot(tie2) == 0) {
                incl2 = inc_scan(tot2);
                total2 = incl2[W - 1];
            }
            const Lanes<uint32_t> incl = inc_scan(tot);
            const Lanes<uint32_t> ex = shfl_up1(incl, 0u);
            for (int lane = 0; lane < W; ++lane) {
                R[lane] = sat_add(B, ex[lane]);
                Rend[lane] = sat_add(B, incl[lane]);
                par[lane] = 0;
            }
        } else {
            Lanes<Xfer> tf;
            for (int lane = 0; lane < W; ++lane) {
                const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
                for (int q = 0; q < kSegPer; ++q)
                    split_term(j0 + q >= kc ? a[lane][q] : 0.0f, E, kk[lane][q], kd[lane][q]);
                Xfer x = xfer_id();
                for (int q = 0; q < kSegPer; ++q) x = xfer_then(x, term_xfer(kk[lane][q], kd[lane][q]));
                tf[lane] = x;
            }
            const Lanes<Xfer> incl = xfer_scan(tf);
            const Lanes<Xfer> ex = shfl_up1(incl, xfer_id());
            for (int lane = 0; lane < W; ++lane) {
                R[lane] = sat_add(B, p0 ? ex[lane].inc1 : ex[lane].inc0);
                par[lane] = (ex[lane].out >> p0) & 1u;
                Rend[lane] = sat_add(B, p0 ? incl[lane].inc1 : incl[lane].inc0);
            }
            incl2.fill(0u);
        }
        Lanes<uint32_t> ev, R_before;
        for (int lane = 0; lane < W; ++lane) {
            const uint32_t j0 = k0 + static_cast<uint32_t>(lane) * kSegPer;
            ev[lane] = kNoEvent;
            R_before[lane] = R[lane];
            bool live = R[lane] < kL;
            uint32_t r = R[lane], p = par[lane];
            for (int q = 0; q < kSegPer; ++q) {
                const uint32_t j = j0 + q;
                if (fast) {
                    const uint32_t d = kk[lane][q];
                    // the device skips the range test here: terms outside [kc, k1) are zeros
                    MODEL_ASSERT(d == 0 || (j >= kc && j < k1), "a nonzero increment outside the segment");
                    const bool cross = live && (r + d >= kL);
                    if (cross) {
                        ev[lane] = 2 * j;
                        R_before[lane] = r;
                    }
                    const bool adv = live && !cross;
                    r = adv ? r + d : r;
                    const bool hit = adv && r >= Tu;
                    if (hit) ev[lane] = 2 * j + 1;
                    live = adv && !hit;
                } else {
                    const uint32_t d = term_inc(kk[lane][q], kd[lane][q], p);
                    const bool go = live && j >= kc && j < k1;
                    const bool cross = go && (r + d >= kL);
                    const bool adv = go && !cross;
                    if (cross) {
                        ev[lane] = 2 * j;
                        R_before[lane] = r;
                    }
                    r = adv ? r + d : r;
                    p = adv ? ((p + d) & 1u) : p;
                    const bool hit = adv && r >= Tu;
                    if (hit) ev[lane] = 2 * j + 1;
                    live = live && !cross && !hit;
                }
            }
            R[lane] = r;
        }
        Lanes<bool> has;
        for (int lane = 0; lane < W; ++lane) has[lane] = ev[lane] != kNoEvent;
        const uint64_t m = ballot(has);
        if (m == 0) {  // lane 63's end, read by every lane
            S = std::ldexp(static_cast<float>(Rend[W - 1]), E - 23);
            break;
        }
        const int owner = ffs64(m);
        const uint32_t e = ev[owner];
        const uint32_t j = e >> 1;
        MODEL_ASSERT(j >= kc && j < k1, "an event inside the terms not yet added");
        if (e & 1u) {
            S = std::ldexp(static_cast<float>(R[owner]), E - 23);
            stop = j;
            break;
        }
        const uint32_t oj0 = k0 + static_cast<uint32_t>(owner) * kSegPer;
        MODEL_ASSERT(j >= oj0 && j < oj0 + kSegPer, "the crossing term is the owner lane's");
        const float aj = a[owner][j - oj0];
        // every lane forms s_new from the owner lane's values (readlane)
        Lanes<float> s_new_l;
        for (int lane = 0; lane < W; ++lane) s_new_l[lane] = std::ldexp(static_cast<float>(R_before[owner]), E - 23) + aj;
        uniform(s_new_l, "the sum after the crossing term");
        const float s_new = s_new_l[0];
        S = s_new;
        S_l.fill(S);
        if (want_stop && s_new >= thr) {
            stop = j;
            break;
        }
        MODEL_ASSERT(j + 1 > kc, "a pass adds at least one term");
        kc = j + 1;
        if (kc >= k1) break;
        if (total2 < kSat) {
            uint32_t B2;
            const int E2 = binade(S, B2);
            if (E2 == E + 1) {
                uint32_t mine = 0u;
                for (int q = 0; q < kSegPer; ++q) mine += oj0 + q > j ? k2[owner][q] : 0u;
                const uint32_t sum2 = mine + (total2 - incl2[owner]);
                const uint32_t Rend2 = B2 + sum2;
                const uint32_t Tu2 = want_stop ? thr_units(thr, E2) : 0xFFFFFFFFu;
                if (Rend2 < kL && Rend2 < Tu2) {
                    S = std::ldexp(static_cast<float>(Rend2), E2 - 23);
                    S_l.fill(S);
                    break;
                }
            }
        }
    }
    if (want_stop) *stop_at = stop;
    return S;
}

// The walk's crossing shortcut for segment [k0, k1) (seg_chain, no stop threshold): when the
// segment carries crossing data for S's binade E and for E + 1, both free of exact half-way
// terms, the lanes' increments in units of E locate the lane c where S leaves E; S before that
// lane is exact, the lane's terms are added with fp32 adds in order (the reference's own
// operations), and, when S has then reached E + 1, the later lanes' increments in units of E + 1
// give the segment's end unless it leaves E + 1 as well. Returns false (S untouched) when the
// data does not apply; otherwise S holds the sum after the segment (the rest of the segment
// summed exactly by wave_seg_sum where the shortcut stops short).
bool crossing(const std::vector<float>& t, const SegRec& R, uint32_t k0, uint32_t k1, uint32_t n, float& S,
              Stats& st) {
    if (!(R.xl & 1u)) return false;
    uint32_t B;
    const int E = binade(S, B);
    const int ce = R.E[0] == E ? 0 : (R.E[1] == E ? 1 : -1);
    if (ce < 0 || R.E[1 - ce] != E + 1 || !((R.xl >> (1 + ce)) & 1u) || !((R.xl >> (2 - ce)) & 1u)) return false;
    Lanes<bool> over;
    for (int lane = 0; lane < W; ++lane) over[lane] = B + R.lane_inc[ce][lane] >= kL;
    const int c = ffs64(ballot(over));
    if (c < 0) return false;  // no lane leaves E: the walk's own test found another reason
    ++st.crossings;
    const uint32_t ex = c > 0 ? R.lane_inc[ce][c - 1] : 0u;
    MODEL_ASSERT(B + ex < kL, "the sum before the crossing lane stays in its binade");
    float s = std::ldexp(static_cast<float>(B + ex), E - 23);
    const uint32_t jc = k0 + static_cast<uint32_t>(c) * kSegPer;
    for (int q = 0; q < kSegPer; ++q) {
        const uint32_t j = jc + static_cast<uint32_t>(q);
        s += (j < k1 && j < n) ? t[j] : 0.0f;
    }
    uint32_t B2;
    const int E2 = binade(s, B2);
    const uint32_t tot1 = R.lane_inc[1 - ce][W - 1], pre1 = R.lane_inc[1 - ce][c];
    if (E2 == E + 1 && tot1 < kSat && B2 + (tot1 - pre1) < kL) {
        S = std::ldexp(static_cast<float>(B2 + (tot1 - pre1)), E2 - 23);
        ++st.crossings_finished;
        return true;
    }
    S = s;
    if (jc + kSegPer < k1) {
        uint32_t at = k1;
        S = wave_seg_sum(t, n, jc + kSegPer, k1, S, 0.0f, false, &at, st);
    }
    return true;
}

// seg_chain: the walk over the records from the head's sum S, 64 records per step
float seg_chain(const std::vector<float>& t, uint32_t n, const std::vector<SegRec>& rec, float S, float thr,
                uint32_t* stop_at, std::vector<float>& start, Stats& st) {
    const uint32_t nseg = seg_count(n);
    MODEL_ASSERT(nseg <= kSegMax && rec.size() == kSegMax && start.size() == kSegMax + 1, "LDS arrays");
    const bool want_stop = stop_at != nullptr;
    uint32_t stop = n;
    uint32_t t_seg = 0;
    while (t_seg < nseg) {
        const uint32_t t_outer = t_seg;
        for (;;) {
            ++st.walk_steps;
            Lanes<int> E_l;
            Lanes<uint32_t> B_l;
            for (int lane = 0; lane < W; ++lane) E_l[lane] = binade(S, B_l[lane]);
            uniform(E_l, "the walk's binade of S");
            uniform(B_l, "the walk's S in units");
            const int E = E_l[0];
            const uint32_t B = B_l[0];
            const uint32_t p0 = B & 1u;
            Lanes<Xfer> f;
            Lanes<int> c;
            for (int lane = 0; lane < W; ++lane) {
                const uint32_t idx = t_seg + static_cast<uint32_t>(lane);
                c[lane] = -1;
                f[lane] = xfer_id();
                if (idx < nseg) {
                    MODEL_ASSERT(idx < kSegMax, "record index");
                    const SegRec& R = rec[idx];
                    c[lane] = R.E[0] == E ? 0 : (R.E[1] == E ? 1 : -1);
                    if (c[lane] >= 0) f[lane] = R.f[c[lane]];
                    if (c[lane] < 0) ++st.mispredicted;
                }
            }
            Lanes<bool> notfree;
            for (int lane = 0; lane < W; ++lane) {
                const Xfer& x = f[lane];
                notfree[lane] = !(x.inc0 == x.inc1 && x.out == ((x.inc0 & 1u) ? 1u : 2u));
            }
            Lanes<uint32_t> b0, b1;
            if (ballot(notfree) == 0) {
                Lanes<uint32_t> i0;
                for (int lane = 0; lane < W; ++lane) i0[lane] = f[lane].inc0;
                const Lanes<uint32_t> incl = inc_scan(i0);
                const Lanes<uint32_t> excl = shfl_up1(incl, 0u);
                for (int lane = 0; lane < W; ++lane) {
                    b0[lane] = B + excl[lane];
                    b1[lane] = B + incl[lane];
                }
            } else {
                const Lanes<Xfer> incl = xfer_scan(f);
                const Lanes<Xfer> excl = shfl_up1(incl, xfer_id());
                for (int lane = 0; lane < W; ++lane) {
                    b0[lane] = B + (p0 ? excl[lane].inc1 : excl[lane].inc0);
                    b1[lane] = B + (p0 ? incl[lane].inc1 : incl[lane].inc0);
                }
            }
            Lanes<float> Se;
            Lanes<bool> bad;
            for (int lane = 0; lane < W; ++lane) {
                Se[lane] = std::ldexp(static_cast<float>(b1[lane]), E - 23);
                const bool good = c[lane] >= 0 && b1[lane] < kL && !(want_stop && Se[lane] >= thr);
                bad[lane] = !good;
            }
            const uint64_t bm = ballot(bad);
            const uint32_t first = bm ? static_cast<uint32_t>(ffs64(bm)) : 64u;
            for (int lane = 0; lane < W; ++lane) {
                const uint32_t idx = t_seg + static_cast<uint32_t>(lane);
                if (static_cast<uint32_t>(lane) <= first && idx < nseg) {
                    MODEL_ASSERT(idx < kSegMax + 1, "start index");
                    start[idx] = std::ldexp(static_cast<float>(b0[lane]), E - 23);
                }
            }
            if (first > 0) S = Se[first - 1];
            t_seg += first;
            if (first < 64 || t_seg >= nseg) break;
        }
        if (t_seg >= nseg) break;
        const uint32_t k0 = kSegHead + t_seg * kSegLen, k1 = std::min(n, k0 + kSegLen);
        uint32_t at = k1;
        if (!want_stop && crossing(t, rec[t_seg], k0, k1, n, S, st)) {
            ++t_seg;
            continue;
        }
        S = wave_seg_sum(t, n, k0, k1, S, thr, want_stop, &at, st);
        if (want_stop && at < k1) {
            stop = at;
            break;
        }
        ++t_seg;
        MODEL_ASSERT(t_seg > t_outer, "the walk advances");
    }
    start[nseg] = S;
    if (want_stop) *stop_at = stop;
    return S;
}

struct RowResult {
    float sum;
    uint32_t stop;
};

// seg_xfer_kernel + seg_row_sum: the records from the double prefix sums, the serial head,
// then the walk (with a stop threshold when want_stop)
RowResult engine(const std::vector<float>& t, uint32_t n, float thr, bool want_stop, std::vector<float>& start,
                 Stats& st) {
    const uint32_t nseg = seg_count(n);
    // the double sums of the head and of each segment (any order: they only predict binades)
    std::vector<double> d(nseg + 1, 0.0);
    for (uint32_t j = 0; j < std::min(n, kSegHead); ++j) d[0] += t[j];
    for (uint32_t s = 0; s < nseg; ++s)
        for (uint32_t j = kSegHead + s * kSegLen; j < std::min(n, kSegHead + (s + 1) * kSegLen); ++j)
            d[1 + s] += t[j];
    std::vector<SegRec> rec(kSegMax);
    double D = 0.0;
    for (uint32_t s = 0; s < nseg; ++s) {
        D += d[s];
        rec[s] = make_record(t, n, s, D, D + d[s + 1]);
    }
    // the serial head, staged in LDS (kSegHead entries)
    std::vector<float> hterm(kSegHead, 0.0f);
    const uint32_t nh = std::min(n, kSegHead);
    for (uint32_t j = 0; j < kSegHead; ++j) {
        MODEL_ASSERT(j < kSegHead, "head staging index");
        hterm[j] = j < nh ? t[j] : 0.0f;
    }
    float S = 0.0f;
    uint32_t hstop = n;
    if (want_stop) {
        for (uint32_t j = 0; j < nh; ++j) {
            S += hterm[j];
            if (S >= thr) {
                hstop = j;
                break;
            }
        }
        if (hstop < nh) return RowResult{S, hstop};
    } else {
        for (uint32_t j = 0; j < kSegHead; ++j) S += hterm[j];  // zeros past nh leave S as it is
    }
    uint32_t stop = n;
    const float sum = seg_chain(t, n, rec, S, thr, want_stop ? &stop : nullptr, start, st);
    return RowResult{sum, stop};
}

// seg_residual_block's draw: the sum without a stop, then the first index whose prefix reaches
// r = u2 * sum, searched in the head or in the one segment whose recorded start lies below r
RowResult residual_draw(const std::vector<float>& t, uint32_t n, float u2, Stats& st) {
    std::vector<float> start(kSegMax + 1, 0.0f);
    const RowResult all = engine(t, n, 0.0f, false, start, st);
    const float r = u2 * all.sum;
    const uint32_t nseg = seg_count(n);
    const uint32_t nh = std::min(n, kSegHead);
    uint32_t at = n;
    float S = 0.0f;
    if (nseg == 0 || start[0] >= r) {
        for (uint32_t j = 0; j < nh; ++j) {  // block_seq_sum's serial start over the head
            S += t[j];
            if (S >= r) {
                at = j;
                break;
            }
        }
    } else {
        // each of the block's 1024 threads counts starts 1 + tid, 1 + tid + 1024, ..., then
        // __syncthreads_count sums the counts
        uint32_t below = 0;
        for (uint32_t tid = 0; tid < 1024; ++tid)
            for (uint32_t i = 1 + tid; i < nseg; i += 1024) {
                MODEL_ASSERT(i < kSegMax + 1, "start index in the search");
                below += start[i] < r;
            }
        MODEL_ASSERT(below < nseg, "search segment");
        for (uint32_t i = 1; i < nseg; ++i) MODEL_ASSERT(start[i] >= start[i - 1], "segment starts never decrease");
        const float S0 = start[below];
        const uint32_t k0 = kSegHead + below * kSegLen, k1 = std::min(n, k0 + kSegLen);
        uint32_t a = k1;
        S = wave_seg_sum(t, n, k0, k1, S0, r, true, &a, st);
        at = a >= k1 ? n : a;
    }
    return RowResult{S, at};
}

RowResult in_order(const std::vector<float>& t, uint32_t n, float thr, bool want_stop) {
    float s = 0.0f;
    for (uint32_t j = 0; j < n; ++j) {
        s += t[j];
        if (want_stop && s >= thr) return RowResult{s, j};
    }
    return RowResult{s, n};
}

// six kinds of rows, as the device tests build them
std::vector<float> make_row(int kind, uint32_t n, std::mt19937_64& g) {
    std::vector<float> t(n);
    std::uniform_real_distribution<double> U(0.0, 1.0);
    std::normal_distribution<double> N(0.0, 1.0);
    switch (kind) {
        case 0: {  // softmax terms expf(l - max), l ~ N(0, sigma^2)
            const double sigma = 0.5 + 4.0 * U(g);
            std::vector<float> l(n);
            float mx = -1e9f;
            for (auto& x : l) {
                x = static_cast<float>(N(g) * sigma);
                mx = x > mx ? x : mx;
            }
            for (uint32_t j = 0; j < n; ++j) t[j] = std::exp(l[j] - mx);
            break;
        }
        case 1: {  // residual terms max(0, p - q) of two nearby normalised rows
            const double sigma = 1.0 + 2.0 * U(g);
            double sp = 0.0, sq = 0.0;
            std::vector<float> p(n), q(n);
            for (uint32_t j = 0; j < n; ++j) {
                const double z = N(g) * sigma;
                p[j] = static_cast<float>(std::exp(z / 3.0));
                q[j] = static_cast<float>(std::exp((0.8 * z + 0.6 * N(g)) / 3.0));
                sp += p[j];
                sq += q[j];
            }
            const float ip = static_cast<float>(1.0 / sp), iq = static_cast<float>(1.0 / sq);
            for (uint32_t j = 0; j < n; ++j) {
                const float x = p[j] * ip - q[j] * iq;
                t[j] = 0.0f < x ? x : 0.0f;
            }
            break;
        }
        case 2: {  // every other addition an exact half-way case: 1, then 2^-24 and 2^-23
            t[0] = 1.0f;
            for (uint32_t j = 1; j < n; ++j) t[j] = (j & 1) ? 0x1p-24f : (U(g) < 0.5 ? 0x1p-23f : 0x1p-22f);
            break;
        }
        case 3: {  // powers of two over a wide range
            for (auto& x : t) x = std::ldexp(1.0f, -static_cast<int>(g() % 40));
            break;
        }
        case 4: {  // terms near 0.5: the sum crosses many binades, ties frequent
            for (auto& x : t) x = static_cast<float>(0.49 + 0.02 * U(g));
            break;
        }
        default: {  // zeros, terms far below half an ulp, sparse big terms
            for (auto& x : t) {
                const double r = U(g);
                x = r < 0.3 ? 0.0f : (r < 0.95 ? static_cast<float>(1e-12 * U(g)) : static_cast<float>(10.0 * U(g)));
            }
            break;
        }
    }
    return t;
}

}  // namespace

int main(int argc, char** argv) {
    const int rows = argc > 1 ? std::atoi(argv[1]) : 1600;
    std::mt19937_64 g(argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 20261202ull);
    static const uint32_t sizes[] = {1000, 2048, 2049, 2560, 3000, 50000, 131072, 262144, 300000};
    long checked[6] = {}, bad = 0;
    Stats st;
    try {
        for (int r = 0; r < rows; ++r) {
            const int kind = r % 6;
            const uint32_t n = (r % 7 == 0) ? sizes[g() % 9] : static_cast<uint32_t>(1000 + g() % 299000);
            const std::vector<float> t = make_row(kind, n, g);
            // the sum alone
            std::vector<float> start(kSegMax + 1, 0.0f);
            const RowResult a = engine(t, n, 0.0f, false, start, st);
            const RowResult ra = in_order(t, n, 0.0f, false);
            // a stop threshold inside the sum (twd_sequential_sum with stop_out)
            const float u = static_cast<float>(std::uniform_real_distribution<double>(0.0, 1.0)(g));
            const float thr = u * ra.sum;
            std::vector<float> start2(kSegMax + 1, 0.0f);
            const RowResult b = engine(t, n, thr, true, start2, st);
            const RowResult rb = in_order(t, n, thr, true);
            // the residual draw's search
            const RowResult c = residual_draw(t, n, u, st);
            const RowResult rc = in_order(t, n, u * ra.sum, true);
            const bool ok = f2u(a.sum) == f2u(ra.sum) && f2u(b.sum) == f2u(rb.sum) && b.stop == rb.stop &&
                            c.stop == rc.stop && (c.stop == n || f2u(c.sum) == f2u(rc.sum));
            if (!ok) {
                if (bad < 5)
                    std::printf("MISMATCH row %d kind %d n %u: sum %a/%a stop %u/%u draw %u/%u\n", r, kind, n,
                                static_cast<double>(a.sum), static_cast<double>(ra.sum), b.stop, rb.stop, c.stop,
                                rc.stop);
                ++bad;
            }
            ++checked[kind];
        }
    } catch (const std::exception& e) {
        std::printf("FAIL %s\n", e.what());
        return 1;
    }
    static const char* names[] = {"softmax", "residual", "half-way ties", "powers of two", "near 0.5",
                                  "zeros/tiny/sparse"};
    for (int k = 0; k < 6; ++k) std::printf("%-18s %ld rows\n", names[k], checked[k]);
    std::printf("exact segments %ld (passes %ld, with a tie %ld), walk steps %ld, record lookups outside both binades %ld\n",
                st.exact_segments, st.passes, st.tie_passes, st.walk_steps, st.mispredicted);
    std::printf("crossings resolved from the crossing data %ld (finished without a pass %ld)\n", st.crossings,
                st.crossings_finished);
    std::printf("mismatches %ld\n", bad);
    if (bad == 0) std::puts("MODEL OK");
    return bad == 0 ? 0 : 1;
}
