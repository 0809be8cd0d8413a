"""The shortlist's exp(double) (turbo-winfare-dense_amd/csrc/exp_libm.h), compiled for the host
from the same header the device code uses, against this host C library's exp, bit for bit.

sample_token forms its shortlist terms as std::exp((double)l - max) and
std::exp(((double)l - max) / T) (src/sampling.cpp:145,157), with l and max floats and T the
float temperature; the reference's std::exp(double) is the host library's exp (x86-64 glibc,
whose ifunc picks the FMA build on CPUs with FMA, as this one and the GPU box's host have).
Checked here:
  * those two argument families: l and max floats in [-60, 0] (l <= max), T in [0.05, 2];
  * random arguments over the whole range where exp is finite and nonzero, and past it;
  * arguments within a few ulps of every point where x * 128/ln2 is half an odd integer (the
    rounding of the reduction step, where a fused and an unfused evaluation differ);
  * the special cases: zeros, infinities, NaN, the overflow and underflow edges, the subnormal
    results, tiny arguments.
"""
import os
import subprocess

from helpers import ROOT

SRC = r'''
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include "exp_libm.h"
static uint64_t s = 0x9E3779B97F4A7C15ull;
static uint64_t rnd() { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }
static double unit() { return static_cast<double>(rnd() >> 11) * 0x1p-53; }
static float unitf() { return static_cast<float>(rnd() >> 40) * 0x1p-24f; }
static unsigned long long bad = 0;
static void check(double x) {
    const double a = std::exp(x), b = twd::exp_libm(x);
    uint64_t ua, ub;
    std::memcpy(&ua, &a, 8);
    std::memcpy(&ub, &b, 8);
    if (ua != ub && !(a != a && b != b)) {
        if (bad < 5) std::printf("x=%a host=%a ours=%a\n", x, a, b);
        ++bad;
    }
}
int main() {
    // the shortlist's arguments
    unsigned long long n0 = 0;
    for (long i = 0; i < 6000000; ++i) {
        float l = -60.0f * unitf(), mx = -60.0f * unitf();
        if (l > mx) { const float t = l; l = mx; mx = t; }
        const double x = static_cast<double>(l) - static_cast<double>(mx);
        const float T = 0.05f + 1.95f * unitf();
        check(x);
        check(x / static_cast<double>(T));
        n0 += 2;
    }
    std::printf("shortlist %llu %llu\n", n0, bad);
    const unsigned long long b0 = bad;
    // random arguments: [-745.2, 0] (every nonzero result of x <= 0), then wider
    for (long i = 0; i < 12000000; ++i) check(-745.2 * unit());
    for (long i = 0; i < 4000000; ++i) check(-1100.0 + 1900.0 * unit());
    for (long i = 0; i < 2000000; ++i) check(std::ldexp(unit() - 0.5, -20 - static_cast<int>(rnd() % 40)));
    std::printf("random 18000000 %llu\n", bad - b0);
    const unsigned long long b1 = bad;
    // around x * 128/ln2 = k + 1/2
    const double inv = 0x1.71547652b82fep0 * 128;
    for (long k = -95500; k < 91000; k += 1) {
        const double x0 = (static_cast<double>(k) + 0.5) / inv;
        uint64_t u;
        std::memcpy(&u, &x0, 8);
        for (int d = -24; d <= 24; ++d) {
            const uint64_t v = u + static_cast<uint64_t>(static_cast<int64_t>(d));
            double x;
            std::memcpy(&x, &v, 8);
            check(x);
        }
    }
    std::printf("halfway %llu\n", bad - b1);
    const unsigned long long b2 = bad;
    const double sp[] = {0.0, -0.0, INFINITY, -INFINITY, NAN, -NAN, 1.0, -1.0, 0x1p-54, -0x1p-54,
                         0x1p-53, -0x1p-60, 0x1p-1074, -0x1p-1074, 709.782712893384, 709.7827128933841,
                         710.0, 1023.9, 1024.0, 5000.0, -708.3964185322641, -708.4, -744.4400719213812,
                         -745.1332191019411, -745.1332191019412, -745.2, -1023.9, -1024.0, -5000.0,
                         511.9999999, 512.0, -512.0, -511.9999999, 1e-300, -1e-300};
    for (double x : sp) check(x);
    for (int e = -1074; e < 1024; ++e) {  // every power of two, both signs
        check(std::ldexp(1.0, e));
        check(-std::ldexp(1.0, e));
    }
    std::printf("special %llu\n", bad - b2);
    return 0;
}
'''


def test_exp_matches_host_libm(tmp_path):
    src = tmp_path / "exp_pin.cpp"
    src.write_text(SRC)
    exe = tmp_path / "exp_pin"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I" + os.path.join(ROOT, "turbo-winfare-dense_amd", "csrc"), str(src), "-o",
                    str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, check=True).stdout
    print(out)
    counts = {}
    for line in out.splitlines():
        f = line.split()
        if f and f[0] in ("shortlist", "random", "halfway", "special"):
            counts[f[0]] = int(f[-1])
    assert counts == {"shortlist": 0, "random": 0, "halfway": 0, "special": 0}, out
