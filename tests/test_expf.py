"""The draft verify's expf (turbo-winfare-dense_amd/csrc/expf_libm.h), compiled for the host
from the same header the device code uses, against this host C library's expf, bit for bit over
every float the softmax of speculator.cpp:14-30 can feed it: x = l / T - max <= 0, where results
are nonzero down to about -103.97 (every float in [-104, 0], 1,120,927,745 values), plus the
special cases of the method (overflow, underflow, infinities, NaN) and a sweep of positive
arguments. The reference's std::exp(float) is the host library's expf (x86-64 glibc, whose
ifunc picks the FMA build on CPUs with FMA, as this one and the GPU box's host have)."""
import os
import subprocess

import pytest

from helpers import ROOT

SRC = r'''
#include <cmath>
#include <cstdio>
#include <cstring>
#include "expf_libm.h"
static unsigned long long mismatches(unsigned lo, unsigned hi, unsigned step, unsigned sign) {
    unsigned long long bad = 0;
    for (unsigned long long m = lo; m <= hi; m += step) {
        unsigned u = static_cast<unsigned>(m) | sign;
        float x;
        std::memcpy(&x, &u, 4);
        const float a = expf(x), b = twd::expf_libm<true>(x);
        unsigned ua, ub;
        std::memcpy(&ua, &a, 4);
        std::memcpy(&ub, &b, 4);
        if (ua != ub && !(a != a && b != b)) {
            if (bad < 5) std::printf("x=%a host=%a ours=%a\n", x, a, b);
            ++bad;
        }
    }
    return bad;
}
int main() {
    unsigned top;
    float lim = 104.0f;
    std::memcpy(&top, &lim, 4);
    std::printf("negative %llu\n", mismatches(0, top, 1, 0x80000000u));
    std::printf("positive %llu\n", mismatches(0, 0x7FFFFFFFu, 97, 0u));
    float sp[] = {INFINITY, -INFINITY, NAN, 88.0f, 88.72f, 89.0f, -103.9f, -104.0f, -150.0f, 0.0f, -0.0f};
    unsigned long long bad = 0;
    for (float x : sp) {
        const float a = expf(x), b = twd::expf_libm<true>(x);
        if (std::memcmp(&a, &b, 4) != 0 && !(a != a && b != b)) ++bad;
    }
    std::printf("special %llu\n", bad);
    return 0;
}
'''


def test_expf_matches_host_libm(tmp_path):
    src = tmp_path / "expf_pin.cpp"
    src.write_text(SRC)
    exe = tmp_path / "expf_pin"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I" + os.path.join(ROOT, "turbo-winfare-dense_amd", "csrc"), str(src), "-o",
                    str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, check=True).stdout
    print(out)
    counts = {line.split()[0]: int(line.split()[1]) for line in out.splitlines() if line.split()[0] in ("negative", "positive", "special")}
    assert counts == {"negative": 0, "positive": 0, "special": 0}, out
