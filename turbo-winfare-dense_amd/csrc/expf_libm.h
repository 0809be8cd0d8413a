// expf by the method of glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, the ARM
// optimized-routines algorithm, glibc 2.27 and later), written for the device so that the
// draft-logits verify's softmax terms equal what the reference's std::exp(float) returns on the
// host it was built on: x * 32/ln2 = k + r with k rounded to an integer (adding and subtracting
// 1.5 * 2^52), 2^(k/32) from a 32-entry table of 2^(i/32) (each the double nearest the exact
// value, stored less i << 47, so that adding k << 47 builds the double directly), and 2^(r/32)
// from a degree-3 polynomial evaluated in double, rounded once to float at the end.
//
// Where a * b + c appears the host library (x86-64 glibc built with FMA, the variant its ifunc
// picks on CPUs that have FMA) computes one fused multiply-add; kFma selects that evaluation.
// The CPU test tests/test_expf.py checks this function bit for bit against the host expf over
// every float in the range the softmax feeds it.
//
// Header-only and dependency-free: compiled for the device by hipcc and for the host by the test.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define TWD_HD __host__ __device__
#else
#define TWD_HD
#endif

namespace twd {

// 2^(i/32) as the bits of the nearest double, less i << 47 (glibc's __exp2f_data.tab).
#if defined(__HIPCC__)
__device__ __constant__ static const uint64_t kExpfTab[32] = {
#else
static const uint64_t kExpfTab[32] = {
#endif
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

TWD_HD inline double expf_as_double(uint64_t u) {
    double d;
    memcpy(&d, &u, sizeof d);
    return d;
}

TWD_HD inline uint64_t expf_as_u64(double d) {
    uint64_t u;
    memcpy(&u, &d, sizeof u);
    return u;
}

// kFma: evaluate each a * b + c of the method as one fused multiply-add.
template <bool kFma>
TWD_HD inline float expf_libm(float x) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
    uint32_t ux;
    memcpy(&ux, &x, sizeof ux);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88 (top 12 bits of 88.0f), inf or NaN
        if (ux == 0xff800000u) return 0.0f;           // -inf
        if (abstop >= 0x7f8) return x + x;             // +inf, NaN
        if (x > 0x1.62e42ep6f) return 0x1p97f * 0x1p97f;   // overflow to +inf
        if (x < -0x1.9fe368p6f) return 0x1p-95f * 0x1p-95f;  // underflow to +0
    }
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = static_cast<double>(x);
    double kd, r;
    if constexpr (kFma) {
        // z = x * 32/ln2 only feeds z + shift and z - kd: both fuse with the product
        kd = __builtin_fma(kInvLn2N, xd, kShift);
        const uint64_t ki = expf_as_u64(kd);
        kd -= kShift;
        r = __builtin_fma(kInvLn2N, xd, -kd);
        uint64_t t = kExpfTab[ki % 32];
        t += ki << 47;
        const double s = expf_as_double(t);
        const double z = __builtin_fma(kC0, r, kC1);
        const double r2 = r * r;
        double y = __builtin_fma(kC2, r, 1.0);
        y = __builtin_fma(z, r2, y);
        return static_cast<float>(y * s);
    } else {
        const double z0 = kInvLn2N * xd;
        kd = z0 + kShift;
        const uint64_t ki = expf_as_u64(kd);
        kd -= kShift;
        r = z0 - kd;
        uint64_t t = kExpfTab[ki % 32];
        t += ki << 47;
        const double s = expf_as_double(t);
        const double z = kC0 * r + kC1;
        const double r2 = r * r;
        double y = kC2 * r + 1.0;
        y = z * r2 + y;
        return static_cast<float>(y * s);
    }
}

}  // namespace twd
