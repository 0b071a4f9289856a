// hf_expf.h -- single-precision exp and the router sigmoid, bit-identical to
// the C library's expf on x86-64 glibc, for host and device code alike.
//
// The reference ranks experts on 1 / (1 + std::exp(-z)) in float
// (moe_router.h:19-21, glm_forward.cpp:522-524), i.e. on glibc's expf, which is
// not correctly rounded: a correctly rounded exp differs from it by one ulp on
// about one input in 13,000, enough to flip a near-tie at the top-k boundary.
// So the device evaluates the same algorithm, not merely an accurate exp.
//
// Method: the table-driven exp of Szabolcs Nagy (ARM optimized-routines,
// glibc's expf since 2.27), in double precision and rounded once to float:
//   z = x * 32/ln2;  k = round-to-nearest(z) (by adding 1.5 * 2^52);  r = z - k,
//   exp(x) = 2^(k/32) * 2^(r/32),
//   2^(k/32) = 2^floor(k/32) * 2^((k mod 32)/32): a table entry whose exponent
//              field receives floor(k/32) by an integer add of k << 47,
//   2^(r/32) ~= 1 + C2 r + C1 r^2 + C0 r^3  (|r| <= 1/2; the degree-3 fit of
//              the method, coefficients pre-divided by 32, 32^2, 32^3).
// Entry i of the table holds the bits of 2^(i/32) rounded to double, minus
// i << 47 (so adding k << 47 for k = 32q + i leaves q in the exponent field).
// x86-64 glibc runs the FMA build of this routine on CPUs that have FMA; its
// r = x * 32/ln2 - k is then one fused multiply-add, and so it is here (an
// unfused r rounds 2 of the 2^32 inputs differently; the fusion of the
// polynomial steps and of k changes no result).  Every float input, NaN
// aside, was checked against the C library's expf (tests/test_expf.py).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define HF_HD __host__ __device__
#else
#define HF_HD
#endif

namespace hf {

namespace expf_detail {

// bits(2^(i/32) rounded to double) - (i << 47), i = 0..31.
#if defined(__HIP_DEVICE_COMPILE__)
__constant__
#endif
static const uint64_t kTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

constexpr double kInvLn2x32 = 0x1.71547652b82fep+0 * 32;  // 32 / ln 2 rounded to double
constexpr double kShift = 0x1.8p+52;                       // 1.5 * 2^52: rounds to an integer
constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;

HF_HD inline uint32_t f2u(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    return u;
}
HF_HD inline uint64_t d2u(double d) {
    uint64_t u;
    __builtin_memcpy(&u, &d, 8);
    return u;
}
HF_HD inline double u2d(uint64_t u) {
    double d;
    __builtin_memcpy(&d, &u, 8);
    return d;
}

}  // namespace expf_detail

// exp(x) rounded as glibc's expf rounds it, for every float x.
HF_HD inline float glibc_expf(float x) {
    using namespace expf_detail;
    const uint32_t ux = f2u(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                  // |x| >= 88 (0x42b is 88.0f's top 12 bits), or NaN
        if (ux == 0xff800000u) return 0.0f;  // -inf
        if (abstop >= 0x7f8u) return x + x;  // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff();  // exp(x) >= 2^128
        if (x < -0x1.9fe368p6f) return 0.0f;             // exp(x) < 2^-150
    }
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2x32, xd, kShift);
    const uint64_t ki = d2u(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2x32, xd, -kd);
    const double s = u2d(kTab[ki % 32] + (ki << 47));
    const double p = __builtin_fma(kC0, r, kC1);
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(p, r * r, y);
    return (float)(y * s);
}

// The router's sigmoid, 1 / (1 + expf(-x)) in float (moe_router.h:19-21): the
// sum and the quotient are each rounded once to float (the quotient is formed
// in double and rounded to float, which for float operands is the correctly
// rounded float quotient: 53 >= 2 * 24 + 2 significand bits).
HF_HD inline float router_sigmoid(float x) {
    const float den = 1.0f + glibc_expf(-x);
    return (float)(1.0 / (double)den);
}

}  // namespace hf
