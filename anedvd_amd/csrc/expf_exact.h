// expf_exact.h -- single-precision exp that returns, bit for bit, what x86-64
// glibc's expf returns (the function Zig's @exp lowers to on Linux), so that the
// GPU router ranks experts with exactly the CPU's probabilities.
//
// Method: the published table-driven algorithm of Szabolcs Nagy (ARM
// optimized-routines, 2017; adopted by glibc 2.27 and musl), evaluated in
// binary64:  x*N/ln2 = k + r,  exp(x) = 2^(k/N) * P(r/N),  N = 32, with
// 2^(i/N) from a 32-entry table (each entry the correctly rounded double
// 2^(i/32), minus i<<52/32 so the exponent can be added as an integer) and a
// degree-3 polynomial.  glibc's x86-64 build runs the FMA variant when the CPU
// has FMA (every MI355X host does), in which the compiler fuses
// `InvLn2N*x + Shift`, `InvLn2N*x - kd` and the three polynomial steps; the
// same five fused operations are spelled out below with fma(), so the device
// code (v_fma_f64) rounds identically.
//
// Pinned by tests/test_expf.py: this header compiled for the host equals libm
// expf on every float in [-inf, 88.72] (4.3e9 inputs, 0 differences).
#pragma once

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define ANEDVD_HD __host__ __device__
#else
#define ANEDVD_HD
#endif

#ifndef __HIPCC__
#include <math.h>
#endif

namespace anedvd {

ANEDVD_HD inline double as_f64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
ANEDVD_HD inline uint64_t as_u64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
ANEDVD_HD inline uint32_t as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
ANEDVD_HD inline float as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

ANEDVD_HD inline double fma_f64(double a, double b, double c)
{
#ifdef __HIP_DEVICE_COMPILE__
    return __builtin_fma(a, b, c);
#else
    return fma(a, b, c);
#endif
}

// bits(2^(i/32)) - (i << 52) / 32, for i = 0..31.
#define ANEDVD_EXP2_TABLE                                                          \
    { 0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull }

// expf for x <= 0x1.62e42ep6 (the routing kernel only evaluates exp(v - max) <= 0).
// NaN propagates; -inf and x < log(2^-150) give +0; larger x overflows to +inf.
ANEDVD_HD inline float expf_exact(float x, const uint64_t *tab)
{
    const uint32_t ux = as_u32(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                  // |x| >= 88, or x is inf/nan
        if (ux == 0xff800000u) return 0.0f;  // -inf
        if (abstop >= 0x7f8u) return x + x;  // nan (or +inf)
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = fma_f64(inv_ln2_n, xd, shift);
    const uint64_t ki = as_u64(kd);
    kd -= shift;
    const double r = fma_f64(inv_ln2_n, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << (52 - 5));
    const double s = as_f64(t);
    const double z = fma_f64(c0, r, c1);
    const double r2 = r * r;
    double y = fma_f64(c2, r, 1.0);
    y = fma_f64(z, r2, y);
    y = y * s;
    return (float)y;
}

}  // namespace anedvd
