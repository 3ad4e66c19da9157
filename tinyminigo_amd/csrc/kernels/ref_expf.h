// expf with the results of the C library the reference calls.
//
// The reference's f32 exp (Rust f32::exp; softmax, src/tensor.rs:1055-1060,
// and silu, src/tensor.rs:1043-1045) is the platform libm's expf.  On Linux
// that is glibc (2.27 and later), whose expf is the published algorithm of
// ARM's optimized-routines (Szabolcs Nagy, 2017; MIT licensed), built for
// x86-64 CPUs with FMA in its FMA variant:
//   k = round(x * 32/ln2),  r = x * 32/ln2 - k          (in double)
//   exp(x) = 2^(k/32) * 2^(r/32)
//   2^(r/32) ~= 1 + c2 r + c1 r^2 + c0 r^3              (c_i its minimax
//                                                         coefficients)
//   2^(k/32) from a 32-entry table of 2^(i/32) rounded to double, with the
//   integer part of k/32 added to the exponent field,
// and the double result rounded once to float.  Evaluated here with the
// same operations, the same fused multiply-adds and the same constants, so
// the result equals glibc's bit for bit (checked over all 2^32 inputs on the
// host and on a sample on the device).  The device's own expf differs from
// glibc's in the last bit for about 1.5% of inputs.
//
// Usable from host C++ and from HIP device code.
#pragma once

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define TMG_HD __host__ __device__
#else
#define TMG_HD
#endif

namespace tmg {

TMG_HD inline float ref_expf(float x) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
    // kTab[i] = bits of 2^(i/32) rounded to double, minus i << 47, so that
    // adding k << 47 to kTab[k % 32] gives the bits of 2^(k/32)
    constexpr uint64_t kTab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;  // 32 / ln 2
    constexpr double kShift = 0x1.8p+52;                    // round-to-int by addition
    constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88, or inf / NaN
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf();  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                  // underflow
    }
    // the FMA build fuses x * 32/ln2 into both of its uses
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = kTab[ki % 32];
    t += ki << 47;
    double s;
    memcpy(&s, &t, 8);
    const double zz = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(zz, r2, y);
    y = y * s;
    return (float)y;
}

}  // namespace tmg
