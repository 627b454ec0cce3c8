// expf of the reference's libm (glibc 2.28 and later, x86-64 with FMA), restated so that
// device code computes the same float bits: the method of ARM's optimized-routines
// (Szabolcs Nagy) that glibc uses. x * 32 / ln 2 = k + r with k integral; 2^(k/32) from a
// table of 2^(i/32) (entry i: the double 2^(i/32) with i << 47 subtracted from its bits,
// so adding k << 47 applies k / 32's integral part to the exponent); 2^(r/32) by a cubic;
// all in double with fused multiply-adds where the FMA build has them, rounded once to
// float. The table is 2^(i/32) rounded to double; the cubic's coefficients and the
// thresholds are the method's. A host test compares this function with the host's expf on
// every float in [-128, 0].
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace tfk {

#define TF_EXP2_TABLE                                                                         \
    {                                                                                         \
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull, \
    }

// tab: the 32 entries of TF_EXP2_TABLE (device code passes its constant-memory copy).
__host__ __device__ inline float expf_libm(float x, const uint64_t* tab) {
    if (x != x) return x + x;
    if (x < -0x1.9fe368p6f) return 0.0f;  // below log(2^-150): rounds to +0
    if (x > 0x1.62e42ep6f) return INFINITY;
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32768.0, c1 = 0x1.ebfce50fac4f3p-3 / 1024.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = fma(kInvLn2N, xd, kShift);
    uint64_t ki;
    __builtin_memcpy(&ki, &kd, 8);
    kd = kd - kShift;
    const double r = fma(kInvLn2N, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    double s;
    __builtin_memcpy(&s, &t, 8);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

}  // namespace tfk
