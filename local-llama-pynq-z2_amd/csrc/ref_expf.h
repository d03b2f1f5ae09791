// expf exactly as the reference's libm computes it, for the reference-order ("strict") mode.
//
// The reference calls the C library's expf in softmax (qwen.c:346-352, runq.c:409-428) and in SiLU
// (qwen.c:558-562, runq.c:589-596).  On the hosts it runs on (x86-64, glibc 2.35) that is glibc's expf,
// the algorithm published with ARM's optimized-routines (sysdeps/ieee754/flt-32/e_expf.c, e_exp2f_data.c),
// selected in its FMA build on any CPU with FMA:
//   x * 32/ln2 = k + r, |r| <= 1/2, k rounded to nearest even by adding 1.5 * 2^52;
//   exp(x) = 2^(k/32) * 2^(r/32),  2^(k/32) from a 32-entry table of 2^(i/32) with k/32's integer part added
//   to the exponent bits,  2^(r/32) ~ C0 r^3 + C1 r^2 + C2 r + 1  evaluated in double with FMA,
//   then one rounding to float.
// glibc's result is not the correctly rounded exp: the cubic leaves up to ~2^-34 relative error, so a
// correctly rounded fp64 exp differs from it in about 1 of 13,000 inputs.  Bit-exact softmax and SiLU
// therefore need this exact evaluation order.  The table holds the bits of the double nearest to 2^(i/32)
// minus i << 47 (so adding k << 47 puts k's integer part /32 into the exponent).  The restatement below
// was compared with glibc 2.35's expf over every float in [-103.9, 88.7] (2,239,836,981 inputs, no
// difference) and is checked again by the tests over a strided sample of all 2^32 bit patterns.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#define REF_EXPF_TAB                                                                                     \
    {                                                                                                    \
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,     \
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,     \
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,     \
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,     \
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,     \
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,     \
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,     \
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,     \
    }

static __constant__ uint64_t ref_expf_tab_dev[32] = REF_EXPF_TAB;
static const uint64_t ref_expf_tab_host[32] = REF_EXPF_TAB;

// The evaluation with the table passed in (the device's constant-memory copy or the host's).
__host__ __device__ inline float ref_expf_with(float x, const uint64_t *tab) {
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                         // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f;          // -inf
        if (abstop >= 0x7f8) return x + x;           // +inf, nan
        if (x > 0x1.62e42ep6f) return INFINITY;      // above log(2^128): overflow
        if (x < -0x1.9fe368p6f) return 0.0f;         // below log(2^-150): underflow to zero
    }
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_32, xd, shift);          // k + 1.5 * 2^52: k in the low mantissa bits
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_32, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double z = fma(c0, r, c1), r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

__device__ __forceinline__ float ref_expf(float x) { return ref_expf_with(x, ref_expf_tab_dev); }
