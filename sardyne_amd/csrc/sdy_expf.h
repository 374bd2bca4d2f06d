/* expf of the host C library, restated so that the device computes the reference's exponentials bit
 * for bit (the reference calls libm expf in op_softmax and op_silu_mul, csrc/ops.c:353-371).
 *
 * The library is glibc 2.35 (x86-64, FMA build), whose expf is the published ARM optimized-routines
 * algorithm (sysdeps/ieee754/flt-32/e_expf.c, EXP2F_TABLE_BITS = 5, EXP2F_POLY_ORDER = 3):
 *   z = x * 32/ln2, k = z rounded to an integer (by adding 1.5 * 2^52), r = x * 32/ln2 - k taken
 *   with one fused multiply-add, s = 2^(k/32) from a table of 2^(i/32) (i = k mod 32) whose exponent
 *   field is raised by k/32, exp(x) ~ s * (c0 r^3 + c1 r^2 + c2 r + 1) in double, rounded to float
 *   once. Above 0x1.62e42ep6 the result is +inf, below -0x1.9fe368p6 it is +0, NaN gives NaN.
 * The table holds 2^(i/32) correctly rounded to double, minus i << 47 (the exponent step that the
 * addition of k << 47 puts back). The result equals the host expf for every one of the 2^32 float
 * inputs (checked exhaustively; tests/test_expf.py runs a strided subset).
 *
 * Included by C (the CPU check) and by HIP sources (device code). */
#ifndef SDY_EXPF_H
#define SDY_EXPF_H
#include <stdint.h>

#ifdef __HIPCC__
#define SDY_EXPF_QUAL __device__ static inline
#define SDY_EXPF_TABLE __constant__ static const
#define SDY_EXPF_FMA(a, b, c) __builtin_fma((a), (b), (c))
#else
#include <math.h>
#include <string.h>
#define SDY_EXPF_QUAL static inline
#define SDY_EXPF_TABLE static const
#define SDY_EXPF_FMA(a, b, c) fma((a), (b), (c))
#endif

SDY_EXPF_TABLE uint64_t sdy_exp2_32_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

SDY_EXPF_QUAL double sdy_expf_bits_to_double(uint64_t u) {
#ifdef __HIPCC__
    return __builtin_bit_cast(double, u);
#else
    double d;
    memcpy(&d, &u, sizeof d);
    return d;
#endif
}

SDY_EXPF_QUAL uint64_t sdy_expf_double_to_bits(double d) {
#ifdef __HIPCC__
    return __builtin_bit_cast(uint64_t, d);
#else
    uint64_t u;
    memcpy(&u, &d, sizeof u);
    return u;
#endif
}

/* Branch-free: the main path runs for every x (its table index is in range for any input) and the
 * special cases are selected at the end, so a device wave issues its table reads without branching. */
SDY_EXPF_QUAL float sdy_expf(float x) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = sdy_expf_double_to_bits(kd);
    kd -= shift;
    const double r = SDY_EXPF_FMA(inv_ln2_n, xd, -kd);
    const uint64_t t = sdy_exp2_32_tab[ki % 32] + (ki << 47);
    const double s = sdy_expf_bits_to_double(t);
    const double p = c0 * r + c1;
    const double r2 = r * r;
    double y = c2 * r + 1.0;
    y = p * r2 + y;
    y = y * s;
    float res = (float)y;
    res = x < -0x1.9fe368p6f ? 0.0f : res;
    res = x > 0x1.62e42ep6f ? __builtin_inff() : res;
    return x != x ? x + x : res;
}

#ifdef __HIPCC__
/* sdy_expf with the table in a register instead of memory: lane i of `tab` holds dword i of
 * sdy_exp2_32_tab (sdy_expf_tab_lane loads it, with the kernel's other loads) and the lookup is two
 * lane reads, so no memory round trip follows the argument. Every lane of the wave must be active. */
__device__ static inline uint32_t sdy_expf_tab_lane(int lane) {
    return reinterpret_cast<const uint32_t *>(sdy_exp2_32_tab)[lane & 63];
}

__device__ static inline float sdy_expf_reg(float x, uint32_t tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = sdy_expf_double_to_bits(kd);
    kd -= shift;
    const double r = SDY_EXPF_FMA(inv_ln2_n, xd, -kd);
    const int i = (int)(ki % 32);
    const uint32_t lo = (uint32_t)__shfl((int)tab, 2 * i), hi = (uint32_t)__shfl((int)tab, 2 * i + 1);
    const uint64_t t = (((uint64_t)hi << 32) | lo) + (ki << 47);
    const double s = sdy_expf_bits_to_double(t);
    const double p = c0 * r + c1;
    const double r2 = r * r;
    double y = c2 * r + 1.0;
    y = p * r2 + y;
    y = y * s;
    float res = (float)y;
    res = x < -0x1.9fe368p6f ? 0.0f : res;
    res = x > 0x1.62e42ep6f ? __builtin_inff() : res;
    return x != x ? x + x : res;
}
#endif

#endif
