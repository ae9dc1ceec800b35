// dev_exp.h -- the host C library's expf on the device (softmax tails of the
// attention kernels).
#ifndef DPUF_DEV_EXP_H
#define DPUF_DEV_EXP_H

#include "dev_common.h"

// exp for x <= 0 with the results of the host C library's expf, which the
// reference calls on the scalar tail of its softmax (dpuf_engine.c:423-426).
// Method: exp(x) = 2^(k/32) * 2^(r/32), k = round(x*32/ln2), with a 32-entry
// table of 2^(i/32) and a cubic polynomial evaluated in double precision,
// rounded once to float (the exp2f-table method of Szabolcs Nagy used by
// glibc's expf).  The table holds bits(2^(i/32)) - (i << 47), i.e. the
// correctly rounded doubles 2^(i/32) with the exponent contribution removed.
// Checked bit-for-bit against glibc expf over every float in [-104, 0].
static __constant__ uint64_t c_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// tab: the 32 table words (c_exp2_tab, or a copy in LDS: a kernel whose
// tail exponentials sit on its critical path copies the table at entry, so
// the lookup does not wait for a global load).
DEV float expf_libc_tab(float x, const uint64_t* tab) {
    if (x < -0x1.9fe368p6f) return 0.0f;  // below log(2^-150): rounds to +0
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki & 31u] + (ki << 47);
    double sc = __longlong_as_double((long long)t);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * sc;
    return (float)y;
}

DEV float expf_libc(float x) { return expf_libc_tab(x, c_exp2_tab); }

#endif
