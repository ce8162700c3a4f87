// gg_exp64.h — the float64 exponential of the sampled draw.
//
// The sampler's softmax (internal/engine/sampling.go:112-136) calls math.Exp in float64.
// A platform exp may differ in the last bit between host and device, so the library
// carries its own: the method of fdlibm's e_exp.c (Sun Microsystems, 1993), which Go's
// portable math.Exp (exp.go) also follows:
//   k = int(x*log2e -+ 0.5) (truncated), hi = x - k*ln2hi, lo = k*ln2lo, r = hi - lo,
//   c = r - r^2*(P1 + r^2*(P2 + ... P5)), y = 1 - ((lo - r*c/(2-c)) - hi), e^x = y*2^k.
// Every operation rounds on its own (no fused multiply-add), the division is IEEE, and
// the scaling by 2^k rounds once (ldexp), so the host C build and the gfx950 build give
// the same bits. Within 1 ulp of glibc's exp.
#pragma once

#ifdef __HIPCC__
#define GG_HD64 __host__ __device__ __forceinline__
#else
#include <math.h>
#define GG_HD64 static inline
#endif

GG_HD64 double gg_exp64(double x) {
#ifdef __clang__
#pragma clang fp contract(off)
#endif
    const double ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10;
    const double log2e = 1.44269504088896338700e+00;
    const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03,
                 P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06,
                 P5 = 4.13813679705723846039e-08;
    if (x != x) return x;                                      // NaN
    if (x > 7.09782712893383973096e+02) return __builtin_inf();  // includes +inf
    if (x < -7.45133219101941108420e+02) return 0.0;           // includes -inf
    if (-3.7252902984619141e-09 < x && x < 3.7252902984619141e-09) return 1.0 + x;  // |x| < 2^-28
    int k = 0;
    if (x < 0) k = (int)(log2e * x - 0.5);
    else if (x > 0) k = (int)(log2e * x + 0.5);
    const double kd = (double)k;
    const double hi = x - kd * ln2hi;
    const double lo = kd * ln2lo;
    const double r = hi - lo;
    const double t = r * r;
    const double c = r - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
    const double y = 1.0 - ((lo - (r * c) / (2.0 - c)) - hi);
    return __builtin_ldexp(y, k);
}

// A cheaper float64 exponential for sums that only need to be close: x = k ln2 + r with
// fused reductions, the degree-11 Taylor polynomial of e^r in Horner form (|r| <= 0.3466,
// truncation below 7e-15) and 2^k. Within 2e-14 relative of gg_exp64 on [-745, 0]
// (tests/test_sampler_oracle.py); 0 below -745.2 and for NaN.
GG_HD64 double gg_fast_exp64(double x) {
    if (!(x >= -745.2)) return 0.0;
    const double kd = __builtin_rint(x * 1.4426950408889634);
    double r = __builtin_fma(kd, -6.93147180369123816490e-01, x);
    r = __builtin_fma(kd, -1.90821492927058770002e-10, r);
    double p = 2.5052108385441720e-08;                // 1/11!
    p = __builtin_fma(p, r, 2.7557319223985893e-07);  // 1/10!
    p = __builtin_fma(p, r, 2.7557319223985888e-06);  // 1/9!
    p = __builtin_fma(p, r, 2.4801587301587302e-05);  // 1/8!
    p = __builtin_fma(p, r, 1.9841269841269841e-04);  // 1/7!
    p = __builtin_fma(p, r, 1.3888888888888889e-03);  // 1/6!
    p = __builtin_fma(p, r, 8.3333333333333332e-03);  // 1/5!
    p = __builtin_fma(p, r, 4.1666666666666664e-02);  // 1/4!
    p = __builtin_fma(p, r, 1.6666666666666666e-01);  // 1/3!
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(p, (int)kd);
}

// The same, table-driven: x = n ln2/64 + r (|r| <= ln2/128), e^x = 2^(n>>6) * T[n&63] * p(r),
// T[j] = gg_exp64(j ln2 / 64), p the degree-5 Taylor polynomial (truncation below 4e-17).
// About half the operations of gg_fast_exp64; within 2e-14 relative of gg_exp64 on
// [-745, 0] (tests/test_sampler_oracle.py). 0 below -745.2 and for NaN.
// T[j] = gg_exp64(j * (ln2 / 64)) for j = 0..63, as literals (printed by gg_exp64 itself;
// tests/test_sampler_oracle.py checks them bit for bit), so a kernel reads the table instead
// of computing it.
#define GG_EXP64_TAB64 \
    0x1p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0, \
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92dep+0, \
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0, \
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0, \
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0, \
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cdp+0, \
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0, \
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5584p+0, 0x1.6623882552224p+0, \
    0x1.6a09e667f3bccp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c8p+0, \
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce12p+0, 0x1.868d99b4492ecp+0, \
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e4fp+0, \
    0x1.9c49182a3f09p+0, 0x1.a0c667b5de564p+0, 0x1.a5503b23e255cp+0, 0x1.a9e6b5579fdcp+0, \
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0, \
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897bp+0, \
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0, \
    0x1.ea4afa2a490d9p+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4541p+0, 0x1.fa7c1819e90d8p+0
GG_HD64 void gg_exp64_table(double* tab) {
    const double t[64] = {GG_EXP64_TAB64};
    for (int j = 0; j < 64; ++j) tab[j] = t[j];
}
GG_HD64 double gg_fast_exp64_tab(double x, const double* tab) {
    if (!(x >= -745.2)) return 0.0;
    const double nd = __builtin_rint(x * (64.0 * 1.4426950408889634));
    double r = __builtin_fma(nd, -6.93147180369123816490e-01 / 64.0, x);
    r = __builtin_fma(nd, -1.90821492927058770002e-10 / 64.0, r);
    const int n = (int)nd;
    double p = 8.3333333333333332e-03;               // 1/5!
    p = __builtin_fma(p, r, 4.1666666666666664e-02);  // 1/4!
    p = __builtin_fma(p, r, 1.6666666666666666e-01);  // 1/3!
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(tab[n & 63] * p, n >> 6);
}
