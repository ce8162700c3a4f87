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
GG_HD64 void gg_exp64_table(double* tab) {
    for (int j = 0; j < 64; ++j) tab[j] = gg_exp64((double)j * (6.93147180559945286227e-01 / 64.0));
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
