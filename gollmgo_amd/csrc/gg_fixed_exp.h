// gg_fixed_exp.h — the exponential and fixed-point weights used by rejection acceptance.
//
// Decisions must be bit-identical wherever the acceptance rule is evaluated, so
// the library does not call a platform exp: exp is computed with Cody–Waite range
// reduction (x = k*ln2 + r, ln2 split into a short high part and a low part) and
// the degree-7 Taylor polynomial of e^r on |r| <= ln2/2, every step an explicit
// fmaf, a correctly rounded IEEE operation on every conforming host and on AMD
// GPUs. Weights are w = floor(e * 2^35) as exact integers, so sums and prefix sums
// do not depend on summation order; vocabularies up to 2^18 keep every sum
// below 2^53, so conversions to double are exact too.
#pragma once

#ifdef __HIPCC__
#define GG_HD __host__ __device__ __forceinline__
#else
#define GG_HD static inline
#endif


// Fixed-point weight w = floor(e^x * 2^35) of logit l given the row max m and 1/T, x =
// (l - m)/T (callers pass x <= 0; x > 0 counts as 0), returned as a float holding that
// integer exactly. e^x is p * 2^k with k in [-116, 0] and p from the polynomial below;
// w = floor(p * 2^(k+35)), the power-of-two scaling exact. Below x = -80 the weight is
// 0 (e^-80 * 2^35 < 2^-80), which clamping x to -80 also gives, so there is no branch or
// select on the result (a NaN x is clamped too). w < 2^36, so sums of up to 2^17 weights
// are exact in double.
GG_HD float gg_weight_f(float l, float m, float inv_t) {
    const float y = (l - m) * inv_t;
    const float x = __builtin_fminf(y >= -80.0f ? y : -80.0f, 0.0f);  // (the compare maps NaN to -80)
    const float kf = __builtin_floorf(__builtin_fmaf(x, 1.44269504088896341f, 0.5f));
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.42860682030941723212e-6f, r);
    float p = 1.98412698412698412698e-4f;               // 1/5040
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f); // 1/720
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f); // 1/120
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f); // 1/24
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f); // 1/6
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = (int)kf;  // in [-116, 0]
    union {
        unsigned int u;
        float f;
    } s;
    s.u = (unsigned int)(k + 127 + 35) << 23;
    return __builtin_floorf(p * s.f);  // floor(e^x * 2^35)
}
// The same weight as a 64-bit integer: two 32-bit conversions, the high word
// floor(w * 2^-32) (at most 15) and the low word w - hi * 2^32 (exact in float: w has 24
// significant bits and is at least hi * 2^32).
GG_HD unsigned long long gg_weight_u64(float w) {
    const float hf = __builtin_floorf(w * 2.3283064365386963e-10f);  // 2^-32
    const unsigned int hi = (unsigned int)hf;
    const unsigned int lo = (unsigned int)__builtin_fmaf(hf, -4294967296.0f, w);
    return ((unsigned long long)hi << 32) | lo;
}
GG_HD unsigned long long gg_weight(float l, float m, float inv_t) { return gg_weight_u64(gg_weight_f(l, m, inv_t)); }
// Monotone order key of a finite logit (larger logit -> larger key; -0 == +0).
GG_HD unsigned int gg_order_key(float l) {
    union {
        float f;
        unsigned int u;
    } v;
    v.f = (l == 0.0f) ? 0.0f : l;
    return (v.u & 0x80000000u) ? ~v.u : (v.u | 0x80000000u);
}

// Coarse nucleus bin: 1/64-nat slices of (m - l)/T, monotone non-increasing in l.
GG_HD int gg_coarse_bin(float l, float m, float inv_t) {
    const float y = -((l - m) * inv_t) * 64.0f;
    return y >= 2047.0f ? 2047 : (int)y;
}

// ---- Exact 128-bit weights (segment-relative) ----
//
// A row is cut into segments of GG_ACCEPT_SEG logits. Logit i of segment s weighs
//     W_i = e_i * f_s,  e_i = gg_weight(l_i, m_s, 1/T),  f_s = gg_weight(m_s, m, 1/T)
// with m_s the segment's max finite logit and m the row's: both factors need only one
// maximum each, so the logits are read once, and every sum is an exact 128-bit
// integer (order-free). Doubles enter only through the two conversions below, written
// out so that host and device round identically.
#define GG_ACCEPT_SEG 8192
typedef unsigned __int128 gg_u128;

// ((x3 * 2^32 + x2) * 2^32 + x1) * 2^32 + x0 over the four 32-bit pieces, each step a
// double operation (the pieces and the power-of-two products are exact).
GG_HD double gg_u128_to_double(gg_u128 x) {
    double d = (double)(unsigned int)(x >> 96) * 4294967296.0 + (double)(unsigned int)(x >> 64);
    d = d * 4294967296.0 + (double)(unsigned int)(x >> 32);
    return d * 4294967296.0 + (double)(unsigned int)x;
}
// floor(d) for 0 <= d < 2^128; 0 for d <= 0 or NaN. Each 32-bit piece is split off with
// exact operations (power-of-two scalings, floors and the subtraction of a value that
// shares d's leading bits), so only 32-bit conversions are needed.
GG_HD gg_u128 gg_u128_floor(double d) {
    if (!(d > 0.0)) return 0;
    const double p32 = 4294967296.0, i32 = 1.0 / 4294967296.0;
    const double hd = __builtin_floor(d * (i32 * i32));
    const double ld = d - hd * (p32 * p32);
    const double hh = __builtin_floor(hd * i32), hl = hd - hh * p32;
    const double lh = __builtin_floor(ld * i32), ll = ld - lh * p32;
    const unsigned long long hi = ((unsigned long long)(unsigned int)hh << 32) | (unsigned int)hl;
    const unsigned long long lo = ((unsigned long long)(unsigned int)lh << 32) | (unsigned int)ll;
    return ((gg_u128)hi << 64) | lo;
}
// A draft probability as the acceptance rule uses it: finite and in (0, 1], else 0.
GG_HD double gg_clean_q(float q) {
    if (!(q > 0.0f) || !(q <= 3.402823466e38f)) return 0.0;
    return q > 1.0f ? 1.0 : (double)q;
}
