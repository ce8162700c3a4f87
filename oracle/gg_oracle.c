/*
 * gg_oracle.c — CPU oracle of the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker / the timed
 * CPU baseline; the product path never calls it.
 *
 * Each function restates the reference behaviour it cites, with plain loops and no
 * cleverness, so that it can be checked by reading. The reference (Go + CUDA) cannot
 * be built in this image (no Go toolchain, no nvcc), so nothing here is compiled
 * from it.
 *
 * Parity pins (see tests/test_oracle.py):
 *   ora_argmax / ora_verify / ora_ngram_draft / softmax / top-p / categorical:
 *       the reference's Go known-answer tests (speculative_test.go, sampling_test.go)
 *       plus brute force on tiny inputs.
 *   ora_fp8_encode: exhaustive nearest-value search, cross-checked against
 *       torch.float8_e4m3fn casts.
 *   ora_attention: torch scaled_dot_product_attention in float64 with an explicit
 *       causal mask, closed forms (one key -> V, equal keys -> mean of V).
 *   ora_expf_fixed: error bound against libm exp (<= 2 ulp on the domain used).
 *   ora_accept_rejection: invariants (one-hot q with p==q -> always accept; q==p ->
 *       accept; distribution of the output token over many uniforms equals p).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ floats */

float ora_bf16_decode(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float ora_f16_decode(uint16_t h) {
    int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400), e - 25);
    return s ? -v : v;
}

/* Round a float to the nearest fp16 value (ties to even), returned as float. */
float ora_f16_round(float x) {
    if (isnan(x) || isinf(x) || x == 0.f) return x;
    int e;
    float f = frexpf(x, &e); /* x = f * 2^e, |f| in [0.5, 1) */
    float r;
    if (e - 1 < -14) r = ldexpf(nearbyintf(ldexpf(x, 24)), -24); /* subnormal step 2^-24 */
    else r = ldexpf(nearbyintf(ldexpf(f, 11)), e - 11);
    if (fabsf(r) > 65504.f) r = copysignf(INFINITY, x);
    return r;
}

/* OCP E4M3 (fn): bias 7, S.1111.111 = NaN, max finite 448. */
float ora_fp8_decode(uint8_t b) {
    int s = b >> 7, e = (b >> 3) & 0xf, m = b & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* Nearest finite E4M3 value, ties to the even code (last mantissa bit 0),
 * saturating at +-448 (the __NV_SATFINITE rule of kernels/gollmgo_model.cu:254):
 * an exhaustive search over the 127 non-negative finite codes. */
uint8_t ora_fp8_encode(float x) {
    if (isnan(x)) return (uint8_t)(signbit(x) ? 0xFF : 0x7F);
    uint8_t sign = signbit(x) ? 0x80 : 0;
    double a = fabs((double)x);
    int best = 0;
    double best_d = INFINITY;
    for (int c = 0; c <= 0x7E; ++c) {
        double v = ora_fp8_decode((uint8_t)c);
        double d = fabs(v - a);
        if (d < best_d || (d == best_d && (c & 1) == 0)) {
            best_d = d;
            best = c;
        }
    }
    return (uint8_t)(sign | best);
}

/* Symmetric int8: round half to even, clamp to +-127 (kernels/gollmgo_model.cu:258-268). */
int8_t ora_int8_encode(float x) {
    if (isnan(x)) return 0;
    float r = nearbyintf(x); /* default rounding mode: to nearest, ties to even */
    if (r > 127.f) r = 127.f;
    if (r < -127.f) r = -127.f;
    return (int8_t)r;
}

/* ------------------------------------------------------------ Go sampler */

/* sampling.go:75-85: first index of the maximum, scanning with `>`. */
int ora_argmax(const float* x, int n) {
    int best = 0;
    float bv = x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] > bv) {
            bv = x[i];
            best = i;
        }
    }
    return best;
}

/* speculative.go:68-84 exactly: rows[nrows][V]. corrected = -1 when every draft is
 * accepted and no extra row is given. */
void ora_verify(const int32_t* drafts, int nd, const float* rows, int nrows, int V, int* accepted,
                int* corrected) {
    for (int i = 0; i < nd; ++i) {
        if (i >= nrows) break;
        int c = ora_argmax(rows + (size_t)i * V, V);
        if (c != drafts[i]) {
            *accepted = i;
            *corrected = c;
            return;
        }
    }
    *accepted = nd;
    *corrected = nrows > nd ? ora_argmax(rows + (size_t)nd * V, V) : -1;
}

/* emitSpeculative (serving.go:514-566) with a greedy sampler: Verify over the K
 * draft rows, then the corrected token, or the bonus = argmax of row n. */
void ora_accept_greedy(const float* logits, int B, int K, int V, const int32_t* drafts,
                       const int32_t* n_drafts, int32_t* out_acc, int32_t* out_tok) {
    for (int b = 0; b < B; ++b) {
        int n = n_drafts[b];
        if (n < 0) n = 0;
        if (n > K) n = K;
        const float* rows = logits + (size_t)b * (K + 1) * V;
        int acc, cor;
        ora_verify(drafts + (size_t)b * K, n, rows, n, V, &acc, &cor);
        out_acc[b] = acc;
        out_tok[b] = acc < n ? cor : ora_argmax(rows + (size_t)n * V, V);
    }
}

/* exp in float64 as fdlibm's e_exp.c computes it (Sun Microsystems, 1993), the method of
 * Go's portable math.Exp (exp.go, used where Go has no assembly version): special cases,
 * k = int(x/ln2 -+ 0.5) truncated, r = (x - k*ln2hi) - k*ln2lo, the degree-5 minimax
 * polynomial c(r) and 1 - ((lo - r*c/(2-c)) - hi) scaled by 2^k (ldexp rounds once). Every
 * operation is rounded on its own (the library is built with -ffp-contract=off), as Go
 * evaluates the expression on amd64. */
double ora_exp64(double x) {
    const double ln2hi = 6.93147180369123816490e-01, ln2lo = 1.90821492927058770002e-10;
    const double log2e = 1.44269504088896338700e+00;
    const double P1 = 1.66666666666666019037e-01, P2 = -2.77777777770155933842e-03,
                 P3 = 6.61375632143793436117e-05, P4 = -1.65339022054652515390e-06,
                 P5 = 4.13813679705723846039e-08;
    if (isnan(x) || (isinf(x) && x > 0)) return x;
    if (isinf(x)) return 0.0;
    if (x > 7.09782712893383973096e+02) return INFINITY;
    if (x < -7.45133219101941108420e+02) return 0.0;
    if (-3.7252902984619141e-09 < x && x < 3.7252902984619141e-09) return 1.0 + x; /* |x| < 2^-28 */
    int k = 0;
    if (x < 0) k = (int)(log2e * x - 0.5);
    else if (x > 0) k = (int)(log2e * x + 0.5);
    const double hi = x - (double)k * ln2hi;
    const double lo = (double)k * ln2lo;
    const double r = hi - lo;
    const double t = r * r;
    const double c = r - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
    const double y = 1.0 - ((lo - (r * c) / (2.0 - c)) - hi);
    return ldexp(y, k);
}

/* softmax (sampling.go:112-136) in float64: max by a `>` scan from element 0, -inf -> 0,
 * the sum in index order, the division only when the sum is > 0. */
void ora_softmax_f64(const double* in, int n, double* out) {
    double mx = in[0];
    for (int i = 1; i < n; ++i)
        if (in[i] > mx) mx = in[i];
    double sum = 0;
    for (int i = 0; i < n; ++i) {
        if (isinf(in[i]) && in[i] < 0) out[i] = 0;
        else {
            out[i] = ora_exp64(in[i] - mx);
            sum += out[i];
        }
    }
    if (sum > 0)
        for (int i = 0; i < n; ++i) out[i] /= sum;
}

typedef struct {
    int idx;
    double v;
} ora_iv;

/* The order of the reference's sort.Slice(... a.v > b.v) (sampling.go:97-99,148-150) with
 * what it leaves open fixed: equal values (-0 == +0) by lower index first, NaN after every
 * number. */
static int cmp_desc_stable(const void* a, const void* b) {
    const ora_iv* x = (const ora_iv*)a;
    const ora_iv* y = (const ora_iv*)b;
    const int xn = isnan(x->v), yn = isnan(y->v);
    if (xn != yn) return xn - yn;
    if (!xn) {
        if (x->v > y->v) return -1;
        if (x->v < y->v) return 1;
    }
    return x->idx - y->idx;
}

/* topKFilter (sampling.go:88-109): the k largest values kept, the rest -inf. */
void ora_top_k_filter_f64(const double* in, int n, int k, double* out) {
    ora_iv* it = (ora_iv*)malloc(sizeof(ora_iv) * (size_t)n);
    for (int i = 0; i < n; ++i) {
        it[i].idx = i;
        it[i].v = in[i];
        out[i] = -INFINITY;
    }
    qsort(it, (size_t)n, sizeof(ora_iv), cmp_desc_stable);
    for (int i = 0; i < k && i < n; ++i) out[it[i].idx] = it[i].v;
    free(it);
}

/* topPFilter (sampling.go:139-173): walk in (prob desc, index asc) order, keep while
 * !(cumulative >= p && cumulative > 0), then renormalise by the index-order sum. */
void ora_top_p_filter_f64(const double* probs, int n, double p, double* out) {
    ora_iv* it = (ora_iv*)malloc(sizeof(ora_iv) * (size_t)n);
    for (int i = 0; i < n; ++i) {
        it[i].idx = i;
        it[i].v = probs[i];
        out[i] = 0;
    }
    qsort(it, (size_t)n, sizeof(ora_iv), cmp_desc_stable);
    double cum = 0;
    for (int k = 0; k < n; ++k) {
        if (cum >= p && cum > 0) break;
        out[it[k].idx] = it[k].v;
        cum += it[k].v;
    }
    double s = 0;
    for (int i = 0; i < n; ++i) s += out[i];
    if (s > 0)
        for (int i = 0; i < n; ++i) out[i] /= s;
    free(it);
}

/* categoricalSample (sampling.go:176-192) with the uniform supplied. */
int ora_categorical_f64(const double* probs, int n, double u) {
    double cum = 0;
    for (int i = 0; i < n; ++i) {
        cum += probs[i];
        if (u < cum) return i;
    }
    for (int i = n - 1; i >= 0; --i)
        if (probs[i] > 0) return i;
    return 0;
}

/* The distribution Sampler.Sample (sampling.go:40-72) hands to categoricalSample, for
 * temperature > 1e-9: scaled = float64(l) * (1/T), topKFilter when 0 < k < n, softmax,
 * topPFilter when 0 < p < 1. out receives n probabilities. */
void ora_sampler_probs_f64(const float* logits, int n, double temperature, int top_k, double top_p,
                           double* out) {
    double* sc = (double*)malloc(sizeof(double) * (size_t)n);
    double* tk = (double*)malloc(sizeof(double) * (size_t)n);
    const double inv_t = 1.0 / temperature;
    for (int i = 0; i < n; ++i) sc[i] = (double)logits[i] * inv_t;
    if (top_k > 0 && top_k < n) {
        ora_top_k_filter_f64(sc, n, top_k, tk);
        memcpy(sc, tk, sizeof(double) * (size_t)n);
    }
    ora_softmax_f64(sc, n, out);
    if (top_p > 0 && top_p < 1.0) {
        ora_top_p_filter_f64(out, n, top_p, tk);
        memcpy(out, tk, sizeof(double) * (size_t)n);
    }
    free(sc);
    free(tk);
}

/* Sampler.Sample (sampling.go:40-72) with the uniform supplied in place of
 * rng.Float64(): temperature <= 1e-9 -> argmax, else the categorical draw over
 * ora_sampler_probs_f64. */
int ora_sample_f64(const float* logits, int n, double temperature, int top_k, double top_p, double u) {
    if (n <= 0) return 0;
    if (temperature <= 1e-9) return ora_argmax(logits, n);
    double* pr = (double*)malloc(sizeof(double) * (size_t)n);
    ora_sampler_probs_f64(logits, n, temperature, top_k, top_p, pr);
    const int t = ora_categorical_f64(pr, n, u);
    free(pr);
    return t;
}

/* gg_accept_greedy_sample's rule: ora_accept_greedy, except that the bonus token (every
 * draft accepted) is Sampler.Sample(row n) with uniforms[b] (serving.go:552-566). */
void ora_accept_greedy_sample(const float* logits, int B, int K, int V, const int32_t* drafts,
                              const int32_t* n_drafts, double temperature, int top_k, double top_p,
                              const double* uniforms, int32_t* out_acc, int32_t* out_tok, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#else
    (void)threads;
#endif
    for (int b = 0; b < B; ++b) {
        int n = n_drafts[b];
        if (n < 0) n = 0;
        if (n > K) n = K;
        const float* rows = logits + (size_t)b * (K + 1) * V;
        int acc, cor;
        ora_verify(drafts + (size_t)b * K, n, rows, n, V, &acc, &cor);
        out_acc[b] = acc;
        out_tok[b] = acc < n ? cor : ora_sample_f64(rows + (size_t)n * V, V, temperature, top_k, top_p, uniforms[b]);
    }
}

/* emitSpeculative's use of StepOutput.LogitsPerPosition (serving.go:496-570) over ragged
 * rows, as Go slices: sequence b owns counts[b] rows, taken in order from rows / lens.
 * Verify over the first min(count, n) rows; on a rejection the corrected token; on full
 * acceptance Sample(rows[n]) when a row is there, else -1 (no token). n = 0 reduces to
 * the standard path's Sample over the one row. uniforms[b] feeds the sample. */
void ora_emit_positions(int B, int K, const int32_t* drafts, const int32_t* n_drafts,
                        const float* const* rows, const int32_t* lens, const int32_t* counts,
                        double temperature, int top_k, double top_p, const double* uniforms, int32_t* out_acc,
                        int32_t* out_tok) {
    size_t r0 = 0;
    for (int b = 0; b < B; ++b) {
        int n = n_drafts[b];
        if (n < 0) n = 0;
        if (n > K) n = K;
        const int cnt = counts[b];
        const float* const* rw = rows + r0;
        const int32_t* ln = lens + r0;
        r0 += (size_t)cnt;
        const int nv = cnt < n ? cnt : n;
        const int32_t* d = drafts + (size_t)b * K;
        int acc = n, cor = -1;
        for (int i = 0; i < nv; ++i) { /* Verify, speculative.go:68-84 (fewer rows: all accepted) */
            const int c = ora_argmax(rw[i], ln[i]);
            if (c != d[i]) {
                acc = i;
                cor = c;
                break;
            }
        }
        out_acc[b] = acc;
        if (acc < n) out_tok[b] = cor;
        else out_tok[b] = cnt > n ? ora_sample_f64(rw[n], ln[n], temperature, top_k, top_p, uniforms[b]) : -1;
    }
}

/* ------------------------------------------------------------ n-gram drafter */

/* NGramDrafter.Draft (speculative.go:12-62) with an explicit hash map whose
 * entries are overwritten in history order, so the latest occurrence wins. */
typedef struct {
    int32_t key[8];
    int32_t val;
    int used;
} ora_slot;

static uint64_t key_hash(const int32_t* k, int kl) {
    uint64_t h = 1469598103934665603ull;
    for (int i = 0; i < kl; ++i) {
        h ^= (uint32_t)k[i];
        h *= 1099511628211ull;
    }
    return h;
}

int ora_ngram_draft(const int32_t* hist, int len, int n, int max_drafts, int32_t* out) {
    if (n < 2) n = 2;
    if (max_drafts < 1) max_drafts = 4;
    if (n > 9) return -1;
    if (len < n) return 0;
    const int kl = n - 1;
    size_t cap = 16;
    while (cap < (size_t)len * 2 + 16) cap <<= 1;
    ora_slot* tab = (ora_slot*)calloc(cap, sizeof(ora_slot));
    for (int i = 0; i <= len - n; ++i) {
        uint64_t h = key_hash(hist + i, kl) & (cap - 1);
        while (tab[h].used && memcmp(tab[h].key, hist + i, sizeof(int32_t) * kl) != 0) h = (h + 1) & (cap - 1);
        tab[h].used = 1;
        memcpy(tab[h].key, hist + i, sizeof(int32_t) * kl);
        tab[h].val = hist[i + kl];
    }
    int32_t suffix[8];
    memcpy(suffix, hist + len - kl, sizeof(int32_t) * kl);
    int cnt = 0;
    while (cnt < max_drafts) {
        uint64_t h = key_hash(suffix, kl) & (cap - 1);
        int found = 0;
        while (tab[h].used) {
            if (memcmp(tab[h].key, suffix, sizeof(int32_t) * kl) == 0) {
                found = 1;
                break;
            }
            h = (h + 1) & (cap - 1);
        }
        if (!found) break;
        int32_t next = tab[h].val;
        out[cnt++] = next;
        memmove(suffix, suffix + 1, sizeof(int32_t) * (kl - 1));
        suffix[kl - 1] = next;
    }
    free(tab);
    return cnt;
}

/* ------------------------------------------------- fixed-point acceptance */

/* The acceptance rule's exponential: Cody-Waite reduction with ln2 = hi + lo and
 * the degree-7 Taylor polynomial of e^r, every step an fmaf (correctly rounded). */
float ora_expf_fixed(float x) {
    if (!(x >= -80.0f)) return 0.0f;
    if (x > 0.0f) x = 0.0f;
    float kf = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
    float r = fmaf(kf, -0.693145751953125f, x);
    r = fmaf(kf, -1.42860682030941723212e-6f, r);
    float p = 1.98412698412698412698e-4f;
    p = fmaf(p, r, 1.38888888888888888889e-3f);
    p = fmaf(p, r, 8.33333333333333333333e-3f);
    p = fmaf(p, r, 4.16666666666666666667e-2f);
    p = fmaf(p, r, 1.66666666666666666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return p * ldexpf(1.0f, (int)kf);
}

uint64_t ora_weight(float l, float m, float inv_t) {
    float x = (l - m) * inv_t;
    float e = ora_expf_fixed(x);
    return (uint64_t)floorf(e * 34359738368.0f); /* 2^35 */
}

typedef struct {
    int idx;
    float l;
} ora_il;

static int cmp_logit_desc(const void* a, const void* b) {
    const ora_il* x = (const ora_il*)a;
    const ora_il* y = (const ora_il*)b;
    if (x->l > y->l) return -1;
    if (x->l < y->l) return 1;
    return x->idx - y->idx;
}

/* Exact 128-bit weights. A row is cut into segments of ORA_SEG logits (the device's
 * segment size). Logit i of segment s weighs
 *     W_i = e_i * f_s,   e_i = weight(l_i, m_s),   f_s = weight(m_s, m)
 * with m_s the segment's max finite logit, m the row's, and weight(l, a) =
 * floor(exp_gg((l - a) / T) * 2^35) (ora_weight). Both factors need only one maximum
 * each, so a device reads every logit once; W_i / Z equals the softmax probability to
 * within the exp's ~4e-7 relative error. Sums are exact 128-bit integers; conversions
 * to double are written out over 32-bit pieces below, identical on host and device
 * (gollmgo_amd/csrc/gg_fixed_exp.h states the same rule). */
#define ORA_SEG 8192
typedef unsigned __int128 u128;
static double u128_to_double(u128 x) {
    double d = (double)(uint32_t)(x >> 96) * 4294967296.0 + (double)(uint32_t)(x >> 64);
    d = d * 4294967296.0 + (double)(uint32_t)(x >> 32);
    return d * 4294967296.0 + (double)(uint32_t)x;
}
/* floor(d) for 0 <= d < 2^128 (0 for d <= 0 or NaN). */
static u128 u128_floor(double d) {
    if (!(d > 0.0)) return 0;
    const double hd = floor(d / 18446744073709551616.0);
    const double ld = d - hd * 18446744073709551616.0;
    return ((u128)(uint64_t)hd << 64) | (u128)(uint64_t)ld;
}
/* A draft probability as the rule uses it: finite and in (0, 1], anything else 0. */
static double clean_q(float q) {
    if (!(q > 0.0f) || !isfinite(q)) return 0.0;
    return q > 1.0f ? 1.0 : (double)q;
}

/* Nucleus-filtered weights of one row: w_out[i] (0 outside the nucleus), returns Zp.
 * When e_out / f_out are given they receive e_i (0 outside the nucleus) and f_s. */
static u128 row_weights_ef(const float* row, int V, float inv_t, float top_p, u128* w_out, ora_il* scratch,
                           uint64_t* e_out, uint64_t* f_out) {
    const int nseg = (V + ORA_SEG - 1) / ORA_SEG;
    float* ms = (float*)malloc(sizeof(float) * (size_t)nseg);
    float m = -INFINITY;
    for (int s = 0; s < nseg; ++s) {
        ms[s] = -INFINITY;
        for (int i = s * ORA_SEG; i < V && i < (s + 1) * ORA_SEG; ++i)
            if (isfinite(row[i]) && row[i] > ms[s]) ms[s] = row[i];
        if (ms[s] > m) m = ms[s];
    }
    if (!isfinite(m)) {
        memset(w_out, 0, sizeof(u128) * (size_t)V);
        if (e_out) memset(e_out, 0, sizeof(uint64_t) * (size_t)V);
        if (f_out) memset(f_out, 0, sizeof(uint64_t) * (size_t)nseg);
        free(ms);
        return 0;
    }
    if (f_out)
        for (int s = 0; s < nseg; ++s) f_out[s] = isfinite(ms[s]) ? ora_weight(ms[s], m, inv_t) : 0;
    u128 z = 0;
    int nf = 0;
    for (int i = 0; i < V; ++i) {
        const int s = i / ORA_SEG;
        w_out[i] = 0;
        if (e_out) e_out[i] = 0;
        if (isfinite(row[i])) {
            const uint64_t f = ora_weight(ms[s], m, inv_t);
            const uint64_t e = ora_weight(row[i], ms[s], inv_t);
            w_out[i] = (u128)e * f;
            if (e_out) e_out[i] = e;
            scratch[nf].idx = i;
            scratch[nf].l = row[i] == 0.0f ? 0.0f : row[i];
            ++nf;
        }
        z += w_out[i];
    }
    free(ms);
    if (!(top_p > 0.f && top_p < 1.f) || z == 0) return z;
    /* topPFilter: walk in (logit desc, index asc) order; keep while the mass before
     * the item is below p (cumulative >= p && cumulative > 0 stops the walk). */
    const u128 tp = u128_floor(ceil((double)top_p * u128_to_double(z)));
    qsort(scratch, (size_t)nf, sizeof(ora_il), cmp_logit_desc);
    u128 cum = 0;
    int k = 0;
    for (; k < nf; ++k) {
        if (cum >= tp && cum > 0) break;
        cum += w_out[scratch[k].idx];
    }
    for (; k < nf; ++k) {
        w_out[scratch[k].idx] = 0;
        if (e_out) e_out[scratch[k].idx] = 0;
    }
    return cum;
}
static u128 row_weights(const float* row, int V, float inv_t, float top_p, u128* w_out, ora_il* scratch) {
    return row_weights_ef(row, V, inv_t, top_p, w_out, scratch, NULL, NULL);
}

/* The final draw of the rejection acceptance in float64, with Sampler's rules: p =
 * ora_sampler_probs_f64(row) (temperature, top-p; sampling.go:57-71). Plain (x < 0): the
 * categorical draw over p, i.e. Sampler.Sample. Residual after the rejected draft x:
 * r_i = p_i - q_i where p_i > q_i, for i != x (q_i = clean_q of the draft distribution,
 * 0 without one: a one-hot q puts its mass on x alone), normalised by its index-order sum;
 * a zero sum falls back to p without x, normalised, and that being zero too, to p. */
int ora_final_draw_f64(const float* row, int V, double temperature, int top_k, double top_p, int x,
                       const float* qrow, double u) {
    double* p = (double*)malloc(sizeof(double) * (size_t)V);
    double* r = (double*)malloc(sizeof(double) * (size_t)V);
    ora_sampler_probs_f64(row, V, temperature, top_k, top_p, p);
    const double* dist = p;
    if (x >= 0) {
        double s = 0;
        for (int i = 0; i < V; ++i) {
            const double q = qrow ? clean_q(qrow[i]) : 0.0;
            r[i] = (i != x && p[i] > q) ? p[i] - q : 0.0;
        }
        for (int i = 0; i < V; ++i) s += r[i];
        if (!(s > 0)) {
            s = 0;
            for (int i = 0; i < V; ++i) r[i] = i != x ? p[i] : 0.0;
            for (int i = 0; i < V; ++i) s += r[i];
        }
        if (s > 0) {
            for (int i = 0; i < V; ++i) r[i] /= s;
            dist = r;
        }
    }
    const int t = ora_categorical_f64(dist, V, u);
    free(p);
    free(r);
    return t;
}

/* Speculative sampling (Leviathan et al. 2023, Alg. 1). The acceptance tests use the exact
 * fixed-point weights W:
 *   accept draft j iff u_j * q_j(x_j) * Zp_j < W_j(x_j)   (doubles, left to right;
 *     q as clean_q; W and Zp through u128_to_double; q one-hot at the draft when no draft
 *     distribution is given);
 * the token is drawn in float64 by ora_final_draw_f64 with uniforms[b][K]: after the
 * first rejection at row a, the residual of row a against q_a without the rejected draft;
 * when every draft passes, the bonus from row n (Sampler.Sample).
 * logits [B][K+1][V] (fp32 values), dprobs [B][K][V] or NULL (one-hot q),
 * uniforms [B][K+1] (element K drives the final draw). */
void ora_accept_rejection(const float* logits, int B, int K, int V, const float* dprobs,
                          const int32_t* drafts, const int32_t* n_drafts, const float* uniforms,
                          float temperature, float top_p, int32_t* out_acc, int32_t* out_tok) {
    const float inv_t = 1.0f / temperature;
    u128* w = (u128*)malloc(sizeof(u128) * (size_t)V);
    ora_il* scratch = (ora_il*)malloc(sizeof(ora_il) * (size_t)V);
    for (int b = 0; b < B; ++b) {
        int n = n_drafts[b];
        if (n < 0) n = 0;
        if (n > K) n = K;
        const float* lg = logits + (size_t)b * (K + 1) * V;
        int a = n;
        for (int j = 0; j < n; ++j) {
            const u128 zp = row_weights(lg + (size_t)j * V, V, inv_t, top_p, w, scratch);
            int x = drafts[(size_t)b * K + j];
            int ok = 0;
            if (x >= 0 && x < V) {
                double q = dprobs ? clean_q(dprobs[((size_t)b * K + j) * V + x]) : 1.0;
                double u = (double)uniforms[(size_t)b * (K + 1) + j];
                ok = u * q * u128_to_double(zp) < u128_to_double(w[x]);
            }
            if (!ok) {
                a = j;
                break;
            }
        }
        const int x = a < n ? drafts[(size_t)b * K + a] : -1;
        const float* qrow = (a < n && dprobs) ? dprobs + ((size_t)b * K + a) * V : NULL;
        out_acc[b] = a;
        out_tok[b] = ora_final_draw_f64(lg + (size_t)a * V, V, (double)temperature, 0, (double)top_p, x, qrow,
                                        (double)uniforms[(size_t)b * (K + 1) + K]);
    }
    free(w);
    free(scratch);
}

/* The exact weights of one row as float64 values W_i / 2^70 (tests read the
 * distribution through this; Zp is returned the same way). */
double ora_row_weights_f64(const float* row, int V, float temperature, float top_p, double* out) {
    u128* w = (u128*)malloc(sizeof(u128) * (size_t)V);
    ora_il* scratch = (ora_il*)malloc(sizeof(ora_il) * (size_t)V);
    const u128 zp = row_weights(row, V, 1.0f / temperature, top_p, w, scratch);
    for (int i = 0; i < V; ++i) out[i] = u128_to_double(w[i]) / 1180591620717411303424.0; /* 2^70 */
    free(w);
    free(scratch);
    return u128_to_double(zp) / 1180591620717411303424.0;
}

/* ------------------------------------------------------------- KV cache */

/* Pool element access for the block layouts
 *   K[blk][Hkv][bs][D], V[blk][Hkv][D][bs]; dtype codes as gg_dtype_t
 *   (0 f32, 1 f16, 2 bf16, 3 fp8-e4m3, 4 int8). */
static size_t k_off(int blk, int h, int o, int d, int H, int bs, int D) {
    return (((size_t)blk * H + h) * bs + o) * D + d;
}
static size_t v_off(int blk, int h, int o, int d, int H, int bs, int D) {
    return (((size_t)blk * H + h) * D + d) * bs + o;
}
static float raw_elem(const uint8_t* p, int dt, size_t i) {
    switch (dt) {
        case 0: {
            float f;
            memcpy(&f, p + 4 * i, 4);
            return f;
        }
        case 1: {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            return ora_f16_decode(h);
        }
        case 2: {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            return ora_bf16_decode(h);
        }
        case 3: return ora_fp8_decode(p[i]);
        case 4: return (float)(int8_t)p[i];
    }
    return 0.f;
}

/* Quantised append for 1-byte pools (the float pools are written with numpy casts
 * by the Python side). Mirrors the rules stated in gg_verify.h:
 *   fp8 (dt 3): q = E4M3_sat(x * inv_scale[h]) with inv_scale = 1/scale (fp32);
 *   int8 (dt 4): per block b and head h, new scale = max(old, fp16(amax(new rows)/127))
 *     where old = 0 if the block's first new row sits at offset 0; existing tokens are
 *     re-quantised as int8(q_old * old * (1/new)) when the scale changes.
 * rows: k,v [n][H][D] fp32; f16 scales are held as float values here. */
void ora_kv_append_q(uint8_t* kc, uint8_t* vc, int dt, int H, int D, int bs, const float* k,
                     const float* v, const int32_t* slots, int n, const float* k_inv,
                     const float* v_inv, float* k_bscale, float* v_bscale) {
    if (dt == 3) {
        for (int r = 0; r < n; ++r) {
            if (slots[r] < 0) continue;
            int blk = slots[r] / bs, o = slots[r] % bs;
            for (int h = 0; h < H; ++h)
                for (int d = 0; d < D; ++d) {
                    size_t s = ((size_t)r * H + h) * D + d;
                    kc[k_off(blk, h, o, d, H, bs, D)] = ora_fp8_encode(k[s] * k_inv[h]);
                    vc[v_off(blk, h, o, d, H, bs, D)] = ora_fp8_encode(v[s] * v_inv[h]);
                }
        }
        return;
    }
    /* int8 per block: process runs of adjacent rows in the same block (skipped rows, slot
     * < 0, may sit inside a run and are passed over). */
    int r = 0;
    while (r < n) {
        if (slots[r] < 0) {
            ++r;
            continue;
        }
        int blk = slots[r] / bs;
        int e = r;
        while (e < n && (slots[e] < 0 || slots[e] / bs == blk)) ++e;
        int lead_off = slots[r] % bs;
        for (int h = 0; h < H; ++h) {
            for (int which = 0; which < 2; ++which) {
                const float* src = which ? v : k;
                uint8_t* pool = which ? vc : kc;
                float* sc = which ? v_bscale : k_bscale;
                float am = 0.f;
                for (int rr = r; rr < e; ++rr)
                    for (int d = 0; d < D && slots[rr] >= 0; ++d) {
                        float a = fabsf(src[((size_t)rr * H + h) * D + d]);
                        if (a == a && a > am) am = a;
                    }
                float old_s = lead_off == 0 ? 0.f : sc[(size_t)blk * H + h];
                float cand = ora_f16_round(am / 127.0f);
                float new_s = cand > old_s ? cand : old_s;
                float inv = new_s > 0.f ? 1.0f / new_s : 0.f;
                if (new_s != old_s)
                    for (int o = 0; o < lead_off; ++o)
                        for (int d = 0; d < D; ++d) {
                            size_t i = which ? v_off(blk, h, o, d, H, bs, D) : k_off(blk, h, o, d, H, bs, D);
                            pool[i] = (uint8_t)ora_int8_encode(((float)(int8_t)pool[i] * old_s) * inv);
                        }
                for (int rr = r; rr < e; ++rr) {
                    if (slots[rr] < 0) continue;
                    int o = slots[rr] % bs;
                    for (int d = 0; d < D; ++d) {
                        size_t i = which ? v_off(blk, h, o, d, H, bs, D) : k_off(blk, h, o, d, H, bs, D);
                        pool[i] = (uint8_t)ora_int8_encode(src[((size_t)rr * H + h) * D + d] * inv);
                    }
                }
                sc[(size_t)blk * H + h] = new_s;
            }
        }
        r = e;
    }
}

/* Textbook softmax attention in float64 for the verify rows
 * (kernels/gollmgo_paged_attn.cu:38-119 per row; causal rule of
 * kernels/gollmgo_ops.cu:178 across the R rows of a sequence).
 *   q [B][R][Hq][D] fp32 values; out [B][R][Hq][D] fp32.
 *   kc/vc pools of dtype dt; k_scale/v_scale: per-head [H] (dt 3) or per-block
 *   [blocks][H] (dt 4) as floats, NULL otherwise.
 *   row_counts may be NULL (all R). Rows j >= row_counts[b] are left untouched.
 *   Boundary semantics of gg_verify_attention (no reference counterpart: the
 *   reference trusts its slot tables): ctx_lens are clamped to [0, max_blocks*bs];
 *   a sequence with no rows or with more rows than keys is left untouched; keys whose
 *   block id is outside [0, num_blocks) take no part in the softmax. */
void ora_attention(const float* q, float* out, const uint8_t* kc, const uint8_t* vc, int dt, int H,
                   int D, int bs, const float* k_scale, const float* v_scale, const int32_t* ctx_lens,
                   const int32_t* row_counts, const int32_t* block_tables, int max_blocks, int B, int R,
                   int Hq, float scale, int threads, int num_blocks) {
    const int G = Hq / H;
    /* One work item per (sequence, row, query head), so that a single long sequence
     * still spreads over every thread. */
    const long items = (long)B * R * Hq;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#else
    (void)threads;
#endif
    for (long w = 0; w < items; ++w) {
        const int b = (int)(w / ((long)R * Hq)), j = (int)((w / Hq) % R), hq = (int)(w % Hq);
        int ctx = ctx_lens[b];
        if (ctx < 0) ctx = 0;
        if (ctx > max_blocks * bs) ctx = max_blocks * bs;
        const int nr = row_counts ? row_counts[b] : R;
        if (nr <= 0 || nr > ctx || j >= nr) continue;
        double* sc = (double*)malloc(sizeof(double) * (size_t)(ctx > 0 ? ctx : 1));
        double* acc = (double*)malloc(sizeof(double) * (size_t)D);
        {
            const int pos = ctx - nr + j;
            {
                const int h = hq / G;
                const float* qv = q + (((size_t)b * R + j) * Hq + hq) * D;
                double mx = -INFINITY;
                for (int t = 0; t <= pos; ++t) {
                    int blk = block_tables[(size_t)b * max_blocks + t / bs], o = t % bs;
                    if (blk < 0 || blk >= num_blocks) {
                        sc[t] = -INFINITY;
                        continue;
                    }
                    double ks = dt == 3 ? k_scale[h] : dt == 4 ? k_scale[(size_t)blk * H + h] : 1.0;
                    double dot = 0;
                    for (int d = 0; d < D; ++d)
                        dot += (double)qv[d] * (double)raw_elem(kc, dt, k_off(blk, h, o, d, H, bs, D));
                    sc[t] = dot * ks * (double)scale;
                    if (sc[t] > mx) mx = sc[t];
                }
                double sum = 0;
                for (int t = 0; t <= pos; ++t) {
                    sc[t] = mx == -INFINITY ? 0.0 : exp(sc[t] - mx);
                    sum += sc[t];
                }
                for (int d = 0; d < D; ++d) acc[d] = 0;
                for (int t = 0; t <= pos; ++t) {
                    int blk = block_tables[(size_t)b * max_blocks + t / bs], o = t % bs;
                    if (blk < 0 || blk >= num_blocks) continue;
                    double vs = dt == 3 ? v_scale[h] : dt == 4 ? v_scale[(size_t)blk * H + h] : 1.0;
                    double p = sum > 0 ? sc[t] / sum * vs : 0.0;
                    for (int d = 0; d < D; ++d)
                        acc[d] += p * (double)raw_elem(vc, dt, v_off(blk, h, o, d, H, bs, D));
                }
                float* ov = out + (((size_t)b * R + j) * Hq + hq) * D;
                for (int d = 0; d < D; ++d) ov[d] = (float)acc[d];
            }
        }
        free(sc);
        free(acc);
    }
}

/* The reference's v1 paged attention (kernels/gollmgo_paged_attn.cu:38-119) in fp32, as a
 * host loop: per (sequence, verify row, query head) the dot products over the visible keys
 * in fp32 (q * k, summed over d in order, then * scale), the max, expf(s - max) summed in
 * key order, a reciprocal of the sum, and the fp32 weighted sum of V. Causal rows, block
 * tables and the fp8 / int8 scales as ora_attention. This is the CPU baseline bench.py
 * times (the reference semantics at the reference's precision); ora_attention, in fp64, is
 * the checker. */
void ora_attention_ref_f32(const float* q, float* out, const uint8_t* kc, const uint8_t* vc, int dt, int H,
                           int D, int bs, const float* k_scale, const float* v_scale, const int32_t* ctx_lens,
                           const int32_t* row_counts, const int32_t* block_tables, int max_blocks, int B, int R,
                           int Hq, float scale, int threads, int num_blocks) {
    const int G = Hq / H;
    const long items = (long)B * R * Hq;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#else
    (void)threads;
#endif
    for (long w = 0; w < items; ++w) {
        const int b = (int)(w / ((long)R * Hq)), j = (int)((w / Hq) % R), hq = (int)(w % Hq);
        int ctx = ctx_lens[b];
        if (ctx < 0) ctx = 0;
        if (ctx > max_blocks * bs) ctx = max_blocks * bs;
        const int nr = row_counts ? row_counts[b] : R;
        if (nr <= 0 || nr > ctx || j >= nr) continue;
        const int pos = ctx - nr + j, n = pos + 1, h = hq / G;
        float* sc = (float*)malloc(sizeof(float) * (size_t)n);
        const float* qv = q + (((size_t)b * R + j) * Hq + hq) * D;
        float mx = -1e30f;
        for (int t = 0; t < n; ++t) {
            const int blk = block_tables[(size_t)b * max_blocks + t / bs], o = t % bs;
            if (blk < 0 || blk >= num_blocks) {
                sc[t] = -INFINITY;
                continue;
            }
            const float ks = dt == 3 ? k_scale[h] : dt == 4 ? k_scale[(size_t)blk * H + h] : 1.0f;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qv[d] * (raw_elem(kc, dt, k_off(blk, h, o, d, H, bs, D)) * ks);
            sc[t] = dot * scale;
            if (sc[t] > mx) mx = sc[t];
        }
        float sum = 0.0f;
        for (int t = 0; t < n; ++t) {
            sc[t] = expf(sc[t] - mx);
            sum += sc[t];
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int t = 0; t < n; ++t) sc[t] *= inv;
        float* ov = out + (((size_t)b * R + j) * Hq + hq) * D;
        for (int d = 0; d < D; ++d) {
            float acc = 0.0f;
            for (int t = 0; t < n; ++t) {
                if (sc[t] == 0.0f) continue;
                const int blk = block_tables[(size_t)b * max_blocks + t / bs], o = t % bs;
                const float vs = dt == 3 ? v_scale[h] : dt == 4 ? v_scale[(size_t)blk * H + h] : 1.0f;
                acc += sc[t] * (raw_elem(vc, dt, v_off(blk, h, o, d, H, bs, D)) * vs);
            }
            ov[d] = acc;
        }
        free(sc);
    }
}

/* ------------------------------------------------------- array helpers */

void ora_fp8_encode_n(const float* x, uint8_t* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = ora_fp8_encode(x[i]);
}
void ora_fp8_decode_n(const uint8_t* x, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = ora_fp8_decode(x[i]);
}
void ora_int8_encode_n(const float* x, int8_t* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = ora_int8_encode(x[i]);
}
void ora_f16_round_n(const float* x, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = ora_f16_round(x[i]);
}
void ora_exp64_n(const double* x, double* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = ora_exp64(x[i]);
}
void ora_expf_fixed_n(const float* x, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = ora_expf_fixed(x[i]);
}
/* Greedy/rejection/n-gram over a batch, timed as the CPU baseline. */
void ora_ngram_draft_batch(const int32_t* hist, int stride, const int32_t* lens, int B, int n, int K,
                           int32_t* out, int32_t* out_n, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#else
    (void)threads;
#endif
    for (int b = 0; b < B; ++b) {
        int c = ora_ngram_draft(hist + (size_t)b * stride, lens[b], n, K, out + (size_t)b * (K < 1 ? 4 : K));
        out_n[b] = c < 0 ? 0 : c;
    }
}
