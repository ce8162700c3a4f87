// gg_draw.h — the float64 token draw's per-row state, shared by its launches
// (accept_sample.hip) and by the acceptance launches that set a row up themselves
// (accept_rejection.hip: its decide kernel knows the drawn row, so no launch of its own).
#pragma once
#include "gg_common.h"

namespace gg {
namespace fd {

constexpr int kBins = 4096;       // coarse bins: 1/64-nat slices below the row max (bin_of)

enum : int { ST_NONE = 0, ST_DRAW = 1, ST_EXACT = 2 };

struct RowInfo {
    double m;                 // max scaled logit of the drawn row
    unsigned long long cut;   // kept <=> comp_key >= cut (0 keeps every element)
    double tot;               // the kept e summed (the nucleus mass with top-p)
    int row;                  // row of the sequence drawn from
    int x;                    // residual draw: the rejected draft (excluded); -1: plain draw
    int cbin;                 // the coarse bin the gather launch collects (-1: none); with a
                              // range hint the highest bin of the range
    int cbin_lo;              // the lowest bin gathered (cbin but for a range hint)
    int need;                 // top-k: how many of that bin's elements the filter keeps
    double above;             // histogram mass of the bins above cbin (top-p without top-k)
    double S;                 // top-p without top-k: the row's e summed
    int kept_pass;            // the kept launch computes the draw's segment sums
    int pregather;            // cbin known before the pass (a hint), which gathers it
    unsigned long long hint;  // the hinted cut element's key (comp_key order), or 0
    double Sest;              // dense residual without filters: the caller's estimate of the
                              // row's e sum (0: none), see split_residual
};

// Everything the draw launches share (passed by value).
struct DrawParams {
    const void* logits;       // [B][K+1][V]
    gg_dtype_t dt;
    int B, K, V, nseg;
    double inv_t;
    int top_k;
    double top_p;
    int use_k, use_p, filtered;
    int hint_mode;            // top-p alone with the caller's cut hints: select1 / gather not launched
    int kept_launched;        // the kept launch runs (a row that needs it otherwise goes exact)
    int vec;                  // rows allow 16-byte loads
    int vec_q;                // so do the draft distributions' rows
    double tau;
    const double* ud;         // uniform of sequence b: ud[b], or else
    const float* uf;          //   uf[b * (K + 1) + K]
    const float* q;           // residual draws: dense draft distributions [B][K][V], or null
    int* state;
    RowInfo* info;
    uint32_t* hcnt;
    double* hmass;
    double* segsum;
    double* segkept;
    double* segabove;         // per segment: e summed over the bins above cbin
    double* segep;            // per segment (estimated residuals): e of the sure-positive elements
    double* segqp;            //   and their q
    int* ncand;               // per sequence: elements of cbin gathered
    unsigned long long* cand; // per sequence: kCap gathered keys
    int32_t* out_tok;
};

__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Coarse bin of a logit: 1/64-nat slices of its distance below the row max, x = (m - l/T)
// * 64, the highest bin holding the max; everything more than (kBins - 1)/64 nats below
// (and -inf, NaN) in bin 0. Monotone in the value, and a bin holds a few hundred of a
// 128k-entry row where a nucleus cut falls (a 1/8-octave slice of the value holds thousands).
// Elements below bin c have e <= gg_exp64(-(kBins - c) / 64) exactly: x is 64 * fl(m - v)
// and e = gg_exp64(-fl(m - v)), with gg_exp64 monotone.
// bin_of_scaled takes the scaled value v = l / T itself (clamped to the top bin above m).
__device__ __forceinline__ int bin_of_scaled(double v, double m) {
    const double x = (m - v) * 64.0;
    if (!(x >= 0.0)) return x < 0.0 ? kBins - 1 : 0;
    return x < (double)(kBins - 1) ? kBins - 1 - (int)x : 0;
}
__device__ __forceinline__ int bin_of(float l, double inv_t, double m) {
    const double x = (m - (double)l * inv_t) * 64.0;
    return x < (double)(kBins - 1) ? kBins - 1 - (int)x : 0;
}

// A residual draw against a dense q without filters, with the caller's estimate S~ of the
// row's e sum S: |S - S~| <= kSestTol * S~ (the fixed-point total of the rejection
// acceptance; its exponential, the float32 arguments and the truncations stay within
// about 1e-5). The residual of element i is max(0, e_i / S - q_i); it is e_i/S - q_i for
// sure when e_i > q_i * S~ (1 + kSestTol) and 0 for sure when e_i < q_i * S~ (1 - kSestTol).
// So the pass sums e and q of the sure-positive elements per segment, lists the few in
// between (their p and q nearly tie), and the draw forms each segment's residual mass as
// E+/S - Q+ plus the listed elements' own residuals, with S from the pass. More listed
// elements than a list holds (a draft distribution close to p): the kept launch computes
// the sums from S instead.
constexpr double kSestTol = 1e-4;
__device__ __forceinline__ bool split_residual(const DrawParams& P, const RowInfo& ri) {
    return ri.x >= 0 && P.q && !P.filtered && ri.Sest > 0.0;
}

// One sequence's draw set up (by one thread, after the acceptance decided it): row `row` of
// sequence b (-1: no draw), residual after draft x (-1: plain), mx the row's max logit and
// any whether it has a finite one, hint the caller's cut element (0: none), sest the
// caller's estimate of the row's e sum (0: none). Without a cut element, vlo < vhi hints
// the cut by a range of scaled values l / T instead: the pass gathers the bins from
// bin_of_scaled(vlo) to bin_of_scaled(vhi). Either hint only steers where the draw looks:
// when the cut is not among the gathered elements, the select finds no cut that clears
// its margins and the row takes the literal rule.
__device__ inline void prep_row(const DrawParams& P, int b, int row, int x, float mx, bool any,
                                unsigned long long hint, double sest, int force_exact, double vlo = 0.0,
                                double vhi = 0.0) {
    if (row < 0) {
        P.state[b] = ST_NONE;
        return;
    }
    const double m = (double)mx * P.inv_t;
    int st = ST_DRAW;
    // No finite maximum (all -inf / NaN, or +inf present), or a non-finite scale:
    // the literal rule decides.
    if (!any || !(mx > -INFINITY && mx < INFINITY) || !(m > -INFINITY && m < INFINITY) || force_exact)
        st |= ST_EXACT;
    // Hint mode launches no select1 / gather: a row without a hint (the caller's
    // nucleus kept every finite logit, or was not computed) takes the literal rule.
    const bool range = hint == 0 && vhi > vlo;
    if (P.hint_mode && hint == 0 && !range) st |= ST_EXACT;
    RowInfo ri;
    ri.m = m;
    ri.cut = 0;
    ri.tot = 0.0;
    ri.row = row;
    ri.x = x;
    ri.cbin = -1;
    ri.cbin_lo = -1;
    ri.need = 0;
    ri.above = 0.0;
    ri.S = 0.0;
    // Without filters only a dense residual needs the kept launch's sums, and with an
    // estimate of S only when the pass lists too many near-ties.
    ri.Sest = sest;
    ri.kept_pass = !P.filtered && P.q && x >= 0 && !(ri.Sest > 0.0);
    if (ri.kept_pass && !P.kept_launched) st |= ST_EXACT;
    ri.pregather = hint != 0 || range;
    ri.hint = hint;
    if (split_residual(P, ri)) P.ncand[b] = 0;
    if (hint != 0) {
        ri.cbin = ri.cbin_lo = bin_of(key_value((uint32_t)(hint >> 32)), P.inv_t, m);
        P.ncand[b] = 0;
    } else if (range) {
        ri.cbin = bin_of_scaled(vhi, m);
        ri.cbin_lo = bin_of_scaled(vlo, m);
        P.ncand[b] = 0;
    }
    P.info[b] = ri;
    P.state[b] = st;
}

// The launches' shared parameters for a call (workspace views included).
DrawParams final_draw_params(const FinalDraw& d, void* ws);

}  // namespace fd
}  // namespace gg
