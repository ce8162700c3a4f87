// accept_sample.hip — the float64 token draw of the acceptance, as the reference samples.
//
// The reference's emitSpeculative (internal/engine/serving.go:514-566) runs the greedy
// Verify over the draft rows, then, when every draft was accepted, draws the bonus token
// with Sampler.Sample(posLogits[K]) (internal/engine/sampling.go:40-72): temperature,
// top-k, softmax, top-p and a categorical draw, all in float64. This file adds that draw
// to the greedy acceptance (accept_greedy.hip), with the uniform supplied in place of
// rng.Float64(). The rejection acceptance (accept_rejection.hip) uses the same draw for its
// final token: the bonus as above, or after a rejected draft x the residual
// max(0, p - q) over tokens other than x, normalised, p being Sampler's distribution of
// that row and q the draft distribution (one-hot at x for a deterministic drafter).
//
// The draw must give the token the float64 sequential rule gives, for every uniform. The
// rule's sums run in index order (or in sorted order for top-p), one rounding per term, so
// they are inherently sequential. Two paths:
//   fast  : every quantity in float64 with parallel sums. A parallel sum differs from the
//           sequential one by at most a few n*2^-53 relative; the fast path takes a decision
//           (the nucleus cut, the drawn index) only when it clears the rule's boundary by
//           more than tau = 8*(V + 4096)*2^-53, a bound on both sums' rounding. Otherwise the
//           row goes to the exact path.
//   exact : one workgroup replays the rule literally: the same float64 operations in the
//           same order (sorted orders by a bitonic sort), every sequential sum in one wave.
//           6-17 ms per row; a row lands here with probability ~1e-4 (rows with NaN or
//           +inf logits always do).
// Orders the reference leaves open (sort.Slice is not stable) are fixed as value desc,
// then index asc, NaN last; exp is gg_exp64 (gg_exp64.h), identical on host and device.
//
// Launches after the acceptance has decided which row of each sequence is drawn from:
//   prep   (B blocks)       : which sequences draw, from which row; the row max from the
//                             acceptance's segment maxima (the rejection acceptance's
//                             decide kernel does this itself, fd::prep_row).
//   pass   (segments x B)   : e_i = exp(l_i/T - m) per element, segment sums, NaN/+inf
//                             check; with top-k or top-p the coarse histograms (count and
//                             mass per 1/64-nat slice below the row max), or, with the
//                             caller's hint of the nucleus cut, the hinted bins' elements
//                             and the mass above them; for a dense residual with an
//                             estimate of its total, the residual's sums.
//   select (B, top-k/p only): from the histograms, the crossing bin (select1) and its
//                             elements (gather), unless hinted; then the top-k threshold
//                             and the nucleus cut in LDS (select2), which draws itself
//                             when no kept launch follows.
//   kept   (segments x B)   : the draw's weight per segment (kept e, or the residual).
//   draw   (B)              : the segment and then the element where u * total falls.
//   exact  (a few blocks)   : the literal rule for the rows flagged on the way.
#include "gg_common.h"
#include "gg_exp64.h"
#include "gg_draw.h"

#pragma clang fp contract(off)

namespace gg {
namespace {

using namespace fd;

constexpr int kSeg = 8192;        // elements per block of the pass and kept launches
constexpr int kSegThreads = 512;
constexpr int kCap = 4096;        // items of one bin the select launch can gather
constexpr int kRowThreads = 1024;
constexpr int kChunk = 4096;      // exact path: bitonic sort entries held in LDS at once
constexpr int kExactSlots = 4;    // exact path: workgroups (each with its own scratch)
constexpr int kGreedySeg = 4096;  // accept_greedy.hip's segment length
constexpr int kNone = 0x7fffffff; // accept_greedy.hip's "no element" index



struct Ent {                  // exact path sort entry, ordered by (hi, lo) descending
    unsigned long long hi, lo;
};

struct Layout {
    size_t state, info, hcnt, hmass, segsum, segkept, segabove, segep, segqp, ncand, cand, exact, total;
    size_t slot_bytes, vpad, npow;
};


__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Layout layout(int B, int V) {
    Layout L{};
    const int nseg = (V + kSeg - 1) / kSeg;
    size_t o = 0;
    L.state = o;   o = align256(o + (size_t)B * sizeof(int));
    L.info = o;    o = align256(o + (size_t)B * sizeof(RowInfo));
    L.hcnt = o;    o = align256(o + (size_t)B * kBins * sizeof(uint32_t));
    L.hmass = o;   o = align256(o + (size_t)B * kBins * sizeof(double));
    L.segsum = o;  o = align256(o + (size_t)B * nseg * sizeof(double));
    L.segkept = o; o = align256(o + (size_t)B * nseg * sizeof(double));
    L.segabove = o; o = align256(o + (size_t)B * nseg * sizeof(double));
    L.segep = o;   o = align256(o + (size_t)B * nseg * sizeof(double));
    L.segqp = o;   o = align256(o + (size_t)B * nseg * sizeof(double));
    L.ncand = o;   o = align256(o + (size_t)B * sizeof(int));
    L.cand = o;    o = align256(o + (size_t)B * kCap * sizeof(unsigned long long));
    L.vpad = ((size_t)V + 63) & ~(size_t)63;
    size_t np = kChunk;
    while (np < (size_t)V) np <<= 1;
    L.npow = np;
    L.slot_bytes = align256(2 * L.vpad * sizeof(double) + np * sizeof(Ent));
    L.exact = o;
    o += (size_t)(B < kExactSlots ? B : kExactSlots) * L.slot_bytes;
    L.total = o;
    return L;
}

// Order key of a float: ascending in value, -0 == +0 (NaN is handled by the callers).
__device__ __forceinline__ uint32_t order_key(float l) {
    const uint32_t u = __float_as_uint(l == 0.0f ? 0.0f : l);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// (value desc, index asc) as one descending 64-bit key; every element's key is > 0.
__device__ __forceinline__ unsigned long long comp_key(uint32_t key, int idx) {
    return ((unsigned long long)key << 32) | (unsigned long long)(uint32_t)(~(uint32_t)idx);
}
__device__ __forceinline__ int comp_index(unsigned long long c) { return (int)(~(uint32_t)c); }


__device__ __forceinline__ int clamp_n(const int32_t* n_drafts, int b, int K) {
    const int n = n_drafts[b];
    return n < 0 ? 0 : (n > K ? K : n);
}

__device__ __forceinline__ double exp_term(float l, double inv_t, double m) {
    if (l == -INFINITY) return 0.0;
    const double v = (double)l * inv_t;
    return gg_exp64(v - m);
}

// The parallel path's exponential (gg_fast_exp64_tab, gg_exp64.h): within 2e-14 relative of
// gg_exp64; the margins count 1e-12. Nothing the rule decides depends on its bits, only sums
// that clear a margin.
constexpr double kFastExpErr = 1e-12;
__device__ __forceinline__ double fast_term(float l, double inv_t, double m, const double* tab) {
    const double v = (double)l * inv_t;
    return gg_fast_exp64_tab(v - m, tab);  // -inf logits give -inf, hence 0
}
// Each block's copy of the exponential's table (64 doubles in LDS).
__constant__ double c_exp_tab[64] = {GG_EXP64_TAB64};
__device__ __forceinline__ void load_exp_table(double* s_tab) {
    if (threadIdx.x < 64) s_tab[threadIdx.x] = c_exp_tab[threadIdx.x];
    __syncthreads();
}

// Eight consecutive elements e0.. of a row as floats: one 16-byte load (two for f32) when
// the row allows it, else element loads (past V: -inf).
template <gg_dtype_t DT>
__device__ __forceinline__ void load8(const void* row, int V, int e0, bool vec, float (&x)[8]) {
    if (vec && e0 + 8 <= V) {
        if constexpr (DT == GG_DTYPE_F32) {
            const uint4 a = *(const uint4*)((const float*)row + e0);
            const uint4 c = *(const uint4*)((const float*)row + e0 + 4);
            const uint32_t w[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = __uint_as_float(w[k]);
        } else {
            const uint4 a = *(const uint4*)((const uint16_t*)row + e0);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint16_t h = (uint16_t)(w[k >> 1] >> ((k & 1) * 16));
                x[k] = DT == GG_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
            }
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = e0 + k < V ? load_as_f32(row, DT, e0 + k) : -INFINITY;
}

// Eight draft probabilities e0.. of a row (0 past V, or with no row).
__device__ __forceinline__ void load8q(const float* qr, int V, int e0, bool vec, float (&y)[8]) {
    if (!qr) {
#pragma unroll
        for (int k = 0; k < 8; ++k) y[k] = 0.0f;
        return;
    }
    if (vec && e0 + 8 <= V) {
        const float4 a = *(const float4*)(qr + e0);
        const float4 c = *(const float4*)(qr + e0 + 4);
        y[0] = a.x; y[1] = a.y; y[2] = a.z; y[3] = a.w;
        y[4] = c.x; y[5] = c.y; y[6] = c.z; y[7] = c.w;
        return;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = e0 + k < V ? qr[e0 + k] : 0.0f;
}

__device__ __forceinline__ const void* drawn_row(const DrawParams& P, int b, int row) {
    return (const uint8_t*)P.logits + ((size_t)b * (P.K + 1) + row) * P.V * dtype_bytes(P.dt);
}
__device__ __forceinline__ double uniform_of(const DrawParams& P, int b) {
    return P.ud ? P.ud[b] : (double)P.uf[(size_t)b * (P.K + 1) + P.K];
}
__device__ __forceinline__ const float* q_row(const DrawParams& P, int b, const RowInfo& ri) {
    return (P.q && ri.x >= 0) ? P.q + ((size_t)b * P.K + ri.row) * P.V : nullptr;
}
// A draft probability as the rule uses it: finite and in (0, 1], anything else 0.
__device__ __forceinline__ double clean_q(float q) {
    if (!(q > 0.0f) || !(q <= 3.402823466e38f)) return 0.0;
    return q > 1.0f ? 1.0 : (double)q;
}
// The draw's weight of element e (logit l): its e if kept (plain draw, e units), or its
// residual max(0, e/tot - q) (probability units; 0 at the rejected draft). inv_tot is
// 1/tot: one more rounding per element, far inside the margins.
__device__ __forceinline__ double draw_weight(const DrawParams& P, const RowInfo& ri, float q, float l,
                                              int e, const double* tab, double inv_tot) {
    if (comp_key(order_key(l), e) < ri.cut) return 0.0;
    const double ev = fast_term(l, P.inv_t, ri.m, tab);
    if (ri.x < 0) return ev;
    if (e == ri.x) return 0.0;
    const double p = ev * inv_tot;
    const double qv = clean_q(q);
    return p > qv ? p - qv : 0.0;
}


// The pass's segment sums added in segment order (the row's e total without filters); every
// kernel that needs it adds them the same way.
__device__ __forceinline__ double seg_total(const DrawParams& P, int b) {
    double t = 0.0;
    for (int s = 0; s < P.nseg; ++s) t += P.segsum[(size_t)b * P.nseg + s];
    return t;
}

__device__ __forceinline__ double lane_val(double x, int l) {
    const int lo = __builtin_amdgcn_readlane(__double2loint(x), l);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(x), l);
    return __hiloint2double(hi, lo);
}

// Block-wide sum (blockDim.x a multiple of 64, at most 1024); every thread gets it.
__device__ double block_sum(double v, double* sh) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    double s = 0;
    for (int i = 0; i < nw; ++i) s += sh[i];
    __syncthreads();
    return s;
}

// Block-wide exclusive scan of one double per thread (in thread order) and the total.
__device__ double block_excl_scan(double v, double* sh, double* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    double inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    __syncthreads();
    if (lane == 63) sh[w] = inc;
    __syncthreads();
    double before = 0, tot = 0;
    for (int i = 0; i < nw; ++i) {
        if (i < w) before += sh[i];
        tot += sh[i];
    }
    double ex = __shfl_up(inc, 1);
    if (lane == 0) ex = 0.0;
    __syncthreads();
    *total = tot;
    return before + ex;
}
__device__ uint32_t block_excl_scan_u32(uint32_t v, uint32_t* sh, uint32_t* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    __syncthreads();
    if (lane == 63) sh[w] = inc;
    __syncthreads();
    uint32_t before = 0, tot = 0;
    for (int i = 0; i < nw; ++i) {
        if (i < w) before += sh[i];
        tot += sh[i];
    }
    __syncthreads();
    *total = tot;
    return before + inc - v;
}

// ------------------------------------------------------------------------ prep

// Sequence b draws from row spec_row[b] (-1: no draw), residual after draft spec_x[b]
// (-1: plain) — or, for the greedy acceptance, from row n when all n drafts were accepted.
// The row max comes from the acceptance's segment maxima: the greedy (value, index) pairs
// of 4096-element segments (gws), or the rejection's finite maxima of 8192-element
// segments (seg_max).
__global__ void __launch_bounds__(256) sample_prep_kernel(
    DrawParams P, const float2* __restrict__ gws, const float* __restrict__ seg_max, int nseg_m,
    const int32_t* __restrict__ n_drafts, const int32_t* __restrict__ acc, const int* __restrict__ spec_row,
    const int* __restrict__ spec_x, const unsigned long long* __restrict__ spec_key,
    const double* __restrict__ spec_s, int force_exact) {
    const int b = blockIdx.x;
    const int K = P.K, R = K + 1;
    int row, x = -1;
    if (gws) {
        const int n = clamp_n(n_drafts, b, K);
        row = acc[b] == n ? n : -1;
    } else {
        row = spec_row[b];
        x = spec_x[b];
    }
    if (row < 0) {
        if (threadIdx.x == 0) P.state[b] = ST_NONE;
        return;
    }
    // top-p alone with a hint of the cut element: the pass gathers its bin itself
    const unsigned long long hint = P.hint_mode ? spec_key[b] : 0ull;
    if (P.filtered && !P.hint_mode)
        for (int i = threadIdx.x; i < kBins; i += blockDim.x) {
            P.hcnt[(size_t)b * kBins + i] = 0;
            P.hmass[(size_t)b * kBins + i] = 0.0;
        }
    if (threadIdx.x < 64) {
        float mx = -INFINITY;
        int any = 0;
        for (int s = threadIdx.x; s < nseg_m; s += 64) {
            if (gws) {
                const float2 p = gws[((size_t)b * R + row) * nseg_m + s];
                if (__float_as_int(p.y) != kNone) {
                    any = 1;
                    mx = fmaxf(mx, p.x);
                }
            } else {
                const float v = seg_max[((size_t)b * R + row) * nseg_m + s];
                if (v > -INFINITY) any = 1;
                mx = fmaxf(mx, v);
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            mx = fmaxf(mx, __shfl_xor(mx, o));
            any |= __shfl_xor(any, o);
        }
        if (threadIdx.x == 0) prep_row(P, b, row, x, mx, any != 0, hint, spec_s && x >= 0 ? spec_s[b] : 0.0, force_exact);
    }
}

// ------------------------------------------------------------------------ pass

// The draw itself, by one block of NT threads: the segment where u * total falls (sums
// per segment of the draw's weights), then the element inside it (kSeg / NT per thread). A plain
// draw's margins are tau * total (e units); a residual's tau * (1 + total) (probability
// units: the parallel p carries up to tau of error summed over the row, whatever q is). A
// residual total within a few margins of 0 may be 0 in the rule, whose fallbacks then
// apply. Undecided: the row is left to the literal rule.
template <gg_dtype_t DT, int NT>
__device__ void draw_in_block(const DrawParams& P, int b, const RowInfo& ri, const double* sums,
                              const double* s_tab) {
    __shared__ double s_red[16];
    __shared__ int s_seg, s_tok, s_bad;
    __shared__ double s_base, s_tot;
    const double tau = P.tau;
    const double u = uniform_of(P, b);
    const int nseg = P.nseg;
    const double inv_tot = 1.0 / ri.tot;
    if (threadIdx.x == 0) {
        double tot = 0.0;
        for (int s = 0; s < nseg; ++s) tot += sums[s];
        const double t = u * tot;
        double run = 0.0;
        int sel = -1;
        for (int s = 0; s < nseg; ++s) {
            if (run + sums[s] > t) {
                sel = s;
                break;
            }
            run += sums[s];
        }
        const double marg = ri.x < 0 ? tau * tot : tau * (1.0 + tot);
        if (ri.x >= 0 && tot <= 8.0 * marg) sel = -1;
        if (!(u >= tau && u < 1.0 - tau)) sel = -1;  // near 0, near or past 1, NaN
        s_seg = sel;
        s_base = run;
        s_tot = tot;
        s_tok = -1;
        s_bad = 0;
    }
    __syncthreads();
    const int seg = s_seg;
    if (seg < 0) {
        if (threadIdx.x == 0) atomicOr(&P.state[b], ST_EXACT);
        return;
    }
    const double tot = s_tot, t = u * tot;
    const double marg = ri.x < 0 ? tau * tot : tau * (1.0 + tot);
    const void* row = drawn_row(P, b, ri.row);
    const float* qr = q_row(P, b, ri);
    constexpr int kPer = kSeg / NT;
    static_assert(kPer == 8 || kPer == 16, "eight or sixteen elements per thread");
    const int e0 = seg * kSeg + threadIdx.x * kPer;
    double ev[kPer];
    double loc = 0.0;
    float xl[kPer / 8][8], ql[kPer / 8][8];
#pragma unroll
    for (int h = 0; h < kPer / 8; ++h) {
        load8<DT>(row, P.V, e0 + 8 * h, P.vec, xl[h]);
        load8q(qr, P.V, e0 + 8 * h, P.vec_q, ql[h]);
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int e = e0 + q;
        ev[q] = e < P.V ? draw_weight(P, ri, ql[q >> 3][q & 7], xl[q >> 3][q & 7], e, s_tab, inv_tot) : 0.0;
        loc += ev[q];
    }
    double btot;
    double run = s_base + block_excl_scan(loc, s_red, &btot);
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const double nx = run + ev[q];
        if (run <= t && nx > t) {
            const bool ok = (t - run) > marg && (nx - t) > marg;
            if (ok) s_tok = e0 + q;
            else s_bad = 1;
        }
        run = nx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (s_tok >= 0 && !s_bad) P.out_tok[b] = s_tok;
        else atomicOr(&P.state[b], ST_EXACT);
    }
}

// Per (segment, sequence): e of every element (the parallel exponential), the segment's
// sum, the NaN / +inf check, and with top-k / top-p the coarse histograms.
// Stage the elements of one coarse bin found by a block in LDS, one counter update per wave.
constexpr int kBlockCap = 2048;  // a segment's hits staged in LDS; more: the row goes exact
__device__ __forceinline__ void stage_hit(bool hit, unsigned long long comp, int* s_cnt, unsigned long long* s_buf) {
    const int lane = threadIdx.x & 63;
    const unsigned long long mask = __ballot(hit);
    if (mask) {
        int base = 0;
        const int leader = __ffsll((long long)mask) - 1;
        if (lane == leader) base = atomicAdd(s_cnt, __popcll(mask));
        base = __shfl(base, leader);
        if (hit) {
            const int slot = base + __popcll(mask & ((1ull << lane) - 1ull));
            if (slot < kBlockCap) s_buf[slot] = comp;
        }
    }
}
// The staged elements appended to the sequence's list (one global update per block; an
// overflow forces the count past kCap, so the row goes exact).
__device__ __forceinline__ void flush_hits(const DrawParams& P, int b, int* s_cnt, int* s_base,
                                           const unsigned long long* s_buf) {
    __syncthreads();
    const int n = *s_cnt;
    if (threadIdx.x == 0 && n > 0) *s_base = atomicAdd(&P.ncand[b], n > kBlockCap ? kCap + 1 : n);
    __syncthreads();
    if (n > 0 && n <= kBlockCap)
        for (int i = threadIdx.x; i < n; i += blockDim.x)
            if (*s_base + i < kCap) P.cand[(size_t)b * kCap + *s_base + i] = s_buf[i];
}

// Per (segment, sequence): e of every element (the parallel exponential), the segment's
// sum, the NaN / +inf check, and with top-k / top-p the coarse histograms — or, when the
// cut's bin is known beforehand, that bin's elements and the sum of e above it.
// kMode: kPassPlain without filters (a split residual's staging at most); kPassHist builds
// the histograms (filters without hints); kPassPre gathers the hinted bin (hint mode, where
// every drawn row has its hint). Only kPassHist holds the 48 KB of histograms: the others
// stage in 16 KB, so four blocks share a CU.
constexpr int kPassPlain = 0, kPassHist = 1, kPassPre = 2;
template <gg_dtype_t DT, int kMode>
__global__ void __launch_bounds__(kSegThreads) sample_pass_kernel(DrawParams P) {
    constexpr bool kHist = kMode == kPassHist;
    const int b = blockIdx.y, seg = blockIdx.x;
    if (P.state[b] != ST_DRAW) return;
    __shared__ uint32_t s_cnt[kHist ? kBins : 1];
    __shared__ double s_mass[kHist ? kBins : 1];
    __shared__ unsigned long long s_stage[kHist ? 1 : kBlockCap];
    __shared__ double s_red[16];
    __shared__ double s_tab[64];
    __shared__ int s_hits, s_base;
    // the staging buffer of a pregather or a split residual
    unsigned long long* s_buf = s_stage;
    load_exp_table(s_tab);
    const RowInfo ri = P.info[b];
    if (kMode == kPassPre && !ri.pregather) {  // hint mode marks rows without a hint exact
        if (threadIdx.x == 0) atomicOr(&P.state[b], ST_EXACT);
        return;
    }
    const bool pre = kMode == kPassPre;
    const bool split = kMode == kPassPlain && split_residual(P, ri);
    const float* qr = split ? q_row(P, b, ri) : nullptr;
    // The bounds in float, widened by 1e-6 for the float rounding of e, q and the products.
    const float shi = (float)(ri.Sest * (1.0 + kSestTol) * (1.0 + 1e-6));
    const float slo = (float)(ri.Sest * (1.0 - kSestTol) * (1.0 - 1e-6));
    const int want_cnt = kHist && P.use_k && !pre, want_mass = kHist && P.filtered && !pre;
    const int V = P.V;
    const double inv_t = P.inv_t;
    const void* row = drawn_row(P, b, ri.row);
    const double m = ri.m;
    if (want_cnt || want_mass) {
        for (int i = threadIdx.x; i < kBins; i += blockDim.x) {
            s_cnt[i] = 0;
            s_mass[i] = 0.0;
        }
    }
    if (threadIdx.x == 0) s_hits = 0;
    __syncthreads();
    double acc = 0.0, above = 0.0, ep = 0.0, qp = 0.0;
    int bad = 0;
    for (int c0 = 0; c0 < kSeg / 8; c0 += blockDim.x) {
        const int e0 = seg * kSeg + (c0 + threadIdx.x) * 8;
        float x[8], y[8];
        load8<DT>(row, V, e0, P.vec, x);
        if (split) load8q(qr, V, e0, P.vec_q, y);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float l = x[k];
            const bool in = e0 + k < V;
            if (in && (l != l || l == INFINITY)) bad = 1;
            const double ev = (!in || l != l || l == INFINITY) ? 0.0 : fast_term(l, inv_t, m, s_tab);
            acc += ev;
            const uint32_t key = order_key(l);
            const int bin = bin_of(l, inv_t, m);
            if (pre) {
                if (in && bin > ri.cbin) above += ev;
                stage_hit(in && bin <= ri.cbin && bin >= ri.cbin_lo, comp_key(key, e0 + k), &s_hits, s_buf);
            } else if (split) {
                const int e = e0 + k;
                const bool cand = in && e != ri.x;
                const float qf = (y[k] > 0.0f && y[k] <= 3.402823466e38f) ? fminf(y[k], 1.0f) : 0.0f;  // clean_q
                const float ef = (float)ev;
                const bool pos = cand && ef > qf * shi;
                const bool amb = cand && !pos && ef != 0.0f && ef >= qf * slo;
                if (pos) {
                    ep += ev;
                    qp += (double)qf;
                }
                if (__any(amb)) stage_hit(amb, (unsigned long long)e, &s_hits, s_buf);
            } else if ((want_cnt || want_mass) && in) {
                if (want_cnt) atomicAdd(&s_cnt[bin], 1u);
                if (want_mass && ev != 0.0) atomicAdd(&s_mass[bin], ev);
            }
        }
    }
    if (__syncthreads_or(bad)) {
        if (threadIdx.x == 0) atomicOr(&P.state[b], ST_EXACT);
        return;
    }
    const double tot = block_sum(acc, s_red);
    if (threadIdx.x == 0) P.segsum[(size_t)b * P.nseg + seg] = tot;
    if (split) {
        const double E = block_sum(ep, s_red), Q = block_sum(qp, s_red);
        if (threadIdx.x == 0) {
            P.segep[(size_t)b * P.nseg + seg] = E;
            P.segqp[(size_t)b * P.nseg + seg] = Q;
        }
        flush_hits(P, b, &s_hits, &s_base, s_buf);
        return;
    }
    if (pre) {
        const double ab = block_sum(above, s_red);
        if (threadIdx.x == 0) P.segabove[(size_t)b * P.nseg + seg] = ab;
        flush_hits(P, b, &s_hits, &s_base, s_buf);
        return;
    }
    if (want_cnt || want_mass) {
        for (int i = threadIdx.x; i < kBins; i += blockDim.x) {
            if (want_cnt && s_cnt[i]) atomicAdd(&P.hcnt[(size_t)b * kBins + i], s_cnt[i]);
            if (want_mass && s_mass[i] != 0.0) unsafeAtomicAdd(&P.hmass[(size_t)b * kBins + i], s_mass[i]);
        }
    }
}

// ---------------------------------------------------------------------- select

// Gather the elements of the row whose order key falls in bin `bin` into s_comp (in no
// particular order) and their e into s_e. Returns the count, or -1 when the bin holds more
// than kCap elements.
template <gg_dtype_t DT>
__device__ int gather_bin(const void* row, int V, bool vec, int bin, double inv_t, double m,
                          unsigned long long* s_comp, double* s_e, int* s_n) {
    if (threadIdx.x == 0) *s_n = 0;
    __syncthreads();
    const int nch = (V + 7) / 8;
    const int lane = threadIdx.x & 63;
    for (int c0 = threadIdx.x; c0 - (int)threadIdx.x < nch; c0 += 4 * blockDim.x) {
        float x[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = c0 + u * blockDim.x;
            if (c < nch) load8<DT>(row, V, c * 8, vec, x[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = c0 + u * blockDim.x;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int e = c * 8 + k;
                const uint32_t key = c < nch ? order_key(x[u][k]) : 0u;
                const bool hit = c < nch && e < V && bin_of(x[u][k], inv_t, m) == bin;
                // one LDS atomic per wave: the wave's hits take consecutive slots
                const unsigned long long mask = __ballot(hit);
                if (mask) {
                    int base = 0;
                    const int leader = __ffsll((long long)mask) - 1;
                    if (lane == leader) base = atomicAdd(s_n, __popcll(mask));
                    base = __shfl(base, leader);
                    if (hit) {
                        const int slot = base + __popcll(mask & ((1ull << lane) - 1ull));
                        if (slot < kCap) s_comp[slot] = comp_key(key, e);
                    }
                }
            }
        }
    }
    __syncthreads();
    const int ng = *s_n;
    __syncthreads();
    if (ng > kCap) return -1;
    for (int i = threadIdx.x; i < ng; i += blockDim.x)
        s_e[i] = exp_term(key_value((uint32_t)(s_comp[i] >> 32)), inv_t, m);
    __syncthreads();
    return ng;
}

// Among the ng gathered items (unique 64-bit keys, unordered), the first in descending key
// order whose running total (of e with by_mass, else of 1) reaches `target`: a radix
// descent in 8-bit digits over the key bits below the highest one in which the items
// differ (from their minimum and maximum), each digit a 256-entry LDS histogram and a scan
// from the top digit. Returns the item's position in the list (-1 if the total stays below
// target) and, through before, the total of the items above it. The items are left in place.
__device__ int select_desc(const unsigned long long* s_comp, const double* s_e, int ng, double target, bool by_mass,
                           double* before, double* s_h, double* s_red, int* s_i) {
    __shared__ unsigned long long s_lo[16], s_hi[16];
    unsigned long long lo = ~0ull, hi = 0;
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
        const unsigned long long c = s_comp[i];
        lo = c < lo ? c : lo;
        hi = c > hi ? c : hi;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long a = __shfl_xor(lo, o), c = __shfl_xor(hi, o);
        lo = a < lo ? a : lo;
        hi = c > hi ? c : hi;
    }
    if ((threadIdx.x & 63) == 0) {
        s_lo[threadIdx.x >> 6] = lo;
        s_hi[threadIdx.x >> 6] = hi;
    }
    __syncthreads();
    lo = ~0ull;
    hi = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
        lo = s_lo[w] < lo ? s_lo[w] : lo;
        hi = s_hi[w] > hi ? s_hi[w] : hi;
    }
    const unsigned long long diff = lo ^ hi;
    int nbits = diff ? 64 - __clzll((long long)diff) : 0;  // the items share every bit above these
    nbits = nbits < 8 ? 8 : nbits;
    unsigned long long pmask = nbits >= 64 ? 0ull : ~((1ull << nbits) - 1ull);
    unsigned long long prefix = hi & pmask;
    double above = 0.0;
    // items per digit: once the chosen digit holds one item, that item is the answer
    __shared__ int s_hc[256];
    __shared__ int s_one;
    for (int shift = nbits - 8; shift > -8; shift -= 8) {
        const int sh = shift < 0 ? 0 : shift;
        const int width = shift < 0 ? 8 + shift : 8;
        const unsigned long long dmask = ((1ull << width) - 1ull) << sh;
        for (int i = threadIdx.x; i < 256; i += blockDim.x) {
            s_h[i] = 0.0;
            s_hc[i] = 0;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < ng; i += blockDim.x) {
            const unsigned long long c = s_comp[i];
            if ((c & pmask) == prefix) {
                const int d = (int)((c & dmask) >> sh);
                atomicAdd(&s_h[d], by_mass ? s_e[i] : 1.0);
                atomicAdd(&s_hc[d], 1);
            }
        }
        __syncthreads();
        // digits from the top: thread t < 256 holds digit 255 - t
        const int t = threadIdx.x;
        const double hv = t < 256 ? s_h[255 - t] : 0.0;
        double tot;
        const double ex = block_excl_scan(hv, s_red, &tot);
        if (t == 0) *s_i = -1;
        __syncthreads();
        // rounding may let two neighbouring digits both claim the crossing: the first in
        // order (the larger digit) wins, and only its thread writes the total above it
        const bool claim = t < 256 && hv > 0.0 && above + ex < target && above + ex + hv >= target;
        if (claim) atomicMax(s_i, 255 - t);
        __syncthreads();
        if (claim && *s_i == 255 - t) {
            s_h[256] = above + ex;
            s_one = s_hc[255 - t] == 1;
        }
        __syncthreads();
        const int dgt = *s_i;
        if (dgt < 0) {  // rounding between the histogram and the target: the caller's margin fails
            __syncthreads();
            return -1;
        }
        above = s_h[256];
        prefix |= (unsigned long long)dgt << sh;
        pmask |= dmask;
        const bool one = s_one;
        __syncthreads();
        if (one) break;
    }
    // prefix now names exactly one item (the keys are unique; or the digit held one)
    if (threadIdx.x == 0) *s_i = -1;
    __syncthreads();
    for (int i = threadIdx.x; i < ng; i += blockDim.x)
        if ((s_comp[i] & pmask) == prefix) *s_i = i;
    __syncthreads();
    const int r = *s_i;
    __syncthreads();
    *before = above;
    return r;
}

// The largest gathered key below `c` (0 if none): the next item in descending order.
__device__ unsigned long long next_below(const unsigned long long* s_comp, int ng, unsigned long long c,
                                         unsigned long long* s_u) {
    unsigned long long best = 0;
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
        const unsigned long long v = s_comp[i];
        if (v < c && v > best) best = v;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long v = __shfl_xor(best, o);
        if (v > best) best = v;
    }
    if ((threadIdx.x & 63) == 0) s_u[threadIdx.x >> 6] = best;
    __syncthreads();
    unsigned long long r = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w)
        if (s_u[w] > r) r = s_u[w];
    __syncthreads();
    return r;
}

// The caller's hinted cut among the gathered items: the lowest key with the hint's order key
// that is >= the hint (the ties the hint keeps), i.e. the hint itself, or the last tie when
// the hint keeps them all. If the rule's condition holds for it (the mass above it below
// `target`, with it at least `target`), returns its position and, through before, the mass
// above it; otherwise -1 and the radix descent decides.
__device__ int hint_cut(const unsigned long long* s_comp, const double* s_e, int ng, unsigned long long h,
                        double target, double* before, double* s_red, unsigned long long* s_u, int* s_i) {
    unsigned long long best = ~0ull;
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
        const unsigned long long v = s_comp[i];
        if ((v >> 32) == (h >> 32) && v >= h && v < best) best = v;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long v = __shfl_xor(best, o);
        if (v < best) best = v;
    }
    if ((threadIdx.x & 63) == 0) s_u[threadIdx.x >> 6] = best;
    if (threadIdx.x == 0) *s_i = -1;
    __syncthreads();
    unsigned long long c = ~0ull;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w)
        if (s_u[w] < c) c = s_u[w];
    if (c == ~0ull) {  // the same for every thread
        __syncthreads();
        return -1;
    }
    double a = 0.0;
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
        const unsigned long long v = s_comp[i];
        if (v > c) a += s_e[i];
        else if (v == c) *s_i = i;
    }
    const double A = block_sum(a, s_red);  // its barriers publish s_i
    const int ci = *s_i;
    __syncthreads();
    if (ci < 0 || !(A < target && A + s_e[ci] >= target)) return -1;
    *before = A;
    return ci;
}

// Select, first part (one block per sequence, with filters and no hints): from the coarse
// histograms, the bin the gather launch collects — the top-k threshold bin, or without
// top-k the nucleus cut's bin and the histogram mass above it.
__global__ void __launch_bounds__(kRowThreads) sample_select1_kernel(DrawParams P) {
    const int b = blockIdx.x;
    if (P.state[b] != ST_DRAW) return;
    __shared__ double s_red[16];
    __shared__ uint32_t s_redu[16];
    __shared__ int s_bin;
    __shared__ double s_above;
    __shared__ uint32_t s_cabove;
    const int per = kBins / kRowThreads;  // bins per thread, positions counted from the top bin
    const int nseg = P.nseg;
    RowInfo* info = P.info;
    if (threadIdx.x == 0) P.ncand[b] = 0;
    if (P.use_k) {
        // The bin where the count from the top first reaches k.
        uint32_t c = 0;
        for (int q = 0; q < per; ++q) c += P.hcnt[(size_t)b * kBins + (kBins - 1 - (threadIdx.x * per + q))];
        uint32_t tot;
        const uint32_t before = block_excl_scan_u32(c, s_redu, &tot);
        if (threadIdx.x == 0) s_bin = -1;
        __syncthreads();
        if (before < (uint32_t)P.top_k && before + c >= (uint32_t)P.top_k) {
            uint32_t run = before;
            for (int q = 0; q < per; ++q) {
                const int bin = kBins - 1 - (threadIdx.x * per + q);
                const uint32_t cq = P.hcnt[(size_t)b * kBins + bin];
                if (run + cq >= (uint32_t)P.top_k) {
                    s_bin = bin;
                    s_cabove = run;
                    break;
                }
                run += cq;
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            if (s_bin < 0) atomicOr(&P.state[b], ST_EXACT);  // fewer counted elements than k
            info[b].cbin = info[b].cbin_lo = s_bin;
            info[b].need = P.top_k - (int)s_cabove;
        }
        return;
    }
    // top-p alone: the bin where the mass from the top first reaches p * S.
    double sv = 0.0;
    for (int i = threadIdx.x; i < nseg; i += blockDim.x) sv += P.segsum[(size_t)b * nseg + i];
    const double S = block_sum(sv, s_red);
    const double pS = P.top_p * S;
    double c = 0.0;
    for (int q = 0; q < per; ++q) c += P.hmass[(size_t)b * kBins + kBins - 1 - (threadIdx.x * per + q)];
    double tot;
    const double before = block_excl_scan(c, s_red, &tot);
    // Rounding can let two neighbouring threads both see the crossing; the first in order
    // wins (atomicMax on the bin) and only its owner writes the mass above it.
    if (threadIdx.x == 0) s_bin = -1;
    __syncthreads();
    double run = before;
    int mine = -1;
    double mine_above = 0.0;
    if (before < pS && before + c >= pS) {
        for (int q = 0; q < per; ++q) {
            const int bin = kBins - 1 - (threadIdx.x * per + q);
            const double mq = P.hmass[(size_t)b * kBins + bin];
            if (run + mq >= pS) {
                mine = bin;
                mine_above = run;
                break;
            }
            run += mq;
        }
        if (mine >= 0) atomicMax(&s_bin, mine);
    }
    __syncthreads();
    if (mine >= 0 && mine == s_bin) s_above = mine_above;
    __syncthreads();
    if (threadIdx.x == 0) {
        if (s_bin < 0) atomicOr(&P.state[b], ST_EXACT);  // p * S at the very end: rounding decides
        info[b].cbin = info[b].cbin_lo = s_bin;
        info[b].above = s_above;
        info[b].S = S;
    }
}

// Gather (per segment and sequence): the elements of bin cbin appended to the sequence's
// list (one counter update per wave), and the e of the elements above that bin summed
// per segment.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) sample_gather_kernel(DrawParams P) {
    const int b = blockIdx.y, seg = blockIdx.x;
    if (P.state[b] != ST_DRAW) return;
    const RowInfo ri = P.info[b];
    if (ri.cbin < 0 || ri.pregather) return;
    __shared__ double s_red[16];
    __shared__ unsigned long long s_buf[kBlockCap];
    __shared__ int s_cnt, s_base;
    __shared__ double s_tab[64];
    load_exp_table(s_tab);
    const void* row = drawn_row(P, b, ri.row);
    if (threadIdx.x == 0) s_cnt = 0;
    __syncthreads();
    double acc = 0.0;
    for (int c0 = 0; c0 < kSeg / 8; c0 += blockDim.x) {
        const int e0 = seg * kSeg + (c0 + threadIdx.x) * 8;
        float x[8];
        load8<DT>(row, P.V, e0, P.vec, x);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int e = e0 + k;
            const uint32_t key = order_key(x[k]);
            const int bin = bin_of(x[k], P.inv_t, ri.m);
            const bool in = e < P.V;
            if (in && bin > ri.cbin) acc += fast_term(x[k], P.inv_t, ri.m, s_tab);
            stage_hit(in && bin == ri.cbin, comp_key(key, e), &s_cnt, s_buf);
        }
    }
    flush_hits(P, b, &s_cnt, &s_base, s_buf);
    const double tot = block_sum(acc, s_red);
    if (threadIdx.x == 0) P.segabove[(size_t)b * P.nseg + seg] = tot;
}

// Select, second part (one block per sequence): the gathered bin resolved in LDS — the
// top-k threshold and/or the nucleus cut — with the margins, then the draw's segment sums
// (the mass above the bin plus the bin's kept elements), unless the kept launch has to
// compute them.
// Returns whether the row is still drawn (ri then holds its cut, total and kept_pass, and
// s_segk its segment sums unless the kept launch computes them); every return is uniform
// across the block.
template <gg_dtype_t DT>
__device__ bool select2_row(const DrawParams& P, int b, RowInfo& ri, double* s_segk, double* s_tab) {
    int* __restrict__ state = P.state;
    const int V = P.V, nseg = P.nseg;
    const double inv_t = P.inv_t, tau = P.tau, m = ri.m;
    __shared__ double s_mass[kBins];
    __shared__ unsigned long long s_comp[kCap];
    __shared__ double s_e[kCap];
    __shared__ double s_h[257];
    __shared__ double s_red[16];
    __shared__ unsigned long long s_u[16];
    __shared__ int s_n, s_bin, s_i, s_ok;
    __shared__ double s_above;
    const void* row = drawn_row(P, b, ri.row);
    const int per = kBins / kRowThreads;
    int ng = P.ncand[b];
    if (ng > kCap) {  // a crowded bin: the literal rule decides
        if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
        return false;
    }
    for (int i = threadIdx.x; i < ng; i += blockDim.x) {
        s_comp[i] = P.cand[(size_t)b * kCap + i];
        s_e[i] = exp_term(key_value((uint32_t)(s_comp[i] >> 32)), inv_t, m);
    }
    if (threadIdx.x == 0) s_ok = 1;
    __syncthreads();
    if (ri.pregather) {  // hint mode: the pass gathered the hinted bin and summed e above it
        double sv = 0.0, av = 0.0;
        for (int i = threadIdx.x; i < nseg; i += blockDim.x) {
            sv += P.segsum[(size_t)b * nseg + i];
            av += P.segabove[(size_t)b * nseg + i];
        }
        ri.S = block_sum(sv, s_red);
        ri.above = block_sum(av, s_red);
    }

    unsigned long long cut = 0, tk = 0;
    double tot = 0.0;
    int cbin = ri.cbin;  // the bin whose kept elements complete the segment sums
    if (P.use_k) {
        double dummy;
        const int ck = ng < ri.need ? -1 : select_desc(s_comp, s_e, ng, (double)ri.need, false, &dummy, s_h, s_red, &s_i);
        if (ck < 0) {
            if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
            return false;
        }
        tk = s_comp[ck];
        cut = tk;
        double part = 0.0, above = 0.0;
        for (int i = threadIdx.x; i < ng; i += blockDim.x)
            if (s_comp[i] >= tk) part += s_e[i];
        for (int i = ri.cbin + 1 + threadIdx.x; i < kBins; i += blockDim.x) above += P.hmass[(size_t)b * kBins + i];
        part = block_sum(part, s_red);
        above = block_sum(above, s_red);
        tot = above + part;
        if (P.use_p) {
            const double S = tot, pS = P.top_p * S;
            // Kept mass per bin: bins above the threshold bin whole, that bin in part.
            for (int i = threadIdx.x; i < kBins; i += blockDim.x)
                s_mass[i] = i > ri.cbin ? P.hmass[(size_t)b * kBins + i] : (i == ri.cbin ? part : 0.0);
            __syncthreads();
            double c = 0.0;
            for (int q = 0; q < per; ++q) c += s_mass[kBins - 1 - (threadIdx.x * per + q)];
            double btot;
            const double before = block_excl_scan(c, s_red, &btot);
            if (threadIdx.x == 0) s_bin = -1;
            __syncthreads();
            double run = before;
            int mine = -1;
            double mine_above = 0.0;
            if (before < pS && before + c >= pS) {
                for (int q = 0; q < per; ++q) {
                    const int bin = kBins - 1 - (threadIdx.x * per + q);
                    const double mq = s_mass[bin];
                    if (run + mq >= pS) {
                        mine = bin;
                        mine_above = run;
                        break;
                    }
                    run += mq;
                }
                if (mine >= 0) atomicMax(&s_bin, mine);
            }
            __syncthreads();
            if (mine >= 0 && mine == s_bin) s_above = mine_above;
            __syncthreads();
            const int pbin = s_bin;
            if (pbin < 0) {
                if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
                return false;
            }
            if (pbin != ri.cbin) {
                // The cut lies above the threshold bin: that bin's elements (one block gathers
                // them), and the kept launch computes the segment sums.
                ng = gather_bin<DT>(row, V, P.vec, pbin, inv_t, m, s_comp, s_e, &s_n);
                if (ng < 0) {
                    if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
                    return false;
                }
                ri.kept_pass = 1;
                cbin = pbin;
            }
            ri.above = s_above;
            ri.S = S;
        }
    }
    if (P.use_p) {
        const double S = ri.S, pS = P.top_p * S, above = ri.above;
        // The cut: the first item (value desc, index asc) whose running mass reaches p * S.
        double inbin = 0.0;
        int ci = -1;
        if (ri.hint != 0 && !P.use_k) ci = hint_cut(s_comp, s_e, ng, ri.hint, pS - above, &inbin, s_red, s_u, &s_i);
        if (ci < 0) ci = select_desc(s_comp, s_e, ng, pS - above, true, &inbin, s_h, s_red, &s_i);
        if (ci < 0) {
            if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
            return false;
        }
        const unsigned long long cc = s_comp[ci];
        const unsigned long long nb = next_below(s_comp, ng, cc, s_u);
        if (threadIdx.x == 0) {
            const double A = above + inbin, ec = s_e[ci];
            bool ok = (pS - A) > tau * S && (A + ec - pS) > tau * S;
            if (P.use_k && cc < tk) ok = false;  // past the top-k set: only rounding gets here
            // An element after the cut with the same probability but another value would come
            // first in the rule's (probability desc, index asc) order if its index is lower.
            if (nb != 0 && !(P.use_k && nb < tk)) {
                const double en = exp_term(key_value((uint32_t)(nb >> 32)), inv_t, m);
                if (en == ec && (nb >> 32) != (cc >> 32)) ok = false;
            } else if (nb == 0 && !(P.use_k && cbin == ri.cbin) && (ri.pregather ? ri.cbin_lo : cbin) > 0) {
                // bound of the bins below the gathered ones
                const double e_edge = gg_exp64(-(double)(kBins - (ri.pregather ? ri.cbin_lo : cbin)) / 64.0);
                if (e_edge >= ec) ok = false;
            }
            if (!ok) {
                atomicOr(&state[b], ST_EXACT);
                s_ok = 0;
            }
            s_above = A + ec;
        }
        __syncthreads();
        cut = cc;
        tot = s_above;
    }
    if (!s_ok) return false;
    if (P.q && ri.x >= 0) ri.kept_pass = 1;  // dense residual weights need the kept launch
    if (!ri.kept_pass) {
        // segment sums: the bins above cbin (gather launch) plus cbin's kept elements
        for (int i = threadIdx.x; i < nseg; i += blockDim.x) s_segk[i] = P.segabove[(size_t)b * nseg + i];
        __syncthreads();
        for (int i = threadIdx.x; i < ng; i += blockDim.x)
            if (s_comp[i] >= cut)
                atomicAdd(&s_segk[comp_index(s_comp[i]) / kSeg],
                          fast_term(key_value((uint32_t)(s_comp[i] >> 32)), inv_t, m, s_tab));
        __syncthreads();
        for (int i = threadIdx.x; i < nseg; i += blockDim.x) P.segkept[(size_t)b * nseg + i] = s_segk[i];
    }
    if (threadIdx.x == 0) {
        P.info[b].cut = cut;
        P.info[b].tot = tot;
        P.info[b].kept_pass = ri.kept_pass;
    }
    ri.cut = cut;
    ri.tot = tot;
    return true;
}

template <gg_dtype_t DT, int NT>
__device__ void draw_seq(const DrawParams& P, int b, RowInfo ri, const double* kept, const double* s_tab);

// kFuse: no kept launch follows, so the block draws right after its select, from the
// segment sums in its LDS, and the draw launch is not made.
template <gg_dtype_t DT, bool kFuse>
__global__ void __launch_bounds__(kRowThreads) sample_select2_kernel(DrawParams P) {
    const int b = blockIdx.x;
    if (P.state[b] != ST_DRAW) return;
    RowInfo ri = P.info[b];
    if (ri.cbin < 0) {  // (select1 marks such a row exact)
        if (kFuse && threadIdx.x == 0) atomicOr(&P.state[b], ST_EXACT);
        return;
    }
    __shared__ double s_segk[64];
    __shared__ double s_tab[64];
    load_exp_table(s_tab);
    if (!select2_row<DT>(P, b, ri, s_segk, s_tab)) return;
    if constexpr (kFuse) {
        if (ri.kept_pass) {  // (needs the kept launch, which a fused select rules out)
            if (threadIdx.x == 0) atomicOr(&P.state[b], ST_EXACT);
            return;
        }
        draw_seq<DT, kRowThreads>(P, b, ri, s_segk, s_tab);
    }
}

// ------------------------------------------------------------------------ kept

// Per (segment, sequence): the draw's weights summed (kept e, or the residual).
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) sample_kept_kernel(DrawParams P) {
    const int b = blockIdx.y, seg = blockIdx.x;
    if (P.state[b] != ST_DRAW) return;
    __shared__ double s_red[16];
    RowInfo ri = P.info[b];
    if (!ri.kept_pass) return;
    if (!P.filtered) ri.tot = seg_total(P, b);  // a dense residual without filters
    const double inv_tot = 1.0 / ri.tot;
    __shared__ double s_tab[64];
    load_exp_table(s_tab);
    const void* row = drawn_row(P, b, ri.row);
    const float* qr = q_row(P, b, ri);
    double acc = 0.0;
    constexpr int kIt = kSeg / 8 / kSegThreads;  // both chunks' loads issued before the math
    float x[kIt][8], y[kIt][8];
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
        const int e0 = seg * kSeg + (threadIdx.x + i * kSegThreads) * 8;
        load8<DT>(row, P.V, e0, P.vec, x[i]);
        load8q(qr, P.V, e0, P.vec_q, y[i]);
    }
#pragma unroll
    for (int i = 0; i < kIt; ++i) {
        const int e0 = seg * kSeg + (threadIdx.x + i * kSegThreads) * 8;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (e0 + k < P.V) acc += draw_weight(P, ri, y[i][k], x[i][k], e0 + k, s_tab, inv_tot);
    }
    const double tot = block_sum(acc, s_red);
    if (threadIdx.x == 0) P.segkept[(size_t)b * P.nseg + seg] = tot;
}

// ------------------------------------------------------------------------ draw

// The draw of sequence b by one block of NT threads, from its row's state ri: over the
// segment sums of the pass (no filters, unless a dense residual) or of the kept e or
// residuals (select or the kept launch; `kept`: a fused select's own, in LDS). A one-hot
// residual whose sums are kept e takes them as (kept e - e of the rejected draft) / total,
// its weights r = e / total.
template <gg_dtype_t DT, int NT>
__device__ void draw_seq(const DrawParams& P, int b, RowInfo ri, const double* kept, const double* s_tab) {
    __shared__ double s_sums[64];
    if (!P.filtered) ri.tot = seg_total(P, b);
    const bool split = split_residual(P, ri);
    const double* src = kept ? kept
                             : (!P.filtered && !ri.kept_pass && !split ? P.segsum : P.segkept) + (size_t)b * P.nseg;
    if (split && P.ncand[b] > kCap) {
        // More near-ties than the list holds (q close to p): this block sums the row's
        // residual by segment itself, 16 elements per thread and round.
        const double inv = 1.0 / ri.tot;
        if ((int)threadIdx.x < P.nseg) s_sums[threadIdx.x] = 0.0;
        __syncthreads();
        const float* qr = q_row(P, b, ri);
        const void* row = drawn_row(P, b, ri.row);
        for (int e0 = threadIdx.x * 16; e0 < P.V; e0 += blockDim.x * 16) {  // 16 | kSeg: one segment
            float xl[2][8], ql[2][8];
            load8<DT>(row, P.V, e0, P.vec, xl[0]);
            load8<DT>(row, P.V, e0 + 8, P.vec, xl[1]);
            load8q(qr, P.V, e0, P.vec_q, ql[0]);
            load8q(qr, P.V, e0 + 8, P.vec_q, ql[1]);
            double part = 0.0;
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (e0 + q < P.V) part += draw_weight(P, ri, ql[q >> 3][q & 7], xl[q >> 3][q & 7], e0 + q, s_tab, inv);
            atomicAdd(&s_sums[e0 / kSeg], part);
        }
        __syncthreads();
        src = s_sums;
    } else if (split) {
        // Segment residual masses: the sure-positive elements' E+/S - Q+, plus the listed
        // near-ties' own residuals (the same weight the draw below gives each element).
        const double inv = 1.0 / ri.tot;
        if ((int)threadIdx.x < P.nseg)
            s_sums[threadIdx.x] = P.segep[(size_t)b * P.nseg + threadIdx.x] * inv - P.segqp[(size_t)b * P.nseg + threadIdx.x];
        __syncthreads();
        const int n = P.ncand[b];
        const float* qr = q_row(P, b, ri);
        const void* row = drawn_row(P, b, ri.row);
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const int e = (int)P.cand[(size_t)b * kCap + i];
            atomicAdd(&s_sums[e / kSeg], draw_weight(P, ri, qr[e], load_as_f32(row, P.dt, e), e, s_tab, inv));
        }
        __syncthreads();
        src = s_sums;
    } else if (ri.x >= 0 && !ri.kept_pass && !split) {
        if (threadIdx.x < P.nseg) {
            double v = src[threadIdx.x];
            if (ri.x < P.V && ri.x / kSeg == (int)threadIdx.x) {
                const float lx = load_as_f32(drawn_row(P, b, ri.row), P.dt, ri.x);
                if (comp_key(order_key(lx), ri.x) >= ri.cut) v -= fast_term(lx, P.inv_t, ri.m, s_tab);
            }
            s_sums[threadIdx.x] = v / ri.tot;
        }
        __syncthreads();
        src = s_sums;
    }
    draw_in_block<DT, NT>(P, b, ri, src, s_tab);
}

template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) sample_draw_kernel(DrawParams P) {
    const int b = blockIdx.x;
    if (P.state[b] != ST_DRAW) return;
    __shared__ double s_tab[64];
    load_exp_table(s_tab);
    draw_seq<DT, kSegThreads>(P, b, P.info[b], nullptr, s_tab);
}

// ----------------------------------------------------------------------- exact

__device__ __forceinline__ bool ent_less(const Ent& a, const Ent& c) {
    return a.hi < c.hi || (a.hi == c.hi && a.lo < c.lo);
}

// One compare-exchange pass of a descending bitonic sort over g[0, N) (global memory).
__device__ void bitonic_pass_global(Ent* g, int N, int k, int j) {
    for (int p = threadIdx.x; p < N / 2; p += blockDim.x) {
        const int i = (p / j) * 2 * j + (p % j), l = i + j;
        const Ent x = g[i], y = g[l];
        const bool desc = (i & k) == 0;
        if (desc ? ent_less(x, y) : ent_less(y, x)) {
            g[i] = y;
            g[l] = x;
        }
    }
    __syncthreads();
}

// Passes j = jmax .. 1 of stage k on each kChunk-entry chunk of g, in LDS.
__device__ void bitonic_chunks_lds(Ent* g, int N, int kmin, int kmax, Ent* sh) {
    for (int c0 = 0; c0 < N; c0 += kChunk) {
        for (int i = threadIdx.x; i < kChunk; i += blockDim.x) sh[i] = g[c0 + i];
        __syncthreads();
        for (int k = kmin; k <= kmax; k <<= 1)
            for (int j = (k > kChunk ? kChunk : k) >> 1; j > 0; j >>= 1) {
                for (int p = threadIdx.x; p < kChunk / 2; p += blockDim.x) {
                    const int i = (p / j) * 2 * j + (p % j), l = i + j;
                    const Ent x = sh[i], y = sh[l];
                    const bool desc = ((c0 + i) & k) == 0;
                    if (desc ? ent_less(x, y) : ent_less(y, x)) {
                        sh[i] = y;
                        sh[l] = x;
                    }
                }
                __syncthreads();
            }
        for (int i = threadIdx.x; i < kChunk; i += blockDim.x) g[c0 + i] = sh[i];
        __syncthreads();
    }
}

// Descending sort of g[0, N), N a power of two >= kChunk.
__device__ void bitonic_sort_desc(Ent* g, int N, Ent* sh) {
    bitonic_chunks_lds(g, N, 2, kChunk, sh);
    for (int k = 2 * kChunk; k <= N; k <<= 1) {
        for (int j = k >> 1; j >= kChunk; j >>= 1) bitonic_pass_global(g, N, k, j);
        bitonic_chunks_lds(g, N, k, k, sh);
    }
}

// Sequential float64 sum of a[0, V) in index order, computed by wave 0 (every lane holds
// it), as the rule's `sum += x` loop does.
__device__ double wave_seq_sum(const double* a, int V) {
    const int lane = threadIdx.x & 63;
    double s = 0.0;
    for (int base = 0; base < V; base += 64) {
        const double x = base + lane < V ? a[base + lane] : 0.0;
        for (int l = 0; l < 64; ++l) s = s + lane_val(x, l);
    }
    return s;
}

// Sequential float64 sum of a[0, V) computed by wave 0, stored for the whole block.
__device__ double block_seq_sum(const double* a, int V, double* s_red) {
    if (threadIdx.x < 64) {
        const double s = wave_seq_sum(a, V);
        if (threadIdx.x == 0) s_red[0] = s;
    }
    __syncthreads();
    const double s = s_red[0];
    __syncthreads();
    return s;
}

// The rule of Sampler.Sample for one row (temperature > 1e-9), literally:
// internal/engine/sampling.go:57-71 and the helpers at :88-192. With x >= 0 the draw is the
// residual one of the rejection acceptance: r_i = p_i - q_i where p_i > q_i, for i != x
// (q_i the cleaned draft probability from qr, 0 without qr), r / sum(r); a zero sum falls
// back to p without x, normalised, and that being 0 too, to p.
__device__ int exact_draw(const void* row, gg_dtype_t dt, int V, double inv_t, int top_k, double top_p,
                          double u, int x, const float* qr, double* A, double* E, Ent* ent, int N, Ent* sh,
                          double* s_red, int* s_i) {
    const int tid = threadIdx.x;
    // scaled[i] = float64(l) * invT (:57-61)
    for (int i = tid; i < V; i += blockDim.x) A[i] = (double)load_as_f32(row, dt, i) * inv_t;
    __syncthreads();
    // topKFilter (:88-109): value desc, index asc, NaN last; the rest -inf.
    if (top_k > 0 && top_k < V) {
        // Numbers: (1, comp key); NaN: (0, ~index), after every number; padding (0, 0).
        for (int i = tid; i < N; i += blockDim.x) {
            Ent e{0ull, 0ull};
            if (i < V) {
                const float l = load_as_f32(row, dt, i);
                if (l == l) e = Ent{1ull, comp_key(order_key(l), i)};
                else e = Ent{0ull, (unsigned long long)(uint32_t)(~(uint32_t)i)};
            }
            ent[i] = e;
        }
        __syncthreads();
        bitonic_sort_desc(ent, N, sh);
        for (int j = top_k + tid; j < V; j += blockDim.x) {
            const Ent e = ent[j];
            A[comp_index(e.lo)] = -INFINITY;
        }
        __syncthreads();
    }
    // softmax (:112-136): max by `>` from element 0, exp, sequential sum, division.
    double mx = -INFINITY;
    for (int i = tid; i < V; i += blockDim.x) {
        const double v = A[i];
        if (v == v && v > mx) mx = v;
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
    if ((tid & 63) == 0) s_red[tid >> 6] = mx;
    __syncthreads();
    if (tid == 0) {
        double r = s_red[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmax(r, s_red[w]);
        if (A[0] != A[0]) r = A[0];  // nothing is `>` a NaN first element
        s_red[0] = r;
    }
    __syncthreads();
    mx = s_red[0];
    __syncthreads();
    for (int i = tid; i < V; i += blockDim.x) {
        const double v = A[i];
        E[i] = (v == -INFINITY) ? 0.0 : gg_exp64(v - mx);
    }
    __syncthreads();
    if (tid < 64) {
        const double s = wave_seq_sum(E, V);
        if (tid == 0) s_red[0] = s;
    }
    __syncthreads();
    const double sum = s_red[0];
    __syncthreads();
    if (sum > 0)
        for (int i = tid; i < V; i += blockDim.x) E[i] = E[i] / sum;
    __syncthreads();
    const double* fin = E;
    // topPFilter (:139-173)
    if (top_p > 0 && top_p < 1.0) {
        for (int i = tid; i < N; i += blockDim.x) {
            Ent e{0ull, 0ull};
            if (i < V) {
                const double p = E[i];
                // probability desc (NaN last), then index asc
                e.hi = p != p ? 0ull : (unsigned long long)__double_as_longlong(p) + 1ull;
                e.lo = (unsigned long long)(uint32_t)(~(uint32_t)i);
            }
            ent[i] = e;
            if (i < V) A[i] = 0.0;
        }
        __syncthreads();
        bitonic_sort_desc(ent, N, sh);
        if (tid < 64) {
            const int lane = tid;
            double cum = 0.0;
            bool stop = false;
            for (int j0 = 0; j0 < V && !stop; j0 += 64) {
                const bool real = j0 + lane < V;
                const int idx = real ? comp_index(ent[j0 + lane].lo) : 0;
                const double pr = real ? E[idx] : 0.0;
                bool kept = false;
                for (int l = 0; l < 64; ++l) {
                    if (j0 + l >= V || (cum >= top_p && cum > 0)) {
                        stop = true;
                        break;
                    }
                    if (lane == l) kept = true;
                    cum = cum + lane_val(pr, l);
                }
                if (kept) A[idx] = pr;
            }
        }
        __syncthreads();
        if (tid < 64) {
            const double s = wave_seq_sum(A, V);
            if (tid == 0) s_red[0] = s;
        }
        __syncthreads();
        const double s2 = s_red[0];
        __syncthreads();
        if (s2 > 0)
            for (int i = tid; i < V; i += blockDim.x) A[i] = A[i] / s2;
        __syncthreads();
        fin = A;
    }
    if (x >= 0) {
        double* r = fin == A ? E : A;
        for (int i = tid; i < V; i += blockDim.x) {
            const double qv = qr ? clean_q(qr[i]) : 0.0;
            r[i] = (i != x && fin[i] > qv) ? fin[i] - qv : 0.0;
        }
        __syncthreads();
        double sr = block_seq_sum(r, V, s_red);
        if (!(sr > 0)) {
            for (int i = tid; i < V; i += blockDim.x) r[i] = i != x ? fin[i] : 0.0;
            __syncthreads();
            sr = block_seq_sum(r, V, s_red);
        }
        if (sr > 0) {
            for (int i = tid; i < V; i += blockDim.x) r[i] = r[i] / sr;
            __syncthreads();
            fin = r;
        }
    }
    // categoricalSample (:176-192): first i with u < cumulative, else the last nonzero.
    if (tid < 64) {
        const int lane = tid;
        double cum = 0.0;
        int found = -1;
        for (int base = 0; base < V && found < 0; base += 64) {
            const double x = base + lane < V ? fin[base + lane] : 0.0;
            for (int l = 0; l < 64; ++l) {
                cum = cum + lane_val(x, l);
                if (u < cum) {
                    found = base + l;
                    break;
                }
            }
        }
        if (tid == 0) *s_i = found;
    }
    __syncthreads();
    int tok = *s_i;
    __syncthreads();
    if (tok < 0) {
        int last = -1;
        for (int i = tid; i < V; i += blockDim.x)
            if (fin[i] > 0) last = i;
        for (int o = 32; o > 0; o >>= 1) last = max(last, __shfl_xor(last, o));
        if ((tid & 63) == 0) s_red[tid >> 6] = (double)last;
        __syncthreads();
        if (tid == 0) {
            int r = -1;
            for (int w = 0; w < (int)(blockDim.x >> 6); ++w) r = max(r, (int)s_red[w]);
            *s_i = r < 0 ? 0 : r;
        }
        __syncthreads();
        tok = *s_i;
        __syncthreads();
    }
    return tok;
}

__global__ void __launch_bounds__(kRowThreads) sample_exact_kernel(DrawParams P, uint8_t* __restrict__ scratch,
                                                                    size_t slot_bytes, size_t vpad, int npow) {
    __shared__ Ent sh[kChunk];
    __shared__ double s_red[16];
    __shared__ int s_i;
    uint8_t* slot = scratch + (size_t)blockIdx.x * slot_bytes;
    double* A = (double*)slot;
    double* E = A + vpad;
    Ent* ent = (Ent*)(E + vpad);
    for (int b = blockIdx.x; b < P.B; b += gridDim.x) {
        if (!(P.state[b] & ST_EXACT)) continue;
        const RowInfo ri = P.info[b];
        const int tok = exact_draw(drawn_row(P, b, ri.row), P.dt, P.V, P.inv_t, P.top_k, P.top_p, uniform_of(P, b),
                                   ri.x, q_row(P, b, ri), A, E, ent, npow, sh, s_red, &s_i);
        if (threadIdx.x == 0) P.out_tok[b] = tok;
        __syncthreads();
    }
}

}  // namespace

size_t final_draw_workspace_bytes(int num_seqs, int vocab) { return layout(num_seqs, vocab).total; }

fd::DrawParams fd::final_draw_params(const FinalDraw& d, void* ws) {
    const int B = d.num_seqs, K = d.max_drafts, V = d.vocab;
    const Layout L = layout(B, V);
    uint8_t* w = (uint8_t*)ws;
    DrawParams P{};
    P.logits = d.logits;
    P.dt = d.dt;
    P.B = B;
    P.K = K;
    P.V = V;
    P.nseg = (V + kSeg - 1) / kSeg;
    P.inv_t = 1.0 / d.temperature;
    P.top_k = d.top_k;
    P.top_p = d.top_p;
    P.use_k = d.top_k > 0 && d.top_k < V;
    P.use_p = d.top_p > 0 && d.top_p < 1.0;
    P.filtered = P.use_k || P.use_p;
    P.hint_mode = d.spec_key && P.use_p && !P.use_k;
    P.kept_launched = (d.draft_probs && (P.filtered || !d.spec_s)) || (P.use_k && P.use_p);
    {
        const size_t eb = dtype_bytes(d.dt);
        P.vec = ((size_t)V * eb % 16 == 0) && ((uintptr_t)d.logits % 16 == 0);
        P.vec_q = (V % 4 == 0) && ((uintptr_t)d.draft_probs % 16 == 0);
    }
    // Bound on the rounding of a sequential or parallel float64 sum over the row (plus the
    // 4096 histogram bins), relative to the sum: 8 * (V + 4096) * 2^-53, plus twice the
    // parallel path's exponential error.
    P.tau = 8.0 * ((double)V + 4096.0) * 0x1p-53 + 2.0 * kFastExpErr;
    P.ud = d.uniforms_f64;
    P.uf = d.uniforms_f32;
    P.q = d.draft_probs;
    P.state = (int*)(w + L.state);
    P.info = (RowInfo*)(w + L.info);
    P.hcnt = (uint32_t*)(w + L.hcnt);
    P.hmass = (double*)(w + L.hmass);
    P.segsum = (double*)(w + L.segsum);
    P.segkept = (double*)(w + L.segkept);
    P.segabove = (double*)(w + L.segabove);
    P.segep = (double*)(w + L.segep);
    P.segqp = (double*)(w + L.segqp);
    P.ncand = (int*)(w + L.ncand);
    P.cand = (unsigned long long*)(w + L.cand);
    P.out_tok = d.out_tok;
    return P;
}

gg_status_t launch_final_draw(const FinalDraw& d, void* ws, hipStream_t s) {
    const int B = d.num_seqs, V = d.vocab;
    const Layout L = layout(B, V);
    uint8_t* w = (uint8_t*)ws;
    const DrawParams P = fd::final_draw_params(d, ws);
    const int force = d.force_exact ? 1 : 0;
    const int nseg_m = d.greedy_seg ? (V + kGreedySeg - 1) / kGreedySeg : d.nseg_max;
    if (!d.prepped)
        sample_prep_kernel<<<B, 256, 0, s>>>(P, d.greedy_seg, d.seg_max, nseg_m, d.n_drafts, d.accepted, d.spec_row,
                                             d.spec_x, d.spec_key, d.spec_s, force);
    // Without filters the draw takes the pass's segment sums (a dense residual: the kept
    // launch's). With filters: the bin of the cut (select1), its elements and the sums above
    // it (gather) — both done by the pass when the caller hints the cut — then the cut and
    // the segment sums (select2); the kept launch only for dense residuals and for a nucleus
    // cut above the top-k bin.
    // (A dense residual without filters but with the caller's estimate of S needs none: the
    // pass and the draw form its sums.)
    const bool kept = P.kept_launched;
#define GG_DRAW(DTV)                                                                                 \
    if (P.hint_mode) sample_pass_kernel<DTV, kPassPre><<<dim3(P.nseg, B), kSegThreads, 0, s>>>(P);   \
    else if (P.filtered) sample_pass_kernel<DTV, kPassHist><<<dim3(P.nseg, B), kSegThreads, 0, s>>>(P); \
    else sample_pass_kernel<DTV, kPassPlain><<<dim3(P.nseg, B), kSegThreads, 0, s>>>(P);             \
    if (P.filtered && !P.hint_mode) {                                                                \
        sample_select1_kernel<<<B, kRowThreads, 0, s>>>(P);                                          \
        sample_gather_kernel<DTV><<<dim3(P.nseg, B), kSegThreads, 0, s>>>(P);                        \
    }                                                                                                \
    if (P.filtered && !kept) sample_select2_kernel<DTV, true><<<B, kRowThreads, 0, s>>>(P);           \
    if (P.filtered && kept) sample_select2_kernel<DTV, false><<<B, kRowThreads, 0, s>>>(P);           \
    if (kept) sample_kept_kernel<DTV><<<dim3(P.nseg, B), kSegThreads, 0, s>>>(P);                    \
    if (!(P.filtered && !kept)) sample_draw_kernel<DTV><<<B, kSegThreads, 0, s>>>(P);
    switch (d.dt) {
        case GG_DTYPE_F32: GG_DRAW(GG_DTYPE_F32) break;
        case GG_DTYPE_BF16: GG_DRAW(GG_DTYPE_BF16) break;
        case GG_DTYPE_F16: GG_DRAW(GG_DTYPE_F16) break;
        default: return fail(GG_ERR_INVALID, "final draw: logits dtype");
    }
#undef GG_DRAW
    const int slots = B < kExactSlots ? B : kExactSlots;
    sample_exact_kernel<<<slots, kRowThreads, 0, s>>>(P, w + L.exact, L.slot_bytes, L.vpad, (int)L.npow);
    return check_hip(hipGetLastError(), "final draw launch");
}

size_t sample_workspace_bytes(int num_seqs, int max_drafts, int vocab) {
    return ((greedy_workspace_bytes(num_seqs, max_drafts, vocab) + 255) & ~(size_t)255) +
           final_draw_workspace_bytes(num_seqs, vocab);
}

gg_status_t launch_accept_greedy_sample(const void* logits, gg_dtype_t dt, int B, int K, int V,
                                        const int32_t* drafts, const int32_t* n_drafts, double temperature,
                                        int top_k, double top_p, const double* uniforms, unsigned flags,
                                        int32_t* out_acc, int32_t* out_tok, void* ws, hipStream_t s) {
    uint8_t* w = (uint8_t*)ws;
    gg_status_t st = launch_accept_greedy(logits, dt, B, K, V, drafts, n_drafts, out_acc, out_tok, w, s);
    if (st != GG_OK) return st;
    if (temperature <= 1e-9) return GG_OK;  // Sampler.Sample's greedy case (sampling.go:54-56)
    FinalDraw d{};
    d.logits = logits;
    d.dt = dt;
    d.num_seqs = B;
    d.max_drafts = K;
    d.vocab = V;
    d.temperature = temperature;
    d.top_k = top_k;
    d.top_p = top_p;
    d.uniforms_f64 = uniforms;
    d.n_drafts = n_drafts;
    d.accepted = out_acc;
    d.greedy_seg = (const float2*)w;
    d.force_exact = (flags & GG_SAMPLE_EXACT) != 0;
    d.out_tok = out_tok;
    return launch_final_draw(d, w + ((greedy_workspace_bytes(B, K, V) + 255) & ~(size_t)255), s);
}

}  // namespace gg
