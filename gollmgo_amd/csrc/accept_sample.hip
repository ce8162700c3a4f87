// accept_sample.hip — greedy verify with the bonus token drawn as the reference samples it.
//
// The reference's emitSpeculative (internal/engine/serving.go:514-566) runs the greedy
// Verify over the draft rows, then, when every draft was accepted, draws the bonus token
// with Sampler.Sample(posLogits[K]) (internal/engine/sampling.go:40-72): temperature,
// top-k, softmax, top-p and a categorical draw, all in float64. This file adds that draw
// to the greedy acceptance (accept_greedy.hip), with the uniform supplied in place of
// rng.Float64().
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
//           About 3 ms per row; a row lands here with probability ~1e-4 (rows with NaN or
//           +inf logits always do).
// Orders the reference leaves open (sort.Slice is not stable) are fixed as value desc,
// then index asc, NaN last; exp is gg_exp64 (gg_exp64.h), identical on host and device.
//
// Launches after the greedy pair (segment argmax, decide):
//   prep   (B blocks)       : which sequences draw; row max from the greedy segments.
//   pass   (segments x B)   : e_i = exp(l_i/T - m) per element, segment sums, NaN/+inf
//                             check, coarse histograms (count and mass per 4096 bins of
//                             the value's order key) when top-k or top-p is on.
//   select (B, top-k/p only): top-k threshold and nucleus cut from the histograms, the
//                             crossing bin's items gathered and sorted in LDS.
//   kept   (segments x B, top-k/p only): kept mass per segment.
//   draw   (B)              : the segment and then the element where u * total falls.
//   exact  (a few blocks)   : the literal rule for the rows flagged on the way.
#include "gg_common.h"
#include "gg_exp64.h"

#pragma clang fp contract(off)

namespace gg {
namespace {

constexpr int kSeg = 8192;        // elements per block of the pass and kept launches
constexpr int kSegThreads = 512;
constexpr int kBins = 4096;       // coarse bins: the top 12 bits of the order key
constexpr int kCap = 4096;        // items of one bin the select launch can gather
constexpr int kRowThreads = 1024;
constexpr int kChunk = 4096;      // exact path: bitonic sort entries held in LDS at once
constexpr int kExactSlots = 4;    // exact path: workgroups (each with its own scratch)
constexpr int kGreedySeg = 4096;  // accept_greedy.hip's segment length
constexpr int kNone = 0x7fffffff; // accept_greedy.hip's "no element" index

enum : int { ST_NONE = 0, ST_DRAW = 1, ST_EXACT = 2 };

struct RowInfo {
    double m;                 // max scaled logit of the bonus row
    unsigned long long cut;   // kept <=> comp_key >= cut (0 keeps every element)
};

struct Ent {                  // exact path sort entry, ordered by (hi, lo) descending
    unsigned long long hi, lo;
};

struct Layout {
    size_t greedy, state, info, hcnt, hmass, segsum, segkept, exact, total;
    size_t slot_bytes, vpad, npow;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Layout layout(int B, int K, int V) {
    Layout L{};
    const int nseg = (V + kSeg - 1) / kSeg;
    size_t o = align256(greedy_workspace_bytes(B, K, V));
    L.greedy = 0;
    L.state = o;   o = align256(o + (size_t)B * sizeof(int));
    L.info = o;    o = align256(o + (size_t)B * sizeof(RowInfo));
    L.hcnt = o;    o = align256(o + (size_t)B * kBins * sizeof(uint32_t));
    L.hmass = o;   o = align256(o + (size_t)B * kBins * sizeof(double));
    L.segsum = o;  o = align256(o + (size_t)B * nseg * sizeof(double));
    L.segkept = o; o = align256(o + (size_t)B * nseg * sizeof(double));
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
__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
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

__global__ void __launch_bounds__(256) sample_prep_kernel(
    const float2* __restrict__ gws, int K, int nseg_g, const int32_t* __restrict__ n_drafts,
    const int32_t* __restrict__ acc, double inv_t, int hist, int force_exact, uint32_t* __restrict__ hcnt,
    double* __restrict__ hmass, int* __restrict__ state, RowInfo* __restrict__ info) {
    const int b = blockIdx.x;
    const int R = K + 1;
    const int n = clamp_n(n_drafts, b, K);
    if (acc[b] != n) {
        if (threadIdx.x == 0) state[b] = ST_NONE;
        return;
    }
    if (hist)
        for (int i = threadIdx.x; i < kBins; i += blockDim.x) {
            hcnt[(size_t)b * kBins + i] = 0;
            hmass[(size_t)b * kBins + i] = 0.0;
        }
    if (threadIdx.x < 64) {
        float mx = -INFINITY;
        int any = 0;
        for (int s = threadIdx.x; s < nseg_g; s += 64) {
            const float2 p = gws[((size_t)b * R + n) * nseg_g + s];
            if (__float_as_int(p.y) != kNone) {
                any = 1;
                mx = fmaxf(mx, p.x);
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            mx = fmaxf(mx, __shfl_xor(mx, o));
            any |= __shfl_xor(any, o);
        }
        if (threadIdx.x == 0) {
            const double m = (double)mx * inv_t;
            int st = ST_DRAW;
            // No finite maximum (all -inf / NaN, or +inf present), or a non-finite scale:
            // the literal rule decides.
            if (!any || !(mx > -INFINITY && mx < INFINITY) || !(m > -INFINITY && m < INFINITY) || force_exact)
                st |= ST_EXACT;
            info[b].m = m;
            info[b].cut = 0;
            state[b] = st;
        }
    }
}

// ------------------------------------------------------------------------ pass

__global__ void __launch_bounds__(kSegThreads) sample_pass_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int K, int V, int nseg,
    const int32_t* __restrict__ n_drafts, double inv_t, int want_cnt, int want_mass,
    int* __restrict__ state, const RowInfo* __restrict__ info, uint32_t* __restrict__ hcnt,
    double* __restrict__ hmass, double* __restrict__ segsum) {
    const int b = blockIdx.y, seg = blockIdx.x;
    if (state[b] != ST_DRAW) return;
    __shared__ uint32_t s_cnt[kBins];
    __shared__ double s_mass[kBins];
    __shared__ double s_red[16];
    const int n = clamp_n(n_drafts, b, K);
    const void* row = (const uint8_t*)logits + ((size_t)b * (K + 1) + n) * V * dtype_bytes(dt);
    const double m = info[b].m;
    if (want_cnt || want_mass) {
        for (int i = threadIdx.x; i < kBins; i += blockDim.x) {
            s_cnt[i] = 0;
            s_mass[i] = 0.0;
        }
        __syncthreads();
    }
    double acc = 0.0;
    int bad = 0;
    const int end = min(V, (seg + 1) * kSeg);
    for (int e = seg * kSeg + threadIdx.x; e < end; e += blockDim.x) {
        const float l = load_as_f32(row, dt, e);
        if (l != l || l == INFINITY) {
            bad = 1;
            continue;
        }
        const double ev = exp_term(l, inv_t, m);
        acc += ev;
        if (want_cnt || want_mass) {
            const int bin = (int)(order_key(l) >> 20);
            if (want_cnt) atomicAdd(&s_cnt[bin], 1u);
            if (want_mass && ev != 0.0) atomicAdd(&s_mass[bin], ev);
        }
    }
    if (__syncthreads_or(bad)) {
        if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
        return;
    }
    const double tot = block_sum(acc, s_red);
    if (threadIdx.x == 0) segsum[(size_t)b * nseg + seg] = tot;
    if (want_cnt || want_mass) {
        for (int i = threadIdx.x; i < kBins; i += blockDim.x) {
            if (want_cnt && s_cnt[i]) atomicAdd(&hcnt[(size_t)b * kBins + i], s_cnt[i]);
            if (want_mass && s_mass[i] != 0.0) unsafeAtomicAdd(&hmass[(size_t)b * kBins + i], s_mass[i]);
        }
    }
}

// ---------------------------------------------------------------------- select

// Bitonic sort of n_pad (a power of two, <= kCap) keys in LDS, descending.
__device__ void lds_sort_desc(unsigned long long* a, int n_pad) {
    for (int k = 2; k <= n_pad; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int p = threadIdx.x; p < n_pad / 2; p += blockDim.x) {
                const int i = (p / j) * 2 * j + (p % j), l = i + j;
                const unsigned long long x = a[i], y = a[l];
                const bool desc = (i & k) == 0;
                if (desc ? x < y : x > y) {
                    a[i] = y;
                    a[l] = x;
                }
            }
            __syncthreads();
        }
}

// Gather the elements of the row whose order key falls in bin `bin` into s_comp (sorted
// descending, padded with 0) and their e into s_e. Returns the count, or -1 when the bin
// holds more than kCap elements.
__device__ int gather_bin(const void* row, gg_dtype_t dt, int V, int bin, double inv_t, double m,
                          unsigned long long* s_comp, double* s_e, int* s_n) {
    if (threadIdx.x == 0) *s_n = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < V; e += blockDim.x) {
        const float l = load_as_f32(row, dt, e);
        const uint32_t key = order_key(l);
        if ((int)(key >> 20) == bin) {
            const int slot = atomicAdd(s_n, 1);
            if (slot < kCap) s_comp[slot] = comp_key(key, e);
        }
    }
    __syncthreads();
    const int ng = *s_n;
    __syncthreads();
    if (ng > kCap) return -1;
    int np = 1;
    while (np < ng) np <<= 1;
    for (int i = ng + threadIdx.x; i < np; i += blockDim.x) s_comp[i] = 0ull;
    __syncthreads();
    lds_sort_desc(s_comp, np);
    for (int i = threadIdx.x; i < ng; i += blockDim.x)
        s_e[i] = exp_term(key_value((uint32_t)(s_comp[i] >> 32)), inv_t, m);
    __syncthreads();
    return ng;
}

__global__ void __launch_bounds__(kRowThreads) sample_select_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int K, int V, int nseg,
    const int32_t* __restrict__ n_drafts, double inv_t, int top_k, int use_p, double top_p, double tau,
    int* __restrict__ state, RowInfo* __restrict__ info, const uint32_t* __restrict__ hcnt,
    const double* __restrict__ hmass, const double* __restrict__ segsum) {
    const int b = blockIdx.x;
    if (state[b] != ST_DRAW) return;
    __shared__ double s_mass[kBins];
    __shared__ unsigned long long s_comp[kCap];
    __shared__ double s_e[kCap];
    __shared__ double s_red[16];
    __shared__ uint32_t s_redu[16];
    __shared__ int s_n, s_bin, s_flag;
    __shared__ double s_above;
    __shared__ uint32_t s_cabove;
    const int n = clamp_n(n_drafts, b, K);
    const void* row = (const uint8_t*)logits + ((size_t)b * (K + 1) + n) * V * dtype_bytes(dt);
    const double m = info[b].m;
    const bool use_k = top_k > 0 && top_k < V;
    const int per = kBins / kRowThreads;  // bins per thread, positions counted from the top bin
    for (int i = threadIdx.x; i < kBins; i += blockDim.x) s_mass[i] = hmass[(size_t)b * kBins + i];
    if (threadIdx.x == 0) s_flag = 0;
    __syncthreads();

    unsigned long long cut = 0;
    double S;
    int kbin = -1, need = 0;
    if (use_k) {
        // The bin where the count from the top first reaches k.
        uint32_t c = 0;
        for (int q = 0; q < per; ++q) c += hcnt[(size_t)b * kBins + (kBins - 1 - (threadIdx.x * per + q))];
        uint32_t tot;
        uint32_t before = block_excl_scan_u32(c, s_redu, &tot);
        if (threadIdx.x == 0) s_bin = -1;
        __syncthreads();
        if (before < (uint32_t)top_k && before + c >= (uint32_t)top_k) {
            uint32_t run = before;
            for (int q = 0; q < per; ++q) {
                const int bin = kBins - 1 - (threadIdx.x * per + q);
                const uint32_t cq = hcnt[(size_t)b * kBins + bin];
                if (run + cq >= (uint32_t)top_k) {
                    s_bin = bin;
                    s_cabove = run;
                    break;
                }
                run += cq;
            }
        }
        __syncthreads();
        kbin = s_bin;
        if (kbin < 0) {  // fewer counted elements than k: cannot happen for a clean row
            if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
            return;
        }
        need = top_k - (int)s_cabove;
        const int ng = gather_bin(row, dt, V, kbin, inv_t, m, s_comp, s_e, &s_n);
        if (ng < need) {  // more than kCap elements in the bin (or a count mismatch)
            if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
            return;
        }
        cut = s_comp[need - 1];
        double part = 0.0, above = 0.0;
        for (int i = threadIdx.x; i < need; i += blockDim.x) part += s_e[i];
        for (int i = kbin + 1 + threadIdx.x; i < kBins; i += blockDim.x) above += s_mass[i];
        part = block_sum(part, s_red);
        above = block_sum(above, s_red);
        S = above + part;
        // Kept mass per bin: bins above the threshold bin whole, that bin in part, none below.
        for (int i = threadIdx.x; i < kbin; i += blockDim.x) s_mass[i] = 0.0;
        if (threadIdx.x == 0) s_mass[kbin] = part;
        __syncthreads();
    } else {
        double s = 0.0;
        for (int i = threadIdx.x; i < nseg; i += blockDim.x) s += segsum[(size_t)b * nseg + i];
        S = block_sum(s, s_red);
    }

    if (use_p) {
        const double pS = top_p * S;
        // The bin where the kept mass from the top first reaches p * S.
        double c = 0.0;
        for (int q = 0; q < per; ++q) c += s_mass[kBins - 1 - (threadIdx.x * per + q)];
        double tot;
        const double before = block_excl_scan(c, s_red, &tot);
        // Rounding can let two neighbouring threads both see the crossing; the first in
        // order wins (atomicMax on the bin) and only its owner writes the mass above it.
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
        if (pbin < 0) {  // p * S at the very end of the mass: the rounding decides
            if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
            return;
        }
        const double above = s_above;
        int nk;
        if (use_k && pbin == kbin) {
            nk = need;
        } else {
            nk = gather_bin(row, dt, V, pbin, inv_t, m, s_comp, s_e, &s_n);
            if (nk < 0) {
                if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
                return;
            }
        }
        // Inclusive prefix of e in (value desc, index asc) order; the cut is the first item
        // whose inclusive mass reaches p * S.
        const int q0 = threadIdx.x * (kCap / kRowThreads);
        double loc = 0.0;
        for (int q = 0; q < kCap / kRowThreads; ++q)
            if (q0 + q < nk) loc += s_e[q0 + q];
        double btot;
        double irun = above + block_excl_scan(loc, s_red, &btot);
        if (threadIdx.x == 0) s_n = 0x7fffffff;
        __syncthreads();
        int ic = -1;
        double ic_above = 0.0;
        for (int q = 0; q < kCap / kRowThreads; ++q) {
            const int i = q0 + q;
            if (i >= nk) break;
            const double nx = irun + s_e[i];
            if (irun < pS && nx >= pS) {
                ic = i;
                ic_above = irun;
                break;
            }
            irun = nx;
        }
        if (ic >= 0) atomicMin(&s_n, ic);
        __syncthreads();
        if (ic >= 0 && ic == s_n) s_above = ic_above;
        __syncthreads();
        if (threadIdx.x == 0 && s_n == 0x7fffffff) s_n = -1;
        __syncthreads();
        const int ci = s_n;
        if (ci < 0) {
            if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
            return;
        }
        if (threadIdx.x == 0) {
            const double A = s_above, ec = s_e[ci];
            bool ok = (pS - A) > tau * S && (A + ec - pS) > tau * S;
            // An element after the cut with the same probability but another value would come
            // first in the rule's (probability desc, index asc) order if its index is lower.
            if (ci + 1 < nk) {
                if (s_e[ci + 1] == ec && (s_comp[ci + 1] >> 32) != (s_comp[ci] >> 32)) ok = false;
            } else if (!(use_k && pbin == kbin) && pbin > 0) {
                const double e_edge = exp_term(key_value(((uint32_t)pbin << 20) - 1u), inv_t, m);
                if (e_edge >= ec) ok = false;
            }
            if (!ok) atomicOr(&state[b], ST_EXACT);
            info[b].cut = s_comp[ci];
        }
        return;
    }
    if (threadIdx.x == 0) info[b].cut = cut;
}

// ------------------------------------------------------------------------ kept

__global__ void __launch_bounds__(kSegThreads) sample_kept_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int K, int V, int nseg,
    const int32_t* __restrict__ n_drafts, double inv_t, const int* __restrict__ state,
    const RowInfo* __restrict__ info, double* __restrict__ segkept) {
    const int b = blockIdx.y, seg = blockIdx.x;
    if (state[b] != ST_DRAW) return;
    __shared__ double s_red[16];
    const int n = clamp_n(n_drafts, b, K);
    const void* row = (const uint8_t*)logits + ((size_t)b * (K + 1) + n) * V * dtype_bytes(dt);
    const double m = info[b].m;
    const unsigned long long cut = info[b].cut;
    double acc = 0.0;
    const int end = min(V, (seg + 1) * kSeg);
    for (int e = seg * kSeg + threadIdx.x; e < end; e += blockDim.x) {
        const float l = load_as_f32(row, dt, e);
        if (comp_key(order_key(l), e) >= cut) acc += exp_term(l, inv_t, m);
    }
    const double tot = block_sum(acc, s_red);
    if (threadIdx.x == 0) segkept[(size_t)b * nseg + seg] = tot;
}

// ------------------------------------------------------------------------ draw

__global__ void __launch_bounds__(kRowThreads) sample_draw_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int K, int V, int nseg,
    const int32_t* __restrict__ n_drafts, double inv_t, int filtered, const double* __restrict__ uniforms,
    double tau, int* __restrict__ state, const RowInfo* __restrict__ info,
    const double* __restrict__ segsum, const double* __restrict__ segkept, int32_t* __restrict__ out_tok) {
    const int b = blockIdx.x;
    if (state[b] != ST_DRAW) return;
    __shared__ double s_red[16];
    __shared__ int s_seg, s_tok, s_bad;
    __shared__ double s_base, s_tot;
    const double u = uniforms[b];
    if (!(u >= tau && u < 1.0 - tau)) {  // near 0, near or past 1, NaN: the literal rule
        if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
        return;
    }
    const double* sums = (filtered ? segkept : segsum) + (size_t)b * nseg;
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
        s_seg = sel;
        s_base = run;
        s_tot = tot;
        s_tok = -1;
        s_bad = 0;
    }
    __syncthreads();
    const int seg = s_seg;
    if (seg < 0) {
        if (threadIdx.x == 0) atomicOr(&state[b], ST_EXACT);
        return;
    }
    const double tot = s_tot, t = u * tot;
    const int n = clamp_n(n_drafts, b, K);
    const void* row = (const uint8_t*)logits + ((size_t)b * (K + 1) + n) * V * dtype_bytes(dt);
    const double m = info[b].m;
    const unsigned long long cut = info[b].cut;
    constexpr int kPer = kSeg / kRowThreads;
    const int e0 = seg * kSeg + threadIdx.x * kPer;
    double ev[kPer];
    double loc = 0.0;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int e = e0 + q;
        ev[q] = 0.0;
        if (e < V) {
            const float l = load_as_f32(row, dt, e);
            if (comp_key(order_key(l), e) >= cut) ev[q] = exp_term(l, inv_t, m);
        }
        loc += ev[q];
    }
    double btot;
    double run = s_base + block_excl_scan(loc, s_red, &btot);
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const double nx = run + ev[q];
        if (run <= t && nx > t) {
            const bool ok = (t - run) > tau * tot && (nx - t) > tau * tot;
            if (ok) s_tok = e0 + q;
            else s_bad = 1;
        }
        run = nx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (s_tok >= 0 && !s_bad) out_tok[b] = s_tok;
        else atomicOr(&state[b], ST_EXACT);
    }
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

// The rule of Sampler.Sample for one row (temperature > 1e-9), literally:
// internal/engine/sampling.go:57-71 and the helpers at :88-192.
__device__ int exact_draw(const void* row, gg_dtype_t dt, int V, double inv_t, int top_k, double top_p,
                          double u, double* A, double* E, Ent* ent, int N, Ent* sh, double* s_red,
                          int* s_i) {
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

__global__ void __launch_bounds__(kRowThreads) sample_exact_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int B, int K, int V, const int32_t* __restrict__ n_drafts,
    double inv_t, int top_k, double top_p, const double* __restrict__ uniforms, const int* __restrict__ state,
    uint8_t* __restrict__ scratch, size_t slot_bytes, size_t vpad, int npow, int32_t* __restrict__ out_tok) {
    __shared__ Ent sh[kChunk];
    __shared__ double s_red[16];
    __shared__ int s_i;
    uint8_t* slot = scratch + (size_t)blockIdx.x * slot_bytes;
    double* A = (double*)slot;
    double* E = A + vpad;
    Ent* ent = (Ent*)(E + vpad);
    for (int b = blockIdx.x; b < B; b += gridDim.x) {
        if (!(state[b] & ST_EXACT)) continue;
        const int n = clamp_n(n_drafts, b, K);
        const void* row = (const uint8_t*)logits + ((size_t)b * (K + 1) + n) * V * dtype_bytes(dt);
        const int tok = exact_draw(row, dt, V, inv_t, top_k, top_p, uniforms[b], A, E, ent, npow, sh, s_red, &s_i);
        if (threadIdx.x == 0) out_tok[b] = tok;
        __syncthreads();
    }
}

}  // namespace

size_t sample_workspace_bytes(int num_seqs, int max_drafts, int vocab) {
    return layout(num_seqs, max_drafts, vocab).total;
}

gg_status_t launch_accept_greedy_sample(const void* logits, gg_dtype_t dt, int B, int K, int V,
                                        const int32_t* drafts, const int32_t* n_drafts, double temperature,
                                        int top_k, double top_p, const double* uniforms, unsigned flags,
                                        int32_t* out_acc, int32_t* out_tok, void* ws, hipStream_t s) {
    const Layout L = layout(B, K, V);
    uint8_t* w = (uint8_t*)ws;
    gg_status_t st = launch_accept_greedy(logits, dt, B, K, V, drafts, n_drafts, out_acc, out_tok, w + L.greedy, s);
    if (st != GG_OK) return st;
    if (temperature <= 1e-9) return GG_OK;  // Sampler.Sample's greedy case (sampling.go:54-56)
    const double inv_t = 1.0 / temperature;
    const bool use_k = top_k > 0 && top_k < V;
    const bool use_p = top_p > 0 && top_p < 1.0;
    const bool filtered = use_k || use_p;
    const int nseg = (V + kSeg - 1) / kSeg;
    const int nseg_g = (V + kGreedySeg - 1) / kGreedySeg;
    const double tau = 8.0 * ((double)V + 4096.0) * 0x1p-53;
    int* state = (int*)(w + L.state);
    RowInfo* info = (RowInfo*)(w + L.info);
    uint32_t* hcnt = (uint32_t*)(w + L.hcnt);
    double* hmass = (double*)(w + L.hmass);
    double* segsum = (double*)(w + L.segsum);
    double* segkept = (double*)(w + L.segkept);
    const int force = (flags & GG_SAMPLE_EXACT) ? 1 : 0;
    sample_prep_kernel<<<B, 256, 0, s>>>((const float2*)(w + L.greedy), K, nseg_g, n_drafts, out_acc, inv_t,
                                         filtered ? 1 : 0, force, hcnt, hmass, state, info);
    sample_pass_kernel<<<dim3(nseg, B), kSegThreads, 0, s>>>(logits, dt, K, V, nseg, n_drafts, inv_t, use_k ? 1 : 0,
                                                             filtered ? 1 : 0, state, info, hcnt, hmass, segsum);
    if (filtered) {
        sample_select_kernel<<<B, kRowThreads, 0, s>>>(logits, dt, K, V, nseg, n_drafts, inv_t, top_k, use_p ? 1 : 0,
                                                       top_p, tau, state, info, hcnt, hmass, segsum);
        sample_kept_kernel<<<dim3(nseg, B), kSegThreads, 0, s>>>(logits, dt, K, V, nseg, n_drafts, inv_t, state, info,
                                                                 segkept);
    }
    sample_draw_kernel<<<B, kRowThreads, 0, s>>>(logits, dt, K, V, nseg, n_drafts, inv_t, filtered ? 1 : 0, uniforms,
                                                 tau, state, info, segsum, segkept, out_tok);
    const int slots = B < kExactSlots ? B : kExactSlots;
    sample_exact_kernel<<<slots, kRowThreads, 0, s>>>(logits, dt, B, K, V, n_drafts, inv_t, top_k, top_p, uniforms,
                                                      state, w + L.exact, L.slot_bytes, L.vpad, (int)L.npow, out_tok);
    return check_hip(hipGetLastError(), "accept_greedy_sample launch");
}

}  // namespace gg
