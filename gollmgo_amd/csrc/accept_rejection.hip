// accept_rejection.hip — speculative (rejection) sampling acceptance on the device.
//
// The reference accepts greedily only (internal/engine/speculative.go:68-84) and
// samples the bonus token with Sampler.Sample (internal/engine/serving.go:560-565,
// internal/engine/sampling.go:40-72). This file implements speculative sampling
// (Leviathan et al. 2023, Alg. 1; Chen et al. 2023) with that sampler's rules:
// temperature as logit*(1/T) (sampling.go:59-62), softmax with -inf -> 0
// (sampling.go:112-136), the top-p nucleus kept in descending order while the
// mass before an item is below p (sampling.go:139-173), and the categorical
// draw "first index whose running sum exceeds u" (sampling.go:176-192).
//
// Arithmetic is exact integer fixed point (see gg_fixed_exp.h): w_i =
// floor(exp((l_i - max)/T) * 2^35); nucleus order is (logit desc, index asc).
//   kernel 1 (row_stats), one 1024-thread block per (sequence, row <= n):
//     max; Z = sum w; with top-p the boundary logit of the nucleus is found by a
//     2048-bin histogram of (max-l)/T in 1/64-nat slices followed by three
//     11/11/10-bit radix levels on the order key (LDS u64 atomics: exact), and a
//     9+9-bit index select when the boundary value is tied and cut.
//   kernel 2 (decide), one block per sequence: walks the drafts
//     (accept iff u*q(x)*Zp < w(x)), then draws the corrected token from
//     max(0, w - floor(q*Zp)) or the bonus token from row n with a block-wide
//     exclusive scan over the row.
#pragma clang fp contract(off)

#include "gg_common.h"
#include "gg_fixed_exp.h"

namespace gg {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kBins = 2048;
typedef unsigned long long u64;

struct RowStats {
    float m;          // max finite logit (or -inf when none)
    int idx_cut;      // ties at the boundary key are kept for index <= idx_cut
    u64 zp;           // nucleus mass (== Z without top-p)
    unsigned int lam; // boundary order key (0 = keep every finite logit)
    int valid;        // row was evaluated
    u64 wx;           // weight of the drafted token (0 if outside the nucleus)
};

__device__ __forceinline__ u64 shfl_xor_u64(u64 v, int o) {
    unsigned int lo = (unsigned int)v, hi = (unsigned int)(v >> 32);
    lo = __shfl_xor(lo, o);
    hi = __shfl_xor(hi, o);
    return ((u64)hi << 32) | lo;
}
__device__ __forceinline__ u64 shfl_up_u64(u64 v, int o) {
    unsigned int lo = (unsigned int)v, hi = (unsigned int)(v >> 32);
    lo = __shfl_up(lo, o);
    hi = __shfl_up(hi, o);
    return ((u64)hi << 32) | lo;
}

__device__ u64 block_sum_u64(u64 v, u64* red) {
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    u64 t = 0;
    for (int i = 0; i < kWaves; ++i) t += red[i];
    return t;
}

__device__ float block_max_f(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < kWaves; ++i) t = fmaxf(t, red[i]);
    return t;
}

__device__ int block_max_i(int v, int* red) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    int t = red[0];
    for (int i = 1; i < kWaves; ++i) t = max(t, red[i]);
    return t;
}

__device__ __forceinline__ bool finite_f(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// Wave 0 scans the histogram from bin `top` downward (descending key order when
// `desc`) and returns the LAST non-empty bin whose mass-above C satisfies C < tp ||
// C == 0; *c_above receives its C. Bins are ordered so that larger logits come first.
__device__ void pick_bin(const u64* mass, const unsigned int* cnt, int nbins, bool desc, u64 base,
                         u64 tp, int* out_bin, u64* out_c) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const int per = nbins / 64;
    // Logical position p runs over bins in order of decreasing logit.
    auto bin_at = [&](int p) { return desc ? nbins - 1 - p : p; };
    u64 local = 0;
    for (int k = 0; k < per; ++k) local += mass[bin_at(lane * per + k)];
    // Exclusive prefix over lanes.
    u64 incl = local;
    for (int o = 1; o < 64; o <<= 1) {
        u64 t = shfl_up_u64(incl, o);
        if (lane >= o) incl += t;
    }
    u64 c = base + incl - local;
    int best = -1;
    u64 best_c = 0;
    for (int k = 0; k < per; ++k) {
        const int bn = bin_at(lane * per + k);
        if (cnt[bn] > 0 && (c < tp || c == 0)) {
            best = lane * per + k;
            best_c = c;
        }
        c += mass[bn];
    }
    // Highest qualifying logical position across lanes.
    int bp = best;
    for (int o = 32; o > 0; o >>= 1) bp = max(bp, __shfl_xor(bp, o));
    if (best == bp && best >= 0) {
        *out_bin = bin_at(bp);
        *out_c = best_c;
    }
}

template <gg_dtype_t DT>
__device__ __forceinline__ float ld(const void* p, size_t i) {
    if constexpr (DT == GG_DTYPE_F32) return ((const float*)p)[i];
    else if constexpr (DT == GG_DTYPE_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    else return f16_bits_to_f32(((const uint16_t*)p)[i]);
}

struct Nucleus {
    float m, inv_t;
    unsigned int lam;
    int idx_cut;
    __device__ __forceinline__ bool kept(float l, int i) const {
        if (!finite_f(l)) return false;
        const unsigned int k = gg_order_key(l);
        return k > lam || (k == lam && i <= idx_cut);
    }
    __device__ __forceinline__ u64 weight(float l, int i) const {
        return kept(l, i) ? gg_weight(l, m, inv_t) : 0ull;
    }
};

template <gg_dtype_t DT>
__global__ void __launch_bounds__(kThreads) rejection_row_stats_kernel(
    const void* __restrict__ logits, int K, int V, const int32_t* __restrict__ drafts,
    const int32_t* __restrict__ n_drafts, float inv_t, float top_p, int use_topp,
    RowStats* __restrict__ stats) {
    const int row = blockIdx.x;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);

    __shared__ u64 hmass[kBins];
    __shared__ unsigned int hcnt[kBins];
    __shared__ u64 red64[kWaves];
    __shared__ float redf[kWaves];
    __shared__ int redi[kWaves];
    __shared__ int s_bin;
    __shared__ u64 s_c;

    // Pass 1: max over finite logits.
    float m = -INFINITY;
    for (int i = threadIdx.x; i < V; i += kThreads) {
        const float l = ld<DT>(lp, i);
        if (finite_f(l)) m = fmaxf(m, l);
    }
    m = block_max_f(m, redf);

    RowStats st{};
    st.m = m;
    st.valid = 1;
    st.lam = 0;
    st.idx_cut = 0x7fffffff;
    if (!finite_f(m)) {
        // No finite logit: every weight is zero.
        if (threadIdx.x == 0) {
            st.zp = 0;
            st.wx = 0;
            stats[row] = st;
        }
        return;
    }

    // Pass 2: Z (and the coarse histogram when top-p is on).
    if (use_topp) {
        for (int i = threadIdx.x; i < kBins; i += kThreads) {
            hmass[i] = 0;
            hcnt[i] = 0;
        }
        __syncthreads();
    }
    u64 z = 0;
    for (int i = threadIdx.x; i < V; i += kThreads) {
        const float l = ld<DT>(lp, i);
        if (!finite_f(l)) continue;
        const u64 w = gg_weight(l, m, inv_t);
        z += w;
        if (use_topp) {
            const int bn = gg_coarse_bin(l, m, inv_t);
            atomicAdd(&hmass[bn], w);
            atomicAdd(&hcnt[bn], 1u);
        }
    }
    z = block_sum_u64(z, red64);

    u64 zp = z;
    unsigned int lam = 0;
    int idx_cut = 0x7fffffff;
    if (use_topp && z > 0) {
        const u64 tp = (u64)ceil((double)top_p * (double)z);
        __syncthreads();
        pick_bin(hmass, hcnt, kBins, false, 0, tp, &s_bin, &s_c);
        __syncthreads();
        const int cbin = s_bin;
        u64 c_above = s_c;
        // Radix levels over the order key of elements in the coarse bin.
        unsigned int prefix = 0, pmask = 0;
        const int shifts[3] = {21, 10, 0};
        const int widths[3] = {11, 11, 10};
        for (int lv = 0; lv < 3; ++lv) {
            const int nb = 1 << widths[lv];
            __syncthreads();
            for (int i = threadIdx.x; i < kBins; i += kThreads) {
                hmass[i] = 0;
                hcnt[i] = 0;
            }
            __syncthreads();
            for (int i = threadIdx.x; i < V; i += kThreads) {
                const float l = ld<DT>(lp, i);
                if (!finite_f(l)) continue;
                if (gg_coarse_bin(l, m, inv_t) != cbin) continue;
                const unsigned int key = gg_order_key(l);
                if ((key & pmask) != prefix) continue;
                const int d = (key >> shifts[lv]) & (nb - 1);
                atomicAdd(&hmass[d], gg_weight(l, m, inv_t));
                atomicAdd(&hcnt[d], 1u);
            }
            __syncthreads();
            // Pad unused bins (10-bit level) with empties: the scan covers kBins.
            pick_bin(hmass, hcnt, kBins, true, c_above, tp, &s_bin, &s_c);
            __syncthreads();
            const unsigned int dsel = (unsigned int)s_bin;
            c_above = s_c;
            prefix |= dsel << shifts[lv];
            pmask |= (unsigned int)(nb - 1) << shifts[lv];
        }
        lam = prefix;
        // Ties at the boundary key: count and weight.
        const unsigned int n_tie = hcnt[prefix & 0x3ff];
        const u64 m_tie = hmass[prefix & 0x3ff];
        const u64 w_tie = n_tie ? m_tie / n_tie : 0;
        u64 n_keep = n_tie;
        if (w_tie > 0) {
            const u64 need = (tp - c_above + w_tie - 1) / w_tie;
            if (need < n_keep) n_keep = need;
        }
        zp = c_above + n_keep * w_tie;
        if (n_keep < n_tie) {
            // Index of the n_keep-th smallest index among the ties (two 9-bit levels).
            unsigned int iprefix = 0, imask = 0;
            unsigned int remaining = (unsigned int)n_keep;  // >= 1
            const int ish[2] = {9, 0};
            for (int lv = 0; lv < 2; ++lv) {
                __syncthreads();
                for (int i = threadIdx.x; i < 512; i += kThreads) hcnt[i] = 0;
                __syncthreads();
                for (int i = threadIdx.x; i < V; i += kThreads) {
                    const float l = ld<DT>(lp, i);
                    if (!finite_f(l) || gg_order_key(l) != lam) continue;
                    if (((unsigned int)i & imask) != iprefix) continue;
                    atomicAdd(&hcnt[((unsigned int)i >> ish[lv]) & 511u], 1u);
                }
                __syncthreads();
                if (threadIdx.x == 0) {
                    unsigned int acc = 0;
                    int d = 0;
                    for (; d < 512; ++d) {
                        if (acc + hcnt[d] >= remaining) break;
                        acc += hcnt[d];
                    }
                    s_bin = d;
                    s_c = acc;
                }
                __syncthreads();
                remaining -= (unsigned int)s_c;
                iprefix |= (unsigned int)s_bin << ish[lv];
                imask |= 511u << ish[lv];
            }
            idx_cut = (int)iprefix;
        }
    }

    if (threadIdx.x == 0) {
        st.zp = zp;
        st.lam = lam;
        st.idx_cut = idx_cut;
        st.wx = 0;
        if (j < n) {
            const int x = drafts[(size_t)b * K + j];
            if (x >= 0 && x < V) {
                Nucleus nu{m, inv_t, lam, idx_cut};
                st.wx = nu.weight(ld<DT>(lp, x), x);
            }
        }
        stats[row] = st;
    }
}

// Block-wide inclusive scan of u64 (1024 threads), returns inclusive value.
__device__ u64 block_scan_u64(u64 v, u64* red, u64* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    u64 incl = v;
    for (int o = 1; o < 64; o <<= 1) {
        u64 t = shfl_up_u64(incl, o);
        if (lane >= o) incl += t;
    }
    __syncthreads();
    if (lane == 63) red[w] = incl;
    __syncthreads();
    u64 before = 0, tot = 0;
    for (int i = 0; i < kWaves; ++i) {
        if (i < w) before += red[i];
        tot += red[i];
    }
    *total = tot;
    return before + incl;
}

template <gg_dtype_t DT>
__global__ void __launch_bounds__(kThreads) rejection_decide_kernel(
    const void* __restrict__ logits, const float* __restrict__ dprobs, int K, int V,
    const int32_t* __restrict__ drafts, const int32_t* __restrict__ n_drafts,
    const float* __restrict__ uniforms, float inv_t, const RowStats* __restrict__ stats,
    int32_t* __restrict__ out_acc, int32_t* __restrict__ out_tok) {
    const int b = blockIdx.x;
    const int R = K + 1;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    __shared__ u64 red64[kWaves];
    __shared__ int redi[kWaves];
    __shared__ int s_found;

    // Sequential acceptance walk (uniform across the block).
    int a = n;
    for (int j = 0; j < n; ++j) {
        const RowStats& st = stats[(size_t)b * R + j];
        const int x = drafts[(size_t)b * K + j];
        double q = 1.0;
        if (dprobs) q = (x >= 0 && x < V) ? (double)dprobs[((size_t)b * K + j) * V + x] : 0.0;
        const double u = (double)uniforms[(size_t)b * R + j];
        const bool ok = (x >= 0 && x < V) && (u * q * (double)st.zp < (double)st.wx);
        if (!ok) {
            a = j;
            break;
        }
    }
    const bool residual = a < n;
    const int f = a;  // row of the final draw
    const RowStats st = stats[(size_t)b * R + f];
    const void* lp = (const uint8_t*)logits + (size_t)((size_t)b * R + f) * V * dtype_bytes(DT);
    Nucleus nu{st.m, inv_t, st.lam, st.idx_cut};
    const float* qrow = (residual && dprobs) ? dprobs + ((size_t)b * K + f) * V : nullptr;
    const int xr = residual ? drafts[(size_t)b * K + f] : -1;
    const double zp_d = (double)st.zp;

    auto r_at = [&](int i, bool use_res) -> u64 {
        if (!finite_f(st.m)) return 0ull;
        const u64 w = nu.weight(ld<DT>(lp, i), i);
        if (!use_res) return w;
        u64 qf;
        if (qrow) qf = (u64)(qrow[i] < 0.f ? 0.0 : (double)qrow[i] * zp_d);
        else qf = (i == xr) ? st.zp : 0ull;
        return w > qf ? w - qf : 0ull;
    };

    bool use_res = residual;
    u64 tot = 0;
    int last_nz = -1;
    for (int pass = 0; pass < 2; ++pass) {
        u64 s = 0;
        int lnz = -1;
        for (int i = threadIdx.x; i < V; i += kThreads) {
            const u64 r = r_at(i, use_res);
            s += r;
            if (r) lnz = i;
        }
        tot = block_sum_u64(s, red64);
        last_nz = block_max_i(lnz, redi);
        if (tot > 0 || !use_res) break;
        use_res = false;  // residual vanished: draw from the target row itself
    }
    int token = 0;
    if (tot > 0) {
        const double u = (double)uniforms[(size_t)b * R + K];
        const u64 t = (u64)(u * (double)tot);
        if (threadIdx.x == 0) s_found = -1;
        u64 carry = 0;
        for (int base = 0; base < V; base += kThreads) {
            const int i = base + threadIdx.x;
            const u64 r = i < V ? r_at(i, use_res) : 0ull;
            u64 tile_total;
            const u64 incl = block_scan_u64(r, red64, &tile_total) + carry;
            const bool hit = r > 0 && incl > t && (incl - r) <= t;
            __syncthreads();
            if (hit) s_found = i;
            __syncthreads();
            if (s_found >= 0) break;
            carry += tile_total;
        }
        token = s_found >= 0 ? s_found : (last_nz >= 0 ? last_nz : 0);
    }
    if (threadIdx.x == 0) {
        out_acc[b] = a;
        out_tok[b] = token;
    }
}

}  // namespace

size_t rejection_workspace_bytes(int num_seqs, int max_drafts, int vocab) {
    size_t own = (size_t)num_seqs * (max_drafts + 1) * sizeof(RowStats);
    size_t g = greedy_workspace_bytes(num_seqs, max_drafts, vocab);
    return own > g ? own : g;
}

gg_status_t launch_accept_rejection(const void* logits, gg_dtype_t dt, const float* q, int num_seqs,
                                    int max_drafts, int vocab, const int32_t* drafts,
                                    const int32_t* n_drafts, const float* uniforms, float temperature,
                                    float top_p, int32_t* out_acc, int32_t* out_tok, void* ws,
                                    hipStream_t s) {
    const float inv_t = 1.0f / temperature;
    const int use_topp = (top_p > 0.f && top_p < 1.f) ? 1 : 0;
    RowStats* st = (RowStats*)ws;
    const int rows = num_seqs * (max_drafts + 1);
#define GG_REJ(DTV)                                                                                  \
    rejection_row_stats_kernel<DTV><<<rows, kThreads, 0, s>>>(logits, max_drafts, vocab, drafts,     \
                                                              n_drafts, inv_t, top_p, use_topp, st); \
    rejection_decide_kernel<DTV><<<num_seqs, kThreads, 0, s>>>(logits, q, max_drafts, vocab, drafts, \
                                                               n_drafts, uniforms, inv_t, st,        \
                                                               out_acc, out_tok);
    switch (dt) {
        case GG_DTYPE_F32: GG_REJ(GG_DTYPE_F32) break;
        case GG_DTYPE_BF16: GG_REJ(GG_DTYPE_BF16) break;
        case GG_DTYPE_F16: GG_REJ(GG_DTYPE_F16) break;
        default: return fail(GG_ERR_INVALID, "accept_rejection: logits dtype");
    }
#undef GG_REJ
    return check_hip(hipGetLastError(), "accept_rejection launch");
}

}  // namespace gg
