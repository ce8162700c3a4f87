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
//     Without top-p the same statistics come from two segmented launches (segment
//     max, then segment sums of w) over (row, 8192-logit segment) blocks.
//   draw sums, one block per (sequence, segment): walks the drafts (accept iff
//     u*q(x)*Zp < w(x)), then sums the final row's segment of max(0, w -
//     floor(q*Zp)) (first rejection) or of w (bonus, row n);
//   draw find, one block per sequence: locates floor(u*total) among the segment sums,
//     then inside that one segment.
// The draft distributions are read only at drafted tokens and on the final row.
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

constexpr int kCandCap = 4096;
constexpr int kFindThreads = 1024;  // draw find: threads per sequence

// Coarse-bin masses of one row. (Only the mass: weights do not increase down the bins,
// so a bin with no mass sits where the whole row's mass lies before it and can never
// hold the boundary; the boundary bin's element count comes from the gather.)
struct RowHist {
    u64 mass[kBins];
};

struct RowPick {
    int cbin;        // boundary coarse bin (-1: nothing to resolve)
    int n_cand;      // elements of that bin gathered so far
    u64 c_above;     // mass of the bins before it
    u64 tp;          // ceil(top_p * Z)
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
// `desc`) and returns the LAST non-empty bin (count > 0; mass > 0 when cnt is null)
// whose mass-above C satisfies C < tp || C == 0; *c_above receives its C. Bins are ordered so that larger logits come first.
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
        const bool nonempty = cnt ? cnt[bn] > 0 : mass[bn] > 0;
        if (nonempty && (c < tp || c == 0)) {
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

// Exact per-row statistics in one 1024-thread block (passes over the whole row). With
// `only_flagged`, rows whose nucleus boundary the segmented path already resolved
// (flag 0) are skipped: this kernel is then the fallback for crowded boundary bins.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kThreads) rejection_row_stats_kernel(
    const void* __restrict__ logits, int K, int V, const int32_t* __restrict__ drafts,
    const int32_t* __restrict__ n_drafts, float inv_t, float top_p, int use_topp,
    RowStats* __restrict__ stats, const int* __restrict__ only_flagged) {
    const int row = blockIdx.x;
    if (only_flagged && only_flagged[row] == 0) return;
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
// ---------------------------------------------------------------------------
// Segmented path. A row of V logits is cut into segments of kSegElems; every
// (row, segment) pair is one 256-thread block, so a launch has thousands of blocks.
// All cross-segment combinations are max of floats or sums of integers: exact and
// order-free, so the result is the same bit pattern whatever the schedule.

constexpr int kSegThreads = 256;
constexpr int kSegElems = 8192;  // 32 logits per thread
// Segments per block of the top-p weight launch (measured on MI355X, config 5: one, two,
// four or sixteen segments per block take 418, 387, 382, 391 µs per acceptance call).
constexpr int kZhistSegs = 4;

struct SegOut {
    u64 sum_res;     // residual weights of the segment (final row)
    u64 sum_plain;   // nucleus weights of the segment (final row)
    int last_res;    // last index with a non-zero residual weight (-1: none)
    int last_plain;
};

struct SeqDecision {
    int accepted;
    int row;         // row of the final draw
    int residual;    // 1: draw from max(0, w - floor(q*Zp)), 0: from w
};

__device__ __forceinline__ float seg_block_max(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
    for (int i = 1; i < kSegThreads / 64; ++i) t = fmaxf(t, red[i]);
    return t;
}
__device__ __forceinline__ u64 seg_block_sum(u64 v, u64* red) {
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    u64 t = 0;
    for (int i = 0; i < kSegThreads / 64; ++i) t += red[i];
    return t;
}
__device__ __forceinline__ int seg_block_maxi(int v, int* red) {
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    int t = red[0];
    for (int i = 1; i < kSegThreads / 64; ++i) t = max(t, red[i]);
    return t;
}

// The 32 logits a thread owns in a segment: elements base + 8*threadIdx + {0..7} of each
// of the four 2048-element quarters (16-byte loads; scalar fallback for odd rows).
template <gg_dtype_t DT>
__device__ __forceinline__ void load_seg(const void* row, int V, int seg, bool vec_ok, float (&x)[32],
                                         int (&idx)[32]) {
    const int base = seg * kSegElems;
#pragma unroll
    for (int qtr = 0; qtr < 4; ++qtr) {
        const int e0 = base + qtr * 2048 + 8 * threadIdx.x;
#pragma unroll
        for (int k = 0; k < 8; ++k) idx[qtr * 8 + k] = e0 + k;
        if (vec_ok && e0 + 8 <= V) {
            if constexpr (DT == GG_DTYPE_F32) {
                const float4 a = *(const float4*)((const float*)row + e0);
                const float4 b = *(const float4*)((const float*)row + e0 + 4);
                x[qtr * 8 + 0] = a.x; x[qtr * 8 + 1] = a.y; x[qtr * 8 + 2] = a.z; x[qtr * 8 + 3] = a.w;
                x[qtr * 8 + 4] = b.x; x[qtr * 8 + 5] = b.y; x[qtr * 8 + 6] = b.z; x[qtr * 8 + 7] = b.w;
            } else {
                const uint4 r = *(const uint4*)((const uint16_t*)row + e0);
                const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint16_t h = (uint16_t)(w[k >> 1] >> ((k & 1) * 16));
                    x[qtr * 8 + k] = DT == GG_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) x[qtr * 8 + k] = (e0 + k < V) ? ld<DT>(row, e0 + k) : NAN;
        }
    }
}

// A: per (row, segment) max over finite logits.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) seg_max_kernel(const void* __restrict__ logits, int K, int V,
                                                              int nseg, int vec_ok,
                                                              const int32_t* __restrict__ n_drafts,
                                                              float* __restrict__ seg_max, void* __restrict__ hist) {
    const int seg = blockIdx.x, row = blockIdx.y;
    // Top-p: segment 0 clears the row's coarse histogram for the weight launch.
    if (hist && seg == 0) {
        u64* h = (u64*)hist + (size_t)row * (sizeof(RowHist) / sizeof(u64));
        for (int i = threadIdx.x; i < (int)(sizeof(RowHist) / sizeof(u64)); i += kSegThreads) h[i] = 0;
    }
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    float x[32];
    int idx[32];
    load_seg<DT>(lp, V, seg, vec_ok, x, idx);
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if (finite_f(x[k])) m = fmaxf(m, x[k]);
    __shared__ float red[kSegThreads / 64];
    m = seg_block_max(m, red);
    if (threadIdx.x == 0) seg_max[(size_t)row * nseg + seg] = m;
}

// Row max and weight sum over the per-segment values, by a whole wave (lane s reads
// segment s; nseg <= 64): one load round trip rather than a chain of nseg, which every
// block of a launch would otherwise wait for.
__device__ __forceinline__ float row_max_wave(const float* seg_max, int row, int nseg) {
    const int lane = threadIdx.x & 63;
    float m = lane < nseg ? seg_max[(size_t)row * nseg + lane] : -INFINITY;
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    return m;
}
__device__ __forceinline__ u64 row_z_wave(const u64* seg_z, int row, int nseg) {
    const int lane = threadIdx.x & 63;
    u64 z = lane < nseg ? seg_z[(size_t)row * nseg + lane] : 0ull;
    for (int o = 32; o > 0; o >>= 1) z += shfl_xor_u64(z, o);
    return z;
}

// B: per (row, segment) sum of fixed-point weights.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) seg_z_kernel(const void* __restrict__ logits, int K, int V,
                                                            int nseg, int vec_ok, float inv_t,
                                                            const int32_t* __restrict__ n_drafts,
                                                            const float* __restrict__ seg_max,
                                                            u64* __restrict__ seg_z) {
    const int seg = blockIdx.x, row = blockIdx.y;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    __shared__ u64 red[kSegThreads / 64];
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    float x[32];
    int idx[32];
    load_seg<DT>(lp, V, seg, vec_ok, x, idx);
    const float m = row_max_wave(seg_max, row, nseg);  // (requested after the segment)
    u64 z = 0;
    if (finite_f(m)) {
#pragma unroll
        for (int k = 0; k < 32; ++k)
            if (finite_f(x[k])) z += gg_weight(x[k], m, inv_t);
    }
    z = seg_block_sum(z, red);
    if (threadIdx.x == 0) seg_z[(size_t)row * nseg + seg] = z;
}

// ---- Segmented top-p: the nucleus boundary without whole-row passes per block ----
//
// The boundary is the last element, in (logit desc, index asc) order, whose mass before
// it is below Tp = ceil(p*Z) (or zero). Coarse bins of 1/64 nat on (m - l)/T are ordered
// the same way, so: (B') the weights of each segment also go into a per-row histogram of
// coarse bins (integer sums: exact in any order); (C') a block per row finds the boundary
// bin and the mass above it; (D') the elements of that bin are gathered (usually a few
// hundred); (E') a block per row sorts them by (key desc, index asc) and walks the
// weights to the cut. A bin with more than kCandCap elements flags its row for the exact
// row kernel instead.

// B': per (row, segment) weight sum and coarse histogram (the row's histogram and pick
// were cleared by segment 0 of the max launch).
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) seg_zhist_kernel(const void* __restrict__ logits, int K, int V,
                                                                int nseg, int vec_ok, float inv_t,
                                                                const int32_t* __restrict__ n_drafts,
                                                                const float* __restrict__ seg_max,
                                                                u64* __restrict__ seg_z, RowHist* __restrict__ hist) {
    const int row = blockIdx.y;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    __shared__ u64 red[kSegThreads / 64];
    __shared__ u64 h_mass[kBins];
    for (int i = threadIdx.x; i < kBins; i += kSegThreads) h_mass[i] = 0;
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    // kZhistSegs consecutive segments per block: their weights meet in one LDS histogram,
    // flushed to the row's once (the global atomics are the launch's cost, not the loads).
    // The next segment's logits are requested before the current one is weighed.
    const int seg0 = blockIdx.x * kZhistSegs;
    const int seg1 = min(seg0 + kZhistSegs, nseg);
    float xn[32];
    int idxn[32];
    load_seg<DT>(lp, V, seg0, vec_ok, xn, idxn);
    const float m = row_max_wave(seg_max, row, nseg);  // (requested after the first segment)
    __syncthreads();  // the cleared histogram
    for (int seg = seg0; seg < seg1; ++seg) {
        float x[32];
#pragma unroll
        for (int k = 0; k < 32; ++k) x[k] = xn[k];
        if (seg + 1 < seg1) load_seg<DT>(lp, V, seg + 1, vec_ok, xn, idxn);
        u64 z = 0;
        if (finite_f(m)) {
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const bool fin = finite_f(x[k]);
                const u64 w = fin ? gg_weight(x[k], m, inv_t) : 0ull;
                z += w;
                if (w) atomicAdd(&h_mass[gg_coarse_bin(x[k], m, inv_t)], w);
            }
        }
        z = seg_block_sum(z, red);  // (its barriers also complete the LDS histogram)
        if (threadIdx.x == 0) seg_z[(size_t)row * nseg + seg] = z;
    }
    RowHist& h = hist[row];
    for (int i = threadIdx.x; i < kBins; i += kSegThreads) {
        if (h_mass[i]) atomicAdd(&h.mass[i], h_mass[i]);
    }
}

// C': per row, the boundary coarse bin and the mass above it.
__global__ void __launch_bounds__(kSegThreads) row_pick_kernel(int K, int nseg, float top_p,
                                                               const int32_t* __restrict__ n_drafts,
                                                               const float* __restrict__ seg_max,
                                                               const u64* __restrict__ seg_z,
                                                               const RowHist* __restrict__ hist,
                                                               RowPick* __restrict__ pick) {
    const int row = blockIdx.x;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    __shared__ int s_bin;
    __shared__ u64 s_c;
    const float m = row_max_wave(seg_max, row, nseg);
    const u64 z = row_z_wave(seg_z, row, nseg);
    if (!finite_f(m) || z == 0) {
        if (threadIdx.x == 0) pick[row] = RowPick{-1, 0, 0, 0};
        return;
    }
    const u64 tp = (u64)ceil((double)top_p * (double)z);
    if (threadIdx.x == 0) s_bin = -1;
    __syncthreads();
    pick_bin(hist[row].mass, nullptr, kBins, false, 0, tp, &s_bin, &s_c);
    __syncthreads();
    if (threadIdx.x == 0) pick[row] = RowPick{s_bin, 0, s_c, tp};
}

// D': per (row, segment), gather the elements of the boundary bin.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) seg_gather_kernel(const void* __restrict__ logits, int K, int V,
                                                                 int nseg, int vec_ok, float inv_t,
                                                                 const int32_t* __restrict__ n_drafts,
                                                                 const float* __restrict__ seg_max,
                                                                 RowPick* __restrict__ pick,
                                                                 uint2* __restrict__ cand) {
    const int seg = blockIdx.x, row = blockIdx.y;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    float x[32];
    int idx[32];
    load_seg<DT>(lp, V, seg, vec_ok, x, idx);
    // The boundary bin and the row max are requested after the segment.
    const int cbin = pick[row].cbin;
    const float m = row_max_wave(seg_max, row, nseg);
    if (cbin < 0) return;
    // The lane's hits as a bit mask first (vector work only), then one counter update per
    // lane that has any, and its candidates written in order.
    uint32_t hits = 0;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const bool hit = idx[k] < V && finite_f(x[k]) && gg_coarse_bin(x[k], m, inv_t) == cbin;
        hits |= (uint32_t)hit << k;
    }
    if (hits) {
        int slot = atomicAdd(&pick[row].n_cand, __popc(hits));
        while (hits) {
            const int k = __ffs(hits) - 1;
            hits &= hits - 1;
            float xv = 0.f;
            int iv = 0;
#pragma unroll
            for (int kk = 0; kk < 32; ++kk)
                if (kk == k) xv = x[kk], iv = idx[kk];
            if (slot < kCandCap) cand[(size_t)row * kCandCap + slot] = make_uint2(__float_as_uint(xv), (unsigned)iv);
            ++slot;
        }
    }
}

// E': per row, sort the boundary bin's elements by (key desc, index asc) and cut; fills
// the row's statistics, or flags the row for the exact row kernel (too many elements).
template <gg_dtype_t DT>
__global__ void __launch_bounds__(1024) row_select_kernel(const void* __restrict__ logits, int K, int V,
                                                          int nseg, float inv_t,
                                                          const int32_t* __restrict__ drafts,
                                                          const int32_t* __restrict__ n_drafts,
                                                          const float* __restrict__ seg_max,
                                                          const RowPick* __restrict__ pick,
                                                          const uint2* __restrict__ cand,
                                                          RowStats* __restrict__ stats, int* __restrict__ flag) {
    const int row = blockIdx.x;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    if (j > n) return;
    __shared__ u64 s_key[kCandCap];    // order key << 32 | (~index): descending = the nucleus order
    __shared__ u64 red[1024 / 64];
    __shared__ int s_last;
    const RowPick pk = pick[row];
    const float m = row_max_wave(seg_max, row, nseg);
    if (pk.cbin < 0) {  // no finite logit or Z == 0: no nucleus
        if (threadIdx.x == 0) {
            stats[row] = RowStats{m, 0x7fffffff, 0ull, 0u, 1, 0ull};
            flag[row] = 0;
        }
        return;
    }
    const int nc = pk.n_cand;
    if (nc > kCandCap) {
        if (threadIdx.x == 0) flag[row] = 1;
        return;
    }
    int np2 = 1;
    while (np2 < nc) np2 <<= 1;
    for (int i = threadIdx.x; i < np2; i += 1024) {
        if (i < nc) {
            const uint2 c = cand[(size_t)row * kCandCap + i];
            s_key[i] = ((u64)gg_order_key(__uint_as_float(c.x)) << 32) | (u64)(~c.y);
        } else {
            s_key[i] = 0;  // sorts last
        }
    }
    __syncthreads();
    // Bitonic sort, descending.
    for (int k = 2; k <= np2; k <<= 1) {
        for (int jj = k >> 1; jj > 0; jj >>= 1) {
            for (int i = threadIdx.x; i < np2; i += 1024) {
                const int ix = i ^ jj;
                if (ix > i) {
                    const u64 a = s_key[i], c = s_key[ix];
                    const bool desc = (i & k) == 0;
                    if (desc ? (a < c) : (a > c)) {
                        s_key[i] = c;
                        s_key[ix] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    // Weights in that order (the logit is recovered from the order key). Thread t owns
    // elements [4t, 4t+4): an exclusive block scan of the thread sums gives each
    // element's mass before it; the kept elements are a prefix (that mass never drops),
    // so the cut is the largest kept position.
    const int e0 = 4 * (int)threadIdx.x;
    u64 w[4];
    u64 tsum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w[k] = 0;
        if (e0 + k < nc) {
            const unsigned int key = (unsigned int)(s_key[e0 + k] >> 32);
            const unsigned int bits = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
            w[k] = gg_weight(__uint_as_float(bits), m, inv_t);
        }
        tsum += w[k];
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    u64 incl = tsum;
    for (int o = 1; o < 64; o <<= 1) {
        const u64 t = shfl_up_u64(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) red[wv] = incl;
    __syncthreads();
    u64 before = pk.c_above + incl - tsum;
    for (int i = 0; i < wv; ++i) before += red[i];
    int last = -1;
    u64 zp = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (e0 + k < nc && (before < pk.tp || before == 0)) {
            last = e0 + k;
            zp = before + w[k];
        }
        before += w[k];
    }
    if (threadIdx.x == 0) s_last = -1;
    __syncthreads();
    if (last >= 0) atomicMax(&s_last, last);
    __syncthreads();
    if (last >= 0 && last == s_last) {  // the owner of the cut (position 0 always qualifies)
        const unsigned int lam = (unsigned int)(s_key[last] >> 32);
        // Ties at the boundary key kept for index <= idx_cut; every index when all are.
        const bool all_ties = last + 1 >= nc || (unsigned int)(s_key[last + 1] >> 32) != lam;
        const int idx_cut = all_ties ? 0x7fffffff : (int)(~(unsigned int)(s_key[last] & 0xffffffffu));
        RowStats st{m, idx_cut, zp, lam, 1, 0ull};
        if (j < n) {
            const int x = drafts[(size_t)b * K + j];
            if (x >= 0 && x < V) {
                const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
                Nucleus nu{m, inv_t, lam, idx_cut};
                st.wx = nu.weight(ld<DT>(lp, x), x);
            }
        }
        stats[row] = st;
        flag[row] = 0;
    }
}

// Per-row statistics seen by the decision: max, nucleus mass and nucleus boundary.
struct RowView {
    float m;
    u64 zp;
    unsigned int lam;
    int idx_cut;
};

// The view of one row the decision needs (max, nucleus mass and boundary), evaluated by a
// whole wave: lane s < nseg reads segment s (nseg <= 64), the wave reduces. Every lane
// returns the same view.
__device__ __forceinline__ RowView row_view_wave(int row, int nseg, int use_topp, const RowStats* stats,
                                                 const float* seg_max, const u64* seg_z) {
    RowView v;
    if (use_topp) {
        const RowStats& st = stats[row];
        v.m = st.m;
        v.zp = st.zp;
        v.lam = st.lam;
        v.idx_cut = st.idx_cut;
        return v;
    }
    const int lane = threadIdx.x & 63;
    float m = lane < nseg ? seg_max[(size_t)row * nseg + lane] : -INFINITY;
    u64 z = lane < nseg ? seg_z[(size_t)row * nseg + lane] : 0ull;
    for (int o = 32; o > 0; o >>= 1) {
        m = fmaxf(m, __shfl_xor(m, o));
        z += shfl_xor_u64(z, o);
    }
    v.m = m;
    v.zp = z;
    v.lam = 0;
    v.idx_cut = 0x7fffffff;
    return v;
}

// The acceptance walk of one sequence, run by a whole wave (every lane gets the result).
// The rows' tests do not depend on each other, so they are evaluated together: groups of
// g = 2^ceil(log2 nseg) lanes take one row each (lane s of a group reads segment s), 64/g
// rows per pass; the walk then stops at the first failed row.
template <gg_dtype_t DT>
__device__ SeqDecision decide_seq_wave(const void* logits, const float* dprobs, int K, int V, int b, int n,
                                       const int32_t* drafts, const float* uniforms, float inv_t, int nseg,
                                       int use_topp, const RowStats* stats, const float* seg_max,
                                       const u64* seg_z) {
    const int R = K + 1;
    const int lane = threadIdx.x & 63;
    int g = 1;
    while (g < nseg) g <<= 1;
    const int per_pass = 64 / g;
    const int jl = lane / g, sl = lane % g;
    for (int j0 = 0; j0 < n; j0 += per_pass) {
        const int j = j0 + jl;
        const bool live = j < n;
        const int row = b * R + (live ? j : 0);
        float m;
        u64 zp;
        unsigned int lam = 0;
        int idx_cut = 0x7fffffff;
        if (use_topp) {
            const RowStats& st = stats[row];
            m = st.m;
            zp = st.zp;
            lam = st.lam;
            idx_cut = st.idx_cut;
        } else {
            m = sl < nseg ? seg_max[(size_t)row * nseg + sl] : -INFINITY;
            zp = sl < nseg ? seg_z[(size_t)row * nseg + sl] : 0ull;
            for (int o = g >> 1; o > 0; o >>= 1) {
                m = fmaxf(m, __shfl_xor(m, o));
                zp += shfl_xor_u64(zp, o);
            }
        }
        bool ok = true;
        if (live) {
            const int x = drafts[(size_t)b * K + j];
            ok = false;
            if (x >= 0 && x < V && finite_f(m)) {
                const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
                Nucleus nu{m, inv_t, lam, idx_cut};
                const u64 wx = nu.weight(ld<DT>(lp, x), x);
                const double q = dprobs ? (double)dprobs[((size_t)b * K + j) * V + x] : 1.0;
                const double u = (double)uniforms[(size_t)b * R + j];
                ok = u * q * (double)zp < (double)wx;
            }
        }
        const unsigned long long bad = __ballot(!ok && sl == 0);
        if (bad) {
            const int jf = j0 + (__ffsll((long long)bad) - 1) / g;
            return SeqDecision{jf, jf, 1};
        }
    }
    return SeqDecision{n, n, 0};
}

// D: per (sequence, segment): decide, then the segment's residual and plain weight
// sums on the final row (and the last non-zero index of each).
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) seg_draw_sums_kernel(
    const void* __restrict__ logits, const float* __restrict__ dprobs, int K, int V, int nseg, int vec_ok,
    float inv_t, int use_topp, const int32_t* __restrict__ drafts, const int32_t* __restrict__ n_drafts,
    const float* __restrict__ uniforms, const RowStats* __restrict__ stats,
    const float* __restrict__ seg_max, const u64* __restrict__ seg_z, SeqDecision* __restrict__ dec,
    SegOut* __restrict__ seg_out) {
    const int seg = blockIdx.x, b = blockIdx.y;
    const int R = K + 1;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    __shared__ SeqDecision s_d;
    __shared__ RowView s_rv;
    __shared__ u64 red[kSegThreads / 64];
    __shared__ int redi[kSegThreads / 64];
    if (threadIdx.x < 64) {
        const SeqDecision dd = decide_seq_wave<DT>(logits, dprobs, K, V, b, n, drafts, uniforms, inv_t, nseg,
                                                   use_topp, stats, seg_max, seg_z);
        const RowView rv = row_view_wave(b * R + dd.row, nseg, use_topp, stats, seg_max, seg_z);
        if (threadIdx.x == 0) {
            s_d = dd;
            s_rv = rv;
            if (seg == 0) dec[b] = dd;
        }
    }
    __syncthreads();
    const SeqDecision d = s_d;
    const RowView rv = s_rv;
    const int row = b * R + d.row;
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    float x[32];
    int idx[32];
    load_seg<DT>(lp, V, seg, vec_ok, x, idx);
    const Nucleus nu{rv.m, inv_t, rv.lam, rv.idx_cut};
    const float* qrow = (d.residual && dprobs) ? dprobs + ((size_t)b * K + d.row) * V : nullptr;
    const int xr = d.residual ? drafts[(size_t)b * K + d.row] : -1;
    const double zp_d = (double)rv.zp;
    u64 s_res = 0, s_pl = 0;
    int l_res = -1, l_pl = -1;
    const bool row_ok = finite_f(rv.m);
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int i = idx[k];
        if (i >= V || !row_ok) continue;
        const u64 w = nu.weight(x[k], i);
        u64 r = w;
        if (d.residual) {
            u64 qf;
            if (qrow) {
                const float qi = qrow[i];
                qf = (u64)(qi < 0.f ? 0.0 : (double)qi * zp_d);
            } else {
                qf = (i == xr) ? rv.zp : 0ull;
            }
            r = w > qf ? w - qf : 0ull;
        }
        s_res += r;
        s_pl += w;
        if (r) l_res = max(l_res, i);
        if (w) l_pl = max(l_pl, i);
    }
    s_res = seg_block_sum(s_res, red);
    s_pl = seg_block_sum(s_pl, red);
    l_res = seg_block_maxi(l_res, redi);
    l_pl = seg_block_maxi(l_pl, redi);
    if (threadIdx.x == 0) seg_out[(size_t)b * nseg + seg] = SegOut{s_res, s_pl, l_res, l_pl};
}

// E: per sequence: pick the segment holding floor(u * total), then the element inside it.
// Wave 0 reduces and scans the segment sums (lane s = segment s); in the chosen segment
// thread k of 1024 owns the 8 consecutive elements [8k, 8k+8) and a block scan of the
// thread sums finds the thread whose run crosses the target.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kFindThreads) seg_draw_find_kernel(
    const void* __restrict__ logits, const float* __restrict__ dprobs, int K, int V, int nseg, float inv_t,
    int use_topp, const int32_t* __restrict__ drafts, const float* __restrict__ uniforms,
    const RowStats* __restrict__ stats, const float* __restrict__ seg_max, const u64* __restrict__ seg_z,
    const SeqDecision* __restrict__ dec, const SegOut* __restrict__ seg_out, int32_t* __restrict__ out_acc,
    int32_t* __restrict__ out_tok) {
    const int b = blockIdx.x;
    const int R = K + 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __shared__ int s_seg, s_use_res, s_found;
    __shared__ u64 s_t;
    __shared__ u64 s_wsum[kFindThreads / 64];
    const SeqDecision d = dec[b];
    if (wave == 0) {
        const SegOut o = lane < nseg ? seg_out[(size_t)b * nseg + lane] : SegOut{0ull, 0ull, -1, -1};
        u64 tot_res = o.sum_res, tot_pl = o.sum_plain;
        int last_res = o.last_res, last_pl = o.last_plain;
        for (int off = 32; off > 0; off >>= 1) {
            tot_res += shfl_xor_u64(tot_res, off);
            tot_pl += shfl_xor_u64(tot_pl, off);
            last_res = max(last_res, __shfl_xor(last_res, off));
            last_pl = max(last_pl, __shfl_xor(last_pl, off));
        }
        // A vanished residual falls back to the target row itself.
        const int use_res = (d.residual && tot_res > 0) ? 1 : 0;
        const u64 tot = use_res ? tot_res : tot_pl;
        const int last = use_res ? last_res : last_pl;
        int seg = -1;
        u64 tt = 0;
        if (tot > 0) {
            const double u = (double)uniforms[(size_t)b * R + K];
            const u64 t = (u64)(u * (double)tot);
            const u64 v = use_res ? o.sum_res : o.sum_plain;
            u64 incl = v;
            for (int off = 1; off < 64; off <<= 1) {
                const u64 y = shfl_up_u64(incl, off);
                if (lane >= off) incl += y;
            }
            // First segment whose inclusive prefix passes t.
            const unsigned long long hit = __ballot(lane < nseg && incl > t);
            if (hit) {
                seg = __ffsll((long long)hit) - 1;
                const u64 excl = incl - v;
                tt = t - __shfl(excl, seg);
            }
        }
        if (lane == 0) {
            s_use_res = use_res;
            s_seg = seg;
            s_t = tt;
            s_found = tot > 0 ? (last >= 0 ? last : 0) : 0;  // no segment crosses (u >= 1)
            out_acc[b] = d.accepted;
        }
    }
    __syncthreads();
    if (s_seg < 0) {
        if (threadIdx.x == 0) out_tok[b] = s_found;
        return;
    }
    const int row = b * R + d.row;
    const RowView rv = row_view_wave(row, nseg, use_topp, stats, seg_max, seg_z);
    const Nucleus nu{rv.m, inv_t, rv.lam, rv.idx_cut};
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    const bool use_res = s_use_res;
    const float* qrow = (use_res && dprobs) ? dprobs + ((size_t)b * K + d.row) * V : nullptr;
    const int xr = use_res ? drafts[(size_t)b * K + d.row] : -1;
    const double zp_d = (double)rv.zp;
    constexpr int kPer = kSegElems / kFindThreads;
    const int e0 = s_seg * kSegElems + kPer * threadIdx.x;
    u64 r[kPer];
    u64 mine = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = e0 + k;
        u64 w = 0;
        if (i < V) {
            w = nu.weight(ld<DT>(lp, i), i);
            if (use_res) {
                u64 qf;
                if (qrow) {
                    const float qi = qrow[i];
                    qf = (u64)(qi < 0.f ? 0.0 : (double)qi * zp_d);
                } else {
                    qf = (i == xr) ? rv.zp : 0ull;
                }
                w = w > qf ? w - qf : 0ull;
            }
        }
        r[k] = w;
        mine += w;
    }
    // Exclusive block scan of the thread sums.
    u64 incl = mine;
    for (int off = 1; off < 64; off <<= 1) {
        const u64 y = shfl_up_u64(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    u64 before = incl - mine;
    for (int w = 0; w < wave; ++w) before += s_wsum[w];
    const u64 t = s_t;
    if (before <= t && before + mine > t) {
        u64 c = before;
        int found = e0 + kPer - 1;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            c += r[k];
            if (c > t) {
                found = e0 + k;
                break;
            }
        }
        s_found = found;
    }
    __syncthreads();
    if (threadIdx.x == 0) out_tok[b] = s_found;
}

}  // namespace

static int rej_nseg(int vocab) { return (vocab + kSegElems - 1) / kSegElems; }

struct RejWs {
    RowStats* stats;
    float* seg_max;
    u64* seg_z;
    SeqDecision* dec;
    SegOut* seg_out;
    RowHist* hist;   // top-p only: coarse histogram per row
    RowPick* pick;
    uint2* cand;     // boundary-bin elements per row (logit bits, index)
    int* flag;       // 1: the row needs the exact row kernel
    size_t bytes;
};

static RejWs rej_layout(void* base, int num_seqs, int max_drafts, int vocab, bool topp) {
    const size_t rows = (size_t)num_seqs * (max_drafts + 1);
    const int nseg = rej_nseg(vocab);
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    size_t off = 0;
    RejWs w{};
    uint8_t* p = (uint8_t*)base;
    w.stats = (RowStats*)(p + off);
    off += al(rows * sizeof(RowStats));
    w.seg_max = (float*)(p + off);
    off += al(rows * nseg * sizeof(float));
    w.seg_z = (u64*)(p + off);
    off += al(rows * nseg * sizeof(u64));
    w.dec = (SeqDecision*)(p + off);
    off += al((size_t)num_seqs * sizeof(SeqDecision));
    w.seg_out = (SegOut*)(p + off);
    off += al((size_t)num_seqs * nseg * sizeof(SegOut));
    if (topp) {
        w.hist = (RowHist*)(p + off);
        off += al(rows * sizeof(RowHist));
        w.pick = (RowPick*)(p + off);
        off += al(rows * sizeof(RowPick));
        w.cand = (uint2*)(p + off);
        off += al(rows * kCandCap * sizeof(uint2));
        w.flag = (int*)(p + off);
        off += al(rows * sizeof(int));
    }
    w.bytes = off;
    return w;
}

size_t rejection_workspace_bytes(int num_seqs, int max_drafts, int vocab) {
    size_t own = rej_layout(nullptr, num_seqs, max_drafts, vocab, true).bytes;
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
    const RejWs w = rej_layout(ws, num_seqs, max_drafts, vocab, use_topp != 0);
    const int rows = num_seqs * (max_drafts + 1);
    const int nseg = rej_nseg(vocab);
    const int K = max_drafts;
    const size_t eb = dtype_bytes(dt);
    const int vec_ok = ((vocab * eb) % 16 == 0) && (((uintptr_t)logits) % 16 == 0);
#define GG_REJ(DTV)                                                                                        \
    seg_max_kernel<DTV><<<dim3(nseg, rows), kSegThreads, 0, s>>>(logits, K, vocab, nseg, vec_ok, n_drafts,  \
                                                                 w.seg_max, use_topp ? w.hist : nullptr);  \
    if (use_topp) {                                                                                        \
        seg_zhist_kernel<DTV><<<dim3((nseg + kZhistSegs - 1) / kZhistSegs, rows), kSegThreads, 0, s>>>(                                    \
            logits, K, vocab, nseg, vec_ok, inv_t, n_drafts, w.seg_max, w.seg_z, w.hist);                  \
        row_pick_kernel<<<rows, kSegThreads, 0, s>>>(K, nseg, top_p, n_drafts, w.seg_max, w.seg_z, w.hist, \
                                                     w.pick);                                              \
        seg_gather_kernel<DTV><<<dim3(nseg, rows), kSegThreads, 0, s>>>(                                   \
            logits, K, vocab, nseg, vec_ok, inv_t, n_drafts, w.seg_max, w.pick, w.cand);                   \
        row_select_kernel<DTV><<<rows, 1024, 0, s>>>(logits, K, vocab, nseg, inv_t, drafts, n_drafts,      \
                                                     w.seg_max, w.pick, w.cand, w.stats, w.flag);          \
        rejection_row_stats_kernel<DTV><<<rows, kThreads, 0, s>>>(logits, K, vocab, drafts, n_drafts,      \
                                                                  inv_t, top_p, use_topp, w.stats, w.flag); \
    } else {                                                                                               \
        seg_z_kernel<DTV><<<dim3(nseg, rows), kSegThreads, 0, s>>>(logits, K, vocab, nseg, vec_ok, inv_t,  \
                                                                   n_drafts, w.seg_max, w.seg_z);          \
    }                                                                                                      \
    seg_draw_sums_kernel<DTV><<<dim3(nseg, num_seqs), kSegThreads, 0, s>>>(                                \
        logits, q, K, vocab, nseg, vec_ok, inv_t, use_topp, drafts, n_drafts, uniforms, w.stats,           \
        w.seg_max, w.seg_z, w.dec, w.seg_out);                                                             \
    seg_draw_find_kernel<DTV><<<num_seqs, kFindThreads, 0, s>>>(logits, q, K, vocab, nseg, inv_t, use_topp, \
                                                               drafts, uniforms, w.stats, w.seg_max,       \
                                                               w.seg_z, w.dec, w.seg_out, out_acc, out_tok);
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
