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
// Arithmetic is exact integer fixed point (gg_fixed_exp.h): a row is cut into segments
// of 8192 logits and logit i of segment s weighs W_i = e_i * f_s, e_i = weight(l_i, m_s),
// f_s = weight(m_s, m) (m_s the segment max, m the row max, weight(l, a) =
// floor(exp_gg((l - a)/T) * 2^35)); sums are exact 128-bit integers. The nucleus order
// is (logit desc, index asc). Launches:
//   seg_pass, one block per (row, segment): the segment max m_s and E_s = sum of e_i (with
//     top-p also the segment's coarse histogram of e on an absolute 1/16-nat grid, and the
//     counters of the next launch cleared). The only read of the whole logits: m and
//     Z = sum f_s * E_s follow from the segments.
//   top-p only:
//     row_pick (per row, the segment histograms merged exactly into the row's, and its
//       boundary bin); the last row block of each sequence then runs the bounds walk:
//       every draft the bounds of the nucleus mass already decide; the rows left open are
//       flagged and listed for the exact nucleus, or, when the bounds settle the walk,
//       the row of the final draw is marked as only drawn from;
//     seg_gather (listed rows: the boundary bin's elements), row_select (listed rows: a
//       sort of those elements to the exact cut). The later kernels are sized for about
//       one listed row per sequence and loop over the list, so no block is launched for a
//       row that needs nothing. A row whose boundary bin is crowded falls back to the
//       exact single-block row passes (three 11/11/10-bit radix levels on the order key
//       and a 9+9-bit index select of a tied cut).
//   rej_decide, one wave per sequence: the acceptance walk (accept iff u*q(x)*Zp < W(x))
//     and the set-up of the sequence's final draw (its row, the rejected draft, and with
//     top-p the exact cut element of a listed row, or the range of l/T of a marked row's
//     boundary bin, as the draw's hint).
//   The float64 draw's launches (accept_sample.hip) draw the token.
// The draft distributions are read only at drafted tokens and, by the draw, on the drawn row.
#pragma clang fp contract(off)

#include "gg_common.h"
#include "gg_fixed_exp.h"
#include "gg_draw.h"

namespace gg {
namespace {

constexpr int kThreads = 512;  // exact row passes: threads per row
constexpr int kBins = 2048;
typedef unsigned long long u64;
typedef gg_u128 u128;

struct RowStats {
    u128 zp;          // nucleus mass
    u128 wx;          // weight of the drafted token (0 if outside the nucleus)
    float m;          // max finite logit (or -inf when none)
    int idx_cut;      // ties at the boundary key are kept for index <= idx_cut
    unsigned int lam; // boundary order key (0 = keep every finite logit)
    int valid;        // row was evaluated
};

constexpr int kCandCap = 4096;
constexpr int kFindThreads = 1024;  // draw find: threads per sequence

// The nucleus boundary of one row (top-p), from the coarse histogram: the boundary bin,
// the mass of the bins before it and its own mass.
struct RowPick {
    u128 c_above;    // mass of the bins before the boundary bin
    u128 m_bin;      // mass of the boundary bin
    u128 tp;         // ceil(top_p * Z)
    float m;         // the row's max finite logit (-inf when none)
    int cbin;        // boundary coarse bin (-1: no finite logit or Z == 0)
    int n_cand;      // elements of that bin gathered so far
};

// A RowPick written and read across workgroups of one launch: device-scope relaxed stores
// and loads (the ordering argument is at row_pick_kernel).
__device__ __forceinline__ void store_pick(RowPick* p, const RowPick& v) {
    u64* d = (u64*)p;
    const u64* w = (const u64*)&v;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(RowPick) / 8); ++i) __hip_atomic_store(d + i, w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ RowPick load_pick(const RowPick* p) {
    RowPick v;
    u64* w = (u64*)&v;
    const u64* d = (const u64*)p;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(RowPick) / 8); ++i) w[i] = __hip_atomic_load(d + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v;
}
static_assert(sizeof(RowPick) % 8 == 0, "RowPick moves as 64-bit words");

// What the bounds walk (run by row_pick_kernel's last row block of a sequence) takes.
struct DecideBoundsIn {
    const void* logits;
    const float* dprobs;
    int K, V, nseg;
    float inv_t;
    const int32_t* drafts;
    const int32_t* n_drafts;
    const float* uniforms;
    const float* seg_max;
    const u64* seg_e;
    RowPick* pick;
    int* status;
    int* flag;
    int* n_flagged;
    int* flagged;
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
__device__ __forceinline__ u128 shfl_xor_u128(u128 v, int o) {
    return ((u128)shfl_xor_u64((u64)(v >> 64), o) << 64) | shfl_xor_u64((u64)v, o);
}
__device__ __forceinline__ u128 shfl_up_u128(u128 v, int o) {
    return ((u128)shfl_up_u64((u64)(v >> 64), o) << 64) | shfl_up_u64((u64)v, o);
}
__device__ __forceinline__ u128 shfl_u128(u128 v, int src) {
    const u64 lo = (u64)v, hi = (u64)(v >> 64);
    const unsigned int a = __shfl((unsigned int)lo, src), b = __shfl((unsigned int)(lo >> 32), src);
    const unsigned int c = __shfl((unsigned int)hi, src), d = __shfl((unsigned int)(hi >> 32), src);
    return ((u128)(((u64)d << 32) | c) << 64) | (((u64)b << 32) | a);
}
// Exact 128-bit add into (lo, hi) words with atomics (LDS or global): the carry out of
// the low word goes into the high word.
__device__ __forceinline__ void atomic_add_u128(u64* lo, u64* hi, u128 v) {
    const u64 vl = (u64)v, vh = (u64)(v >> 64);
    const u64 old = vl ? atomicAdd(lo, vl) : 0ull;
    const u64 carry = (vl && old + vl < old) ? 1ull : 0ull;
    if (vh + carry) atomicAdd(hi, vh + carry);
}

__device__ __forceinline__ bool finite_f(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// Wave 0 scans the histogram from bin 0 upward (larger logits first; descending bin
// index order when `desc`) and returns the LAST non-empty bin (count > 0; mass > 0
// when cnt is null) whose mass-above C satisfies C < tp || C == 0; *out_c receives
// its C. Masses are (lo, hi) word pairs.
__device__ void pick_bin(const u64* mlo, const u64* mhi, const unsigned int* cnt, int nbins, bool desc, u128 base,
                         u128 tp, int* out_bin, u128* out_c) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const int per = nbins / 64;
    auto bin_at = [&](int p) { return desc ? nbins - 1 - p : p; };
    auto mass = [&](int bn) { return ((u128)mhi[bn] << 64) | mlo[bn]; };
    u128 local = 0;
    for (int k = 0; k < per; ++k) local += mass(bin_at(lane * per + k));
    u128 incl = local;
    for (int o = 1; o < 64; o <<= 1) {
        const u128 t = shfl_up_u128(incl, o);
        if (lane >= o) incl += t;
    }
    u128 c = base + incl - local;
    int best = -1;
    u128 best_c = 0;
    for (int k = 0; k < per; ++k) {
        const int bn = bin_at(lane * per + k);
        const u128 mb = mass(bn);
        const bool nonempty = cnt ? cnt[bn] > 0 : mb > 0;
        if (nonempty && (c < tp || c == 0)) {
            best = lane * per + k;
            best_c = c;
        }
        c += mb;
    }
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

// The segment factor f_s of segment max ms against row max m (0 for an empty segment).
__device__ __forceinline__ u64 seg_factor(float ms, float m, float inv_t) {
    return finite_f(ms) ? gg_weight(ms, m, inv_t) : 0ull;
}

// The nucleus of one row and the weights inside it.
struct Nucleus {
    float m, inv_t;
    unsigned int lam;
    int idx_cut;
    __device__ __forceinline__ bool kept(float l, int i) const {
        if (!finite_f(l)) return false;
        const unsigned int k = gg_order_key(l);
        return k > lam || (k == lam && i <= idx_cut);
    }
    // W of logit l at index i, given its segment max ms.
    __device__ __forceinline__ u128 weight(float l, int i, float ms) const {
        if (!kept(l, i)) return 0;
        return (u128)gg_weight(l, ms, inv_t) * seg_factor(ms, m, inv_t);
    }
};

// ---------------------------------------------------------------------------
// Segmented path. A row of V logits is cut into segments of kSegElems; every
// (row, segment) pair is one 256-thread block, so a launch has thousands of blocks.
// All cross-segment combinations are max of floats or sums of integers: exact and
// order-free, so the result is the same bit pattern whatever the schedule.

constexpr int kSegThreads = 256;
constexpr int kSegElems = GG_ACCEPT_SEG;  // 32 logits per thread
static_assert(kSegElems == kSegThreads * 32, "segment = 32 logits per thread");
// Coarse nucleus bins, 1/16 nat wide on an absolute grid: cb(l) = floor(l/T * 16), and a
// logit's bin relative to a maximum a is cb(a) - cb(l). Both terms are integers, so a bin
// relative to a segment max turns into the bin relative to the row max by adding
// cb(m) - cb(m_s): the segments' histograms merge exactly. cb is monotone, so the bins
// follow the nucleus order. (l * (16/T) is the same float as l/T * 16 outside the
// subnormal range, the power-of-two factor being exact; the loop-invariant 16/T leaves
// one multiply per logit.)
constexpr int kSegBins = 400;   // per segment: e > 0 needs (m_s - l)/T < 24.3 nats (389 bins)
constexpr int kRowBins = 1024;  // per row (the last bin takes everything further down)
__device__ __forceinline__ int cb_abs(float l, float inv_t) {
    const float y = fminf(fmaxf(l * (inv_t * 16.0f), -1.0e9f), 1.0e9f);
    return (int)__builtin_floorf(y);
}


// Per-row state of the top-p decision: certain outcome from the coarse bounds, or
// resolved from the exact nucleus.
constexpr int kRowAccept = 1, kRowReject = 2, kRowUnsure = 3;

struct SeqDecision {
    int accepted;
    int row;         // row of the final draw
    int residual;    // 1: draw from W - min(W, floor(q*Zp)), 0: from W
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
// The 32 logits a thread owns in a segment: elements base + 8*threadIdx + {0..7} of each
// of the four 2048-element quarters (16-byte loads; scalar fallback for odd rows).
// Elements past the row read as NaN (never finite, never weighed).
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

__device__ __forceinline__ int live_rows(const int32_t* n_drafts, int b, int K) {
    int n = n_drafts[b];
    return n < 0 ? 0 : (n > K ? K : n);
}

// Row max and Z = sum of f_s * E_s over the per-segment values, by a whole wave (lane s
// reads segment s; nseg <= 64): one load round trip rather than a chain of nseg. Every
// lane returns the same values.
__device__ __forceinline__ float row_max_wave(const float* seg_max, int row, int nseg) {
    const int lane = threadIdx.x & 63;
    float m = lane < nseg ? seg_max[(size_t)row * nseg + lane] : -INFINITY;
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    return m;
}
__device__ __forceinline__ u128 row_z_wave(const float* seg_max, const u64* seg_e, int row, int nseg, float m,
                                           float inv_t) {
    const int lane = threadIdx.x & 63;
    u128 z = 0;
    if (lane < nseg && finite_f(m)) {
        const float ms = seg_max[(size_t)row * nseg + lane];
        z = (u128)seg_e[(size_t)row * nseg + lane] * seg_factor(ms, m, inv_t);
    }
    for (int o = 32; o > 0; o >>= 1) z += shfl_xor_u128(z, o);
    return z;
}

// Eight consecutive logits [e0, e0 + 8) of a row (16-byte loads when aligned; NaN past
// the row).
template <gg_dtype_t DT>
__device__ __forceinline__ void load8(const void* row, int V, int e0, bool vec_ok, float (&x)[8]) {
    if (vec_ok && e0 + 8 <= V) {
        if constexpr (DT == GG_DTYPE_F32) {
            const float4 a = *(const float4*)((const float*)row + e0), c = *(const float4*)((const float*)row + e0 + 4);
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
        } else {
            const uint4 r4 = *(const uint4*)((const uint16_t*)row + e0);
            const uint32_t wv[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint16_t h = (uint16_t)(wv[k >> 1] >> ((k & 1) * 16));
                x[k] = DT == GG_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = e0 + k < V ? ld<DT>(row, e0 + k) : NAN;
    }
}

// A: per (row, segment): the segment max m_s and E_s = sum of weight(l, m_s); with top-p
// also the segment's coarse histogram of e over bins cb(m_s) - cb(l) (written out: the
// row max, needed to merge, is not known yet), and the counters the next launch counts
// in cleared: each sequence's row count, and the flagged-row and crowded-row list lengths.
// The only full read of the logits.
template <gg_dtype_t DT, bool kTopP>
__global__ void __launch_bounds__(kSegThreads) seg_pass_kernel(const void* __restrict__ logits, int K, int V,
                                                               int nseg, int vec_ok, float inv_t,
                                                               const int32_t* __restrict__ n_drafts,
                                                               float* __restrict__ seg_max, u64* __restrict__ seg_e,
                                                               u64* __restrict__ seg_hist, int* __restrict__ seq_cnt,
                                                               int* __restrict__ n_flagged) {
    const int seg = blockIdx.x, row = blockIdx.y;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    if constexpr (kTopP) {
        if (seg == 0 && j == 0 && threadIdx.x == 0) seq_cnt[b] = 0;
        if (seg == 0 && row == 0 && threadIdx.x < 2) n_flagged[threadIdx.x] = 0;
    }
    if (j > live_rows(n_drafts, b, K)) return;
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    float x[32];
    int idx[32];
    load_seg<DT>(lp, V, seg, vec_ok, x, idx);
    __shared__ float redf[kSegThreads / 64];
    __shared__ u64 red[kSegThreads / 64];
    __shared__ u64 h[kTopP ? kSegBins : 1];
    if constexpr (kTopP) {
        for (int i = threadIdx.x; i < kSegBins; i += kSegThreads) h[i] = 0;
    }
    // Non-finite logits become -inf: no effect on the max, and weight 0 (gg_weight
    // clamps x = -inf to -80), so neither loop branches per element.
    float ms = -INFINITY;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        x[k] = finite_f(x[k]) ? x[k] : -INFINITY;
        ms = fmaxf(ms, x[k]);
    }
    ms = seg_block_max(ms, redf);  // (its barriers also publish the cleared histogram)
    // The thread's 32 weights (integers below 2^36, held in floats) summed exactly in a
    // double.
    double ed = 0.0;
    if (finite_f(ms)) {
        const int cbm = kTopP ? cb_abs(ms, inv_t) : 0;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float w = gg_weight_f(x[k], ms, inv_t);
            ed += (double)w;
            if constexpr (kTopP) {
                if (w != 0.0f) atomicAdd(&h[min(cbm - cb_abs(x[k], inv_t), kSegBins - 1)], gg_weight_u64(w));
            }
        }
    }
    const u64 e = seg_block_sum((u64)ed, red);  // (its barriers also complete the histogram)
    if (threadIdx.x == 0) {
        seg_max[(size_t)row * nseg + seg] = ms;
        seg_e[(size_t)row * nseg + seg] = e;
    }
    if constexpr (kTopP) {
        u64* out = seg_hist + ((size_t)row * nseg + seg) * kSegBins;
        for (int i = threadIdx.x; i < kSegBins; i += kSegThreads) out[i] = h[i];
    }
}

// The row bin of logit l: cb(m) - cb(l), capped at the last bin.
__device__ __forceinline__ int row_bin(float l, int cbm, float inv_t) {
    return min(cbm - cb_abs(l, inv_t), kRowBins - 1);
}

// ---- Top-p: the nucleus boundary ----
//
// The boundary is the last element, in (logit desc, index asc) order, whose mass before
// it is below Tp = ceil(p*Z) (or zero). (B) A block per row merges the segments'
// histograms into the row's (bins shifted by cb(m) - cb(m_s), masses scaled by f_s:
// exact) and finds the boundary bin and the mass above it. (C) In the same launch, the
// last of a sequence's row blocks to finish decides with one wave every draft whose
// outcome the bounds already fix: the nucleus mass lies in [C, C + M] (C the mass above
// the boundary bin, M its mass), a draft in a bin above the boundary bin is in the nucleus
// and one below is out. The rows left open are flagged for the exact nucleus; the row of
// the final draw, when the bounds settle the walk, only for the draw's range hint. (D) For
// the rows flagged exact, the boundary bin's elements are gathered (usually a few hundred
// to a few thousand); (E) a block per such row sorts them by (key desc, index asc) and
// walks the weights to the exact cut. A boundary bin with more than kCandCap elements
// falls back to the exact single-block row kernel.

// B: per row, merge the segment histograms; the boundary bin, the mass above it and its
// own mass. Thread t owns row bins t, t + 256, ...: row bin r gathers f_s * H_s[r - shift_s]
// over the segments (the last row bin everything from there down), no atomics. A thread's
// loads for a batch of segments are issued together. The row's RowPick goes out with
// device-scope stores; then the block counts itself in its sequence's counter (cleared by
// seg_pass_kernel), and the last of the sequence's rows runs the bounds walk (C) for it.
constexpr int kPickBatch = 8;
template <gg_dtype_t DT>
__device__ void bounds_walk(const DecideBoundsIn& in, int b);
__device__ __forceinline__ void row_pick_merge(int nseg, float inv_t, float top_p, const float* __restrict__ seg_max,
                               const u64* __restrict__ seg_hist, RowPick* __restrict__ pick, int row, float m,
                               u128 z, u64* hlo, u64* hhi, int* s_shift, u64* s_f, int* p_bin, u128* p_c);
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) row_pick_kernel(int nseg, float top_p, const u64* __restrict__ seg_hist,
                                                               int* __restrict__ seq_cnt, DecideBoundsIn in) {
    const int row = blockIdx.x;
    const int K = in.K;
    const float inv_t = in.inv_t;
    const float* __restrict__ seg_max = in.seg_max;
    const u64* __restrict__ seg_e = in.seg_e;
    const int R = K + 1;
    const int b = row / R, j = row % R;
    const int n = live_rows(in.n_drafts, b, K);
    if (j > n) return;
    __shared__ u64 hlo[kRowBins], hhi[kRowBins];
    __shared__ int s_shift[64];
    __shared__ u64 s_f[64];
    __shared__ int s_bin;
    __shared__ u128 s_c;
    __shared__ int s_last;
    const float m = row_max_wave(seg_max, row, nseg);
    const u128 z = row_z_wave(seg_max, seg_e, row, nseg, m, inv_t);
    if (!finite_f(m) || z == 0) {
        if (threadIdx.x == 0) store_pick(&in.pick[row], RowPick{0, 0, 0, m, -1, 0});
    } else {
        row_pick_merge(nseg, inv_t, top_p, seg_max, seg_hist, in.pick, row, m, z, hlo, hhi, s_shift, s_f, &s_bin,
                       &s_c);
    }
    // Ordering (gfx950; the library has no code object for other devices): a device-scope
    // relaxed store is written through the XCD's L2 to the coherence point and counts in
    // vmcnt until acknowledged, so after `s_waitcnt vmcnt(0)` the row's RowPick is visible
    // there. The barrier puts that before thread 0's counter add (performed at the coherence
    // point); the last row sees the full count in the add's return value and only then
    // reads the sequence's RowPicks, with device-scope loads (served from the coherence
    // point, never from a stale line of its own L2).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&seq_cnt[b], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n;
    __syncthreads();
    if (!s_last || threadIdx.x >= 64) return;
    bounds_walk<DT>(in, b);
}

// B's merge for one row with a finite max m and Z > 0.
__device__ __forceinline__ void row_pick_merge(int nseg, float inv_t, float top_p, const float* __restrict__ seg_max,
                               const u64* __restrict__ seg_hist, RowPick* __restrict__ pick, int row, float m,
                               u128 z, u64* hlo, u64* hhi, int* s_shift, u64* s_f, int* p_bin, u128* p_c) {
    const int cbm = cb_abs(m, inv_t);
    if (threadIdx.x < 64) {
        int sh = kRowBins;
        u64 f = 0;
        if (threadIdx.x < nseg) {
            const float ms = seg_max[(size_t)row * nseg + threadIdx.x];
            f = seg_factor(ms, m, inv_t);
            if (f) sh = cbm - cb_abs(ms, inv_t);  // (no mass: no bins)
        }
        s_f[threadIdx.x] = f;
        s_shift[threadIdx.x] = sh;
    }
    __syncthreads();
    const u64* hrow = seg_hist + (size_t)row * nseg * kSegBins;
    constexpr int kPer = kRowBins / kSegThreads;
    u128 acc[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) acc[k] = 0;
    for (int sg0 = 0; sg0 < nseg; sg0 += kPickBatch) {
        u64 v[kPer][kPickBatch];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int r = threadIdx.x + k * kSegThreads;
#pragma unroll
            for (int i = 0; i < kPickBatch; ++i) {
                const int lo = r - s_shift[sg0 + i];  // (s_shift is kRowBins past nseg)
                v[k][i] = (lo >= 0 && lo < kSegBins) ? hrow[(size_t)(sg0 + i) * kSegBins + lo] : 0ull;
            }
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k)
#pragma unroll
            for (int i = 0; i < kPickBatch; ++i) acc[k] += (u128)v[k][i] * s_f[sg0 + i];
    }
    // The last row bin also takes every segment bin below its own.
    if (threadIdx.x == kSegThreads - 1) {
        constexpr int r = kRowBins - 1;
        for (int sg = 0; sg < nseg; ++sg) {
            if (!s_f[sg]) continue;
            u128 t = 0;
            for (int bn = max(r - s_shift[sg] + 1, 0); bn < kSegBins; ++bn) t += hrow[(size_t)sg * kSegBins + bn];
            acc[kPer - 1] += t * s_f[sg];
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int r = threadIdx.x + k * kSegThreads;
        hlo[r] = (u64)acc[k];
        hhi[r] = (u64)(acc[k] >> 64);
    }
    const u128 tp = gg_u128_floor(ceil((double)top_p * gg_u128_to_double(z)));
    if (threadIdx.x == 0) *p_bin = -1;
    __syncthreads();
    pick_bin(hlo, hhi, nullptr, kRowBins, false, 0, tp, p_bin, p_c);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int cb = *p_bin;
        store_pick(&pick[row], RowPick{*p_c, ((u128)hhi[cb] << 64) | hlo[cb], tp, m, cb, 0});
    }
}

// The bounds test of one draft: kRowAccept / kRowReject when the coarse bounds decide
// it, kRowUnsure otherwise. W of the draft token x is e_x * f_x when x lies above the
// boundary bin.
template <gg_dtype_t DT>
__device__ __forceinline__ int bounds_test(const void* lp, const float* rsm, const RowPick& pk, float m, float inv_t,
                                           int x, int V, double u, double q) {
    if (pk.cbin < 0 || x < 0 || x >= V) return kRowReject;  // no mass, or no token: W(x) = 0
    const float l = ld<DT>(lp, x);
    if (!finite_f(l)) return kRowReject;
    const int rb = row_bin(l, cb_abs(m, inv_t), inv_t);
    if (rb > pk.cbin) return kRowReject;  // below the boundary bin: outside the nucleus
    if (rb == pk.cbin) return kRowUnsure;
    const float ms = rsm[x / kSegElems];
    const double wx = gg_u128_to_double((u128)gg_weight(l, ms, inv_t) * seg_factor(ms, m, inv_t));
    if (u * q * gg_u128_to_double(pk.c_above + pk.m_bin) < wx) return kRowAccept;  // Zp <= C + M
    if (!(u * q * gg_u128_to_double(pk.c_above) < wx)) return kRowReject;          // Zp >= C
    return kRowUnsure;
}

// C: per sequence, one wave (threads 0..63 of the block): the rows' bound outcomes; flags
// the rows that need the exact nucleus (an open row and every row after it through the
// first certain rejection) and appends them to the flagged-row list (order free: each
// listed row is processed on its own), or flags just the row of the final draw when the
// bounds settle the walk. Lane j tests draft j (max_drafts <= 64), so the rows' loads
// overlap. The sequence's RowPicks come from other blocks of the same launch: device-scope
// loads.
template <gg_dtype_t DT>
__device__ void bounds_walk(const DecideBoundsIn& in, int b) {
    const void* __restrict__ logits = in.logits;
    const float* __restrict__ dprobs = in.dprobs;
    const int K = in.K, V = in.V, nseg = in.nseg;
    const float inv_t = in.inv_t;
    const int32_t* __restrict__ drafts = in.drafts;
    const float* __restrict__ uniforms = in.uniforms;
    const float* __restrict__ seg_max = in.seg_max;
    const RowPick* __restrict__ pick = in.pick;
    int* __restrict__ status = in.status;
    int* __restrict__ flag = in.flag;
    int* __restrict__ n_flagged = in.n_flagged;
    int* __restrict__ flagged = in.flagged;
    const int R = K + 1;
    const int n = live_rows(in.n_drafts, b, K);
    const int lane = threadIdx.x;
    int st = kRowAccept;
    if (lane < n) {
        const int row = b * R + lane;
        const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
        const int x = drafts[(size_t)b * K + lane];
        const double q = (dprobs && x >= 0 && x < V) ? gg_clean_q(dprobs[((size_t)b * K + lane) * V + x]) : 1.0;
        const double u = (double)uniforms[(size_t)b * R + lane];
        const RowPick pk = load_pick(&pick[row]);
        st = bounds_test<DT>(lp, seg_max + (size_t)row * nseg, pk, pk.m, inv_t, x, V, u, q);
        status[row] = st;
    }
    // Walk: the first row that is not a certain acceptance, then (if it is open) every
    // row through the first certain rejection after it.
    const unsigned long long not_acc = __ballot(lane < n && st != kRowAccept);
    const int j0 = not_acc ? __ffsll((long long)not_acc) - 1 : n;
    int jend = j0;  // flag rows j0 .. jend
    if (j0 < n && __shfl(st, j0) == kRowUnsure) {
        const unsigned long long rej = __ballot(lane > j0 && lane < n && st == kRowReject);
        jend = rej ? __ffsll((long long)rej) - 1 : n;
    }
    // When the bounds settle the walk, row j0 is only drawn from: it is flagged 2 and not
    // listed, and the draw gets its coarse boundary bin as a range hint instead of the exact
    // cut (rej_decide_kernel), unless that bin is the last row bin, which holds everything
    // below it. Rows 0 .. n (n <= 64): lane j writes row j, lane 0 also row 64.
    const bool settled = !(j0 < n && __shfl(st, j0) == kRowUnsure);
    int mine = 0, mine64 = 0;
    if (lane <= n) {
        mine = lane >= j0 && lane <= jend;
        if (mine && settled) {
            const int cb = load_pick(&pick[b * R + lane]).cbin;
            if (cb >= 0 && cb < kRowBins - 1) mine = 2;
        }
        flag[b * R + lane] = mine;
    }
    if (lane == 0 && n == 64) {
        mine64 = jend >= 64;
        if (mine64 && settled) {
            const int cb = load_pick(&pick[b * R + 64]).cbin;
            if (cb >= 0 && cb < kRowBins - 1) mine64 = 2;
        }
        flag[b * R + 64] = mine64;
        mine64 = mine64 == 1;
    }
    mine = mine == 1;
    const unsigned long long fl = __ballot(mine);
    const int cnt = __popcll(fl) + __shfl(mine64, 0);
    int base = 0;
    if (lane == 0) base = atomicAdd(n_flagged, cnt);
    base = __shfl(base, 0);
    if (mine) flagged[base + __popcll(fl & ((1ull << lane) - 1))] = b * R + lane;
    if (mine64) flagged[base + cnt - 1] = b * R + 64;
}

// D: per (flagged row, segment): the boundary bin's elements gathered for the cut. Block
// (seg, y) takes the listed rows y, y + gridDim.y, ... (the grid is sized for about one
// flagged row per sequence, so no block is launched for an unflagged row).
template <gg_dtype_t DT>
__device__ __forceinline__ void seg_gather_row(const void* __restrict__ logits, int V, int nseg, int vec_ok,
                                               float inv_t, int seg, int row, const float* __restrict__ seg_max,
                                               RowPick* __restrict__ pick, uint2* __restrict__ cand);
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kSegThreads) seg_gather_kernel(const void* __restrict__ logits, int V,
                                                                 int nseg, int vec_ok, float inv_t,
                                                                 const int* __restrict__ n_flagged,
                                                                 const int* __restrict__ flagged,
                                                                 const float* __restrict__ seg_max,
                                                                 RowPick* __restrict__ pick,
                                                                 uint2* __restrict__ cand) {
    const int nf = *n_flagged;
    for (int li = blockIdx.y; li < nf; li += gridDim.y)
        seg_gather_row<DT>(logits, V, nseg, vec_ok, inv_t, blockIdx.x, flagged[li], seg_max, pick, cand);
}
template <gg_dtype_t DT>
__device__ __forceinline__ void seg_gather_row(const void* __restrict__ logits, int V, int nseg, int vec_ok,
                                               float inv_t, int seg, int row, const float* __restrict__ seg_max,
                                               RowPick* __restrict__ pick, uint2* __restrict__ cand) {
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    __shared__ int s_hits[kSegThreads / 64];
    __shared__ int s_base;
    const int cbin = pick[row].cbin;
    const float m = pick[row].m;
    const float ms = seg_max[(size_t)row * nseg + seg];
    const int cbm = cb_abs(m, inv_t);
    // The boundary bin's elements: a bit mask per thread, bit k for load_seg's element k.
    // The thread's 32 logits are taken in two halves of 16, so fewer registers are live and
    // more waves fit per SIMD.
    uint32_t hits = 0;
    if (cbin >= 0 && finite_f(ms)) {
#pragma unroll 1
        for (int half = 0; half < 2; ++half) {
            float xa[8], xb[8];
            const int e0 = seg * kSegElems + 2 * half * 2048 + 8 * (int)threadIdx.x;
            load8<DT>(lp, V, e0, vec_ok, xa);
            load8<DT>(lp, V, e0 + 2048, vec_ok, xb);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float xk = k < 8 ? xa[k] : xb[k - 8];
                const bool fin = finite_f(xk);
                const float xv = fin ? xk : -INFINITY;
                const int rb = row_bin(xv, cbm, inv_t);
                hits |= (uint32_t)(fin && rb == cbin) << (16 * half + k);
            }
        }
    }
    // The candidates' slots: an exclusive scan of the per-thread counts within the block
    // and one counter update per block.
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nh = __popc(hits);
    int incl = nh;
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) s_hits[wv] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int tot = 0;
        for (int i = 0; i < kSegThreads / 64; ++i) tot += s_hits[i];
        s_base = tot ? atomicAdd(&pick[row].n_cand, tot) : 0;
    }
    __syncthreads();
    if (hits) {
        int slot = s_base + incl - nh;
        for (int i = 0; i < wv; ++i) slot += s_hits[i];
        while (hits) {
            const int k = __ffs(hits) - 1;
            hits &= hits - 1;
            // (load_seg's element order; the logit read again, from cache, so that the
            // loaded values need not stay live)
            const int iv = seg * kSegElems + (k >> 3) * 2048 + 8 * (int)threadIdx.x + (k & 7);
            const float xv = ld<DT>(lp, iv);
            if (slot < kCandCap) cand[(size_t)row * kCandCap + slot] = make_uint2(__float_as_uint(xv), (unsigned)iv);
            ++slot;
        }
    }
}

// The logit of an order key (inverse of gg_order_key).
__device__ __forceinline__ float logit_of_key(unsigned int key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Exact per-row nucleus statistics by one block of kThreads (passes over the whole row),
// for a row whose boundary bin is crowded (more than kCandCap elements). Uses the segment
// maxima and sums of seg_pass_kernel.
template <gg_dtype_t DT>
__device__ void row_stats_exact(const void* __restrict__ logits, int K, int V, int nseg,
                                const int32_t* __restrict__ drafts, const int32_t* __restrict__ n_drafts,
                                float inv_t, float top_p, const float* __restrict__ seg_max,
                                const u64* __restrict__ seg_e, RowStats* __restrict__ stats, int row) {
    const int R = K + 1;
    const int b = row / R, j = row % R;
    const int n = live_rows(n_drafts, b, K);
    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
    const float* rms = seg_max + (size_t)row * nseg;

    __shared__ u64 hlo[kBins], hhi[kBins];
    __shared__ unsigned int hcnt[kBins];
    __shared__ int s_bin;
    __shared__ u128 s_c;

    const float m = row_max_wave(seg_max, row, nseg);  // (every wave computes it)
    const u128 z = row_z_wave(seg_max, seg_e, row, nseg, m, inv_t);
    // Crowded rows have a finite max and Z > 0 (row_pick found a boundary bin).
    const u128 tp = gg_u128_floor(ceil((double)top_p * gg_u128_to_double(z)));
    auto w_of = [&](float l, int i) -> u128 {
        const float ms = rms[i / kSegElems];
        return (u128)gg_weight(l, ms, inv_t) * seg_factor(ms, m, inv_t);
    };
    auto clear = [&]() {
        __syncthreads();
        for (int i = threadIdx.x; i < kBins; i += kThreads) {
            hlo[i] = hhi[i] = 0;
            hcnt[i] = 0;
        }
        __syncthreads();
    };

    // Coarse bins (1/64 nat of (m - l)/T), then three radix levels on the order key
    // within the boundary bin, then the ties at the boundary key by index.
    clear();
    for (int i = threadIdx.x; i < V; i += kThreads) {
        const float l = ld<DT>(lp, i);
        if (!finite_f(l)) continue;
        const int bn = gg_coarse_bin(l, m, inv_t);
        atomic_add_u128(&hlo[bn], &hhi[bn], w_of(l, i));
        atomicAdd(&hcnt[bn], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) s_bin = -1;
    __syncthreads();
    pick_bin(hlo, hhi, hcnt, kBins, false, 0, tp, &s_bin, &s_c);
    __syncthreads();
    const int cbin = s_bin;
    u128 c_above = s_c;
    unsigned int prefix = 0, pmask = 0;
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    for (int lv = 0; lv < 3; ++lv) {
        const int nb = 1 << widths[lv];
        clear();
        for (int i = threadIdx.x; i < V; i += kThreads) {
            const float l = ld<DT>(lp, i);
            if (!finite_f(l)) continue;
            if (gg_coarse_bin(l, m, inv_t) != cbin) continue;
            const unsigned int key = gg_order_key(l);
            if ((key & pmask) != prefix) continue;
            const int d = (key >> shifts[lv]) & (nb - 1);
            atomic_add_u128(&hlo[d], &hhi[d], w_of(l, i));
            atomicAdd(&hcnt[d], 1u);
        }
        __syncthreads();
        // (Unused bins of the 10-bit level stay empty: the scan covers kBins.)
        pick_bin(hlo, hhi, hcnt, kBins, true, c_above, tp, &s_bin, &s_c);
        __syncthreads();
        prefix |= (unsigned int)s_bin << shifts[lv];
        pmask |= (unsigned int)(nb - 1) << shifts[lv];
        c_above = s_c;
    }
    const unsigned int lam = prefix;
    // The ties at the boundary key, in index order: a tie is kept while the mass before
    // it is below tp (or zero), i.e. every tie through the first one whose inclusive mass
    // reaches tp. Two 9-bit levels over the index find that tie; when none reaches tp,
    // every tie is kept.
    const unsigned int dl = prefix & 0x3ffu;
    const u128 m_tie = ((u128)hhi[dl] << 64) | hlo[dl];
    int idx_cut = 0x7fffffff;
    u128 zp = c_above + m_tie;
    if (c_above + m_tie >= tp) {
        unsigned int iprefix = 0, imask = 0;
        u128 base = c_above;
        const int ish[2] = {9, 0};
        for (int lv = 0; lv < 2; ++lv) {
            clear();
            for (int i = threadIdx.x; i < V; i += kThreads) {
                const float l = ld<DT>(lp, i);
                if (!finite_f(l) || gg_order_key(l) != lam) continue;
                if (((unsigned int)i & imask) != iprefix) continue;
                const int d = ((unsigned int)i >> ish[lv]) & 511u;
                atomic_add_u128(&hlo[d], &hhi[d], w_of(l, i));
                atomicAdd(&hcnt[d], 1u);
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                // The first index bin, in order, holding a tie at which the inclusive
                // mass reaches tp (the mass before the first tie is c_above: below tp,
                // or zero, in which case the first tie is kept whatever its weight).
                u128 acc = base;
                int d = 0;
                for (; d < 511; ++d) {
                    const u128 md = ((u128)hhi[d] << 64) | hlo[d];
                    if (hcnt[d] && acc + md >= tp) break;
                    acc += md;
                }
                s_bin = d;
                s_c = acc;
            }
            __syncthreads();
            base = s_c;
            iprefix |= (unsigned int)s_bin << ish[lv];
            imask |= 511u << ish[lv];
        }
        idx_cut = (int)iprefix;
        zp = base + w_of(logit_of_key(lam), idx_cut);
    }
    const Nucleus nu{m, inv_t, lam, idx_cut};
    if (threadIdx.x == 0) {
        RowStats st{zp, 0, m, idx_cut, lam, 1};
        if (j < n) {
            const int x = drafts[(size_t)b * K + j];
            if (x >= 0 && x < V) st.wx = nu.weight(ld<DT>(lp, x), x, rms[x / kSegElems]);
        }
        stats[row] = st;
    }
}

// Bitonic sort of s[0, np2) into descending order (np2 a power of two <= 4 * 1024, 1024
// threads). Element i = t + 1024 * r is held by thread t as v[r] while the compare
// distance is below 64: its partner i ^ jj is then in the same wave, reached by a
// shuffle with no barrier. Longer distances go through LDS, a barrier per step.
__device__ __forceinline__ void sort_desc_1024(u64* s, int np2) {
    const int t = threadIdx.x;
    const int nr = (np2 + 1023) >> 10;
    u64 v[4];
    auto in_wave = [&](int k, int jj0) {
        for (int jj = jj0; jj > 0; jj >>= 1) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (r >= nr) break;
                const int i = t + (r << 10);
                const u64 c = shfl_xor_u64(v[r], jj);
                const bool keep_max = ((i & k) == 0) == ((i & jj) == 0);
                v[r] = keep_max ? (v[r] > c ? v[r] : c) : (v[r] < c ? v[r] : c);
            }
        }
    };
    auto load = [&]() {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = t + (r << 10);
            v[r] = (r < nr && i < np2) ? s[i] : 0ull;
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = t + (r << 10);
            if (r < nr && i < np2) s[i] = v[r];
        }
    };
    load();
    for (int k = 2; k <= np2 && k <= 64; k <<= 1) in_wave(k, k >> 1);
    for (int k = 128; k <= np2; k <<= 1) {
        store();
        __syncthreads();
        for (int jj = k >> 1; jj >= 64; jj >>= 1) {
            for (int i = t; i < np2; i += 1024) {
                const int ix = i ^ jj;
                if (ix > i) {
                    const u64 a = s[i], c = s[ix];
                    const bool desc = (i & k) == 0;
                    if (desc ? (a < c) : (a > c)) {
                        s[i] = c;
                        s[ix] = a;
                    }
                }
            }
            __syncthreads();
        }
        load();
        in_wave(k, 32);
    }
    store();
    __syncthreads();
}

// E: per flagged row, sort the boundary bin's elements by (key desc, index asc) and cut:
// the row's exact statistics.
// A crowded bin (more than kCandCap elements) is left to rejection_row_stats_kernel.
template <gg_dtype_t DT>
__device__ void row_select_row(const void* __restrict__ logits, int K, int V, int nseg, float inv_t, float top_p,
                               const int32_t* __restrict__ drafts, const int32_t* __restrict__ n_drafts,
                               const float* __restrict__ seg_max, const u64* __restrict__ seg_e,
                               const RowPick* __restrict__ pick, const uint2* __restrict__ cand,
                               RowStats* __restrict__ stats, int* __restrict__ n_crowded,
                               int* __restrict__ crowded, int row) {
    const int R = K + 1;
    const int b = row / R, j = row % R;
    const int n = live_rows(n_drafts, b, K);
    __shared__ u64 s_key[kCandCap];    // order key << 32 | (~index): descending = the nucleus order
    __shared__ u128 red[1024 / 64];
    __shared__ int s_last;
    const RowPick pk = pick[row];
    const float m = pk.m;
    if (pk.cbin < 0) {  // no finite logit or Z == 0: no nucleus
        if (threadIdx.x == 0) stats[row] = RowStats{0, 0, m, 0x7fffffff, 0u, 1};
        return;
    }
    const int nc = pk.n_cand;
    if (nc > kCandCap) {  // rejection_row_stats_kernel takes it
        if (threadIdx.x == 0) crowded[atomicAdd(n_crowded, 1)] = row;
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
    sort_desc_1024(s_key, np2);
    // Weights in that order (logit from the order key, segment max from the index).
    // Thread t owns positions [4t, 4t+4): an exclusive block scan of the thread sums gives
    // each element's mass before it; the kept elements are a prefix (that mass never
    // drops), so the cut is the largest kept position. Candidates span at most
    // kCandCap = 4 * 1024 positions.
    const int p0 = 4 * (int)threadIdx.x;
    u128 w[4];
    u64 ev[4];
    int sv[4];
    u128 tsum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w[k] = 0;
        ev[k] = 0;
        sv[k] = 0;
        if (p0 + k < nc) {
            const u64 key = s_key[p0 + k];
            const int i = (int)(~(unsigned int)(key & 0xffffffffu));
            sv[k] = i / kSegElems;
            const float ms = seg_max[(size_t)row * nseg + sv[k]];
            ev[k] = gg_weight(logit_of_key((unsigned int)(key >> 32)), ms, inv_t);
            w[k] = (u128)ev[k] * seg_factor(ms, m, inv_t);
        }
        tsum += w[k];
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    u128 incl = tsum;
    for (int o = 1; o < 64; o <<= 1) {
        const u128 t = shfl_up_u128(incl, o);
        if (lane >= o) incl += t;
    }
    if (lane == 63) red[wv] = incl;
    __syncthreads();
    u128 before = pk.c_above + incl - tsum;
    for (int i = 0; i < wv; ++i) before += red[i];
    int last = -1;
    u128 zp = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (p0 + k < nc && (before < pk.tp || before == 0)) {
            last = p0 + k;
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
        RowStats st{zp, 0, m, idx_cut, lam, 1};
        if (j < n) {
            const int x = drafts[(size_t)b * K + j];
            if (x >= 0 && x < V) {
                const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
                Nucleus nu{m, inv_t, lam, idx_cut};
                st.wx = nu.weight(ld<DT>(lp, x), x, seg_max[(size_t)row * nseg + x / kSegElems]);
            }
        }
        stats[row] = st;
    }
}

template <gg_dtype_t DT>
__global__ void __launch_bounds__(1024) row_select_kernel(const void* __restrict__ logits, int K, int V,
                                                          int nseg, float inv_t, float top_p,
                                                          const int32_t* __restrict__ drafts,
                                                          const int32_t* __restrict__ n_drafts,
                                                          const int* __restrict__ n_flagged,
                                                          const int* __restrict__ flagged,
                                                          const float* __restrict__ seg_max,
                                                          const u64* __restrict__ seg_e,
                                                          const RowPick* __restrict__ pick,
                                                          const uint2* __restrict__ cand,
                                                          RowStats* __restrict__ stats,
                                                          int* __restrict__ n_crowded, int* __restrict__ crowded) {
    const int nf = *n_flagged;
    for (int li = blockIdx.x; li < nf; li += gridDim.x) {
        row_select_row<DT>(logits, K, V, nseg, inv_t, top_p, drafts, n_drafts, seg_max, seg_e, pick, cand, stats,
                           n_crowded, crowded, flagged[li]);
        __syncthreads();  // (the next row reuses the shared arrays)
    }
}

// The rows whose boundary bin is crowded (listed by row_select_kernel), by a few blocks:
// such rows are rare, and with none the kernel only reads the list's count.
constexpr int kRowStatsBlocks = 8;
template <gg_dtype_t DT>
__global__ void __launch_bounds__(kThreads) rejection_row_stats_kernel(
    const void* __restrict__ logits, int K, int V, int nseg, const int32_t* __restrict__ drafts,
    const int32_t* __restrict__ n_drafts, float inv_t, float top_p, const int* __restrict__ n_crowded,
    const int* __restrict__ crowded, const float* __restrict__ seg_max, const u64* __restrict__ seg_e,
    RowStats* __restrict__ stats) {
    const int nc = *n_crowded;
    for (int li = blockIdx.x; li < nc; li += gridDim.x) {
        const int row = crowded[li];
        row_stats_exact<DT>(logits, K, V, nseg, drafts, n_drafts, inv_t, top_p, seg_max, seg_e, stats, row);
        __syncthreads();
    }
}

// Per-row statistics seen by the draw: max, nucleus mass and nucleus boundary.
struct RowView {
    u128 zp;
    float m;
    unsigned int lam;
    int idx_cut;
};

// A sequence's decision and the view of its final row, decided by decide_seq.
struct SeqPlan {
    RowView v;
    SeqDecision d;
};

// The inputs of decide_seq, as the kernels that run it (one wave of theirs) receive them.
struct DecideIn {
    const void* logits;
    const float* dprobs;
    int K, V, nseg;
    float inv_t;
    int use_topp;
    const int32_t* drafts;
    const int32_t* n_drafts;
    const float* uniforms;
    const RowStats* stats;
    const int* status;
    const int* flag;
    const float* seg_max;
    const u64* seg_e;
    const RowPick* pick;
};
// F: per sequence, one wave: the acceptance walk and the view of the final row. Without
// top-p every row's values come from the segment maxima and sums; with top-p a row the
// bounds decided keeps that outcome and a flagged row is tested on its exact nucleus.
// Run by all 64 lanes of one wave (lane = threadIdx.x & 63); the result is uniform.
template <gg_dtype_t DT>
__device__ SeqPlan decide_seq(const DecideIn& in, int b) {
    const void* __restrict__ logits = in.logits;
    const float* __restrict__ dprobs = in.dprobs;
    const int K = in.K, V = in.V, nseg = in.nseg, use_topp = in.use_topp;
    const float inv_t = in.inv_t;
    const int32_t* __restrict__ drafts = in.drafts;
    const int32_t* __restrict__ n_drafts = in.n_drafts;
    const float* __restrict__ uniforms = in.uniforms;
    const RowStats* __restrict__ stats = in.stats;
    const int* __restrict__ status = in.status;
    const int* __restrict__ flag = in.flag;
    const float* __restrict__ seg_max = in.seg_max;
    const u64* __restrict__ seg_e = in.seg_e;
    const int R = K + 1;
    const int n = live_rows(n_drafts, b, K);
    // The rows' tests do not depend on each other, so they run together: groups of
    // g = 2^ceil(log2 nseg) lanes take one row each (lane s of a group reads segment s),
    // 64/g rows per pass; the walk stops at the first failed row.
    const int lane = threadIdx.x & 63;
    int g = 1;
    while (g < nseg) g <<= 1;
    const int per_pass = 64 / g;
    const int jl = lane / g, sl = lane % g;
    int a = n, residual = 0;
    for (int j0 = 0; j0 < n; j0 += per_pass) {
        const int j = j0 + jl;
        const bool live = j < n;
        const int row = b * R + (live ? j : 0);
        const int x = live ? drafts[(size_t)b * K + j] : -1;
        bool ok = true;
        if (use_topp && flag[row] != 1) {  // decided by the bounds (flag 2: only drawn from)
            ok = status[row] == kRowAccept;
        } else {
            float m;
            u128 zp, wx = 0;
            if (use_topp) {
                const RowStats st = stats[row];
                m = st.m;
                zp = st.zp;
                wx = st.wx;
            } else {
                const float ms = sl < nseg ? seg_max[(size_t)row * nseg + sl] : -INFINITY;
                m = ms;
                for (int o = g >> 1; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
                zp = (sl < nseg && finite_f(m)) ? (u128)seg_e[(size_t)row * nseg + sl] * seg_factor(ms, m, inv_t) : 0;
                for (int o = g >> 1; o > 0; o >>= 1) zp += shfl_xor_u128(zp, o);
                if (x >= 0 && x < V && finite_f(m)) {
                    const void* lp = (const uint8_t*)logits + (size_t)row * V * dtype_bytes(DT);
                    const Nucleus nu{m, inv_t, 0u, 0x7fffffff};
                    wx = nu.weight(ld<DT>(lp, x), x, seg_max[(size_t)row * nseg + x / kSegElems]);
                }
            }
            ok = false;
            if (x >= 0 && x < V && finite_f(m)) {
                const double q = dprobs ? gg_clean_q(dprobs[((size_t)b * K + j) * V + x]) : 1.0;
                const double u = (double)uniforms[(size_t)b * R + j];
                ok = u * q * gg_u128_to_double(zp) < gg_u128_to_double(wx);
            }
        }
        const unsigned long long bad = __ballot(live && !ok && sl == 0);
        if (bad) {
            a = j0 + (__ffsll((long long)bad) - 1) / g;
            residual = 1;
            break;
        }
    }
    return SeqPlan{RowView{}, SeqDecision{a, a, residual}};
}

// One wave per sequence: the acceptance walk, then what the final draw takes: the row
// and, after a rejection, the rejected draft (the residual draw excludes it).
// With top-p the row's fixed-point nucleus cut goes along as (boundary key << 32 | ~idx_cut)
// (0: none): the float64 cut is almost always that element, and otherwise almost always in
// its coarse bin, which the draw gathers in its first pass. A row only drawn from (flag 2)
// has no exact cut: its boundary coarse bin goes along as a range of l / T instead, which
// the draw's first pass gathers whole. A residual draw against a dense
// draft distribution without top-p gets the row's fixed-point total Z * 2^-70 as an
// estimate of its float64 softmax sum (0: none), which lets the draw's first pass sum the
// residual for all but the elements whose p and q nearly tie. The kernel then sets the
// sequence's draw up itself (fd::prep_row), so the draw needs no launch for it.
template <gg_dtype_t DT>
__global__ void __launch_bounds__(64) rej_decide_kernel(DecideIn din, int32_t* __restrict__ out_acc,
                                                        int* __restrict__ spec_row, int* __restrict__ spec_x,
                                                        unsigned long long* __restrict__ spec_key,
                                                        double* __restrict__ spec_s, fd::DrawParams P) {
    const int b = blockIdx.x;
    const SeqPlan p = decide_seq<DT>(din, b);
    double sest = 0.0;
    const int frow = b * (din.K + 1) + (p.d.row < 0 ? 0 : p.d.row);
    const float fm = row_max_wave(din.seg_max, frow, din.nseg);  // the drawn row's finite max
    if (p.d.residual && din.dprobs && !din.use_topp && finite_f(fm))  // uniform across the wave
        sest = gg_u128_to_double(row_z_wave(din.seg_max, din.seg_e, frow, din.nseg, fm, din.inv_t)) * 0x1p-70;
    if (threadIdx.x == 0) {
        spec_s[b] = sest;
        out_acc[b] = p.d.accepted;
        spec_row[b] = p.d.row;
        spec_x[b] = p.d.residual ? din.drafts[(size_t)b * din.K + p.d.row] : -1;
        unsigned long long key = 0;
        double vlo = 0.0, vhi = 0.0;
        if (din.use_topp) {
            if (din.flag[frow] == 2) {
                // Only drawn from: the values l / T of its boundary coarse bin (cb_abs bin A
                // holds l * (16 / T) in [A, A + 1)) as the draw's range hint.
                const RowPick pk = din.pick[frow];
                const int A = cb_abs(pk.m, din.inv_t) - pk.cbin;
                vlo = (double)A / 16.0;
                vhi = (double)(A + 1) / 16.0;
            } else {
                const RowStats st = din.stats[frow];
                if (st.valid && st.lam != 0u)
                    key = ((unsigned long long)st.lam << 32) | (unsigned long long)(~(unsigned int)st.idx_cut);
            }
        }
        spec_key[b] = key;
        const int x = p.d.residual ? din.drafts[(size_t)b * din.K + p.d.row] : -1;
        fd::prep_row(P, b, p.d.row, x, fm, fm > -INFINITY, P.hint_mode ? key : 0ull, x >= 0 ? sest : 0.0, 0,
                     P.hint_mode ? vlo : 0.0, P.hint_mode ? vhi : 0.0);
    }
}

}  // namespace

static int rej_nseg(int vocab) { return (vocab + kSegElems - 1) / kSegElems; }

struct RejWs {
    float* seg_max;
    u64* seg_e;
    int* spec_row;     // the final draw's row per sequence
    int* spec_x;       // the rejected draft of a residual draw, -1 for a plain draw
    unsigned long long* spec_key;  // top-p: the final row's fixed-point nucleus cut element
    double* spec_s;                // dense residual draws: the row's fixed-point total (0: none)
    void* draw;        // the final draw's own workspace (launch_final_draw)
    RowStats* stats;   // top-p: exact nucleus statistics of flagged rows
    u64* seg_hist;     // top-p: coarse histogram per (row, segment)
    RowPick* pick;
    int* status;       // top-p: bound outcome per row
    int* flag;         // top-p: row needs the exact nucleus
    int* n_flagged;    // top-p: lengths of the flagged-row and crowded-row lists
    int* crowded;      // top-p: flagged rows whose boundary bin is crowded
    int* flagged;      // top-p: the rows that need the exact nucleus
    uint2* cand;       // top-p: boundary-bin elements per row (logit bits, index)
    int* seq_cnt;      // top-p: rows of each sequence whose RowPick is out (row_pick_kernel)
    size_t bytes;
};

static RejWs rej_layout(void* base, int num_seqs, int max_drafts, int vocab, bool topp) {
    const size_t rows = (size_t)num_seqs * (max_drafts + 1);
    const int nseg = rej_nseg(vocab);
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    size_t off = 0;
    RejWs w{};
    uint8_t* p = (uint8_t*)base;
    auto take = [&](size_t bytes) {
        void* q = p + off;
        off += al(bytes);
        return q;
    };
    w.seg_max = (float*)take(rows * nseg * sizeof(float));
    w.seg_e = (u64*)take(rows * nseg * sizeof(u64));
    w.spec_row = (int*)take((size_t)num_seqs * sizeof(int));
    w.spec_x = (int*)take((size_t)num_seqs * sizeof(int));
    w.spec_key = (unsigned long long*)take((size_t)num_seqs * sizeof(unsigned long long));
    w.spec_s = (double*)take((size_t)num_seqs * sizeof(double));
    w.draw = take(final_draw_workspace_bytes(num_seqs, vocab));
    if (topp) {
        w.stats = (RowStats*)take(rows * sizeof(RowStats));
        w.seg_hist = (u64*)take(rows * nseg * kSegBins * sizeof(u64));
        w.pick = (RowPick*)take(rows * sizeof(RowPick));
        w.status = (int*)take(rows * sizeof(int));
        w.flag = (int*)take(rows * sizeof(int));
        w.n_flagged = (int*)take(2 * sizeof(int));
        w.crowded = (int*)take(rows * sizeof(int));
        w.flagged = (int*)take(rows * sizeof(int));
        w.cand = (uint2*)take(rows * kCandCap * sizeof(uint2));
        w.seq_cnt = (int*)take((size_t)num_seqs * sizeof(int));
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
    // The acceptance walk of each sequence runs inside the residual launch (dense q) or
    // the draw launch (one-hot q), not as a launch of its own.
    const DecideIn din{logits, q, K, vocab, nseg, inv_t, use_topp, drafts, n_drafts, uniforms,
                       w.stats, w.status, w.flag, w.seg_max, w.seg_e, w.pick};
    const DecideBoundsIn dbin{logits, q, K, vocab, nseg, inv_t, drafts, n_drafts, uniforms, w.seg_max, w.seg_e,
                              w.pick, w.status, w.flag, w.n_flagged, w.flagged};
    FinalDraw d{};
    d.logits = logits;
    d.dt = dt;
    d.num_seqs = num_seqs;
    d.max_drafts = K;
    d.vocab = vocab;
    d.temperature = (double)temperature;
    d.top_k = 0;
    d.top_p = (double)top_p;
    d.uniforms_f32 = uniforms;
    d.draft_probs = q;
    d.spec_row = w.spec_row;
    d.spec_x = w.spec_x;
    d.spec_key = w.spec_key;
    d.spec_s = w.spec_s;
    d.seg_max = w.seg_max;
    d.nseg_max = nseg;
    d.out_tok = out_tok;
    d.prepped = true;  // rej_decide_kernel sets each sequence's draw up
    const fd::DrawParams P = fd::final_draw_params(d, w.draw);
#define GG_REJ(DTV)                                                                                          \
    if (use_topp) {                                                                                          \
        seg_pass_kernel<DTV, true><<<dim3(nseg, rows), kSegThreads, 0, s>>>(                                 \
            logits, K, vocab, nseg, vec_ok, inv_t, n_drafts, w.seg_max, w.seg_e, w.seg_hist, w.seq_cnt,       \
            w.n_flagged);                                                                                    \
        row_pick_kernel<DTV><<<rows, kSegThreads, 0, s>>>(nseg, top_p, w.seg_hist, w.seq_cnt, dbin);         \
        seg_gather_kernel<DTV><<<dim3(nseg, num_seqs), kSegThreads, 0, s>>>(logits, vocab, nseg, vec_ok,     \
                                                                            inv_t, w.n_flagged, w.flagged,   \
                                                                            w.seg_max, w.pick, w.cand);      \
        row_select_kernel<DTV><<<num_seqs, 1024, 0, s>>>(logits, K, vocab, nseg, inv_t, top_p, drafts,       \
                                                         n_drafts, w.n_flagged, w.flagged, w.seg_max,        \
                                                         w.seg_e, w.pick, w.cand, w.stats, w.n_flagged + 1,  \
                                                         w.crowded);                                         \
        rejection_row_stats_kernel<DTV><<<kRowStatsBlocks, kThreads, 0, s>>>(                                \
            logits, K, vocab, nseg, drafts, n_drafts, inv_t, top_p, w.n_flagged + 1, w.crowded, w.seg_max,   \
            w.seg_e, w.stats);                                                                               \
    } else {                                                                                                 \
        seg_pass_kernel<DTV, false><<<dim3(nseg, rows), kSegThreads, 0, s>>>(logits, K, vocab, nseg, vec_ok, \
                                                                             inv_t, n_drafts, w.seg_max,     \
                                                                             w.seg_e, nullptr, nullptr,      \
                                                                             nullptr);                       \
    }                                                                                                        \
    rej_decide_kernel<DTV><<<num_seqs, 64, 0, s>>>(din, out_acc, w.spec_row, w.spec_x, w.spec_key, w.spec_s, P);
    switch (dt) {
        case GG_DTYPE_F32: GG_REJ(GG_DTYPE_F32) break;
        case GG_DTYPE_BF16: GG_REJ(GG_DTYPE_BF16) break;
        case GG_DTYPE_F16: GG_REJ(GG_DTYPE_F16) break;
        default: return fail(GG_ERR_INVALID, "accept_rejection: logits dtype");
    }
#undef GG_REJ
    const gg_status_t st = check_hip(hipGetLastError(), "accept_rejection launch");
    if (st != GG_OK) return st;
    return launch_final_draw(d, w.draw, s);
}

}  // namespace gg
