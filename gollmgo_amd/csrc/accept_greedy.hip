// accept_greedy.hip — greedy verify on the device.
//
// Replaces the host-side Verify/argmax loop (internal/engine/speculative.go:68-84,
// internal/engine/sampling.go:75-85) driven by emitSpeculative
// (internal/engine/serving.go:514-566). Two launches:
//   1) segment argmax: grid (segments, rows); each block scans 4096 logits of one
//      row with 16-byte loads and writes (value, index) of its first maximum;
//   2) decide: one block per sequence merges the segments of rows 0..n, every row at
//      once (a lane group per row), then walks the drafts in order: the first row whose
//      argmax differs from its draft ends the accepted prefix and supplies the corrected
//      token; if none differs, row n supplies the bonus token.
// Tie rule: first index of the maximum. NaN never wins; a NaN at element 0 makes
// the row's argmax 0 (the reference scans with `>` from element 0).
#include "gg_common.h"

namespace gg {
namespace {

constexpr int kSeg = 4096;
constexpr int kThreads = 256;
constexpr int kNone = 0x7fffffff;

struct ArgBest {
    float v;
    int i;
};

__device__ __forceinline__ void consider(ArgBest& b, float v, int i) {
    // v == v filters NaN; ties keep the lower index.
    if (v == v && (v > b.v || (v == b.v && i < b.i))) {
        b.v = v;
        b.i = i;
    }
}

__device__ __forceinline__ ArgBest wave_best(ArgBest b) {
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(b.v, o);
        int oi = __shfl_xor(b.i, o);
        if (oi != kNone && (b.i == kNone || ov > b.v || (ov == b.v && oi < b.i))) {
            b.v = ov;
            b.i = oi;
        }
    }
    return b;
}

template <gg_dtype_t DT>
__device__ __forceinline__ void scan_vec(ArgBest& b, const void* row, int base, int V) {
    // base is a multiple of kSeg; every 16-byte chunk is element-aligned because V*eb % 16 == 0.
    constexpr int kPer = DT == GG_DTYPE_F32 ? 4 : 8;
    constexpr int kIters = kSeg / (kThreads * kPer);
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int e0 = base + (it * kThreads + threadIdx.x) * kPer;
        if (e0 >= V) break;
        uint4 raw = *(const uint4*)((const uint8_t*)row + (size_t)e0 * (DT == GG_DTYPE_F32 ? 4 : 2));
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        if constexpr (DT == GG_DTYPE_F32) {
#pragma unroll
            for (int k = 0; k < 4; ++k) consider(b, __uint_as_float(w[k]), e0 + k);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                uint16_t h = (uint16_t)(w[k >> 1] >> ((k & 1) * 16));
                float f = DT == GG_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
                consider(b, f, e0 + k);
            }
        }
    }
}

__global__ void __launch_bounds__(kThreads) greedy_segment_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int R, int V, int nseg, int vec_ok,
    const int32_t* __restrict__ n_drafts, float2* __restrict__ ws) {
    const int row = blockIdx.y;  // b*R + j
    const int b = row / R, j = row % R;
    const int nb = n_drafts[b];
    if (j > (nb < 0 ? 0 : nb)) return;  // rows 0..n, n clamped as the decide kernel clamps it
    const int seg = blockIdx.x;
    const int base = seg * kSeg;
    ArgBest best{-INFINITY, kNone};
    const size_t eb = dtype_bytes(dt);
    const void* rowp = (const uint8_t*)logits + (size_t)row * V * eb;
    if (vec_ok) {
        if (dt == GG_DTYPE_F32) scan_vec<GG_DTYPE_F32>(best, rowp, base, V);
        else if (dt == GG_DTYPE_BF16) scan_vec<GG_DTYPE_BF16>(best, rowp, base, V);
        else scan_vec<GG_DTYPE_F16>(best, rowp, base, V);
    } else {
        const int end = min(base + kSeg, V);
        for (int e = base + threadIdx.x; e < end; e += kThreads) consider(best, load_as_f32(rowp, dt, e), e);
    }
    best = wave_best(best);
    __shared__ ArgBest sb[kThreads / 64];
    const int wv = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) sb[wv] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        ArgBest r = sb[0];
        for (int w = 1; w < kThreads / 64; ++w) {
            ArgBest o = sb[w];
            if (o.i != kNone && (r.i == kNone || o.v > r.v || (o.v == r.v && o.i < r.i))) r = o;
        }
        ws[(size_t)row * nseg + seg] = make_float2(r.v, __int_as_float(r.i));
    }
}

// Lane group of g = 2^ceil(log2 nseg) lanes per row (lane s of a group reads segment s,
// and s + g, ... past 64), kDecideThreads / g rows per pass; each row's argmax lands in LDS
// and thread 0 walks the rows. (Walking row by row, each row's loads waiting for the
// previous row's decision, took 13 us for nine rows.)
constexpr int kDecideThreads = 512;
constexpr int kMaxRows = 65;  // rows per sequence: max_drafts + 1, max_drafts <= 64 (checked by the ABI)
__global__ void __launch_bounds__(kDecideThreads) greedy_decide_kernel(
    const void* __restrict__ logits, gg_dtype_t dt, int K, int V, int nseg,
    const int32_t* __restrict__ drafts, const int32_t* __restrict__ n_drafts,
    const float2* __restrict__ ws, int32_t* __restrict__ out_acc, int32_t* __restrict__ out_tok) {
    const int b = blockIdx.x;
    const int R = K + 1;
    int n = n_drafts[b];
    n = n < 0 ? 0 : (n > K ? K : n);
    __shared__ int s_am[kMaxRows];
    int g = 1;
    while (g < nseg && g < 64) g <<= 1;
    const int per_pass = kDecideThreads / g;
    const int jl = threadIdx.x / g, sl = threadIdx.x % g;
    for (int j0 = 0; j0 <= n; j0 += per_pass) {
        const int j = j0 + jl;
        const bool live = j <= n;
        const int row = b * R + (live ? j : 0);
        const float first = load_as_f32(logits, dt, (size_t)row * V);
        ArgBest best{-INFINITY, kNone};
        for (int s = sl; s < nseg; s += g) {
            const float2 p = ws[(size_t)row * nseg + s];
            const int pi = __float_as_int(p.y);
            if (pi != kNone && (best.i == kNone || p.x > best.v || (p.x == best.v && pi < best.i))) {
                best.v = p.x;
                best.i = pi;
            }
        }
        for (int o = g >> 1; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best.v, o);
            const int oi = __shfl_xor(best.i, o);
            if (oi != kNone && (best.i == kNone || ov > best.v || (ov == best.v && oi < best.i))) {
                best.v = ov;
                best.i = oi;
            }
        }
        if (live && sl == 0) s_am[j] = (first != first || best.i == kNone) ? 0 : best.i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int accepted = n, token = s_am[n];
        for (int j = 0; j < n; ++j) {
            if (s_am[j] != drafts[(size_t)b * K + j]) {
                accepted = j;
                token = s_am[j];
                break;
            }
        }
        out_acc[b] = accepted;
        out_tok[b] = token;
    }
}

}  // namespace

size_t greedy_workspace_bytes(int num_seqs, int max_drafts, int vocab) {
    int nseg = (vocab + kSeg - 1) / kSeg;
    return (size_t)num_seqs * (max_drafts + 1) * nseg * sizeof(float2);
}

gg_status_t launch_accept_greedy(const void* logits, gg_dtype_t dt, int num_seqs, int max_drafts,
                                 int vocab, const int32_t* drafts, const int32_t* n_drafts,
                                 int32_t* out_acc, int32_t* out_tok, void* ws, hipStream_t s) {
    const int R = max_drafts + 1;
    if (R > kMaxRows) return fail(GG_ERR_INVALID, "accept_greedy: more than 64 drafts per sequence");
    const int nseg = (vocab + kSeg - 1) / kSeg;
    const size_t eb = dtype_bytes(dt);
    const int vec_ok = ((vocab * eb) % 16 == 0) && (((uintptr_t)logits) % 16 == 0);
    greedy_segment_kernel<<<dim3(nseg, num_seqs * R), kThreads, 0, s>>>(logits, dt, R, vocab, nseg,
                                                                       vec_ok, n_drafts, (float2*)ws);
    greedy_decide_kernel<<<num_seqs, kDecideThreads, 0, s>>>(logits, dt, max_drafts, vocab, nseg, drafts,
                                                 n_drafts, (const float2*)ws, out_acc, out_tok);
    return check_hip(hipGetLastError(), "accept_greedy launch");
}

}  // namespace gg
