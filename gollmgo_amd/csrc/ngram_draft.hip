// ngram_draft.hip — n-gram draft lookup on the device.
//
// Restates NGramDrafter.Draft (internal/engine/speculative.go:24-62). The
// reference builds a map from every (n-1)-gram at i in [0, len-n] to the token at
// i+n-1, later occurrences overwriting earlier ones, then chains up to max_drafts
// lookups of the running suffix (drafts extend the suffix, never the table).
// Here no table is built: each lookup is a parallel scan for the LARGEST i whose
// (n-1)-gram equals the key, which is exactly the entry the map would hold.
// One 256-thread block per sequence. A history of up to kResident tokens is staged in
// LDS once and every lookup scans it there (the next token is read from LDS too);
// longer histories are streamed through LDS in tiles for each lookup.
#include "gg_common.h"

namespace gg {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 4096;  // tokens staged per LDS tile (plus n-2 halo)
constexpr int kResident = 12288;  // histories up to this length stay in LDS (48 KB)

// Largest i in [0, last] whose (n-1)-gram at i equals key (kl <= 8 tokens), over the
// history in LDS; -1 if none. Thread t checks the 32 consecutive starts [32t, 32t+32) of
// each 8192-start pass from 16-byte LDS reads (its run plus an 8-token halo), so the scan
// has no per-start loads or divergent early exits. All threads return the result.
template <int KL>
__device__ __forceinline__ int scan_resident(const int32_t* hs, int last, const int32_t* key_s, int* best_s) {
    int key[KL];
#pragma unroll
    for (int k = 0; k < KL; ++k) key[k] = key_s[k];
    int local = -1;
    for (int base = 0; base <= last; base += 32 * kThreads) {
        const int p0 = base + 32 * (int)threadIdx.x;
        if (p0 > last) continue;
        int v[40];
#pragma unroll
        for (int q = 0; q < 10; ++q) {
            const int4 w = ((const int4*)(hs + p0))[q];
            v[4 * q] = w.x;
            v[4 * q + 1] = w.y;
            v[4 * q + 2] = w.z;
            v[4 * q + 3] = w.w;
        }
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            bool eq = p0 + j <= last;
#pragma unroll
            for (int k = 0; k < KL; ++k) eq = eq && v[j + k] == key[k];
            if (eq) local = p0 + j;  // ascending j: keeps the largest
        }
    }
    for (int o = 32; o > 0; o >>= 1) local = max(local, __shfl_xor(local, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) best_s[threadIdx.x / 64] = local;
    __syncthreads();
    int m = -1;
    for (int w = 0; w < kThreads / 64; ++w) m = max(m, best_s[w]);
    return m;
}

// The drafts of one sequence whose history is h[0, L): up to K chained lookups, written
// to od[0..) and their count to *on. KL = n - 1 key tokens (1..8), a compile-time
// constant for the resident scan. The whole workgroup calls it.
template <int KL>
__device__ __forceinline__ void draft_one(const int32_t* __restrict__ h, int L, int n, int K,
                                          int32_t* __restrict__ od, int32_t* __restrict__ on) {
    const int kl = n - 1;
    // (A resident history may be read up to 8 + 32 tokens past its end: padding.)
    __shared__ __align__(16) int32_t tile[kResident + 48];
    __shared__ int32_t key[16];
    __shared__ int best_s[kThreads / 64];
    __shared__ int n_out;
    if (threadIdx.x == 0) n_out = 0;
    if (L < n) {
        if (threadIdx.x == 0) *on = 0;
        return;
    }
    if (threadIdx.x < kl) key[threadIdx.x] = h[L - kl + threadIdx.x];
    __syncthreads();
    const int last = L - n;  // largest table start index
    if (L <= kResident) {
        if ((((uintptr_t)h) & 15) == 0) {
            for (int i = threadIdx.x; i < L / 4; i += kThreads) ((int4*)tile)[i] = ((const int4*)h)[i];
            for (int i = (L / 4) * 4 + threadIdx.x; i < L; i += kThreads) tile[i] = h[i];
        } else {
            for (int i = threadIdx.x; i < L; i += kThreads) tile[i] = h[i];
        }
        __syncthreads();
        // Drafts are kept in LDS and written once at the end: a barrier after a global
        // store would wait for that store on every step.
        __shared__ int32_t drafts_s[64];
        int step = 0;
        for (; step < K; ++step) {
            const int best = scan_resident<KL>(tile, last, key, best_s);
            if (best < 0) break;
            const int next = tile[best + kl];
            __syncthreads();
            if (threadIdx.x == 0) {
                drafts_s[step] = next;
                for (int k = 0; k + 1 < kl; ++k) key[k] = key[k + 1];
                key[kl - 1] = next;
            }
            __syncthreads();
        }
        if ((int)threadIdx.x < step) od[threadIdx.x] = drafts_s[threadIdx.x];
        if (threadIdx.x == 0) *on = step;
        return;
    }
    for (int step = 0; step < K; ++step) {
        int best = -1;
        // Scan tiles from the end so most lookups finish in the first tile.
        for (int t_end = last + 1; t_end > 0 && best < 0; t_end -= kTile) {
            const int t_begin = max(0, t_end - kTile);
            const int cnt = t_end - t_begin + kl;  // tokens needed incl. key halo and next token
            __syncthreads();
            for (int i = threadIdx.x; i < cnt; i += kThreads) tile[i] = h[t_begin + i];
            __syncthreads();
            int local = -1;
            for (int i = t_begin + threadIdx.x; i < t_end; i += kThreads) {
                bool eq = true;
                for (int k = 0; k < kl; ++k) eq = eq && (tile[i - t_begin + k] == key[k]);
                if (eq) local = max(local, i);
            }
            for (int o = 32; o > 0; o >>= 1) local = max(local, __shfl_xor(local, o));
            if ((threadIdx.x & 63) == 0) best_s[threadIdx.x / 64] = local;
            __syncthreads();
            int m = -1;
            for (int w = 0; w < kThreads / 64; ++w) m = max(m, best_s[w]);
            best = m;
        }
        if (best < 0) break;
        const int next = h[best + kl];
        __syncthreads();
        if (threadIdx.x == 0) {
            od[step] = next;
            for (int k = 0; k + 1 < kl; ++k) key[k] = key[k + 1];
            key[kl - 1] = next;
            n_out = step + 1;
        }
        __syncthreads();
    }
    __syncthreads();
    if (threadIdx.x == 0) *on = n_out;
}

template <int KL>
__global__ void __launch_bounds__(kThreads) ngram_draft_kernel(
    const int32_t* __restrict__ hist, int stride, const int32_t* __restrict__ hist_len, int n,
    int K, int32_t* __restrict__ out_drafts, int32_t* __restrict__ out_n) {
    const int b = blockIdx.x;
    const int L = min(hist_len[b], stride);
    draft_one<KL>(hist + (size_t)b * stride, L, n, K, out_drafts + (size_t)b * K, out_n + b);
}

// The step's emitted tokens appended to each sequence's history, then its next drafts:
// emitSpeculative (internal/engine/serving.go:541-566) emits the accepted drafts
// drafts[b][0, accepted) and then the corrected or bonus token, and maybeDraft
// (serving.go:608-620) drafts the next step from the whole history. Sequence b's history
// is row rows[b] (b when rows is NULL). A history that the tokens would take past the
// stride is left unchanged and its length set to -1 (no drafts from it until the caller
// reseeds it); a negative length stays -1.
template <int KL>
__global__ void __launch_bounds__(kThreads) history_append_draft_kernel(
    int32_t* __restrict__ hist, int stride, int32_t* __restrict__ hist_len, const int32_t* __restrict__ rows,
    const int32_t* __restrict__ drafts, int k_in, const int32_t* __restrict__ accepted,
    const int32_t* __restrict__ token, int n, int K, int32_t* __restrict__ out_drafts,
    int32_t* __restrict__ out_n) {
    const int b = blockIdx.x;
    const int row = rows ? rows[b] : b;
    int32_t* h = hist + (size_t)row * stride;
    const int L = hist_len[row];
    const int acc = min(max(accepted[b], 0), k_in);
    const int tok = token[b];
    const int cnt = acc + (tok >= 0 ? 1 : 0);
    if (L < 0 || L + cnt > stride) {
        if (threadIdx.x == 0) {
            hist_len[row] = -1;
            out_n[b] = 0;
        }
        return;
    }
    if ((int)threadIdx.x < cnt) h[L + threadIdx.x] = (int)threadIdx.x < acc ? drafts[(size_t)b * k_in + threadIdx.x] : tok;
    // The appended tokens are read back by other threads of the workgroup (the key, the
    // scans): workgroup-scope release and acquire around the barrier.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (threadIdx.x == 0) hist_len[row] = L + cnt;
    draft_one<KL>(h, L + cnt, n, K, out_drafts + (size_t)b * K, out_n + b);
}

}  // namespace

gg_status_t launch_ngram_draft(const int32_t* hist, int stride, const int32_t* hist_len, int num_seqs,
                               int n, int max_drafts, int32_t* out_drafts, int32_t* out_n,
                               hipStream_t s) {
    switch (n - 1) {
#define GG_NG(KLV) \
    case KLV: ngram_draft_kernel<KLV><<<num_seqs, kThreads, 0, s>>>(hist, stride, hist_len, n, max_drafts, out_drafts, out_n); break;
        GG_NG(1) GG_NG(2) GG_NG(3) GG_NG(4) GG_NG(5) GG_NG(6) GG_NG(7)
        default: GG_NG(8)
#undef GG_NG
    }
    return check_hip(hipGetLastError(), "ngram_draft launch");
}

gg_status_t launch_history_append_draft(int32_t* hist, int stride, int32_t* hist_len, const int32_t* rows,
                                        int num_seqs, const int32_t* drafts, int k_in, const int32_t* accepted,
                                        const int32_t* token, int n, int max_drafts, int32_t* out_drafts,
                                        int32_t* out_n, hipStream_t s) {
    switch (n - 1) {
#define GG_HA(KLV)                                                                                               \
    case KLV:                                                                                                    \
        history_append_draft_kernel<KLV><<<num_seqs, kThreads, 0, s>>>(hist, stride, hist_len, rows, drafts, k_in, \
                                                                      accepted, token, n, max_drafts, out_drafts, \
                                                                      out_n);                                     \
        break;
        GG_HA(1) GG_HA(2) GG_HA(3) GG_HA(4) GG_HA(5) GG_HA(6) GG_HA(7)
        default: GG_HA(8)
#undef GG_HA
    }
    return check_hip(hipGetLastError(), "history_append_draft launch");
}

}  // namespace gg
