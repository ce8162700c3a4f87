// ngram_draft.hip — n-gram draft lookup on the device.
//
// Restates NGramDrafter.Draft (internal/engine/speculative.go:24-62). The
// reference builds a map from every (n-1)-gram at i in [0, len-n] to the token at
// i+n-1, later occurrences overwriting earlier ones, then chains up to max_drafts
// lookups of the running suffix (drafts extend the suffix, never the table).
// Here no table is built: each lookup is a parallel scan for the LARGEST i whose
// (n-1)-gram equals the key, which is exactly the entry the map would hold.
// One 256-thread block per sequence; the history is staged through LDS in tiles.
#include "gg_common.h"

namespace gg {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 4096;  // tokens staged per LDS tile (plus n-2 halo)

__global__ void __launch_bounds__(kThreads) ngram_draft_kernel(
    const int32_t* __restrict__ hist, int stride, const int32_t* __restrict__ hist_len, int n,
    int K, int32_t* __restrict__ out_drafts, int32_t* __restrict__ out_n) {
    const int b = blockIdx.x;
    const int32_t* h = hist + (size_t)b * stride;
    int L = hist_len[b];
    if (L > stride) L = stride;
    const int kl = n - 1;
    __shared__ int32_t tile[kTile + 8];
    __shared__ int32_t key[16];
    __shared__ int best_s[kThreads / 64];
    __shared__ int n_out;
    if (threadIdx.x == 0) n_out = 0;
    if (L < n) {
        if (threadIdx.x == 0) out_n[b] = 0;
        return;
    }
    if (threadIdx.x < kl) key[threadIdx.x] = h[L - kl + threadIdx.x];
    __syncthreads();
    const int last = L - n;  // largest table start index
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
            out_drafts[(size_t)b * K + step] = next;
            for (int k = 0; k + 1 < kl; ++k) key[k] = key[k + 1];
            key[kl - 1] = next;
            n_out = step + 1;
        }
        __syncthreads();
    }
    __syncthreads();
    if (threadIdx.x == 0) out_n[b] = n_out;
}

}  // namespace

gg_status_t launch_ngram_draft(const int32_t* hist, int stride, const int32_t* hist_len, int num_seqs,
                               int n, int max_drafts, int32_t* out_drafts, int32_t* out_n,
                               hipStream_t s) {
    ngram_draft_kernel<<<num_seqs, kThreads, 0, s>>>(hist, stride, hist_len, n, max_drafts,
                                                      out_drafts, out_n);
    return check_hip(hipGetLastError(), "ngram_draft launch");
}

}  // namespace gg
