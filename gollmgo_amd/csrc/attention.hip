// attention.hip — multi-query split-K paged attention for the verify rows.
//
// Semantics: textbook softmax attention per (sequence, draft row, query head),
// as the reference's v1 kernel defines it for one query
// (kernels/gollmgo_paged_attn.cu:38-119: GQA kv_head = h / (Hq/Hkv), scores
// q.k*scale, max-subtracted softmax, P.V) extended to R causal rows per sequence
// with the mask of naive_attention (kernels/gollmgo_ops.cu:178: key j is visible
// to row i iff position_j <= position_i). Long contexts are split into
// partitions whose (max, sum, unnormalised P.V) partials are merged with the
// log-sum-exp identity — the job of paged_attention_v2_{phase1,reduce}
// (kernels/gollmgo_paged_attn.cu:234-384), whose reduce is not followed because it
// normalises only in thread 0 and mixes partial strides.
//
// Two phase-1 kernels share one partial format and one combine kernel:
//   - attn_mfma_kernel (attention_mfma.hip): gfx950 MFMA path for head_dim 128,
//     block_size 16, BF16/F16/FP8/INT8 pools, G*R <= 64 rows per kv head;
//   - attn_generic_kernel (here): any head_dim <= 1024 / block size / pool dtype,
//     one wave per (row, head, partition), scalar online softmax. Used for the
//     shapes the MFMA tiling does not cover (e.g. fp32 pools, head_dim 64).
#include "gg_common.h"
#include "attention_common.h"

namespace gg {
namespace {

constexpr int kMaxDC = 16;  // head_dim <= 1024 -> up to 16 dims per lane

template <int DC>
__global__ void __launch_bounds__(64) attn_generic_kernel(AttnArgs a, KVView kv) {
    const int part = blockIdx.x;
    const int h = blockIdx.y;
    const int z = blockIdx.z;  // b*R + j
    const int b = z / a.rows, j = z % a.rows;
    const int nrows = a.row_counts ? a.row_counts[b] : a.rows;
    if (j >= nrows) return;
    const int ctx = seq_keys(a, b, kv.bs);
    if (ctx <= 0 || nrows > ctx) return;
    const int P = a.partition;
    const int nparts = (ctx + P - 1) / P;
    if (part >= nparts) return;
    const int pos = ctx - nrows + j;
    const int t0 = part * P;
    const int t1 = min(t0 + P, pos + 1);
    const int G = a.num_q_heads / kv.Hkv;
    const int kvh = h / G;
    const int lane = threadIdx.x;
    const int D = kv.D;

    float q[DC], acc[DC];
    const size_t qbase = ((size_t)z * a.num_q_heads + h) * D;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
        const int d = lane + 64 * c;
        q[c] = d < D ? load_as_f32(a.q, a.q_dtype, qbase + d) : 0.f;
        acc[c] = 0.f;
    }
    const int32_t* bt = a.block_tables + (size_t)b * a.max_blocks;
    float m = -1e30f, l = 0.f;
    for (int t = t0; t < t1; ++t) {
        const int blk = bt[t / kv.bs];
        const int off = t % kv.bs;
        if (blk < 0 || blk >= kv.num_blocks) continue;  // invalid table entry: key skipped
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) dot += q[c] * kv.k_at(blk, kvh, off, d);
        }
        for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
        const float s = dot * a.scale * kv.k_scale(blk, kvh);
        const float m_new = fmaxf(m, s);
        const float alpha = __expf(m - m_new);
        const float p = __expf(s - m_new);
        l = l * alpha + p;
        const float pv = p * kv.v_scale(blk, kvh);
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const int d = lane + 64 * c;
            const float vv = d < D ? kv.v_at(blk, kvh, off, d) : 0.f;
            acc[c] = acc[c] * alpha + pv * vv;
        }
        m = m_new;
    }
    if (nparts == 1) {
        const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const int d = lane + 64 * c;
            if (d < D) store_from_f32(a.out, a.out_dtype, qbase + d, acc[c] * inv);
        }
        return;
    }
    const size_t pidx = ((size_t)z * a.num_q_heads + h) * a.max_parts + part;
    if (lane == 0) {
        a.ws_ml[pidx * 2 + 0] = m;
        a.ws_ml[pidx * 2 + 1] = l;
    }
#pragma unroll
    for (int c = 0; c < DC; ++c) {
        const int d = lane + 64 * c;
        if (d < D) a.ws_acc[pidx * D + d] = acc[c];
    }
}

// Merge the partitions of one (row, head): out = sum_p e^{m_p-M} acc_p / sum_p e^{m_p-M} l_p.
__global__ void __launch_bounds__(128) attn_combine_kernel(AttnArgs a, int D) {
    const int h = blockIdx.x;
    const int z = blockIdx.y;
    const int b = z / a.rows, j = z % a.rows;
    const int nrows = a.row_counts ? a.row_counts[b] : a.rows;
    if (j >= nrows) return;
    const int ctx = seq_keys(a, b, a.kv_bs);
    const int nparts = (ctx + a.partition - 1) / a.partition;
    if (nparts <= 1 || nrows > ctx) return;
    const size_t base = ((size_t)z * a.num_q_heads + h) * a.max_parts;
    __shared__ float wgt[512];
    __shared__ float inv_total;
    float M = -1e30f;
    for (int p = 0; p < nparts; ++p) M = fmaxf(M, a.ws_ml[(base + p) * 2]);
    // nparts <= max_parts; weights are staged in chunks of 512 partitions.
    float acc_local[8];
    const int DPT = (D + blockDim.x - 1) / blockDim.x;  // <= 8 for D <= 1024
    for (int c = 0; c < 8; ++c) acc_local[c] = 0.f;
    float total = 0.f;
    for (int p0 = 0; p0 < nparts; p0 += 512) {
        const int pn = min(512, nparts - p0);
        __syncthreads();
        for (int p = threadIdx.x; p < pn; p += blockDim.x)
            wgt[p] = __expf(a.ws_ml[(base + p0 + p) * 2] - M);
        __syncthreads();
        for (int p = 0; p < pn; ++p) total += wgt[p] * a.ws_ml[(base + p0 + p) * 2 + 1];
        for (int c = 0; c < DPT; ++c) {
            const int d = threadIdx.x + c * blockDim.x;
            if (d >= D) break;
            float s = 0.f;
            for (int p = 0; p < pn; ++p) s += wgt[p] * a.ws_acc[(base + p0 + p) * D + d];
            acc_local[c] += s;
        }
    }
    if (threadIdx.x == 0) inv_total = total > 0.f ? 1.0f / total : 0.f;
    __syncthreads();
    const size_t obase = ((size_t)z * a.num_q_heads + h) * D;
    for (int c = 0; c < DPT; ++c) {
        const int d = threadIdx.x + c * blockDim.x;
        if (d >= D) break;
        store_from_f32(a.out, a.out_dtype, obase + d, acc_local[c] * inv_total);
    }
}

}  // namespace

AttnPlan attn_plan(const KV* kv, int num_seqs, int rows, int num_q_heads, int max_blocks,
                   int partition_tokens) {
    if (partition_tokens > 0) return {ATTN_SCHED_GRID, partition_tokens};
    if (!attn_mfma_supported(kv, rows, num_q_heads)) return {ATTN_SCHED_GRID, 512};
    // Measured on MI355X: while the (sequence, kv head) items alone fill every resident
    // workgroup slot, longest-first pieces (LPT: items longer than the mean slot load cut
    // in equal pieces, dispatched longest first) balance ragged contexts best; beyond the
    // sequences an LPT workgroup can rank, one workgroup per item (no split, no merge).
    // With fewer items than slots, or keys beyond one MFMA piece, stream-K splits evenly.
    const int G = num_q_heads / kv->num_kv_heads;
    const int nt = (G * rows + 15) / 16;
    const long long max_keys = (long long)max_blocks * kv->block_size;
    const long long items = (long long)num_seqs * kv->num_kv_heads;
    const long long slots = (long long)device_cu_count() * attn_occupancy(nt);
    if (items >= slots && num_seqs <= kLptMaxSeqs) return {ATTN_SCHED_LPT, 0};
    if (items >= slots && max_keys <= kMfmaMaxPartition)
        return {ATTN_SCHED_GRID, (int)((max_keys + 63) / 64 * 64)};
    return {ATTN_SCHED_STREAMK, 0};
}

size_t attn_workspace_bytes(const KV* kv, int num_seqs, int rows, int num_q_heads, int max_blocks,
                            int partition) {
    const int max_parts = (max_blocks * kv->block_size + partition - 1) / partition;
    if (max_parts <= 1) return 0;
    size_t n_ml = (size_t)num_seqs * rows * num_q_heads * max_parts * 2;
    n_ml = ((n_ml + 63) / 64) * 64;
    size_t n_acc = (size_t)num_seqs * rows * num_q_heads * max_parts * kv->head_dim;
    return (n_ml + n_acc) * sizeof(float);
}

gg_status_t launch_verify_attention(const AttnArgs& a, hipStream_t s) {
    const KV* kv = a.kv;
    KVView view = make_kv_view(kv, a.layer);
    if (a.sched != ATTN_SCHED_GRID || (attn_mfma_supported(kv, a.rows, a.num_q_heads) && a.partition % 64 == 0 &&
                                       a.partition <= kMfmaMaxPartition)) {
        // Stream-K and LPT launch their own merge over their record layout.
        gg_status_t st = launch_attn_mfma(a, view, s);
        if (st != GG_OK) return st;
        if (a.sched != ATTN_SCHED_GRID) return check_hip(hipGetLastError(), "verify_attention launch");
    } else {
        const int DC = (kv->head_dim + 63) / 64;
        dim3 grid(a.max_parts, a.num_q_heads, a.num_seqs * a.rows);
#define GG_GEN(N) \
    case N: attn_generic_kernel<N><<<grid, 64, 0, s>>>(a, view); break;
        switch (DC) {
            GG_GEN(1) GG_GEN(2) GG_GEN(3) GG_GEN(4) GG_GEN(5) GG_GEN(6) GG_GEN(7) GG_GEN(8)
            GG_GEN(9) GG_GEN(10) GG_GEN(11) GG_GEN(12) GG_GEN(13) GG_GEN(14) GG_GEN(15) GG_GEN(16)
            default: return fail(GG_ERR_INVALID, "attention: head_dim too large");
        }
#undef GG_GEN
    }
    if (a.max_parts > 1) {
        attn_combine_kernel<<<dim3(a.num_q_heads, a.num_seqs * a.rows), 128, 0, s>>>(a, kv->head_dim);
    }
    static_assert(kMaxDC == 16, "generic kernel instantiations cover head_dim <= 1024");
    return check_hip(hipGetLastError(), "verify_attention launch");
}

}  // namespace gg
