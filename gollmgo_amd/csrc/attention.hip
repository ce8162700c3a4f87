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
#include <type_traits>

#include "gg_common.h"
#include "attention_common.h"

namespace gg {
namespace {

constexpr int kMaxDC = 16;  // head_dim <= 1024 -> up to 16 dims per lane

// One pool element as f32 (raw, before its block / head scale), pool type fixed.
template <gg_dtype_t DT>
__device__ __forceinline__ float pool_elem(const uint8_t* base, size_t i) {
    if constexpr (DT == GG_DTYPE_F32) return ((const float*)base)[i];
    else if constexpr (DT == GG_DTYPE_F16) return f16_bits_to_f32(((const uint16_t*)base)[i]);
    else if constexpr (DT == GG_DTYPE_BF16) return bf16_bits_to_f32(((const uint16_t*)base)[i]);
    else if constexpr (DT == GG_DTYPE_FP8_E4M3) return fp8e4m3_to_f32(base[i]);
    else return (float)((const int8_t*)base)[i];
}

// The pool elements in 16 bytes, as f32.
template <gg_dtype_t DT>
struct Pool16 {
    static constexpr int kN = DT == GG_DTYPE_F32 ? 4 : (DT == GG_DTYPE_F16 || DT == GG_DTYPE_BF16) ? 8 : 16;
    __device__ static __forceinline__ void decode(const uint4 r, float (&f)[kN]) {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int k = 0; k < kN; ++k) {
            if constexpr (DT == GG_DTYPE_F32) f[k] = __uint_as_float(w[k]);
            else if constexpr (DT == GG_DTYPE_F16) f[k] = f16_bits_to_f32((uint16_t)(w[k >> 1] >> (16 * (k & 1))));
            else if constexpr (DT == GG_DTYPE_BF16) f[k] = bf16_bits_to_f32((uint16_t)(w[k >> 1] >> (16 * (k & 1))));
            else if constexpr (DT == GG_DTYPE_FP8_E4M3) f[k] = fp8e4m3_to_f32((uint8_t)(w[k >> 2] >> (8 * (k & 3))));
            else f[k] = (float)(int8_t)(uint8_t)(w[k >> 2] >> (8 * (k & 3)));
        }
    }
};

template <gg_dtype_t DT, int DC>
__global__ void __launch_bounds__(64) attn_generic_kernel(AttnArgs a, KVView kv) {
    const int part = blockIdx.x;
    const int h = blockIdx.y;
    const int z = blockIdx.z;  // b*R + j
    const int b = z / a.rows, j = z % a.rows;
    const int nrows = seq_rows(a, b);
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

    // A tile of 64 keys per step: lane i scores key t0 + 64k + i against the whole query
    // (read from LDS), one wave max / sum per tile, then P.V with each lane owning dims
    // lane + 64c and the tile's probabilities broadcast from their lanes.
    __shared__ float s_q[64 * kMaxDC];
    __shared__ float s_p[64];        // the tile's probabilities (times the V scale)
    __shared__ size_t s_vrow[64];    // element offset of each key's V column 0
    float acc[DC];
    const size_t qbase = ((size_t)z * a.num_q_heads + h) * D;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
        const int d = lane + 64 * c;
        if (d < D) s_q[d] = load_as_f32(a.q, a.q_dtype, qbase + d);
        acc[c] = 0.f;
    }
    __syncthreads();
    const int32_t* bt = a.block_tables + (size_t)b * a.max_blocks;
    float m = -1e30f, l = 0.f;
    for (int tb = t0; tb < t1; tb += 64) {
        const int t = tb + lane;
        int blk = -1, off = 0;
        if (t < t1) {
            blk = bt[t / kv.bs];
            off = t % kv.bs;
            if (blk < 0 || blk >= kv.num_blocks) blk = -1;  // invalid table entry: key skipped
        }
        float sc = -INFINITY;
        if (blk >= 0) {
            // The lane's key row is contiguous: 16-byte loads when rows are whole
            // multiples of 16 bytes (pools are 256-byte aligned), else element loads.
            const uint8_t* krow = kv.kc + (kv.tile0(blk, kvh) + (size_t)off * D) * dtype_bytes(DT);
            float dot = 0.f;
            constexpr int kN = Pool16<DT>::kN;
            if (D % kN == 0) {
#pragma unroll 4
                for (int v = 0; v < D / kN; ++v) {
                    float f[kN];
                    Pool16<DT>::decode(((const uint4*)krow)[v], f);
#pragma unroll
                    for (int e = 0; e < kN; ++e) dot += s_q[v * kN + e] * f[e];
                }
            } else {
#pragma unroll 16
                for (int d = 0; d < D; ++d) dot += s_q[d] * pool_elem<DT>(krow, d);
            }
            sc = dot * a.scale * kv.k_scale(blk, kvh);
        }
        float mt = sc;
        for (int o = 32; o > 0; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o));
        const float m_new = fmaxf(m, mt);
        const float alpha = __expf(m - m_new);
        const float p = blk >= 0 ? __expf(sc - m_new) : 0.f;
        float ps = p;
        for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
        l = l * alpha + ps;
        m = m_new;
#pragma unroll
        for (int c = 0; c < DC; ++c) acc[c] *= alpha;
        // The tile's probabilities and V offsets go through LDS, so the key loop below
        // has no cross-lane operations and unrolls into batches of independent loads.
        // (Masked and skipped keys have p = 0 and read block 0.)
        __syncthreads();  // the previous tile's readers are done
        s_p[lane] = blk >= 0 ? p * kv.v_scale(blk, kvh) : 0.f;
        s_vrow[lane] = kv.tile0(max(blk, 0), kvh) + off;
        __syncthreads();
        const int ntile = min(64, t1 - tb);
        const uint8_t* vc = kv.vc;
#pragma unroll 16
        for (int i = 0; i < ntile; ++i) {
            const float pi = s_p[i];
            const size_t vr = s_vrow[i];
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const int d = lane + 64 * c;
                if (d < D) acc[c] += pi * pool_elem<DT>(vc, vr + (size_t)d * kv.bs);
            }
        }
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
    const int nrows = seq_rows(a, b);
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

// Standalone draft-KV append from the block tables: workgroup (item) = (b, kvh).
__global__ void __launch_bounds__(256) append_from_tables_kernel(AttnArgs a, KVView kv) {
    append_item_rows(a, kv, blockIdx.x / kv.Hkv, blockIdx.x % kv.Hkv);
}

}  // namespace

gg_status_t launch_append_from_tables(const AttnArgs& a, const KVView& kv, hipStream_t s) {
    append_from_tables_kernel<<<a.num_seqs * kv.Hkv, 256, 0, s>>>(a, kv);
    return check_hip(hipGetLastError(), "append launch");
}

AttnPlan attn_plan(const KV* kv, int num_seqs, int rows, int num_q_heads, int max_blocks,
                   int partition_tokens) {
    if (partition_tokens > 0) return {ATTN_SCHED_GRID, partition_tokens};
    if (!attn_mfma_supported(kv, rows, num_q_heads)) {
        // One wave per (row, head, partition): partitions of 64..512 keys, as many as
        // it takes to reach about 2048 waves (the kernel's time is the longest wave's
        // chain of 64-key tiles; the merge costs one small launch).
        const long long waves = (long long)num_seqs * rows * num_q_heads;
        const long long want = waves > 0 ? (2048 + waves - 1) / waves : 1;
        const long long keys = (long long)max_blocks * kv->block_size;
        long long part = (keys + want - 1) / want;
        part = (part + 63) / 64 * 64;
        part = part < 64 ? 64 : (part > 512 ? 512 : part);
        return {ATTN_SCHED_GRID, (int)part};
    }
    // Measured on MI355X: while the (sequence, kv head) items fill at least a quarter of
    // the resident workgroup slots, longest-first pieces (LPT: long items cut in equal
    // pieces, dispatched longest first, split items merged inside the launch) balance
    // ragged contexts best; beyond the sequences an LPT workgroup can rank, one workgroup
    // per item (no split, no merge) when the items fill the slots. Otherwise stream-K
    // splits evenly.
    const int G = num_q_heads / kv->num_kv_heads;
    const int nt = (G * rows + 15) / 16;
    const long long max_keys = (long long)max_blocks * kv->block_size;
    const long long items = (long long)num_seqs * kv->num_kv_heads;
    const long long slots = (long long)device_cu_count() * attn_occupancy((int)dtype_bytes(kv->dtype), nt);
    // (With a merge launch of its own, LPT lost to stream-K at a quarter of the slots,
    // config 4: 164 vs 117 µs. With the merge inside the launch and pieces of 4/3 of the
    // mean slot load it wins there: 110.3 vs 112.7 µs, same box. At an eighth of the slots
    // it loses: config 4 with two workgroups per CU, 120.2 vs 117.4 µs.)
    if (4 * items >= slots && num_seqs <= kLptMaxSeqs) return {ATTN_SCHED_LPT, 0};
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
    const bool mfma = a.sched != ATTN_SCHED_GRID || (attn_mfma_supported(kv, a.rows, a.num_q_heads) &&
                                                     a.partition % 64 == 0 && a.partition <= kMfmaMaxPartition);
    // Draft rows of the call: the MFMA kernels append them piece by piece (start_piece);
    // the generic path takes a launch of its own first.
    if (a.k_new && !mfma) {
        const gg_status_t st = launch_append_from_tables(a, view, s);
        if (st != GG_OK) return st;
    }
    if (mfma) {
        // Stream-K and LPT launch their own merge over their record layout.
        gg_status_t st = launch_attn_mfma(a, view, s);
        if (st != GG_OK) return st;
        if (a.sched != ATTN_SCHED_GRID) return check_hip(hipGetLastError(), "verify_attention launch");
    } else {
        // Dims per lane rounded up to 1, 2, 4, 8 or 16 (the excess lanes idle).
        const int dc = (kv->head_dim + 63) / 64;
        const int DC = dc <= 1 ? 1 : dc <= 2 ? 2 : dc <= 4 ? 4 : dc <= 8 ? 8 : 16;
        if (dc > kMaxDC) return fail(GG_ERR_INVALID, "attention: head_dim too large");
        dim3 grid(a.max_parts, a.num_q_heads, a.num_seqs * a.rows);
        auto launch = [&](auto dt_tag) {
            constexpr gg_dtype_t DT = decltype(dt_tag)::value;
            switch (DC) {
                case 1: attn_generic_kernel<DT, 1><<<grid, 64, 0, s>>>(a, view); break;
                case 2: attn_generic_kernel<DT, 2><<<grid, 64, 0, s>>>(a, view); break;
                case 4: attn_generic_kernel<DT, 4><<<grid, 64, 0, s>>>(a, view); break;
                case 8: attn_generic_kernel<DT, 8><<<grid, 64, 0, s>>>(a, view); break;
                default: attn_generic_kernel<DT, 16><<<grid, 64, 0, s>>>(a, view); break;
            }
        };
        switch (kv->dtype) {
            case GG_DTYPE_F32: launch(std::integral_constant<gg_dtype_t, GG_DTYPE_F32>{}); break;
            case GG_DTYPE_F16: launch(std::integral_constant<gg_dtype_t, GG_DTYPE_F16>{}); break;
            case GG_DTYPE_BF16: launch(std::integral_constant<gg_dtype_t, GG_DTYPE_BF16>{}); break;
            case GG_DTYPE_FP8_E4M3: launch(std::integral_constant<gg_dtype_t, GG_DTYPE_FP8_E4M3>{}); break;
            case GG_DTYPE_INT8: launch(std::integral_constant<gg_dtype_t, GG_DTYPE_INT8>{}); break;
            default: return fail(GG_ERR_INVALID, "attention: pool dtype");
        }
    }
    if (a.max_parts > 1) {
        attn_combine_kernel<<<dim3(a.num_q_heads, a.num_seqs * a.rows), 128, 0, s>>>(a, kv->head_dim);
    }
    static_assert(kMaxDC == 16, "generic kernel instantiations cover head_dim <= 1024");
    return check_hip(hipGetLastError(), "verify_attention launch");
}

}  // namespace gg
