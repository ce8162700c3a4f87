// attention_common.h — pool view and helpers shared by the attention kernels.
#pragma once
#include "gg_common.h"

namespace gg {

constexpr int kMfmaAutoPartition = 1024;
constexpr int kMfmaMaxPartition = 16384;  // longest explicit partition on the MFMA path
constexpr int kStreamKMinChunks = 16;     // least chunks per stream-K workgroup

// One layer of the paged pools, with dequantisation folded in.
struct KVView {
    const uint8_t* kc;
    const uint8_t* vc;
    const float* k_head_scale;     // PER_HEAD [Hkv]
    const float* v_head_scale;
    const uint16_t* k_blk_scale;   // PER_BLOCK fp16 [blocks][Hkv]
    const uint16_t* v_blk_scale;
    gg_dtype_t dt;
    int Hkv, D, bs;
    int num_blocks;  // block ids outside [0, num_blocks) read as empty

#ifdef __HIPCC__
    __device__ __forceinline__ float elem(const uint8_t* base, size_t i) const {
        switch (dt) {
            case GG_DTYPE_F32: return ((const float*)base)[i];
            case GG_DTYPE_F16: return f16_bits_to_f32(((const uint16_t*)base)[i]);
            case GG_DTYPE_BF16: return bf16_bits_to_f32(((const uint16_t*)base)[i]);
            case GG_DTYPE_FP8_E4M3: return fp8e4m3_to_f32(base[i]);
            case GG_DTYPE_INT8: return (float)((const int8_t*)base)[i];
        }
        return 0.f;
    }
    // Raw (unscaled) element of K[blk][h][off][d] and V[blk][h][d][off] (K and V tiles of a
    // (block, head) alternate: tiles of one pool are 2 * bs * D elements apart).
    __device__ __forceinline__ size_t tile0(int blk, int h) const { return ((size_t)blk * Hkv + h) * (2 * (size_t)bs * D); }
    __device__ __forceinline__ float k_at(int blk, int h, int off, int d) const {
        return elem(kc, tile0(blk, h) + (size_t)off * D + d);
    }
    __device__ __forceinline__ float v_at(int blk, int h, int off, int d) const {
        return elem(vc, tile0(blk, h) + (size_t)d * bs + off);
    }
    __device__ __forceinline__ float k_scale(int blk, int h) const {
        if (dt == GG_DTYPE_FP8_E4M3) return k_head_scale[h];
        if (dt == GG_DTYPE_INT8) return f16_bits_to_f32(k_blk_scale[(size_t)blk * Hkv + h]);
        return 1.f;
    }
    __device__ __forceinline__ float v_scale(int blk, int h) const {
        if (dt == GG_DTYPE_FP8_E4M3) return v_head_scale[h];
        if (dt == GG_DTYPE_INT8) return f16_bits_to_f32(v_blk_scale[(size_t)blk * Hkv + h]);
        return 1.f;
    }
#endif
};

inline KVView make_kv_view(const KV* kv, int layer) {
    KVView v{};
    v.kc = kv->k_pool + (size_t)layer * kv->layer_stride;
    v.vc = kv->v_pool + (size_t)layer * kv->layer_stride;
    if (kv->scale_mode == GG_SCALE_PER_HEAD) {
        v.k_head_scale = (const float*)kv->k_scales + (size_t)layer * kv->scale_layer_elems;
        v.v_head_scale = (const float*)kv->v_scales + (size_t)layer * kv->scale_layer_elems;
    } else if (kv->scale_mode == GG_SCALE_PER_BLOCK) {
        v.k_blk_scale = (const uint16_t*)kv->k_scales + (size_t)layer * kv->scale_layer_elems;
        v.v_blk_scale = (const uint16_t*)kv->v_scales + (size_t)layer * kv->scale_layer_elems;
    }
    v.dt = kv->dtype;
    v.Hkv = kv->num_kv_heads;
    v.D = kv->head_dim;
    v.bs = kv->block_size;
    v.num_blocks = kv->num_blocks;
    return v;
}

// Keys of sequence b, clamped to what its block-table row can address.
#ifdef __HIPCC__
__device__ __forceinline__ int seq_keys(const AttnArgs& a, int b, int bs) {
    int c = a.ctx_lens[b];
    const int cap = a.max_blocks * bs;
    return c < 0 ? 0 : (c > cap ? cap : c);
}
// Verify rows of sequence b: row_counts[b], or rows_per_seq when the array is NULL. A count
// above rows_per_seq gives no rows: nothing of the sequence is computed or written.
__device__ __forceinline__ int seq_rows(const AttnArgs& a, int b) {
    const int n = a.row_counts ? a.row_counts[b] : a.rows;
    return n > a.rows ? 0 : n;
}
#endif

inline bool attn_mfma_supported(const KV* kv, int rows, int num_q_heads) {
    const int G = num_q_heads / kv->num_kv_heads;
    return kv->head_dim == 128 && kv->block_size == 16 && G * rows <= 64 &&
           (kv->dtype == GG_DTYPE_BF16 || kv->dtype == GG_DTYPE_F16 ||
            kv->dtype == GG_DTYPE_FP8_E4M3 || kv->dtype == GG_DTYPE_INT8);
}

// MFMA kernel workgroups (of four waves) per CU for a pool's element size and row-tile
// count: two while one wave's registers fit half the file (one or two row tiles; three
// row tiles of a 1-byte pool in 32-token chunks, 217-248 VGPRs), else one. Shared by the
// launch bounds, the stream-K grid (one resident wave of workgroups) and the schedule
// choice.
__host__ __device__ constexpr int attn_occupancy(int elem_bytes, int nt) {
    return nt <= 2 || (elem_bytes == 1 && nt == 3) ? 2 : 1;
}

// Tokens per MFMA chunk for a pool's element size and row-tile count. At one or two row
// tiles a lane moves 256 B of K and V per chunk: 64 tokens of a 1-byte pool, 32 of a
// 2-byte one. From three row tiles on, 1-byte pools take 32-token chunks as well, which
// halves the chunk's K/V, score and P registers next to the three or four O tiles.
__host__ __device__ constexpr int attn_chunk_tokens(int elem_bytes, int nt) {
    return elem_bytes == 1 && nt <= 2 ? 64 : 32;
}

// How one verify_attention call is scheduled.
struct AttnPlan {
    int sched;      // ATTN_SCHED_*
    int partition;  // ATTN_SCHED_GRID: tokens per workgroup
};

// LPT schedule: most sequences the plan kernel ranks (one per thread).
constexpr int kLptMaxSeqs = 1024;
// LPT piece length: T = ceil(C * num / (slots * den)) chunks for C chunks of work over
// `slots` resident workgroups, num/den = 2 of the mean slot load when the (sequence, kv
// head) items fill the slots and 7/5 when they are fewer.
//   - Items that fill the slots are cut into pieces of T chunks and a shorter last piece,
//     which the longest-first order then runs at the end. Measured on MI355X (the call with
//     its append, one layer, mean over eight seeded config-3 layouts, same box): equal
//     pieces at 8/5 (the earlier rule) 127.1 µs; T pieces and a remainder at 8/5 / 9/5 / 2:
//     124.1 / 123.9 / 123.3 (bench layout 123.7 -> 118.5 at 9/5 and 2); at 7/5, 6/5 and 1
//     slower than equal pieces on the bench layout (123.7, 129.2, 132.7). With equal
//     pieces the factors had measured 3/2 / 8/5 / 13/8 / 5/3 / 17/10: 131.0 / 128.4 /
//     129.1 / 130.3 / 130.8 over eight layouts (an older build).
//   - Fewer items than slots: every long item has to be cut to fill the slots, and equal
//     pieces balance them (config 2 with remainder pieces: 71 -> 79 µs). Mean over eight
//     seeded config-2 layouts (items = slots / 2), f = 6/5 / 5/4 / 11/8 / 4/3 / 10/7 / 7/5
//     / 13/9 / 3/2: 69.9 / 67.9 / 61.5 / 63.1 / 61.4 / 60.7 / 61.4 / 62.8 µs (bench layout:
//     7/5 70.4, 4/3 70.8).
//   - Config 5 (items = 2 slots) cuts nothing at any of these factors.
// The factors are tuned constants; the time moves in steps as items cross piece
// boundaries.
constexpr int kLptPieceNum = 2, kLptPieceDen = 1;            // items >= slots
constexpr int kLptPieceNumFew = 7, kLptPieceDenFew = 5;      // items < slots
__host__ __device__ constexpr bool lpt_few_items(int slots, int num_seqs, int num_kv_heads) {
    return num_seqs * num_kv_heads < slots;
}
// Bound on the number of LPT pieces (= main-grid workgroups and partial records): the
// cuts of every item at T chunks give at most C/T + items pieces, C/T <= slots * den / num
// (the smaller factor, 7/5, gives the larger bound). (Stream-K needs grid + items records,
// which is more: the workspace holds the larger of the two.)
__host__ __device__ constexpr int lpt_records(int slots, int num_seqs, int num_kv_heads) {
    return (slots * kLptPieceDenFew + kLptPieceNumFew - 1) / kLptPieceNumFew + num_seqs * num_kv_heads;
}
AttnPlan attn_plan(const KV* kv, int num_seqs, int rows, int num_q_heads, int max_blocks,
                   int partition_tokens);

gg_status_t launch_attn_mfma(const AttnArgs& a, const KVView& kv, hipStream_t s);
gg_status_t launch_append_from_tables(const AttnArgs& a, const KVView& kv, hipStream_t s);

#ifdef __HIPCC__
// The draft-KV rows of item (b, kvh): row b*rows + j, j < the sequence's row count, goes to
// key position ctx - row_count + j, ctx as the attention clamps it to the table row (slot
// from the block table; entries outside the pool are skipped). Same conversions as
// gg_kv_append: rounding to the pool type, FP8 as E4M3-satfinite of x * (1 / per-head
// scale). Not for PER_BLOCK INT8 pools; head_dim a multiple of 8 and 16-byte aligned rows
// (checked by the entry point).
//
// Work item i of rows [j0, j1) is row j0 + i / (D/8), dims [8*(i % (D/8)), +8): K is one
// contiguous run of the row, V eight columns of the dim-major tile. Split in two so that a
// caller can issue the loads early and store later: append_load (block id, source words,
// scales) and append_store (conversion and stores).
struct AppendItem {
    uint4 k[2], v[2];  // source words: f32 sources fill both, 16-bit sources k[0] / v[0]
    size_t ki, vi;     // destination element indices in the K and V pools
    float kinv, vinv;  // FP8: 1 / per-head scale
    bool live;
};
__device__ __forceinline__ AppendItem append_load(const AttnArgs& a, const KVView& kv, int b, int kvh, int ctx,
                                                  int nrows, int j0, int i) {
    AppendItem it;
    const int D = kv.D, bs = kv.bs, groups = D / 8;
    const int j = j0 + i / groups, d0 = (i % groups) * 8;
    const int pos = ctx - nrows + j;
    const int blk = a.block_tables[(size_t)b * a.max_blocks + pos / bs];
    it.live = blk >= 0 && blk < kv.num_blocks;
    const int off = pos % bs;
    const int bsafe = it.live ? blk : 0;
    it.ki = kv.tile0(bsafe, kvh) + (size_t)off * D + d0;
    it.vi = kv.tile0(bsafe, kvh) + (size_t)d0 * bs + off;
    it.kinv = kv.dt == GG_DTYPE_FP8_E4M3 ? kv.k_head_scale[kv.Hkv + kvh] : 1.f;
    it.vinv = kv.dt == GG_DTYPE_FP8_E4M3 ? kv.v_head_scale[kv.Hkv + kvh] : 1.f;
    const size_t src = (((size_t)b * a.rows + j) * kv.Hkv + kvh) * D + d0;
    if (dtype_bytes(a.new_dtype) == 4) {
        const uint4* kp = (const uint4*)((const float*)a.k_new + src);
        const uint4* vp = (const uint4*)((const float*)a.v_new + src);
        it.k[0] = kp[0]; it.k[1] = kp[1]; it.v[0] = vp[0]; it.v[1] = vp[1];
    } else {
        it.k[0] = *(const uint4*)((const uint16_t*)a.k_new + src);
        it.v[0] = *(const uint4*)((const uint16_t*)a.v_new + src);
        it.k[1] = it.v[1] = make_uint4(0, 0, 0, 0);
    }
    return it;
}
// A work item in the pool's format, ready to store: K as one run of 8 elements, V as 8
// columns (element e at column e). FP8 pools use the low 8 bytes of k[0] and v[0], 16-bit
// pools k[0] and v[0], f32 pools both words.
struct AppendBytes {
    uint4 k[2], v[2];
    size_t ki, vi;  // destination element indices; ki == ~0: nothing to store
};
__device__ __forceinline__ AppendBytes append_encode(const AttnArgs& a, const KVView& kv, const AppendItem& it) {
    AppendBytes o;
    o.ki = it.live ? it.ki : ~(size_t)0;
    o.vi = it.vi;
    float kx[8], vx[8];
    if (dtype_bytes(a.new_dtype) == 4) {
        const uint32_t ku[8] = {it.k[0].x, it.k[0].y, it.k[0].z, it.k[0].w, it.k[1].x, it.k[1].y, it.k[1].z, it.k[1].w};
        const uint32_t vu[8] = {it.v[0].x, it.v[0].y, it.v[0].z, it.v[0].w, it.v[1].x, it.v[1].y, it.v[1].z, it.v[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            kx[e] = __uint_as_float(ku[e]);
            vx[e] = __uint_as_float(vu[e]);
        }
    } else {
        const uint32_t ku[4] = {it.k[0].x, it.k[0].y, it.k[0].z, it.k[0].w};
        const uint32_t vu[4] = {it.v[0].x, it.v[0].y, it.v[0].z, it.v[0].w};
        const bool bf = a.new_dtype == GG_DTYPE_BF16;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t kh = (uint16_t)(ku[e >> 1] >> (16 * (e & 1)));
            const uint16_t vh = (uint16_t)(vu[e >> 1] >> (16 * (e & 1)));
            kx[e] = bf ? bf16_bits_to_f32(kh) : f16_bits_to_f32(kh);
            vx[e] = bf ? bf16_bits_to_f32(vh) : f16_bits_to_f32(vh);
        }
    }
    o.k[1] = o.v[1] = make_uint4(0, 0, 0, 0);
    if (kv.dt == GG_DTYPE_FP8_E4M3) {
        uint32_t w[2], u[2];
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            w[e >> 2] = f32x2_to_fp8e4m3_sat(kx[e] * it.kinv, kx[e + 1] * it.kinv) |
                        (f32x2_to_fp8e4m3_sat(kx[e + 2] * it.kinv, kx[e + 3] * it.kinv) << 16);
            u[e >> 2] = f32x2_to_fp8e4m3_sat(vx[e] * it.vinv, vx[e + 1] * it.vinv) |
                        (f32x2_to_fp8e4m3_sat(vx[e + 2] * it.vinv, vx[e + 3] * it.vinv) << 16);
        }
        o.k[0] = make_uint4(w[0], w[1], 0, 0);
        o.v[0] = make_uint4(u[0], u[1], 0, 0);
    } else if (kv.dt == GG_DTYPE_F32) {
        o.k[0] = make_uint4(__float_as_uint(kx[0]), __float_as_uint(kx[1]), __float_as_uint(kx[2]), __float_as_uint(kx[3]));
        o.k[1] = make_uint4(__float_as_uint(kx[4]), __float_as_uint(kx[5]), __float_as_uint(kx[6]), __float_as_uint(kx[7]));
        o.v[0] = make_uint4(__float_as_uint(vx[0]), __float_as_uint(vx[1]), __float_as_uint(vx[2]), __float_as_uint(vx[3]));
        o.v[1] = make_uint4(__float_as_uint(vx[4]), __float_as_uint(vx[5]), __float_as_uint(vx[6]), __float_as_uint(vx[7]));
    } else {
        uint32_t w[4], u[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const bool bf = kv.dt == GG_DTYPE_BF16;
            w[e >> 1] = (uint32_t)(bf ? f32_to_bf16_bits(kx[e]) : f32_to_f16_bits(kx[e])) |
                        ((uint32_t)(bf ? f32_to_bf16_bits(kx[e + 1]) : f32_to_f16_bits(kx[e + 1])) << 16);
            u[e >> 1] = (uint32_t)(bf ? f32_to_bf16_bits(vx[e]) : f32_to_f16_bits(vx[e])) |
                        ((uint32_t)(bf ? f32_to_bf16_bits(vx[e + 1]) : f32_to_f16_bits(vx[e + 1])) << 16);
        }
        o.k[0] = make_uint4(w[0], w[1], w[2], w[3]);
        o.v[0] = make_uint4(u[0], u[1], u[2], u[3]);
    }
    return o;
}
__device__ __forceinline__ void append_write(const KVView& kv, const AppendBytes& o) {
    if (o.ki == ~(size_t)0) return;
    const int bs = kv.bs;
    uint8_t* kc = const_cast<uint8_t*>(kv.kc);
    uint8_t* vc = const_cast<uint8_t*>(kv.vc);
    if (kv.dt == GG_DTYPE_FP8_E4M3) {
        *(uint2*)(kc + o.ki) = make_uint2(o.k[0].x, o.k[0].y);
        const uint32_t u[2] = {o.v[0].x, o.v[0].y};
#pragma unroll
        for (int e = 0; e < 8; ++e) vc[o.vi + (size_t)e * bs] = (uint8_t)(u[e >> 2] >> (8 * (e & 3)));
    } else if (kv.dt == GG_DTYPE_F32) {
        *(uint4*)((float*)kc + o.ki) = o.k[0];
        *(uint4*)((float*)kc + o.ki + 4) = o.k[1];
        const uint32_t u[8] = {o.v[0].x, o.v[0].y, o.v[0].z, o.v[0].w, o.v[1].x, o.v[1].y, o.v[1].z, o.v[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) ((uint32_t*)vc)[o.vi + (size_t)e * bs] = u[e];
    } else {
        *(uint4*)((uint16_t*)kc + o.ki) = o.k[0];
        const uint32_t u[4] = {o.v[0].x, o.v[0].y, o.v[0].z, o.v[0].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) ((uint16_t*)vc)[o.vi + (size_t)e * bs] = (uint16_t)(u[e >> 1] >> (16 * (e & 1)));
    }
}
// The K run of a work item only.
__device__ __forceinline__ void append_write_k(const KVView& kv, const AppendBytes& o) {
    if (o.ki == ~(size_t)0) return;
    uint8_t* kc = const_cast<uint8_t*>(kv.kc);
    if (kv.dt == GG_DTYPE_FP8_E4M3) {
        *(uint2*)(kc + o.ki) = make_uint2(o.k[0].x, o.k[0].y);
    } else if (kv.dt == GG_DTYPE_F32) {
        *(uint4*)((float*)kc + o.ki) = o.k[0];
        *(uint4*)((float*)kc + o.ki + 4) = o.k[1];
    } else {
        *(uint4*)((uint16_t*)kc + o.ki) = o.k[0];
    }
}
__device__ __forceinline__ void append_store(const AttnArgs& a, const KVView& kv, const AppendItem& it) {
    if (it.live) append_write(kv, append_encode(a, kv, it));
}
// PER_BLOCK INT8: rows [jr0, jr1) of item (b, kvh), all landing in one block, by a whole
// workgroup, with gg_kv_append's rule for a run of rows in one block (append_int8_block in
// kv_append.hip): the amax of the rows' K and V over rows and dims, the block's new scale
// max(old, fp16(amax / 127)) (old = 0 when the rows start the block), the rows quantised
// with it, the rows already in the block re-quantised when the scale grew, the scale
// published. A block outside the pool is skipped.
__device__ __forceinline__ void append_int8_run(const AttnArgs& a, const KVView& kv, int b, int kvh, int ctx,
                                                int nrows, int jr0, int jr1) {
    __shared__ float s_red[2][16];
    const int D = kv.D, bs = kv.bs;
    const int pos0 = ctx - nrows + jr0;
    const int blk = a.block_tables[(size_t)b * a.max_blocks + pos0 / bs];
    if (blk < 0 || blk >= kv.num_blocks) return;  // (uniform)
    const int lead_off = pos0 % bs;
    const int nel = (jr1 - jr0) * D;
    auto src_at = [&](int i) { return (((size_t)b * a.rows + jr0 + i / D) * kv.Hkv + kvh) * D + i % D; };
    float mk = 0.f, mv = 0.f;
    for (int i = threadIdx.x; i < nel; i += blockDim.x) {
        const float kx = fabsf(load_as_f32(a.k_new, a.new_dtype, src_at(i)));
        const float vx = fabsf(load_as_f32(a.v_new, a.new_dtype, src_at(i)));
        mk = fmaxf(mk, kx == kx ? kx : 0.f);
        mv = fmaxf(mv, vx == vx ? vx : 0.f);
    }
    for (int o = 32; o > 0; o >>= 1) {
        mk = fmaxf(mk, __shfl_xor(mk, o));
        mv = fmaxf(mv, __shfl_xor(mv, o));
    }
    if ((threadIdx.x & 63) == 0) {
        s_red[0][threadIdx.x >> 6] = mk;
        s_red[1][threadIdx.x >> 6] = mv;
    }
    __syncthreads();
    mk = mv = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
        mk = fmaxf(mk, s_red[0][w]);
        mv = fmaxf(mv, s_red[1][w]);
    }
    __syncthreads();  // (s_red is reused by the next run)
    mk = fminf(mk, 3.0e38f);
    mv = fminf(mv, 3.0e38f);
    uint16_t* ksc = const_cast<uint16_t*>(kv.k_blk_scale);
    uint16_t* vsc = const_cast<uint16_t*>(kv.v_blk_scale);
    const size_t si = (size_t)blk * kv.Hkv + kvh;
    const float k_old = lead_off == 0 ? 0.f : f16_bits_to_f32(ksc[si]);
    const float v_old = lead_off == 0 ? 0.f : f16_bits_to_f32(vsc[si]);
    const float k_new = fmaxf(k_old, f16_bits_to_f32(f32_to_f16_rne_bits(mk / 127.0f)));
    const float v_new = fmaxf(v_old, f16_bits_to_f32(f32_to_f16_rne_bits(mv / 127.0f)));
    const float k_inv = k_new > 0.f ? 1.0f / k_new : 0.f;
    const float v_inv = v_new > 0.f ? 1.0f / v_new : 0.f;
    int8_t* kc = (int8_t*)const_cast<uint8_t*>(kv.kc);
    int8_t* vc = (int8_t*)const_cast<uint8_t*>(kv.vc);
    const size_t t0 = kv.tile0(blk, kvh);
    for (int i = threadIdx.x; i < nel; i += blockDim.x) {
        const int off = lead_off + i / D, d = i % D;
        kc[t0 + (size_t)off * D + d] = f32_to_i8_sat(load_as_f32(a.k_new, a.new_dtype, src_at(i)) * k_inv);
        vc[t0 + (size_t)d * bs + off] = f32_to_i8_sat(load_as_f32(a.v_new, a.new_dtype, src_at(i)) * v_inv);
    }
    if (lead_off > 0 && (k_new != k_old || v_new != v_old)) {  // rows already in the block
        for (int i = threadIdx.x; i < lead_off * D; i += blockDim.x) {
            const int t = i / D, d = i % D;
            if (k_new != k_old) {
                const size_t ki = t0 + (size_t)t * D + d;
                kc[ki] = f32_to_i8_sat(((float)kc[ki] * k_old) * k_inv);
            }
            if (v_new != v_old) {
                const size_t vi = t0 + (size_t)d * bs + t;
                vc[vi] = f32_to_i8_sat(((float)vc[vi] * v_old) * v_inv);
            }
        }
    }
    if (threadIdx.x == 0) {
        ksc[si] = f32_to_f16_rne_bits(k_new);
        vsc[si] = f32_to_f16_rne_bits(v_new);
    }
}

// Rows [j0, j1) of item (b, kvh) (clamped to the sequence's rows), by a whole workgroup,
// before anything reads them. PER_BLOCK INT8 pools go block by block (append_int8_run).
__device__ __forceinline__ void append_item_rows(const AttnArgs& a, const KVView& kv, int b, int kvh, int j0 = 0,
                                                 int j1 = 1 << 30) {
    const int ctx = seq_keys(a, b, kv.bs);
    const int nrows = seq_rows(a, b);
    if (ctx <= 0 || nrows <= 0 || nrows > ctx) return;
    j0 = j0 < 0 ? 0 : j0;
    j1 = j1 > nrows ? nrows : j1;
    if (kv.dt == GG_DTYPE_INT8) {
        for (int j = j0; j < j1;) {
            const int pos = ctx - nrows + j;
            const int je = min(j1, j + (kv.bs - pos % kv.bs));  // the rows in pos's block
            append_int8_run(a, kv, b, kvh, ctx, nrows, j, je);
            j = je;
        }
        return;
    }
    for (int i = threadIdx.x; i < (j1 - j0) * (kv.D / 8); i += blockDim.x)
        append_store(a, kv, append_load(a, kv, b, kvh, ctx, nrows, j0, i));
}
#endif

}  // namespace gg
