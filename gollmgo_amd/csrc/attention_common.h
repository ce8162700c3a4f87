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
    // Raw (unscaled) element of K[blk][h][off][d] and V[blk][h][d][off].
    __device__ __forceinline__ float k_at(int blk, int h, int off, int d) const {
        return elem(kc, (((size_t)blk * Hkv + h) * bs + off) * D + d);
    }
    __device__ __forceinline__ float v_at(int blk, int h, int off, int d) const {
        return elem(vc, (((size_t)blk * Hkv + h) * D + d) * bs + off);
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
    v.kc = kv->k_pool + (size_t)layer * kv->layer_bytes;
    v.vc = kv->v_pool + (size_t)layer * kv->layer_bytes;
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
#endif

inline bool attn_mfma_supported(const KV* kv, int rows, int num_q_heads) {
    const int G = num_q_heads / kv->num_kv_heads;
    return kv->head_dim == 128 && kv->block_size == 16 && G * rows <= 64 &&
           (kv->dtype == GG_DTYPE_BF16 || kv->dtype == GG_DTYPE_F16 ||
            kv->dtype == GG_DTYPE_FP8_E4M3 || kv->dtype == GG_DTYPE_INT8);
}

// MFMA kernel workgroups (of four waves) per CU for a row-tile count: two while one
// wave's registers fit half the file, else one. Shared by the launch bounds, the stream-K
// grid (one resident wave of workgroups) and the schedule choice.
__host__ __device__ constexpr int attn_occupancy(int nt) { return nt <= 2 ? 2 : 1; }

// How one verify_attention call is scheduled.
struct AttnPlan {
    int sched;      // ATTN_SCHED_*
    int partition;  // ATTN_SCHED_GRID: tokens per workgroup
};

// LPT schedule: most sequences the plan kernel ranks (one per thread).
constexpr int kLptMaxSeqs = 1024;
// LPT piece length: at most T = ceil(C * kLptPieceNum / (slots * kLptPieceDen)) chunks
// for C chunks of work over `slots` resident workgroups.
constexpr int kLptPieceNum = 1;
constexpr int kLptPieceDen = 1;
// Bound on the number of LPT pieces (= main-grid workgroups and partial records): the
// cuts of every item at T chunks give at most C/T + items pieces.
__host__ __device__ constexpr int lpt_records(int slots, int num_seqs, int num_kv_heads) {
    return (slots * kLptPieceDen + kLptPieceNum - 1) / kLptPieceNum + num_seqs * num_kv_heads;
}
AttnPlan attn_plan(const KV* kv, int num_seqs, int rows, int num_q_heads, int max_blocks,
                   int partition_tokens);

gg_status_t launch_attn_mfma(const AttnArgs& a, const KVView& kv, hipStream_t s);

}  // namespace gg
