// gg_common.h — shared definitions of the gfx950 verify-path library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/gg_verify.h"

#define GG_API extern "C" __attribute__((visibility("default")))

namespace gg {

// ---- error reporting (per calling thread, like gollmgo_backend_last_error) ----
void set_error(const std::string& msg);
void clear_error();
gg_status_t fail(gg_status_t st, const std::string& msg);
gg_status_t check_hip(hipError_t e, const char* what);

// ---- KV cache handle ----
struct KV {
    int num_layers = 0;
    int num_blocks = 0;
    int block_size = 0;
    int num_kv_heads = 0;
    int head_dim = 0;
    gg_dtype_t dtype = GG_DTYPE_BF16;
    gg_scale_mode_t scale_mode = GG_SCALE_NONE;
    int device = 0;
    size_t elem_bytes = 2;
    size_t layer_bytes = 0;       // bytes of one layer's K (or V) pool
    size_t tile_bytes = 0;        // one (block, head) tile of K (or V): block_size * head_dim elements
    size_t layer_stride = 0;      // bytes between layers (K and V interleaved: 2 * layer_bytes)
    size_t scale_layer_elems = 0; // scales per layer per pool
    uint8_t* k_pool = nullptr;    // [layers][blocks][heads][K tile, V tile]: the allocation
    uint8_t* v_pool = nullptr;    // k_pool + tile_bytes (inside that allocation)
    void* k_scales = nullptr;     // PER_HEAD: float[layers][Hkv]; PER_BLOCK: u16[layers][blocks][Hkv]
    void* v_scales = nullptr;
};

__host__ __device__ inline size_t dtype_bytes(gg_dtype_t t) {
    switch (t) {
        case GG_DTYPE_F32: return 4;
        case GG_DTYPE_F16: return 2;
        case GG_DTYPE_BF16: return 2;
        case GG_DTYPE_FP8_E4M3: return 1;
        case GG_DTYPE_INT8: return 1;
    }
    return 0;
}

__host__ __device__ inline bool is_float_io(gg_dtype_t t) {
    return t == GG_DTYPE_F32 || t == GG_DTYPE_F16 || t == GG_DTYPE_BF16;
}

// ---- launchers (defined in the .hip files) ----
size_t kv_swap_record_bytes(const KV* kv);  // one (block, layer) record of a KV snapshot
gg_status_t launch_kv_snapshot(KV* kv, const int32_t* ids, int n, void* staging, void* host_dst, hipStream_t s);
gg_status_t launch_kv_restore(KV* kv, const int32_t* ids, int n, void* staging, const void* host_src,
                              hipStream_t s);
gg_status_t launch_kv_append(KV* kv, int layer, const void* k, const void* v, gg_dtype_t src,
                             const int32_t* slots, int n_rows, hipStream_t s);

struct AttnArgs {
    const KV* kv;
    int layer;
    const void* q;
    gg_dtype_t q_dtype;
    void* out;
    gg_dtype_t out_dtype;
    const int32_t* ctx_lens;
    const int32_t* row_counts;
    const int32_t* block_tables;
    int max_blocks;
    int num_seqs;
    int rows;
    int num_q_heads;
    float scale;
    int kv_bs;         // block size of the pool
    int partition;     // resolved partition length (tokens)
    int max_parts;
    float* ws_ml;      // partition grid: [seqs][rows][Hq][max_parts][2]; stream-K: [records][G*R][2]
    float* ws_acc;     // partition grid: [seqs][rows][Hq][max_parts][D]; stream-K: [records][G*R][D]
    int sched;         // ATTN_SCHED_*: how the (sequence, kv head) items are cut
    int sk_grid;       // stream-K / LPT: resident workgroup slots (attn_streamk_grid)
    int* plan;         // LPT: piece plan in the workspace, after the records
    int plan_ready;    // LPT: the plan is already in the workspace (gg_verify_attention_plan)
    int sk_min_chunks;    // least chunks a stream-K workgroup takes
    // Draft-KV rows appended by the same call (gg_verify_append_attention_planned): row
    // b*rows + j (j < the sequence's row count) is key position ctx - row_count + j, its
    // slot taken from the block table. The MFMA kernels append each piece's rows before
    // reading them; the generic path runs a launch of its own first.
    const void* k_new;
    const void* v_new;
    gg_dtype_t new_dtype;
};
// Attention schedules on the MFMA path (the generic path always uses the grid).
enum { ATTN_SCHED_GRID = 0, ATTN_SCHED_STREAMK = 1, ATTN_SCHED_LPT = 2 };

// Stream-K and LPT: resident workgroup slots for a shape on the current device, and the
// workspace both need: grid + num_seqs * Hkv partial records of G*rows rows, as (max,
// sum) pairs, then (64-float aligned) P.V rows, then the LPT plan (ints). ml_elems and
// acc_elems receive the float counts of the first two parts.
int attn_streamk_grid(const KV* kv, int rows, int num_q_heads);
size_t attn_streamk_workspace_bytes(const KV* kv, int num_seqs, int rows, int num_q_heads,
                                    size_t* ml_elems, size_t* acc_elems);
int device_cu_count();
size_t attn_workspace_bytes(const KV* kv, int num_seqs, int rows, int num_q_heads,
                            int max_blocks, int partition);
gg_status_t launch_verify_attention(const AttnArgs& a, hipStream_t s);
gg_status_t launch_attn_plan(const AttnArgs& a, hipStream_t s);  // no-op unless LPT

size_t greedy_workspace_bytes(int num_seqs, int max_drafts, int vocab);
gg_status_t launch_accept_greedy(const void* logits, gg_dtype_t dt, int num_seqs, int max_drafts,
                                 int vocab, const int32_t* drafts, const int32_t* n_drafts,
                                 int32_t* out_acc, int32_t* out_tok, void* ws, hipStream_t s);

// The float64 token draw shared by the greedy-with-sampled-bonus and the rejection
// acceptance (accept_sample.hip): per sequence, a row drawn with Sampler.Sample's rule, or
// after a rejected draft the residual of that row's distribution against the draft's.
struct FinalDraw {
    const void* logits;          // [num_seqs][max_drafts + 1][vocab]
    gg_dtype_t dt;
    int num_seqs, max_drafts, vocab;
    double temperature;          // > 1e-9
    int top_k;
    double top_p;
    const double* uniforms_f64;  // uniform of sequence b: uniforms_f64[b], or
    const float* uniforms_f32;   //   uniforms_f32[b * (max_drafts + 1) + max_drafts]
    const float* draft_probs;    // residual draws: [num_seqs][max_drafts][vocab], or null (one-hot)
    // Which row: either greedy (row n_drafts[b] when accepted[b] == n_drafts[b], the row
    // maxima from the greedy segment pairs greedy_seg), or given (spec_row[b], -1 = none;
    // spec_x[b] the rejected draft of a residual draw, -1 = plain; the row maxima from
    // seg_max [rows][nseg_max], finite maxima of 8192-element segments).
    const int32_t* n_drafts;
    const int32_t* accepted;
    const float2* greedy_seg;
    const int* spec_row;
    const int* spec_x;
    const unsigned long long* spec_key;  // given rows, top-p: (order key << 32 | ~index) of an element
                                         // at or near the nucleus cut (0: none)
    const double* spec_s;                // given rows: an estimate of the drawn row's softmax sum
                                         // within 1e-4 relative (0: none; dense residuals)
    const float* seg_max;
    int nseg_max;
    bool force_exact;
    bool prepped;                        // the caller set every sequence's row up (fd::prep_row)
    int32_t* out_tok;
};
size_t final_draw_workspace_bytes(int num_seqs, int vocab);
gg_status_t launch_final_draw(const FinalDraw& d, void* ws, hipStream_t s);

size_t sample_workspace_bytes(int num_seqs, int max_drafts, int vocab);
gg_status_t launch_accept_greedy_sample(const void* logits, gg_dtype_t dt, int num_seqs, int max_drafts, int vocab,
                                        const int32_t* drafts, const int32_t* n_drafts, double temperature,
                                        int top_k, double top_p, const double* uniforms, unsigned flags,
                                        int32_t* out_acc, int32_t* out_tok, void* ws, hipStream_t s);

size_t rejection_workspace_bytes(int num_seqs, int max_drafts, int vocab);
gg_status_t launch_accept_rejection(const void* logits, gg_dtype_t dt, const float* q, int num_seqs,
                                    int max_drafts, int vocab, const int32_t* drafts,
                                    const int32_t* n_drafts, const float* uniforms, float temperature,
                                    float top_p, int32_t* out_acc, int32_t* out_tok, void* ws,
                                    hipStream_t s);

gg_status_t launch_ngram_draft(const int32_t* hist, int stride, const int32_t* hist_len, int num_seqs,
                               int n, int max_drafts, int32_t* out_drafts, int32_t* out_n,
                               hipStream_t s);
gg_status_t launch_history_append_draft(int32_t* hist, int stride, int32_t* hist_len, const int32_t* rows,
                                        int num_seqs, const int32_t* drafts, int k_in, const int32_t* accepted,
                                        const int32_t* token, int n, int max_drafts, int32_t* out_drafts,
                                        int32_t* out_n, hipStream_t s);

}  // namespace gg

// The opaque handle of the C ABI is the KV description itself.
struct gg_kv : public gg::KV {};

// ---- device helpers shared by the kernels ----
#ifdef __HIPCC__
namespace gg {

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load element i of a float-like array of type dt as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, gg_dtype_t dt, size_t i) {
    switch (dt) {
        case GG_DTYPE_F32: return ((const float*)p)[i];
        case GG_DTYPE_F16: return f16_bits_to_f32(((const uint16_t*)p)[i]);
        case GG_DTYPE_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
        default: return 0.f;
    }
}
__device__ __forceinline__ void store_from_f32(void* p, gg_dtype_t dt, size_t i, float v) {
    switch (dt) {
        case GG_DTYPE_F32: ((float*)p)[i] = v; break;
        case GG_DTYPE_F16: ((uint16_t*)p)[i] = f32_to_f16_bits(v); break;
        case GG_DTYPE_BF16: ((uint16_t*)p)[i] = f32_to_bf16_bits(v); break;
        default: break;
    }
}

// OCP FP8 E4M3 ("fn") decode: bias 7, no infinities, S.1111.111 = NaN.
__device__ __forceinline__ float fp8e4m3_to_f32(uint8_t b) {
    uint32_t s = (uint32_t)(b & 0x80) << 24;
    uint32_t e = (b >> 3) & 0xF;
    uint32_t m = b & 0x7;
    if ((b & 0x7F) == 0x7F) return __uint_as_float(0x7fc00000u | s);
    if (e == 0) {
        float v = (float)m * 0.001953125f;  // m * 2^-9
        return s ? -v : v;
    }
    return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// fp32 -> E4M3 with round-to-nearest-even and saturation to +-448 (the __NV_SATFINITE
// convention of kernels/gollmgo_model.cu:254), NaN -> 0x7F | sign. Two values at a time
// (bits 0-7: a, bits 8-15: b) through the gfx950 hardware conversion v_cvt_pk_fp8_f32
// (OCP E4M3, round to nearest even, subnormals kept): the inputs are first clamped to
// +-448, so the conversion never overflows, and NaN inputs are mapped afterwards.
__device__ __forceinline__ uint32_t f32x2_to_fp8e4m3_sat(float a, float b) {
    const float ca = __builtin_amdgcn_fmed3f(a, -448.f, 448.f);
    const float cb = __builtin_amdgcn_fmed3f(b, -448.f, 448.f);
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xffffu;
    if (__builtin_isnan(a)) w = (w & 0xff00u) | ((__float_as_uint(a) >> 24) & 0x80u) | 0x7Fu;
    if (__builtin_isnan(b)) w = (w & 0x00ffu) | (((__float_as_uint(b) >> 24) & 0x80u) << 8) | 0x7F00u;
    return w;
}

__device__ __forceinline__ uint8_t f32_to_fp8e4m3_sat(float f) { return (uint8_t)f32x2_to_fp8e4m3_sat(f, 0.f); }

// fp16 bits of f, round to nearest even (the PER_BLOCK INT8 scales are fp16).
__device__ __forceinline__ uint16_t f32_to_f16_rne_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Symmetric int8: round-half-even, clamp to +-127 (kernels/gollmgo_model.cu:258-268).
__device__ __forceinline__ int8_t f32_to_i8_sat(float f) {
    float r = __builtin_rintf(f);
    if (!(r == r)) r = 0.f;
    r = fminf(fmaxf(r, -127.f), 127.f);
    return (int8_t)(int)r;
}

}  // namespace gg
#endif
