/*
 * gg_verify.h — C ABI of the MI355X (gfx950) speculative-decoding verify path.
 *
 * This is the drop-in boundary a cgo `internal/backend/rocm` runner binds to.
 * It keeps the conventions of the reference's C ABI:
 *   - status codes mirror gollmgo_status_t (kernels/gollmgo_backend.h:21-27);
 *   - a human-readable last-error string mirrors gollmgo_backend_last_error
 *     (kernels/gollmgo_backend.h:43-44, backend.cu:20-31), kept per calling thread;
 *   - opaque handles (gollmgo_kvcache_t, kernels/gollmgo_kvcache.h:16);
 *   - NULL/invalid arguments return GG_ERR_INVALID, never abort; destroy(NULL) is OK.
 *
 * Differences from the reference, on purpose:
 *   - every compute entry point takes DEVICE pointers and a hipStream_t (passed as
 *     void*; NULL = the null stream) and is asynchronous. The reference copies host
 *     buffers and synchronises on every call (gollmgo_kvcache.cu:65-159).
 *   - no entry point allocates device memory. Scratch comes in as a caller-owned
 *     workspace whose size is returned by the matching *_workspace_size() call.
 *   - handles are not thread-safe: one engine thread drives one handle, as the
 *     reference's single engine goroutine does (internal/engine/serving.go:160).
 *
 * KV layout in HBM (per layer), chosen for 16-byte loads:
 *   K tile of (block, head): [block_size][head_dim]   (token-major)
 *   V tile of (block, head): [head_dim][block_size]   (dim-major)
 *   layer: [num_blocks][num_kv_heads][K tile, V tile] — the two tiles of a (block,
 *   head) are adjacent, so one item's block is one contiguous run. Logically the K pool
 *   is K[num_blocks][num_kv_heads][block_size][head_dim] with consecutive tiles
 *   2 * tile bytes apart (tile = block_size * head_dim * element bytes), likewise V.
 * A reference slot index (internal/kvcache/block_table.go:39) still addresses a
 * token: slot = physical_block * block_size + offset.
 */
#ifndef GG_VERIFY_H
#define GG_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors gollmgo_status_t (kernels/gollmgo_backend.h:21-27). */
typedef enum {
    GG_OK = 0,
    GG_ERR_HIP = 1,      /* GOLLMGO_ERR_CUDA */
    GG_ERR_OOM = 2,
    GG_ERR_INVALID = 3,
    GG_ERR_INTERNAL = 4,
} gg_status_t;

/* Element types. FP8 is OCP E4M3 ("e4m3fn": no inf, NaN = S.1111.111). */
typedef enum {
    GG_DTYPE_F32 = 0,
    GG_DTYPE_F16 = 1,
    GG_DTYPE_BF16 = 2,
    GG_DTYPE_FP8_E4M3 = 3,
    GG_DTYPE_INT8 = 4,
} gg_dtype_t;

/* How a quantised KV pool is scaled (dequant: x = q * scale).
 *   PER_HEAD : one fp32 scale per (layer, kv head) for K and one for V, set by
 *              gg_kv_set_head_scales (the reference's amax/448 convention,
 *              kernels/gollmgo_model.cu:415-427, applied per head).
 *   PER_BLOCK: one fp16 scale per (layer, block, kv head) for K and for V,
 *              maintained by gg_kv_append as the running amax/127 of the block
 *              (int8 convention of kernels/gollmgo_model.cu:430-441). */
typedef enum {
    GG_SCALE_NONE = 0,
    GG_SCALE_PER_HEAD = 1,
    GG_SCALE_PER_BLOCK = 2,
} gg_scale_mode_t;

typedef struct gg_kv* gg_kv_t;

/* Last error message of the calling thread ("" if none). */
const char* gg_last_error(void);

/* Library version string and the gfx target it was built for. */
const char* gg_version(void);

/* Select the HIP device used by later calls on this thread.
 * Replaces gollmgo_backend_create's device selection (gollmgo_backend.h:30). */
gg_status_t gg_set_device(int device_id);

/* Block until all work queued on `stream` has finished. */
gg_status_t gg_sync(void* stream);

/* ---------------------------------------------------------------------------
 * Paged KV cache.
 * Replaces gollmgo_kvcache_create / _k_layer_ptr / _v_layer_ptr / _destroy
 * (kernels/gollmgo_kvcache.h:26-35,66). The reference takes num_slots and stores
 * 2-byte elements only (gollmgo_kvcache.cu:39-40); here the pool is sized in
 * blocks and the element type and scale mode are chosen at creation.
 * ------------------------------------------------------------------------- */
gg_status_t gg_kv_create(int num_layers, int num_blocks, int block_size,
                         int num_kv_heads, int head_dim, gg_dtype_t dtype,
                         gg_scale_mode_t scale_mode, gg_kv_t* out);
gg_status_t gg_kv_destroy(gg_kv_t kv);

/* Device pointers to one layer's first K tile and first V tile (NULL on bad
 * arguments); tiles of one pool follow every 2 * tile bytes. */
void* gg_kv_k_layer_ptr(gg_kv_t kv, int layer);
void* gg_kv_v_layer_ptr(gg_kv_t kv, int layer);
/* PER_HEAD: float[num_kv_heads]; PER_BLOCK: uint16 (fp16 bits)[num_blocks][num_kv_heads]. */
void* gg_kv_k_scale_ptr(gg_kv_t kv, int layer);
void* gg_kv_v_scale_ptr(gg_kv_t kv, int layer);
/* Bytes of one layer's K (or V) tiles (num_blocks * num_kv_heads * tile); a layer
 * occupies twice that. */
size_t gg_kv_layer_bytes(gg_kv_t kv);

/* KV swap (preemption with swap semantics). Replaces SnapshotKV / RestoreKV
 * (internal/backend/cuda/swap_bridge.go:53-153; interface internal/backend/runner.go:
 * 94-106). A snapshot of num_blocks blocks holds, for block i of block_ids (device
 * int32[num_blocks]) and every layer, that block's K and V tiles of all kv heads (plus
 * its fp16 K/V scales for PER_BLOCK pools), as gg_kv_snapshot_bytes(kv, num_blocks)
 * bytes ordered [block i][layer]; PER_HEAD scales stay with the pool.
 *   gg_kv_snapshot: gathers the blocks into `staging` (device, 16-byte aligned, at least
 *                   gg_kv_snapshot_bytes) and, if host_dst is not NULL, copies it there
 *                   (hipMemcpyAsync on `stream`: pinned host memory makes it truly
 *                   asynchronous). Ids outside the pool give zero records.
 *   gg_kv_restore:  the reverse: host_src (if not NULL) -> staging -> blocks block_ids
 *                   (any ids, e.g. freshly allocated ones; ids outside the pool are
 *                   skipped). The snapshot is not consumed.
 * Both are asynchronous on `stream`; call gg_sync before reusing host buffers. */
size_t gg_kv_snapshot_bytes(gg_kv_t kv, int num_blocks);
gg_status_t gg_kv_snapshot(gg_kv_t kv, const int32_t* block_ids, int num_blocks, void* staging,
                           size_t staging_bytes, void* host_dst, void* stream);
gg_status_t gg_kv_restore(gg_kv_t kv, const int32_t* block_ids, int num_blocks, void* staging,
                          size_t staging_bytes, const void* host_src, void* stream);

/* PER_HEAD only: upload host arrays k_scales[num_kv_heads], v_scales[num_kv_heads]
 * (synchronous). Scales must be finite and > 0. */
gg_status_t gg_kv_set_head_scales(gg_kv_t kv, int layer, const float* k_scales,
                                  const float* v_scales);

/* Draft-KV append: write n_rows new K/V rows of one layer into their slots,
 * quantising on write for FP8/INT8 pools.
 * Replaces gollmgo_kvcache_write (kernels/gollmgo_kvcache.h:41-45) and the
 * paged_kv_write_{f16,bf16} kernels (kernels/gollmgo_paged_attn.cu:14-35,126-146).
 *   k, v         : device [n_rows][num_kv_heads][head_dim] of src_dtype (F32/F16/BF16)
 *   slot_mapping : device int32[n_rows]; slot = block*block_size + offset; a
 *                  negative slot skips the row.
 * PER_BLOCK pools: rows that land in the same block in one call must be adjacent
 * in slot_mapping (skipped rows may sit between them) with increasing offsets (as
 * BlockTable.Append produces them,
 * internal/kvcache/block_table.go:24-42). Such a block's scale becomes
 * max(old scale, amax(new rows)/127) rounded to fp16; rows already in the block
 * are re-quantised to the new scale. Appends never target a block whose refcount
 * is above one (the kvcache package only shares full blocks). */
gg_status_t gg_kv_append(gg_kv_t kv, int layer, const void* k, const void* v,
                         gg_dtype_t src_dtype, const int32_t* slot_mapping,
                         int n_rows, void* stream);

/* ---------------------------------------------------------------------------
 * Multi-query paged attention over the k+1 verify rows (split-K "v2").
 * Replaces gollmgo_kvcache_attention (kernels/gollmgo_kvcache.h:55-63) and the
 * paged_attention_v1/v2 kernels (kernels/gollmgo_paged_attn.cu:38-119,234-384),
 * generalised from one query per sequence to rows_per_seq causal query rows.
 *   q           : device [num_seqs][rows_per_seq][num_q_heads][head_dim], q_dtype
 *                 F32/F16/BF16
 *   out         : device, same shape, out_dtype F32/F16/BF16
 *   ctx_lens    : device int32[num_seqs], keys in the cache for each sequence
 *                 INCLUDING its appended verify rows (Batch.SeqContextLens,
 *                 internal/backend/runner.go:43-44)
 *   row_counts  : device int32[num_seqs] or NULL (= rows_per_seq for all). Row j
 *                 of sequence b sits at position ctx_lens[b]-row_counts[b]+j and
 *                 attends to keys [0, that position] (causal rule of
 *                 naive_attention, kernels/gollmgo_ops.cu:178). Rows j >=
 *                 row_counts[b] are not written; a count above rows_per_seq
 *                 (or <= 0) writes nothing of that sequence.
 *   block_tables: device int32[num_seqs][max_blocks_per_seq] of physical blocks
 *   scale       : softmax scale (1/sqrt(head_dim) in the reference)
 *   partition_tokens: split-K partition length, a multiple of 64. 0 = automatic:
 *                 longest-first pieces (long items cut, split items merged in the
 *                 same launch) when the (sequence, kv head) items fill at least a
 *                 quarter of the device's workgroup slots; one workgroup per item
 *                 past 1024 sequences; else a stream-K split over a fixed grid
 *                 (results equal to textbook attention in every case).
 * workspace must hold gg_verify_attention_workspace_size(...) bytes (may be 0). */
size_t gg_verify_attention_workspace_size(gg_kv_t kv, int num_seqs, int rows_per_seq,
                                          int num_q_heads, int max_blocks_per_seq,
                                          int partition_tokens);
gg_status_t gg_verify_attention(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype,
                                void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                const int32_t* row_counts, const int32_t* block_tables,
                                int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                int num_q_heads, float scale, int partition_tokens,
                                void* workspace, size_t workspace_bytes, void* stream);

/* One verify step runs the same attention schedule for every layer: it depends only on
 * ctx_lens, row_counts and the shape, not on the layer. These two calls let a caller
 * compute that schedule once per step instead of once per layer. They have no
 * counterpart in the reference (whose attention is one serial loop per query,
 * kernels/gollmgo_paged_attn.cu:38-119).
 *   gg_verify_attention_plan   : computes the schedule of (ctx_lens, row_counts,
 *                                shape) into `workspace` (sized as for
 *                                gg_verify_attention with partition_tokens = 0).
 *   gg_verify_attention_planned: gg_verify_attention with partition_tokens = 0 that
 *                                uses the schedule already in `workspace`.
 * Contract: between the plan and a planned call, the contents of ctx_lens and
 * row_counts, the shape and the workspace must be unchanged (stream order suffices:
 * the plan is a kernel on `stream`). A stale plan gives wrong results. */
gg_status_t gg_verify_attention_plan(gg_kv_t kv, const int32_t* ctx_lens, const int32_t* row_counts,
                                     int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                     int num_q_heads, void* workspace, size_t workspace_bytes,
                                     void* stream);
gg_status_t gg_verify_attention_planned(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype,
                                        void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                        const int32_t* row_counts, const int32_t* block_tables,
                                        int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                        int num_q_heads, float scale, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* Draft-KV append and planned attention of one layer in one call. Replaces the
 * per-layer pair paged_kv_write + paged attention of run_layer
 * (kernels/gollmgo_model.cu:610-625 then :651-687) for the verify rows.
 *   k_new, v_new : device [num_seqs * rows_per_seq][Hkv][head_dim] of F32/F16/BF16; row
 *                  b*rows_per_seq + j (j < the sequence's row count) is written to key
 *                  position ctx_lens[b] - row_count + j through the block table (the slot
 *                  gg_kv_append would be given, block*bs + offset), with gg_kv_append's
 *                  conversions, before the attention reads it. Rows past the row count
 *                  are ignored.
 * Then as gg_verify_attention_planned. The result (pool contents and out) equals
 * gg_kv_append with those slots followed by gg_verify_attention_planned. No slot mapping
 * needs to be built, and on the MFMA path there is no extra launch: each attention
 * workgroup writes the rows of its own key range before it reads them (other shapes run
 * the append as a launch of its own first). PER_BLOCK INT8 pools follow gg_kv_append's
 * block rule: the workgroup that reads a block with new rows first re-scales the block
 * (new scale, the new rows, the old rows re-quantised when the scale grew). */
gg_status_t gg_verify_append_attention_planned(gg_kv_t kv, int layer, const void* k_new, const void* v_new,
                                               gg_dtype_t new_dtype, const void* q, gg_dtype_t q_dtype,
                                               void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                               const int32_t* row_counts, const int32_t* block_tables,
                                               int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                               int num_q_heads, float scale, void* workspace,
                                               size_t workspace_bytes, void* stream);

/* Attention without allocation. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same as gg_verify_attention with partition_tokens = 0 (the
 * automatic schedule; identical results), but its scratch is a fixed device array inside
 * the library, gg_verify_attention_noalloc_max_bytes() bytes (32 MiB) per GPU, held until
 * the process ends. Calls that would need more scratch than that
 * (gg_verify_attention_workspace_size(..., 0) above the limit) return GG_ERR_INVALID before
 * touching the device. The call allocates nothing. Every call on one GPU shares that
 * array: calls that overlap on one GPU (on different streams, or from several threads)
 * race and give wrong results; serialise them on one stream. */
size_t gg_verify_attention_noalloc_max_bytes(void);
gg_status_t gg_verify_attention_noalloc(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype,
                                        void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                        const int32_t* row_counts, const int32_t* block_tables,
                                        int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                        int num_q_heads, float scale, void* stream);

/* ---------------------------------------------------------------------------
 * Greedy acceptance.
 * Replaces Verify + argmax (internal/engine/speculative.go:68-84,
 * internal/engine/sampling.go:75-85) as driven by emitSpeculative
 * (internal/engine/serving.go:514-566) with a greedy sampler.
 *   logits   : device [num_seqs][max_drafts+1][vocab] of F32/F16/BF16; row j scores
 *              the token after position j (row 0 = current token).
 *   drafts   : device int32[num_seqs][max_drafts]
 *   n_drafts : device int32[num_seqs], each in [0, max_drafts]
 * Outputs per sequence: out_accepted = longest prefix j with argmax(row j) ==
 * drafts[j]; out_token = argmax(row out_accepted) (the corrected token, or the bonus
 * token when every draft was accepted). argmax returns the first index of the
 * maximum, skips NaN, and returns 0 when element 0 is NaN (sequential `>` scan).
 * workspace: gg_accept_greedy_workspace_size bytes. */
size_t gg_accept_greedy_workspace_size(int num_seqs, int max_drafts, int vocab);
gg_status_t gg_accept_greedy(const void* logits, gg_dtype_t logits_dtype, int num_seqs,
                             int max_drafts, int vocab, const int32_t* drafts,
                             const int32_t* n_drafts, int32_t* out_accepted,
                             int32_t* out_token, void* workspace, size_t workspace_bytes,
                             void* stream);

/* ---------------------------------------------------------------------------
 * Greedy acceptance with the reference's sampled bonus token.
 * Replaces emitSpeculative at temperature > 0 (internal/engine/serving.go:514-566): the
 * greedy Verify over the draft rows as gg_accept_greedy, and, when every draft is
 * accepted, the bonus token Sampler.Sample(row n) (internal/engine/sampling.go:40-72) with
 * the engine's SamplingParams (sampling.go:10-15) and the draw's uniform supplied:
 *   temperature : SamplingParams.Temperature; <= 1e-9 gives gg_accept_greedy's result
 *   top_k       : SamplingParams.TopK; active when 0 < top_k < vocab (topKFilter, :88-109)
 *   top_p       : SamplingParams.TopP; active when 0 < top_p < 1 (topPFilter, :139-173)
 *   uniforms    : device double[num_seqs], the value rng.Float64() gives the bonus draw of
 *                 sequence b (categoricalSample, :176-192); unused for other sequences
 *   flags       : 0, or GG_SAMPLE_EXACT to take every draw through the sequential path
 * The token is the one the float64 rule gives: scaled = float64(l) * (1/T), the top-k
 * filter, softmax (exp as fdlibm's method, the one Go's portable math.Exp uses), top-p
 * and the first index whose cumulative probability exceeds u, every sum in the rule's
 * order. Orders sort.Slice leaves open are fixed: value (or probability) descending, then
 * index ascending, NaN last. Parallel sums decide whenever they clear the rule's boundary by
 * more than their proven rounding bound; rows that do not (about 1 in 10^4, and rows holding
 * NaN or +inf) are replayed sequentially on the device, about 3 ms per row.
 * workspace: gg_accept_greedy_sample_workspace_size bytes. */
#define GG_SAMPLE_EXACT 1u
size_t gg_accept_greedy_sample_workspace_size(int num_seqs, int max_drafts, int vocab);
gg_status_t gg_accept_greedy_sample(const void* logits, gg_dtype_t logits_dtype, int num_seqs,
                                    int max_drafts, int vocab, const int32_t* drafts,
                                    const int32_t* n_drafts, double temperature, int top_k,
                                    double top_p, const double* uniforms, unsigned flags,
                                    int32_t* out_accepted, int32_t* out_token, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Rejection-sampling acceptance (speculative sampling, Leviathan et al. 2023,
 * Alg. 1) with the reference sampler's temperature and top-p rules
 * (internal/engine/sampling.go:40-72,112-192). Not present in the reference.
 *   target_logits: device [num_seqs][max_drafts+1][vocab], F32/F16/BF16
 *   draft_probs  : device float[num_seqs][max_drafts][vocab], or NULL for a
 *                  deterministic drafter (n-gram), i.e. q = one-hot(draft)
 *   uniforms     : device float[num_seqs][max_drafts+1] in [0,1): element j < n
 *                  decides draft j; element max_drafts drives the final draw
 *   temperature  : > 0 (<= 1e-9 falls back to gg_accept_greedy semantics, as
 *                  Sampler.Sample does at sampling.go:54-56)
 *   top_p        : (0,1) enables the nucleus filter; otherwise disabled
 * Probabilities are fixed-point: w_i = floor(exp_gg((l_i - max) * (1/T)) * 2^35)
 * with the library's own exp (identical on host and device), so every sum and
 * prefix sum is an exact integer and decisions are bit-reproducible. Nucleus
 * order is (logit desc, index asc). Draft j is accepted iff
 * u_j * q_j(x_j) * Zp < w(x_j) (doubles); on the first rejection the token is drawn
 * from max(0, w - floor(q*Zp)); if all drafts pass, the bonus is drawn from row n.
 * A draw picks the first index whose inclusive prefix sum exceeds floor(u*total).
 * workspace: gg_accept_rejection_workspace_size bytes. */
size_t gg_accept_rejection_workspace_size(int num_seqs, int max_drafts, int vocab);
gg_status_t gg_accept_rejection(const void* target_logits, gg_dtype_t logits_dtype,
                                const float* draft_probs, int num_seqs, int max_drafts,
                                int vocab, const int32_t* drafts, const int32_t* n_drafts,
                                const float* uniforms, float temperature, float top_p,
                                int32_t* out_accepted, int32_t* out_token, void* workspace,
                                size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * n-gram draft lookup on the device.
 * Replaces NGramDrafter.Draft (internal/engine/speculative.go:12-62): the table
 * maps each (n-1)-gram of the history to the token that followed its LATEST
 * occurrence; drafting chains up to max_drafts lookups of the running suffix.
 *   history  : device int32[num_seqs][hist_stride]
 *   hist_len : device int32[num_seqs]
 *   n        : n-gram size; values < 2 become 2 (NewNGramDrafter), must be <= 9
 *   max_drafts: values < 1 become 4 (NewNGramDrafter)
 *   out_drafts: device int32[num_seqs][max_drafts]; out_n: device int32[num_seqs] */
gg_status_t gg_ngram_draft(const int32_t* history, int hist_stride, const int32_t* hist_len,
                           int num_seqs, int n, int max_drafts, int32_t* out_drafts,
                           int32_t* out_n, void* stream);

/* ---------------------------------------------------------------------------
 * The step's emitted tokens appended to device-resident histories, then the next
 * drafts: one launch after the acceptance, so a runner can draft on the device
 * without copying histories. Replaces, on the device, the history update of
 * emitSpeculative (internal/engine/serving.go:541-566: accepted drafts, then the
 * corrected or bonus token) followed by maybeDraft's NGramDrafter.Draft over the
 * whole history (serving.go:608-620, speculative.go:24-62). Sequence b:
 *   row       = hist_rows ? hist_rows[b] : b (history row of the sequence)
 *               rows whose hist_len is >= 0 must be distinct within one call (two
 *               sequences on one such row race on its tokens and length); rows of
 *               length -1 may be shared, since they are only set to -1 again
 *   appends     drafts[b][0, accepted[b]) and then token[b] (if >= 0) at
 *               history[row][hist_len[row] ..]; hist_len[row] grows by that count
 *   then        out_drafts[b][0, out_n[b]) = gg_ngram_draft of the updated row
 * A row whose tokens would pass hist_stride (or whose length is negative) is left
 * unchanged with hist_len[row] = -1 and out_n[b] = 0: the caller reseeds it.
 *   history  : device int32[rows][hist_stride]; hist_len: device int32[rows]
 *   drafts   : device int32[num_seqs][drafts_per_seq] (the step's drafts)
 *   accepted, token: device int32[num_seqs] (gg_accept_greedy / gg_accept_rejection)
 *   n, max_drafts: as gg_ngram_draft */
gg_status_t gg_history_append_draft(int32_t* history, int hist_stride, int32_t* hist_len,
                                    const int32_t* hist_rows, int num_seqs, const int32_t* drafts,
                                    int drafts_per_seq, const int32_t* accepted, const int32_t* token,
                                    int n, int max_drafts, int32_t* out_drafts, int32_t* out_n,
                                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GG_VERIFY_H */
