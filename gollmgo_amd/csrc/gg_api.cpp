// gg_api.cpp — C ABI entry points (argument checking, handle management).
//
// Conventions mirror the reference C ABI (kernels/gollmgo_backend.h:21-27,
// kernels/gollmgo_backend.cu:20-31, kernels/gollmgo_kvcache.cu:23-63): status codes,
// a last-error string, NULL/invalid -> GG_ERR_INVALID, destroy(NULL) -> OK.
#include "gg_common.h"
#include "attention_common.h"

#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

namespace gg {

static thread_local std::string t_last_error;

void set_error(const std::string& msg) { t_last_error = msg; }
void clear_error() { t_last_error.clear(); }

gg_status_t fail(gg_status_t st, const std::string& msg) {
    set_error(msg);
    return st;
}

gg_status_t check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return GG_OK;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? GG_ERR_OOM : GG_ERR_HIP;
}

}  // namespace gg

using namespace gg;

#define GG_CHECK_ARG(cond, msg) \
    do {                        \
        if (!(cond)) return fail(GG_ERR_INVALID, msg); \
    } while (0)

GG_API const char* gg_last_error(void) { return t_last_error.c_str(); }

GG_API const char* gg_version(void) { return "gollmgo_amd verify-path 0.1 (gfx950)"; }

GG_API gg_status_t gg_set_device(int device_id) {
    clear_error();
    int n = 0;
    gg_status_t st = check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (st != GG_OK) return st;
    GG_CHECK_ARG(device_id >= 0 && device_id < n, "gg_set_device: device id out of range");
    return check_hip(hipSetDevice(device_id), "hipSetDevice");
}

GG_API gg_status_t gg_sync(void* stream) {
    clear_error();
    return check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

// ---------------------------------------------------------------- KV cache

GG_API gg_status_t gg_kv_create(int num_layers, int num_blocks, int block_size, int num_kv_heads,
                                int head_dim, gg_dtype_t dtype, gg_scale_mode_t scale_mode,
                                gg_kv_t* out) {
    clear_error();
    GG_CHECK_ARG(out != nullptr, "gg_kv_create: out is NULL");
    *out = nullptr;
    GG_CHECK_ARG(num_layers > 0 && num_blocks > 0 && block_size > 0 && num_kv_heads > 0 &&
                     head_dim > 0,
                 "gg_kv_create: sizes must be positive");
    GG_CHECK_ARG(head_dim <= 1024, "gg_kv_create: head_dim must be <= 1024");
    GG_CHECK_ARG(dtype_bytes(dtype) != 0, "gg_kv_create: unknown dtype");
    if (dtype == GG_DTYPE_FP8_E4M3) {
        GG_CHECK_ARG(scale_mode == GG_SCALE_PER_HEAD, "gg_kv_create: FP8 pools need GG_SCALE_PER_HEAD");
    } else if (dtype == GG_DTYPE_INT8) {
        GG_CHECK_ARG(scale_mode == GG_SCALE_PER_BLOCK, "gg_kv_create: INT8 pools need GG_SCALE_PER_BLOCK");
    } else {
        GG_CHECK_ARG(scale_mode == GG_SCALE_NONE, "gg_kv_create: float pools take GG_SCALE_NONE");
    }
    {
        // The code objects are gfx950 only, and the in-launch merge of split attention items
        // relies on gfx950's ordering of device-scope stores, waits and atomics (the stores
        // complete at the device's coherence point before the counter's add is issued), so
        // a pool is only created on a gfx950 device.
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
            return fail(GG_ERR_HIP, "gg_kv_create: no HIP device");
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            return fail(GG_ERR_INVALID, std::string("gg_kv_create: the library is built for gfx950, device is ") +
                                            prop.gcnArchName);
    }
    gg_kv* kv = new gg_kv();
    kv->num_layers = num_layers;
    kv->num_blocks = num_blocks;
    kv->block_size = block_size;
    kv->num_kv_heads = num_kv_heads;
    kv->head_dim = head_dim;
    kv->dtype = dtype;
    kv->scale_mode = scale_mode;
    kv->elem_bytes = dtype_bytes(dtype);
    kv->tile_bytes = (size_t)block_size * head_dim * kv->elem_bytes;
    kv->layer_bytes = (size_t)num_blocks * num_kv_heads * kv->tile_bytes;
    kv->layer_stride = 2 * kv->layer_bytes;
    (void)hipGetDevice(&kv->device);
    // One allocation: the K and V tiles of a (block, head) sit next to each other, so a
    // workgroup reading one item's block reads one contiguous run (a load-only probe of
    // the paged pattern gains ~4 %, the attention kernel ~0.5 %).
    gg_status_t st = check_hip(hipMalloc((void**)&kv->k_pool, kv->layer_stride * num_layers), "hipMalloc(KV pool)");
    if (st == GG_OK) kv->v_pool = kv->k_pool + kv->tile_bytes;
    if (st == GG_OK && scale_mode == GG_SCALE_PER_HEAD) {
        kv->scale_layer_elems = (size_t)2 * num_kv_heads;  // scales then inverse scales
        size_t b = kv->scale_layer_elems * num_layers * sizeof(float);
        st = check_hip(hipMalloc(&kv->k_scales, b), "hipMalloc(K scales)");
        if (st == GG_OK) st = check_hip(hipMalloc(&kv->v_scales, b), "hipMalloc(V scales)");
        if (st == GG_OK) {
            std::vector<float> ones(kv->scale_layer_elems * num_layers, 1.0f);
            st = check_hip(hipMemcpy(kv->k_scales, ones.data(), b, hipMemcpyHostToDevice), "scales init");
            if (st == GG_OK)
                st = check_hip(hipMemcpy(kv->v_scales, ones.data(), b, hipMemcpyHostToDevice), "scales init");
        }
    }
    if (st == GG_OK && scale_mode == GG_SCALE_PER_BLOCK) {
        kv->scale_layer_elems = (size_t)num_blocks * num_kv_heads;
        size_t b = kv->scale_layer_elems * num_layers * sizeof(uint16_t);
        st = check_hip(hipMalloc(&kv->k_scales, b), "hipMalloc(K scales)");
        if (st == GG_OK) st = check_hip(hipMalloc(&kv->v_scales, b), "hipMalloc(V scales)");
        if (st == GG_OK) st = check_hip(hipMemset(kv->k_scales, 0, b), "scales init");
        if (st == GG_OK) st = check_hip(hipMemset(kv->v_scales, 0, b), "scales init");
    }
    if (st != GG_OK) {
        std::string msg = t_last_error;
        (void)hipFree(kv->k_pool);
        (void)hipFree(kv->k_scales);
        (void)hipFree(kv->v_scales);
        delete kv;
        set_error(msg);
        return st;
    }
    *out = kv;
    return GG_OK;
}

GG_API gg_status_t gg_kv_destroy(gg_kv_t kv) {
    clear_error();
    if (!kv) return GG_OK;
    (void)hipFree(kv->k_pool);
    (void)hipFree(kv->k_scales);
    (void)hipFree(kv->v_scales);
    delete kv;
    return GG_OK;
}

GG_API void* gg_kv_k_layer_ptr(gg_kv_t kv, int layer) {
    if (!kv || layer < 0 || layer >= kv->num_layers) return nullptr;
    return kv->k_pool + (size_t)layer * kv->layer_stride;
}
GG_API void* gg_kv_v_layer_ptr(gg_kv_t kv, int layer) {
    if (!kv || layer < 0 || layer >= kv->num_layers) return nullptr;
    return kv->v_pool + (size_t)layer * kv->layer_stride;
}
static void* scale_ptr(gg_kv_t kv, void* base, int layer) {
    if (!kv || !base || layer < 0 || layer >= kv->num_layers) return nullptr;
    size_t eb = kv->scale_mode == GG_SCALE_PER_HEAD ? sizeof(float) : sizeof(uint16_t);
    return (uint8_t*)base + (size_t)layer * kv->scale_layer_elems * eb;
}
GG_API void* gg_kv_k_scale_ptr(gg_kv_t kv, int layer) { return kv ? scale_ptr(kv, kv->k_scales, layer) : nullptr; }
GG_API void* gg_kv_v_scale_ptr(gg_kv_t kv, int layer) { return kv ? scale_ptr(kv, kv->v_scales, layer) : nullptr; }
GG_API size_t gg_kv_layer_bytes(gg_kv_t kv) { return kv ? kv->layer_bytes : 0; }

GG_API gg_status_t gg_kv_set_head_scales(gg_kv_t kv, int layer, const float* k_scales,
                                         const float* v_scales) {
    clear_error();
    GG_CHECK_ARG(kv && k_scales && v_scales, "gg_kv_set_head_scales: NULL argument");
    GG_CHECK_ARG(kv->scale_mode == GG_SCALE_PER_HEAD, "gg_kv_set_head_scales: pool is not PER_HEAD");
    GG_CHECK_ARG(layer >= 0 && layer < kv->num_layers, "gg_kv_set_head_scales: layer out of range");
    const int H = kv->num_kv_heads;
    std::vector<float> kb(2 * H), vb(2 * H);
    for (int h = 0; h < H; ++h) {
        GG_CHECK_ARG(std::isfinite(k_scales[h]) && k_scales[h] > 0.f && std::isfinite(v_scales[h]) &&
                         v_scales[h] > 0.f,
                     "gg_kv_set_head_scales: scales must be finite and > 0");
        kb[h] = k_scales[h];
        vb[h] = v_scales[h];
        kb[H + h] = 1.0f / k_scales[h];  // the reference's scale_inv (gollmgo_model.cu:420)
        vb[H + h] = 1.0f / v_scales[h];
    }
    gg_status_t st = check_hip(hipMemcpy(scale_ptr(kv, kv->k_scales, layer), kb.data(),
                                         2 * H * sizeof(float), hipMemcpyHostToDevice),
                               "upload K scales");
    if (st != GG_OK) return st;
    return check_hip(hipMemcpy(scale_ptr(kv, kv->v_scales, layer), vb.data(), 2 * H * sizeof(float),
                               hipMemcpyHostToDevice),
                     "upload V scales");
}

GG_API size_t gg_kv_snapshot_bytes(gg_kv_t kv, int num_blocks) {
    if (!kv || num_blocks < 0) return 0;
    return (size_t)num_blocks * kv->num_layers * kv_swap_record_bytes(kv);
}

static gg_status_t kv_swap_check(gg_kv_t kv, const int32_t* block_ids, int num_blocks, void* staging,
                                 size_t staging_bytes, const char* who) {
    GG_CHECK_ARG(kv != nullptr, who);
    GG_CHECK_ARG(num_blocks >= 0 && num_blocks <= (1 << 24), "KV swap: bad block count");
    GG_CHECK_ARG(num_blocks == 0 || (block_ids && staging), "KV swap: NULL buffer");
    GG_CHECK_ARG(((uintptr_t)staging % 16) == 0, "KV swap: staging must be 16-byte aligned");
    GG_CHECK_ARG(staging_bytes >= gg_kv_snapshot_bytes(kv, num_blocks), "KV swap: staging too small");
    return GG_OK;
}

GG_API gg_status_t gg_kv_snapshot(gg_kv_t kv, const int32_t* block_ids, int num_blocks, void* staging,
                                  size_t staging_bytes, void* host_dst, void* stream) {
    clear_error();
    const gg_status_t st = kv_swap_check(kv, block_ids, num_blocks, staging, staging_bytes, "gg_kv_snapshot: kv is NULL");
    if (st != GG_OK || num_blocks == 0) return st;
    return launch_kv_snapshot(kv, block_ids, num_blocks, staging, host_dst, (hipStream_t)stream);
}

GG_API gg_status_t gg_kv_restore(gg_kv_t kv, const int32_t* block_ids, int num_blocks, void* staging,
                                 size_t staging_bytes, const void* host_src, void* stream) {
    clear_error();
    const gg_status_t st = kv_swap_check(kv, block_ids, num_blocks, staging, staging_bytes, "gg_kv_restore: kv is NULL");
    if (st != GG_OK || num_blocks == 0) return st;
    return launch_kv_restore(kv, block_ids, num_blocks, staging, host_src, (hipStream_t)stream);
}

GG_API gg_status_t gg_kv_append(gg_kv_t kv, int layer, const void* k, const void* v,
                                gg_dtype_t src_dtype, const int32_t* slot_mapping, int n_rows,
                                void* stream) {
    clear_error();
    GG_CHECK_ARG(kv != nullptr, "gg_kv_append: kv is NULL");
    GG_CHECK_ARG(layer >= 0 && layer < kv->num_layers, "gg_kv_append: layer out of range");
    GG_CHECK_ARG(n_rows >= 0, "gg_kv_append: n_rows < 0");
    if (n_rows == 0) return GG_OK;
    GG_CHECK_ARG(k && v && slot_mapping, "gg_kv_append: NULL buffer");
    GG_CHECK_ARG(is_float_io(src_dtype), "gg_kv_append: src dtype must be F32/F16/BF16");
    GG_CHECK_ARG(n_rows <= (1 << 24), "gg_kv_append: n_rows too large");
    return launch_kv_append(kv, layer, k, v, src_dtype, slot_mapping, n_rows, (hipStream_t)stream);
}

// ---------------------------------------------------------------- attention

namespace gg {
int device_cu_count() {
    static int cache[64] = {0};
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 256;
    if (cache[d] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0) n = 256;
        cache[d] = n;
    }
    return cache[d];
}
}  // namespace gg

static bool attn_shape_ok(gg_kv_t kv, int num_seqs, int rows, int hq, int max_blocks) {
    return kv && num_seqs > 0 && rows > 0 && hq > 0 && max_blocks > 0 && hq % kv->num_kv_heads == 0 &&
           (long long)max_blocks * kv->block_size <= (1LL << 30);
}

GG_API size_t gg_verify_attention_workspace_size(gg_kv_t kv, int num_seqs, int rows_per_seq,
                                                 int num_q_heads, int max_blocks_per_seq,
                                                 int partition_tokens) {
    if (!attn_shape_ok(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq)) return 0;
    if (partition_tokens < 0 || partition_tokens % 64 != 0) return 0;
    const AttnPlan plan = attn_plan(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq, partition_tokens);
    if (plan.sched != ATTN_SCHED_GRID)
        return attn_streamk_workspace_bytes(kv, num_seqs, rows_per_seq, num_q_heads, nullptr, nullptr);
    return attn_workspace_bytes(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq, plan.partition);
}

// What one attention entry point does with the schedule plan.
enum AttnCall { ATTN_CALL_SELF = 0, ATTN_CALL_PLANNED = 1, ATTN_CALL_PLAN_ONLY = 2 };

static gg_status_t verify_attention_impl(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype, void* out,
                                         gg_dtype_t out_dtype, const int32_t* ctx_lens, const int32_t* row_counts,
                                         const int32_t* block_tables, int max_blocks_per_seq, int num_seqs,
                                         int rows_per_seq, int num_q_heads, float scale, int partition_tokens,
                                         void* workspace, size_t workspace_bytes, void* stream, AttnCall call,
                                         const void* k_new = nullptr, const void* v_new = nullptr,
                                         gg_dtype_t new_dtype = GG_DTYPE_BF16) {
    clear_error();
    const bool compute = call != ATTN_CALL_PLAN_ONLY;
    GG_CHECK_ARG(kv != nullptr, "gg_verify_attention: kv is NULL");
    GG_CHECK_ARG(!compute || (layer >= 0 && layer < kv->num_layers), "gg_verify_attention: layer out of range");
    GG_CHECK_ARG(ctx_lens && (!compute || (q && out && block_tables)), "gg_verify_attention: NULL buffer");
    GG_CHECK_ARG(!compute || (is_float_io(q_dtype) && is_float_io(out_dtype)),
                 "gg_verify_attention: q/out dtype must be F32/F16/BF16");
    GG_CHECK_ARG(attn_shape_ok(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq),
                 "gg_verify_attention: bad shape (num_q_heads must be a multiple of num_kv_heads)");
    GG_CHECK_ARG(partition_tokens >= 0 && partition_tokens % 64 == 0,
                 "gg_verify_attention: partition_tokens must be a non-negative multiple of 64");
    GG_CHECK_ARG(std::isfinite(scale), "gg_verify_attention: scale must be finite");
    AttnArgs a{};
    a.kv = kv;
    a.layer = layer;
    a.q = q;
    a.q_dtype = q_dtype;
    a.out = out;
    a.out_dtype = out_dtype;
    a.ctx_lens = ctx_lens;
    a.row_counts = row_counts;
    a.block_tables = block_tables;
    a.max_blocks = max_blocks_per_seq;
    a.num_seqs = num_seqs;
    a.rows = rows_per_seq;
    a.num_q_heads = num_q_heads;
    a.scale = scale;
    a.kv_bs = kv->block_size;
    const AttnPlan plan = attn_plan(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq, partition_tokens);
    a.sched = plan.sched;
    a.partition = plan.sched == ATTN_SCHED_GRID ? plan.partition : kMfmaAutoPartition;
    a.max_parts = (max_blocks_per_seq * kv->block_size + a.partition - 1) / a.partition;
    a.sk_min_chunks = kStreamKMinChunks;
    size_t need, n_ml, n_acc = 0;
    if (a.sched != ATTN_SCHED_GRID) {
        a.sk_grid = attn_streamk_grid(kv, rows_per_seq, num_q_heads);
        need = attn_streamk_workspace_bytes(kv, num_seqs, rows_per_seq, num_q_heads, &n_ml, &n_acc);
    } else {
        need = attn_workspace_bytes(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq, a.partition);
        n_ml = (size_t)num_seqs * rows_per_seq * num_q_heads * a.max_parts * 2;
    }
    GG_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                 "gg_verify_attention: workspace too small");
    if (need) {
        a.ws_ml = (float*)workspace;
        a.ws_acc = (float*)workspace + ((n_ml + 63) / 64) * 64;
        if (a.sched != ATTN_SCHED_GRID) a.plan = (int*)(a.ws_acc + n_acc);
    }
    a.plan_ready = call == ATTN_CALL_PLANNED ? 1 : 0;
    if (k_new) {
        a.k_new = k_new;
        a.v_new = v_new;
        a.new_dtype = new_dtype;
    }
    if (call == ATTN_CALL_PLAN_ONLY) return launch_attn_plan(a, (hipStream_t)stream);
    return launch_verify_attention(a, (hipStream_t)stream);
}

GG_API gg_status_t gg_verify_attention(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype,
                                       void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                       const int32_t* row_counts, const int32_t* block_tables,
                                       int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                       int num_q_heads, float scale, int partition_tokens,
                                       void* workspace, size_t workspace_bytes, void* stream) {
    return verify_attention_impl(kv, layer, q, q_dtype, out, out_dtype, ctx_lens, row_counts, block_tables,
                                 max_blocks_per_seq, num_seqs, rows_per_seq, num_q_heads, scale, partition_tokens,
                                 workspace, workspace_bytes, stream, ATTN_CALL_SELF);
}

GG_API gg_status_t gg_verify_attention_plan(gg_kv_t kv, const int32_t* ctx_lens, const int32_t* row_counts,
                                            int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                            int num_q_heads, void* workspace, size_t workspace_bytes,
                                            void* stream) {
    return verify_attention_impl(kv, 0, nullptr, GG_DTYPE_BF16, nullptr, GG_DTYPE_BF16, ctx_lens, row_counts,
                                 nullptr, max_blocks_per_seq, num_seqs, rows_per_seq, num_q_heads, 1.0f, 0,
                                 workspace, workspace_bytes, stream, ATTN_CALL_PLAN_ONLY);
}

GG_API gg_status_t gg_verify_attention_planned(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype,
                                               void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                               const int32_t* row_counts, const int32_t* block_tables,
                                               int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                               int num_q_heads, float scale, void* workspace,
                                               size_t workspace_bytes, void* stream) {
    return verify_attention_impl(kv, layer, q, q_dtype, out, out_dtype, ctx_lens, row_counts, block_tables,
                                 max_blocks_per_seq, num_seqs, rows_per_seq, num_q_heads, scale, 0, workspace,
                                 workspace_bytes, stream, ATTN_CALL_PLANNED);
}

GG_API gg_status_t gg_verify_append_attention_planned(gg_kv_t kv, int layer, const void* k_new,
                                                      const void* v_new, gg_dtype_t new_dtype, const void* q,
                                                      gg_dtype_t q_dtype, void* out, gg_dtype_t out_dtype,
                                                      const int32_t* ctx_lens, const int32_t* row_counts,
                                                      const int32_t* block_tables, int max_blocks_per_seq,
                                                      int num_seqs, int rows_per_seq, int num_q_heads, float scale,
                                                      void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    GG_CHECK_ARG(kv != nullptr, "gg_verify_append_attention_planned: kv is NULL");
    GG_CHECK_ARG(k_new && v_new, "gg_verify_append_attention_planned: NULL buffer");
    GG_CHECK_ARG(is_float_io(new_dtype), "gg_verify_append_attention_planned: k/v dtype must be F32/F16/BF16");
    GG_CHECK_ARG(kv->head_dim % 8 == 0 && (uintptr_t)k_new % 16 == 0 && (uintptr_t)v_new % 16 == 0,
                 "gg_verify_append_attention_planned: needs head_dim % 8 == 0 and 16-byte aligned k_new/v_new");
    return verify_attention_impl(kv, layer, q, q_dtype, out, out_dtype, ctx_lens, row_counts, block_tables,
                                 max_blocks_per_seq, num_seqs, rows_per_seq, num_q_heads, scale, 0, workspace,
                                 workspace_bytes, stream, ATTN_CALL_PLANNED, k_new, v_new, new_dtype);
}

// ---------------------------------------------------------------- attention without allocation

// Scratch of gg_verify_attention_noalloc: a file-scope device array, one copy per GPU the
// library runs on, held until the process ends. Host code never passes the array's name
// to a kernel (on the host it is only a stand-in for the symbol): it uses the device
// address that hipGetSymbolAddress returns, looked up once per device.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up on the first call on
// that device, with the device current).
gg_status_t scratch_ptr(void** out) {
    int d = 0;
    gg_status_t st = check_hip(hipGetDevice(&d), "hipGetDevice");
    if (st != GG_OK) return st;
    if (d < 0 || d >= kMaxDevices) return fail(GG_ERR_INTERNAL, "gg_verify_attention_noalloc: device id too large");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[d]) {
        void* p = nullptr;
        st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (st != GG_OK) return st;
        g_scratch_ptr[d] = p;
    }
    *out = g_scratch_ptr[d];
    return GG_OK;
}
}  // namespace

GG_API size_t gg_verify_attention_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

GG_API gg_status_t gg_verify_attention_noalloc(gg_kv_t kv, int layer, const void* q, gg_dtype_t q_dtype,
                                               void* out, gg_dtype_t out_dtype, const int32_t* ctx_lens,
                                               const int32_t* row_counts, const int32_t* block_tables,
                                               int max_blocks_per_seq, int num_seqs, int rows_per_seq,
                                               int num_q_heads, float scale, void* stream) {
    clear_error();
    GG_CHECK_ARG(kv != nullptr, "gg_verify_attention_noalloc: kv is NULL");
    GG_CHECK_ARG(attn_shape_ok(kv, num_seqs, rows_per_seq, num_q_heads, max_blocks_per_seq),
                 "gg_verify_attention_noalloc: bad shape (num_q_heads must be a multiple of num_kv_heads)");
    // The size check comes before any device call.
    const size_t need = gg_verify_attention_workspace_size(kv, num_seqs, rows_per_seq, num_q_heads,
                                                           max_blocks_per_seq, 0);
    if (need > kNoAllocScratchBytes)
        return fail(GG_ERR_INVALID, "gg_verify_attention_noalloc: the call needs " + std::to_string(need) +
                                        " bytes of scratch, above the library's fixed " +
                                        std::to_string(kNoAllocScratchBytes) +
                                        " (use gg_verify_attention with a workspace)");
    void* ws = nullptr;
    if (need) {
        const gg_status_t st = scratch_ptr(&ws);
        if (st != GG_OK) return st;
    }
    return verify_attention_impl(kv, layer, q, q_dtype, out, out_dtype, ctx_lens, row_counts, block_tables,
                                 max_blocks_per_seq, num_seqs, rows_per_seq, num_q_heads, scale, 0, ws, need,
                                 stream, ATTN_CALL_SELF);
}

// ---------------------------------------------------------------- acceptance

static bool accept_shape_ok(int num_seqs, int max_drafts, int vocab) {
    return num_seqs > 0 && max_drafts >= 0 && max_drafts <= 64 && vocab > 0 && vocab <= (1 << 18);
}

GG_API size_t gg_accept_greedy_workspace_size(int num_seqs, int max_drafts, int vocab) {
    if (!accept_shape_ok(num_seqs, max_drafts, vocab)) return 0;
    return greedy_workspace_bytes(num_seqs, max_drafts, vocab);
}

GG_API gg_status_t gg_accept_greedy(const void* logits, gg_dtype_t logits_dtype, int num_seqs,
                                    int max_drafts, int vocab, const int32_t* drafts,
                                    const int32_t* n_drafts, int32_t* out_accepted,
                                    int32_t* out_token, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    clear_error();
    GG_CHECK_ARG(accept_shape_ok(num_seqs, max_drafts, vocab),
                 "gg_accept_greedy: bad shape (need num_seqs>0, 0<=max_drafts<=64, 0<vocab<=2^18)");
    GG_CHECK_ARG(logits && n_drafts && out_accepted && out_token && (drafts || max_drafts == 0),
                 "gg_accept_greedy: NULL buffer");
    GG_CHECK_ARG(is_float_io(logits_dtype), "gg_accept_greedy: logits dtype must be F32/F16/BF16");
    size_t need = greedy_workspace_bytes(num_seqs, max_drafts, vocab);
    GG_CHECK_ARG(workspace && workspace_bytes >= need, "gg_accept_greedy: workspace too small");
    return launch_accept_greedy(logits, logits_dtype, num_seqs, max_drafts, vocab, drafts, n_drafts,
                                out_accepted, out_token, workspace, (hipStream_t)stream);
}

GG_API size_t gg_accept_greedy_sample_workspace_size(int num_seqs, int max_drafts, int vocab) {
    if (!accept_shape_ok(num_seqs, max_drafts, vocab)) return 0;
    return sample_workspace_bytes(num_seqs, max_drafts, vocab);
}

GG_API gg_status_t gg_accept_greedy_sample(const void* logits, gg_dtype_t logits_dtype, int num_seqs,
                                           int max_drafts, int vocab, const int32_t* drafts,
                                           const int32_t* n_drafts, double temperature, int top_k,
                                           double top_p, const double* uniforms, unsigned flags,
                                           int32_t* out_accepted, int32_t* out_token, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    clear_error();
    GG_CHECK_ARG(accept_shape_ok(num_seqs, max_drafts, vocab),
                 "gg_accept_greedy_sample: bad shape (need num_seqs>0, 0<=max_drafts<=64, 0<vocab<=2^18)");
    GG_CHECK_ARG(logits && n_drafts && uniforms && out_accepted && out_token && (drafts || max_drafts == 0),
                 "gg_accept_greedy_sample: NULL buffer");
    GG_CHECK_ARG(is_float_io(logits_dtype), "gg_accept_greedy_sample: logits dtype must be F32/F16/BF16");
    GG_CHECK_ARG((flags & ~GG_SAMPLE_EXACT) == 0, "gg_accept_greedy_sample: unknown flags");
    const size_t need = sample_workspace_bytes(num_seqs, max_drafts, vocab);
    GG_CHECK_ARG(workspace && workspace_bytes >= need, "gg_accept_greedy_sample: workspace too small");
    return launch_accept_greedy_sample(logits, logits_dtype, num_seqs, max_drafts, vocab, drafts, n_drafts,
                                       temperature, top_k, top_p, uniforms, flags, out_accepted, out_token,
                                       workspace, (hipStream_t)stream);
}

GG_API size_t gg_accept_rejection_workspace_size(int num_seqs, int max_drafts, int vocab) {
    if (!accept_shape_ok(num_seqs, max_drafts, vocab)) return 0;
    return rejection_workspace_bytes(num_seqs, max_drafts, vocab);
}

GG_API gg_status_t gg_accept_rejection(const void* target_logits, gg_dtype_t logits_dtype,
                                       const float* draft_probs, int num_seqs, int max_drafts,
                                       int vocab, const int32_t* drafts, const int32_t* n_drafts,
                                       const float* uniforms, float temperature, float top_p,
                                       int32_t* out_accepted, int32_t* out_token, void* workspace,
                                       size_t workspace_bytes, void* stream) {
    clear_error();
    GG_CHECK_ARG(accept_shape_ok(num_seqs, max_drafts, vocab),
                 "gg_accept_rejection: bad shape (need num_seqs>0, 0<=max_drafts<=64, 0<vocab<=2^18)");
    GG_CHECK_ARG(target_logits && n_drafts && uniforms && out_accepted && out_token &&
                     (drafts || max_drafts == 0),
                 "gg_accept_rejection: NULL buffer");
    GG_CHECK_ARG(is_float_io(logits_dtype), "gg_accept_rejection: logits dtype must be F32/F16/BF16");
    GG_CHECK_ARG(std::isfinite(temperature) && std::isfinite(top_p), "gg_accept_rejection: non-finite parameter");
    if (temperature <= 1e-9f) {
        size_t need = greedy_workspace_bytes(num_seqs, max_drafts, vocab);
        GG_CHECK_ARG(workspace && workspace_bytes >= need, "gg_accept_rejection: workspace too small");
        return launch_accept_greedy(target_logits, logits_dtype, num_seqs, max_drafts, vocab, drafts,
                                    n_drafts, out_accepted, out_token, workspace, (hipStream_t)stream);
    }
    size_t need = rejection_workspace_bytes(num_seqs, max_drafts, vocab);
    GG_CHECK_ARG(workspace && workspace_bytes >= need, "gg_accept_rejection: workspace too small");
    return launch_accept_rejection(target_logits, logits_dtype, draft_probs, num_seqs, max_drafts,
                                   vocab, drafts, n_drafts, uniforms, temperature, top_p,
                                   out_accepted, out_token, workspace, (hipStream_t)stream);
}

// ---------------------------------------------------------------- n-gram drafts

GG_API gg_status_t gg_ngram_draft(const int32_t* history, int hist_stride, const int32_t* hist_len,
                                  int num_seqs, int n, int max_drafts, int32_t* out_drafts,
                                  int32_t* out_n, void* stream) {
    clear_error();
    // NewNGramDrafter normalisation (internal/engine/speculative.go:12-20).
    if (n < 2) n = 2;
    if (max_drafts < 1) max_drafts = 4;
    GG_CHECK_ARG(n <= 9, "gg_ngram_draft: n must be <= 9 (the reference key holds 8 tokens)");
    GG_CHECK_ARG(num_seqs > 0 && hist_stride >= 0 && max_drafts <= 64, "gg_ngram_draft: bad shape");
    GG_CHECK_ARG(history && hist_len && out_drafts && out_n, "gg_ngram_draft: NULL buffer");
    return launch_ngram_draft(history, hist_stride, hist_len, num_seqs, n, max_drafts, out_drafts,
                              out_n, (hipStream_t)stream);
}

GG_API gg_status_t gg_history_append_draft(int32_t* history, int hist_stride, int32_t* hist_len,
                                           const int32_t* hist_rows, int num_seqs, const int32_t* drafts,
                                           int drafts_per_seq, const int32_t* accepted, const int32_t* token,
                                           int n, int max_drafts, int32_t* out_drafts, int32_t* out_n,
                                           void* stream) {
    clear_error();
    if (n < 2) n = 2;
    if (max_drafts < 1) max_drafts = 4;
    GG_CHECK_ARG(n <= 9, "gg_history_append_draft: n must be <= 9 (the reference key holds 8 tokens)");
    GG_CHECK_ARG(num_seqs > 0 && hist_stride >= 0 && max_drafts <= 64 && drafts_per_seq >= 0 && drafts_per_seq <= 64,
                 "gg_history_append_draft: bad shape");
    GG_CHECK_ARG(history && hist_len && accepted && token && out_drafts && out_n && (drafts || drafts_per_seq == 0),
                 "gg_history_append_draft: NULL buffer");
    return launch_history_append_draft(history, hist_stride, hist_len, hist_rows, num_seqs, drafts, drafts_per_seq,
                                       accepted, token, n, max_drafts, out_drafts, out_n, (hipStream_t)stream);
}
