// kv_append.hip — draft-KV append into the paged cache (quantise-on-write).
//
// Replaces paged_kv_write_{f16,bf16} (kernels/gollmgo_paged_attn.cu:14-35,126-146)
// as called per layer from run_layer (kernels/gollmgo_model.cu:610-625). The
// reference copies 2-byte rows to cache[slot][Hkv][D]; here rows land in the
// block layouts K[blk][Hkv][bs][D] and V[blk][Hkv][D][bs] and are quantised to
// FP8-E4M3 (per-head fp32 scale) or INT8 (per-block fp16 scale) when the pool
// stores them. Quantisation follows the reference's weight conventions:
// q = cvt(x * (1/scale)) with E4M3 satfinite / int8 RNE clamped to +-127
// (kernels/gollmgo_model.cu:248-268).
#include "gg_common.h"

namespace gg {
namespace {

// Element indices from the K and V pool bases. The K and V tiles of a (block, head)
// alternate, so consecutive tiles of one pool are 2 * bs * D elements apart.
__device__ __forceinline__ size_t k_index(int blk, int h, int off, int d, int Hkv, int bs, int D) {
    return ((size_t)blk * Hkv + h) * (2 * (size_t)bs * D) + (size_t)off * D + d;
}
__device__ __forceinline__ size_t v_index(int blk, int h, int off, int d, int Hkv, int bs, int D) {
    return ((size_t)blk * Hkv + h) * (2 * (size_t)bs * D) + (size_t)d * bs + off;
}

struct AppendArgs {
    uint8_t* kc;
    uint8_t* vc;
    const void* k;
    const void* v;
    gg_dtype_t src;
    const int32_t* slots;
    int n_rows;
    int Hkv, D, bs;
    long long num_slots;  // num_blocks * bs: larger slots are skipped
    gg_dtype_t dst;
    const float* k_scale;  // PER_HEAD scales [Hkv]
    const float* v_scale;
    const float* k_inv;    // PER_HEAD inverse scales [Hkv]
    const float* v_inv;
    uint16_t* k_bscale;    // PER_BLOCK fp16 scales [blocks][Hkv]
    uint16_t* v_bscale;
};

// Plain / per-head-scaled append: grid (n_rows), one thread per (head, dim) element.
__global__ void __launch_bounds__(256) append_direct_kernel(AppendArgs a) {
    const int r = blockIdx.x;
    const int slot = a.slots[r];
    if (slot < 0 || slot >= a.num_slots) return;
    const int blk = slot / a.bs, off = slot % a.bs;
    const int n = a.Hkv * a.D;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int h = i / a.D, d = i % a.D;
        const size_t src_i = (size_t)r * n + i;
        float kx = load_as_f32(a.k, a.src, src_i);
        float vx = load_as_f32(a.v, a.src, src_i);
        size_t ki = k_index(blk, h, off, d, a.Hkv, a.bs, a.D);
        size_t vi = v_index(blk, h, off, d, a.Hkv, a.bs, a.D);
        switch (a.dst) {
            case GG_DTYPE_F32:
                ((float*)a.kc)[ki] = kx;
                ((float*)a.vc)[vi] = vx;
                break;
            case GG_DTYPE_F16:
                ((uint16_t*)a.kc)[ki] = f32_to_f16_bits(kx);
                ((uint16_t*)a.vc)[vi] = f32_to_f16_bits(vx);
                break;
            case GG_DTYPE_BF16:
                ((uint16_t*)a.kc)[ki] = f32_to_bf16_bits(kx);
                ((uint16_t*)a.vc)[vi] = f32_to_bf16_bits(vx);
                break;
            case GG_DTYPE_FP8_E4M3:
                a.kc[ki] = f32_to_fp8e4m3_sat(kx * a.k_inv[h]);
                a.vc[vi] = f32_to_fp8e4m3_sat(vx * a.v_inv[h]);
                break;
            default:
                break;
        }
    }
}

// Vectorised plain / per-head-scaled append for head_dim % 8 == 0: one thread per eight
// consecutive elements of one (row, head), all source loads issued together, the
// element types fixed at compile time. Same roundings as append_direct_kernel.
template <gg_dtype_t SRC>
__device__ __forceinline__ void load8(const void* p, size_t i, float* x) {
    if constexpr (SRC == GG_DTYPE_F32) {
        const float4 a = ((const float4*)((const float*)p + i))[0];
        const float4 b = ((const float4*)((const float*)p + i))[1];
        x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
    } else {
        const uint4 w = *(const uint4*)((const uint16_t*)p + i);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint16_t lo = (uint16_t)u[k], hi = (uint16_t)(u[k] >> 16);
            x[2 * k] = SRC == GG_DTYPE_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
            x[2 * k + 1] = SRC == GG_DTYPE_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
    }
}

template <gg_dtype_t SRC, gg_dtype_t DST>
__global__ void __launch_bounds__(256) append_vec_kernel(AppendArgs a) {
    const int groups = a.Hkv * a.D / 8;  // eight-element groups per row
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long long)a.n_rows * groups) return;
    const int r = (int)(gid / groups), g = (int)(gid % groups);
    const int i0 = g * 8, h = i0 / a.D, d0 = i0 % a.D;
    // The source row does not depend on the slot: its loads go out together with the
    // slot's, so the call waits for one round trip before converting, not two.
    const size_t src_i = (size_t)r * a.Hkv * a.D + i0;
    float kx[8], vx[8];
    load8<SRC>(a.k, src_i, kx);
    load8<SRC>(a.v, src_i, vx);
    float kinv = 1.f, vinv = 1.f;
    if constexpr (DST == GG_DTYPE_FP8_E4M3) {
        kinv = a.k_inv[h];
        vinv = a.v_inv[h];
    }
    const int slot = a.slots[r];
    if (slot < 0 || slot >= a.num_slots) return;
    const int blk = slot / a.bs, off = slot % a.bs;
    const size_t ki = k_index(blk, h, off, d0, a.Hkv, a.bs, a.D);  // 8 contiguous elements
    const size_t vi = v_index(blk, h, off, d0, a.Hkv, a.bs, a.D);  // stride bs per element
    if constexpr (DST == GG_DTYPE_F32) {
        float4* kp = (float4*)((float*)a.kc + ki);
        kp[0] = make_float4(kx[0], kx[1], kx[2], kx[3]);
        kp[1] = make_float4(kx[4], kx[5], kx[6], kx[7]);
#pragma unroll
        for (int j = 0; j < 8; ++j) ((float*)a.vc)[vi + (size_t)j * a.bs] = vx[j];
    } else if constexpr (DST == GG_DTYPE_F16 || DST == GG_DTYPE_BF16) {
        uint16_t kb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            kb[j] = DST == GG_DTYPE_BF16 ? f32_to_bf16_bits(kx[j]) : f32_to_f16_bits(kx[j]);
            const uint16_t vb = DST == GG_DTYPE_BF16 ? f32_to_bf16_bits(vx[j]) : f32_to_f16_bits(vx[j]);
            ((uint16_t*)a.vc)[vi + (size_t)j * a.bs] = vb;
        }
        *(uint4*)((uint16_t*)a.kc + ki) = make_uint4(kb[0] | ((uint32_t)kb[1] << 16), kb[2] | ((uint32_t)kb[3] << 16),
                                                     kb[4] | ((uint32_t)kb[5] << 16), kb[6] | ((uint32_t)kb[7] << 16));
    } else {  // FP8-E4M3, per-head scales
        uint32_t kw[2];
#pragma unroll
        for (int j = 0; j < 8; j += 4)
            kw[j >> 2] = f32x2_to_fp8e4m3_sat(kx[j] * kinv, kx[j + 1] * kinv) |
                         (f32x2_to_fp8e4m3_sat(kx[j + 2] * kinv, kx[j + 3] * kinv) << 16);
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const uint32_t vw = f32x2_to_fp8e4m3_sat(vx[j] * vinv, vx[j + 1] * vinv);
            a.vc[vi + (size_t)j * a.bs] = (uint8_t)vw;
            a.vc[vi + (size_t)(j + 1) * a.bs] = (uint8_t)(vw >> 8);
        }
        *(uint2*)(a.kc + ki) = make_uint2(kw[0], kw[1]);
    }
}

// 2-byte sources into 1- and 2-byte pools: one thread per (row, kv head, dim), so a wave
// writes 64 dims of one head's row. Its K run is 64 adjacent stores, and each V store of
// the wave lands in a single dim-major tile at the 16-offset stride (16 or 32 bytes): the
// fewest cache lines per store. (Eight dims per thread spread every V store of a wave over
// eight tiles' worth of lines; two dims per thread, two.)
template <gg_dtype_t SRC, gg_dtype_t DST>
__global__ void __launch_bounds__(256) append_dim_kernel(AppendArgs a) {
    const int per = a.Hkv * a.D;
    const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long long)a.n_rows * per) return;
    const int r = (int)(gid / per), i0 = (int)(gid % per);
    const int h = i0 / a.D, d0 = i0 % a.D;
    const size_t src_i = (size_t)r * a.Hkv * a.D + i0;
    const uint16_t kw = ((const uint16_t*)a.k)[src_i];
    const uint16_t vw = ((const uint16_t*)a.v)[src_i];
    float kinv = 1.f, vinv = 1.f;
    if constexpr (DST == GG_DTYPE_FP8_E4M3) {
        kinv = a.k_inv[h];
        vinv = a.v_inv[h];
    }
    const int slot = a.slots[r];
    if (slot < 0 || slot >= a.num_slots) return;
    const int blk = slot / a.bs, off = slot % a.bs;
    auto f = [](uint16_t b) { return SRC == GG_DTYPE_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b); };
    const size_t ki = k_index(blk, h, off, d0, a.Hkv, a.bs, a.D);
    const size_t vi = v_index(blk, h, off, d0, a.Hkv, a.bs, a.D);
    if constexpr (DST == GG_DTYPE_FP8_E4M3) {
        const uint32_t w = f32x2_to_fp8e4m3_sat(f(kw) * kinv, f(vw) * vinv);
        a.kc[ki] = (uint8_t)w;
        a.vc[vi] = (uint8_t)(w >> 8);
    } else if constexpr (SRC == DST) {
        ((uint16_t*)a.kc)[ki] = kw;
        ((uint16_t*)a.vc)[vi] = vw;
    } else {
        ((uint16_t*)a.kc)[ki] = DST == GG_DTYPE_BF16 ? f32_to_bf16_bits(f(kw)) : f32_to_f16_bits(f(kw));
        ((uint16_t*)a.vc)[vi] = DST == GG_DTYPE_BF16 ? f32_to_bf16_bits(f(vw)) : f32_to_f16_bits(f(vw));
    }
}

template <gg_dtype_t SRC>
void launch_dim(const AppendArgs& a, gg_dtype_t dst, hipStream_t s) {
    const long long threads = (long long)a.n_rows * (a.Hkv * a.D);
    const unsigned grid = (unsigned)((threads + 255) / 256);
    switch (dst) {
        case GG_DTYPE_F16: append_dim_kernel<SRC, GG_DTYPE_F16><<<grid, 256, 0, s>>>(a); break;
        case GG_DTYPE_BF16: append_dim_kernel<SRC, GG_DTYPE_BF16><<<grid, 256, 0, s>>>(a); break;
        default: append_dim_kernel<SRC, GG_DTYPE_FP8_E4M3><<<grid, 256, 0, s>>>(a); break;
    }
}

template <gg_dtype_t SRC>
void launch_vec(const AppendArgs& a, gg_dtype_t dst, hipStream_t s) {
    const long long threads = (long long)a.n_rows * (a.Hkv * a.D / 8);
    const unsigned grid = (unsigned)((threads + 255) / 256);
    switch (dst) {
        case GG_DTYPE_F32: append_vec_kernel<SRC, GG_DTYPE_F32><<<grid, 256, 0, s>>>(a); break;
        case GG_DTYPE_F16: append_vec_kernel<SRC, GG_DTYPE_F16><<<grid, 256, 0, s>>>(a); break;
        case GG_DTYPE_BF16: append_vec_kernel<SRC, GG_DTYPE_BF16><<<grid, 256, 0, s>>>(a); break;
        default: append_vec_kernel<SRC, GG_DTYPE_FP8_E4M3><<<grid, 256, 0, s>>>(a); break;
    }
}

// ---- PER_BLOCK int8: one launch ----
//
// A block's new rows are adjacent in the slot mapping (the verify rows of a sequence are;
// skipped rows may sit between them), so the first row of each run of rows in one block
// (its leader) owns the block for the call. Workgroup (r, h) exits unless row r leads a run; otherwise, for kv head h: amax of
// the run's K and V over its rows and dims, the block's new scale max(old, fp16(amax /
// 127)), the run's rows quantised with it, the rows already in the block re-quantised
// when the scale grew, and the scale published. No atomics, no staging.

__device__ __forceinline__ bool slot_ok(int s, long long num_slots) { return s >= 0 && s < num_slots; }

__global__ void __launch_bounds__(256) append_int8_block_kernel(AppendArgs a) {
    const int r = blockIdx.x, h = blockIdx.y;
    const int slot = a.slots[r];
    if (!slot_ok(slot, a.num_slots)) return;
    const int blk = slot / a.bs;
    // Skipped rows (negative or out-of-range slots) do not break a run: row r leads unless
    // the nearest earlier row that is not skipped lands in the same block.
    for (int p = r - 1; p >= 0; --p) {
        const int q = a.slots[p];
        if (!slot_ok(q, a.num_slots)) continue;
        if (q / a.bs == blk) return;  // not the run's leader
        break;
    }
    // The run spans rows [r, e): up to the next row that lands in another block.
    int e = r + 1;
    while (e < a.n_rows) {
        const int q = a.slots[e];
        if (slot_ok(q, a.num_slots) && q / a.bs != blk) break;
        ++e;
    }
    const int lead_off = slot % a.bs;
    const bool fresh = lead_off == 0;
    int8_t* kc = (int8_t*)a.kc;
    int8_t* vc = (int8_t*)a.vc;
    const int nel = (e - r) * a.D;
    __shared__ float red[2][4];
    // The run's values (at most 8 per thread for runs of <= 2048 elements) stay in registers
    // between the amax and the quantisation; skipped rows read as 0.
    constexpr int kCache = 8;
    const bool cached = nel <= kCache * 256;
    auto row_ok = [&](int j) { return slot_ok(a.slots[r + j], a.num_slots); };
    float kv_k[kCache], kv_v[kCache];
    float mk = 0.f, mv = 0.f;
#pragma unroll
    for (int c = 0; c < kCache; ++c) {
        const int i = threadIdx.x + c * 256;
        kv_k[c] = kv_v[c] = 0.f;
        if (cached && i < nel) {
            const int j = i / a.D, d = i % a.D;
            if (row_ok(j)) {
                const size_t src = ((size_t)(r + j) * a.Hkv + h) * a.D + d;
                kv_k[c] = load_as_f32(a.k, a.src, src);
                kv_v[c] = load_as_f32(a.v, a.src, src);
            }
        }
    }
    for (int i = threadIdx.x; i < nel; i += blockDim.x) {
        float kx = 0.f, vx = 0.f;
        if (cached) {
            kx = kv_k[(i - threadIdx.x) / 256];
            vx = kv_v[(i - threadIdx.x) / 256];
        } else {
            const int j = i / a.D, d = i % a.D;
            if (row_ok(j)) {
                const size_t src = ((size_t)(r + j) * a.Hkv + h) * a.D + d;
                kx = load_as_f32(a.k, a.src, src);
                vx = load_as_f32(a.v, a.src, src);
            }
        }
        kx = fabsf(kx);
        vx = fabsf(vx);
        mk = fmaxf(mk, kx == kx ? kx : 0.f);
        mv = fmaxf(mv, vx == vx ? vx : 0.f);
    }
    for (int o = 32; o > 0; o >>= 1) {
        mk = fmaxf(mk, __shfl_xor(mk, o));
        mv = fmaxf(mv, __shfl_xor(mv, o));
    }
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = mk;
        red[1][threadIdx.x >> 6] = mv;
    }
    __syncthreads();
    mk = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    mv = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    mk = fminf(mk, 3.0e38f);
    mv = fminf(mv, 3.0e38f);
    const size_t si = (size_t)blk * a.Hkv + h;
    const float k_old = fresh ? 0.f : f16_bits_to_f32(a.k_bscale[si]);
    const float v_old = fresh ? 0.f : f16_bits_to_f32(a.v_bscale[si]);
    const float k_new = fmaxf(k_old, f16_bits_to_f32(f32_to_f16_rne_bits(mk / 127.0f)));
    const float v_new = fmaxf(v_old, f16_bits_to_f32(f32_to_f16_rne_bits(mv / 127.0f)));
    const float k_inv = k_new > 0.f ? 1.0f / k_new : 0.f;
    const float v_inv = v_new > 0.f ? 1.0f / v_new : 0.f;
    for (int i = threadIdx.x; i < nel; i += blockDim.x) {
        const int j = i / a.D, d = i % a.D;
        const int sj = a.slots[r + j];
        if (!slot_ok(sj, a.num_slots)) continue;
        const int off = sj % a.bs;
        const size_t src = ((size_t)(r + j) * a.Hkv + h) * a.D + d;
        const float kx = cached ? kv_k[(i - threadIdx.x) / 256] : load_as_f32(a.k, a.src, src);
        const float vx = cached ? kv_v[(i - threadIdx.x) / 256] : load_as_f32(a.v, a.src, src);
        kc[k_index(blk, h, off, d, a.Hkv, a.bs, a.D)] = f32_to_i8_sat(kx * k_inv);
        vc[v_index(blk, h, off, d, a.Hkv, a.bs, a.D)] = f32_to_i8_sat(vx * v_inv);
    }
    // Rows already in the block follow a grown scale.
    if (lead_off > 0 && (k_new != k_old || v_new != v_old)) {
        for (int i = threadIdx.x; i < lead_off * a.D; i += blockDim.x) {
            const int t = i / a.D, d = i % a.D;
            if (k_new != k_old) {
                const size_t ki = k_index(blk, h, t, d, a.Hkv, a.bs, a.D);
                kc[ki] = f32_to_i8_sat(((float)kc[ki] * k_old) * k_inv);
            }
            if (v_new != v_old) {
                const size_t vi = v_index(blk, h, t, d, a.Hkv, a.bs, a.D);
                vc[vi] = f32_to_i8_sat(((float)vc[vi] * v_old) * v_inv);
            }
        }
    }
    if (threadIdx.x == 0) {
        a.k_bscale[si] = f32_to_f16_rne_bits(k_new);
        a.v_bscale[si] = f32_to_f16_rne_bits(v_new);
    }
}

}  // namespace

gg_status_t launch_kv_append(KV* kv, int layer, const void* k, const void* v, gg_dtype_t src,
                             const int32_t* slots, int n_rows, hipStream_t s) {
    if (n_rows == 0) return GG_OK;
    AppendArgs a{};
    a.kc = kv->k_pool + (size_t)layer * kv->layer_stride;
    a.vc = kv->v_pool + (size_t)layer * kv->layer_stride;
    a.k = k;
    a.v = v;
    a.src = src;
    a.slots = slots;
    a.n_rows = n_rows;
    a.Hkv = kv->num_kv_heads;
    a.D = kv->head_dim;
    a.bs = kv->block_size;
    a.num_slots = (long long)kv->num_blocks * kv->block_size;
    a.dst = kv->dtype;
    if (kv->scale_mode == GG_SCALE_PER_HEAD) {
        const float* ks = (const float*)kv->k_scales + (size_t)layer * 2 * kv->num_kv_heads;
        const float* vs = (const float*)kv->v_scales + (size_t)layer * 2 * kv->num_kv_heads;
        a.k_scale = ks;
        a.k_inv = ks + kv->num_kv_heads;
        a.v_scale = vs;
        a.v_inv = vs + kv->num_kv_heads;
    }
    if (kv->scale_mode == GG_SCALE_PER_BLOCK) {
        a.k_bscale = (uint16_t*)kv->k_scales + (size_t)layer * kv->scale_layer_elems;
        a.v_bscale = (uint16_t*)kv->v_scales + (size_t)layer * kv->scale_layer_elems;
        append_int8_block_kernel<<<dim3(n_rows, kv->num_kv_heads), 256, 0, s>>>(a);
    } else if (a.D % 8 == 0 && a.dst != GG_DTYPE_INT8 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0) {
        const bool per_dim = src != GG_DTYPE_F32 && a.dst != GG_DTYPE_F32;
        switch (src) {
            case GG_DTYPE_F32: launch_vec<GG_DTYPE_F32>(a, a.dst, s); break;
            case GG_DTYPE_F16:
                if (per_dim) launch_dim<GG_DTYPE_F16>(a, a.dst, s);
                else launch_vec<GG_DTYPE_F16>(a, a.dst, s);
                break;
            default:
                if (per_dim) launch_dim<GG_DTYPE_BF16>(a, a.dst, s);
                else launch_vec<GG_DTYPE_BF16>(a, a.dst, s);
                break;
        }
    } else {
        append_direct_kernel<<<n_rows, 256, 0, s>>>(a);
    }
    return check_hip(hipGetLastError(), "kv_append launch");
}

}  // namespace gg
