// kv_swap.hip — KV snapshot / restore of a set of blocks across every layer.
//
// Replaces SnapshotKV / RestoreKV of the CUDA runner (internal/backend/cuda/
// swap_bridge.go:53-153), which copies 2 x num_layers block slices per block with
// synchronous cudaMemcpy calls. Here one launch gathers every (block, layer) record into
// a contiguous device staging buffer (or scatters it back) and, when a host buffer is
// given, one hipMemcpyAsync moves the whole snapshot on the caller's stream.
//
// A (block, layer) record is the block's tiles of that layer — for every kv head its K
// tile then its V tile, already adjacent in the pool — followed, for PER_BLOCK INT8
// pools, by the block's fp16 K and V scales of that layer (2 * Hkv values), the record
// padded to 16 bytes. Records are ordered [block i][layer]. PER_HEAD scales belong to the
// layer, not to a block, and stay with the pool.
#include "gg_common.h"

namespace gg {
namespace {

struct SwapArgs {
    uint8_t* pool;          // the KV allocation (layer 0, block 0, head 0, K tile)
    uint16_t* k_bscale;     // PER_BLOCK scales (layer 0) or NULL
    uint16_t* v_bscale;
    const int32_t* ids;
    int n, layers, num_blocks, Hkv;
    size_t tiles_bytes;     // Hkv * 2 * tile: one block's tiles of one layer
    size_t layer_stride;    // bytes between layers in the pool
    size_t scale_layer;     // scales per layer (blocks * Hkv)
    size_t record;          // bytes of one (block, layer) record
    uint8_t* staging;
};

// Workgroup (i, layer): copies one record. RESTORE scatters staging -> pool, else gathers.
template <bool RESTORE>
__global__ void __launch_bounds__(256) swap_kernel(SwapArgs a) {
    const int i = blockIdx.x, layer = blockIdx.y;
    const int blk = a.ids[i];
    uint8_t* rec = a.staging + ((size_t)i * a.layers + layer) * a.record;
    const bool ok = blk >= 0 && blk < a.num_blocks;
    uint8_t* tiles = a.pool + (size_t)layer * a.layer_stride + (size_t)(ok ? blk : 0) * a.tiles_bytes;
    if (a.tiles_bytes % 16 == 0) {  // (every tile size with head_dim * block_size * bytes % 16 == 0)
        const size_t n16 = a.tiles_bytes / 16;
        for (size_t k = threadIdx.x; k < n16; k += blockDim.x) {
            if (RESTORE) {
                if (ok) ((uint4*)tiles)[k] = ((const uint4*)rec)[k];
            } else {
                ((uint4*)rec)[k] = ok ? ((const uint4*)tiles)[k] : make_uint4(0, 0, 0, 0);
            }
        }
    } else {
        for (size_t k = threadIdx.x; k < a.tiles_bytes; k += blockDim.x) {
            if (RESTORE) {
                if (ok) tiles[k] = rec[k];
            } else {
                rec[k] = ok ? tiles[k] : (uint8_t)0;
            }
        }
    }
    if (a.k_bscale) {
        uint16_t* rs = (uint16_t*)(rec + a.tiles_bytes);
        const size_t base = (size_t)layer * a.scale_layer + (size_t)(ok ? blk : 0) * a.Hkv;
        for (int h = threadIdx.x; h < a.Hkv; h += blockDim.x) {
            if (RESTORE) {
                if (ok) {
                    a.k_bscale[base + h] = rs[h];
                    a.v_bscale[base + h] = rs[a.Hkv + h];
                }
            } else {
                rs[h] = ok ? a.k_bscale[base + h] : (uint16_t)0;
                rs[a.Hkv + h] = ok ? a.v_bscale[base + h] : (uint16_t)0;
            }
        }
    }
}

SwapArgs swap_args(KV* kv, const int32_t* ids, int n, void* staging) {
    SwapArgs a{};
    a.pool = kv->k_pool;
    if (kv->scale_mode == GG_SCALE_PER_BLOCK) {
        a.k_bscale = (uint16_t*)kv->k_scales;
        a.v_bscale = (uint16_t*)kv->v_scales;
    }
    a.ids = ids;
    a.n = n;
    a.layers = kv->num_layers;
    a.num_blocks = kv->num_blocks;
    a.Hkv = kv->num_kv_heads;
    a.tiles_bytes = (size_t)kv->num_kv_heads * 2 * kv->tile_bytes;
    a.layer_stride = kv->layer_stride;
    a.scale_layer = kv->scale_layer_elems;
    a.record = kv_swap_record_bytes(kv);
    a.staging = (uint8_t*)staging;
    return a;
}

}  // namespace

size_t kv_swap_record_bytes(const KV* kv) {
    size_t r = (size_t)kv->num_kv_heads * 2 * kv->tile_bytes;
    if (kv->scale_mode == GG_SCALE_PER_BLOCK) r += (size_t)kv->num_kv_heads * 2 * sizeof(uint16_t);
    return (r + 15) / 16 * 16;
}

gg_status_t launch_kv_snapshot(KV* kv, const int32_t* ids, int n, void* staging, void* host_dst, hipStream_t s) {
    const SwapArgs a = swap_args(kv, ids, n, staging);
    swap_kernel<false><<<dim3(n, kv->num_layers), 256, 0, s>>>(a);
    gg_status_t st = check_hip(hipGetLastError(), "kv_snapshot launch");
    if (st == GG_OK && host_dst)
        st = check_hip(hipMemcpyAsync(host_dst, staging, (size_t)n * kv->num_layers * a.record, hipMemcpyDeviceToHost, s),
                       "kv_snapshot copy");
    return st;
}

gg_status_t launch_kv_restore(KV* kv, const int32_t* ids, int n, void* staging, const void* host_src,
                              hipStream_t s) {
    const SwapArgs a = swap_args(kv, ids, n, staging);
    if (host_src) {
        const gg_status_t st = check_hip(hipMemcpyAsync(staging, host_src, (size_t)n * kv->num_layers * a.record,
                                                        hipMemcpyHostToDevice, s),
                                         "kv_restore copy");
        if (st != GG_OK) return st;
    }
    swap_kernel<true><<<dim3(n, kv->num_layers), 256, 0, s>>>(a);
    return check_hip(hipGetLastError(), "kv_restore launch");
}

}  // namespace gg
