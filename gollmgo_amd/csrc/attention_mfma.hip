// attention_mfma.hip — gfx950 MFMA phase-1 kernel of the verify attention.
//
// One 256-thread workgroup per (sequence, kv head, partition). Its G*R query rows
// (G query heads of the kv head x R verify rows, row r = j*G + g) form NT tiles of
// 16 rows; K/V of each 64-token chunk (four 16-token blocks) are read ONCE with
// 16-byte loads and shared by every row — the GQA x draft reuse that turns
// a bandwidth-bound decode into MFMA-friendly tiles. The four waves stream
// disjoint chunks and merge their (max, sum, P.V) states through LDS at the end.
//
// Per chunk (64 tokens for 1-byte pools, 32 for 2-byte pools) and row tile, lane = 16*g4 + c:
//   S^T = K . Q^T   v_mfma_f32_16x16x32_{bf16,f16}: A = K (16 tokens x 32 dims),
//                   B = Q^T. Token m = 4q+i of tile s is (block q, offset 4s+i), so
//                   the output gives lane (g4, c) row c and block g4's offsets 4s..4s+3.
//   P = softmax     online, per row, base-2 exponent; row max via the row-swap permutes.
//   O += P . V      A = P (row c, k = 8*g4+i -> block g4 offset 8*pv+i),
//                   B = V from the dim-major V block: one 16-byte load gives a lane
//                   all 16 offsets of one dim.
// Head dims are permuted consistently in K and Q (lane group g4 owns dims
// 32*g4..32*g4+31), so every K load is a contiguous 32- or 64-byte run.
//
// Pool types: BF16 (bf16 MFMA; P split into bf16 hi+lo for two MFMAs so the
// probabilities keep ~16 bits), F16 (f16 MFMA), FP8-E4M3 and INT8 (decoded in
// registers to exact f16 values: E4M3 by the gfx950 pk_f16_fp8 conversion, int8
// via the 0x6400 magic; the per-head / per-block scales are applied to the fp32
// scores and to P, never to the operands).
#include "gg_common.h"
#include "attention_common.h"

#include <algorithm>
#include <type_traits>

namespace gg {
#ifdef GG_TRACE
// Debug builds (-DGG_TRACE) only: the LPT kernel's per-workgroup timeline in wall-clock
// ticks (100 MHz): [4p] start, [4p+1] end, [4p+2] CU id (__smid) | 1 << 32 | XCC << 40 |
// keys << 44, [4p+3] when wave 0's first chunk had arrived. gg_debug_trace_ptr gives its device address.
__device__ long long g_trace[65536 * 4];
#endif
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef unsigned __int128 u128;

constexpr int kD = 128;
constexpr int kBS = 16;
constexpr int kChunk = 64;
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <gg_dtype_t DT>
struct PoolTraits;
template <>
struct PoolTraits<GG_DTYPE_BF16> {
    static constexpr int kEB = 2;
    static constexpr bool kBf16 = true;
};
template <>
struct PoolTraits<GG_DTYPE_F16> {
    static constexpr int kEB = 2;
    static constexpr bool kBf16 = false;
};
template <>
struct PoolTraits<GG_DTYPE_FP8_E4M3> {
    static constexpr int kEB = 1;
    static constexpr bool kBf16 = false;
};
template <>
struct PoolTraits<GG_DTYPE_INT8> {
    static constexpr int kEB = 1;
    static constexpr bool kBf16 = false;
};

__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c, bool bf16) {
    if (bf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Four E4M3 bytes -> four f16 (exact: every E4M3 value, subnormals included, is an
// f16 value), two hardware conversions (v_cvt_scalef32_pk_f16_fp8, scale 1).
__device__ __forceinline__ uint2 e4m3x4_to_f16x4(uint32_t w) {
    const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
    const f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true);
    return make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
}
// Four int8 -> four f16 (exact): (0x6400 | (b ^ 0x80)) is 1024 + b + 128. Each half is
// one byte permute of (0x64646464 : w), bytes (b, 0x64, b', 0x64): five instructions per
// four bytes with the sign flip and the two subtractions (shift-and-mask takes ten).
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t w) {
    w ^= 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    f16x2 a = __builtin_bit_cast(f16x2, lo) - bias;
    f16x2 b = __builtin_bit_cast(f16x2, hi) - bias;
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}
// Eight 1-byte elements (two dwords) -> one 16-byte MFMA operand of f16.
template <gg_dtype_t DT>
__device__ __forceinline__ uint4 bytes8_to_f16x8(uint32_t w0, uint32_t w1) {
    uint2 a, b;
    if constexpr (DT == GG_DTYPE_FP8_E4M3) {
        a = e4m3x4_to_f16x4(w0);
        b = e4m3x4_to_f16x4(w1);
    } else {
        a = i8x4_to_f16x4(w0);
        b = i8x4_to_f16x4(w1);
    }
    return make_uint4(a.x, a.y, b.x, b.y);
}

// Hardware round-to-nearest-even pair conversions (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32)
// for probabilities, which are finite and non-negative.
__device__ __forceinline__ uint32_t cvt_pk_f16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// Max over lanes l, l^16, l^32, l^48 (the four 16-lane rows of the wave) with the gfx950
// row-swap permutes, which stay in the VALU instead of going through the LDS crossbar.
__device__ __forceinline__ float max_over_rows(float v) {
    const uint32_t u = __float_as_uint(v);
    const auto h = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    const uint32_t w = __float_as_uint(v);
    const auto r = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Zero the 1-byte elements at offsets >= nvalid of a 16-offset run.
__device__ __forceinline__ uint4 mask_bytes16(uint4 v, int nvalid) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int lo = 4 * k;
        uint32_t m;
        if (nvalid >= lo + 4) m = 0xFFFFFFFFu;
        else if (nvalid <= lo) m = 0u;
        else m = 0xFFFFFFFFu >> (8 * (lo + 4 - nvalid));
        w[k] &= m;
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}
// Zero the 2-byte elements at offsets >= nvalid of an 8-offset run starting at `first`.
// Bytes of an 8-byte run that starts at offset `first`: offsets >= nvalid cleared.
__device__ __forceinline__ uint2 mask_bytes8(uint2 v, int nvalid, int first) {
    const int n = nvalid - first;
    const uint32_t m0 = n >= 4 ? 0xFFFFFFFFu : (n <= 0 ? 0u : 0xFFFFFFFFu >> (8 * (4 - n)));
    const uint32_t m1 = n >= 8 ? 0xFFFFFFFFu : (n <= 4 ? 0u : 0xFFFFFFFFu >> (8 * (8 - n)));
    return make_uint2(v.x & m0, v.y & m1);
}
__device__ __forceinline__ uint4 mask_halves8(uint4 v, int nvalid, int first) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int o0 = first + 2 * k;
        uint32_t m = (o0 < nvalid ? 0x0000FFFFu : 0u) | (o0 + 1 < nvalid ? 0xFFFF0000u : 0u);
        w[k] &= m;
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Chunk geometry. A chunk is kTok consecutive tokens (kTok/16 blocks). 1-byte pools use
// 64-token chunks, 2-byte pools 32-token chunks, so that in both cases a lane moves
// 256 bytes per chunk: K rows of kTok/16 tiles (32 dims each) and one 16-byte run
// of V offsets for each of the eight dim tiles.
//
// S tile s, M index m = 4q + i (q = m/4) holds token (block bq(q), offset ob(q) + 4s + i):
//   64-token chunks: bq(q) = q,    ob(q) = 0       (tiles s = 0..3)
//   32-token chunks: bq(q) = q/2,  ob(q) = 8*(q%2) (tiles s = 0..1)
// The MFMA output gives lane (g4, c16) row c16 and tokens (bq(g4), ob(g4) + 4s + i), so the
// lane's P values are the consecutive offsets ob(g4) .. ob(g4) + 4*NS - 1 of one block,
// which is exactly the A operand of P.V (k = 8*g4 + i' -> offset ob(g4) + 8*pv + i') and
// one contiguous run of the dim-major V block.
template <int kEB, int TOK>
struct Geo {
    static constexpr int kTok = TOK;
    static constexpr int kNS = kTok / 16;                 // S tiles (and blocks) per chunk
    static constexpr int kNPV = kNS / 2;                  // P.V MFMAs per dim tile
    static constexpr int kKVec = 32 * kEB / 16;           // 16-byte loads per lane per K tile
    static constexpr int kVBytes = 8 * kNPV * kEB;        // V bytes per lane per dim tile (16, or 8)
    using VReg = std::conditional_t<kVBytes == 16, uint4, uint2>;
    __device__ static __forceinline__ int bq(int q) { return kTok == 64 ? q : (q >> 1); }
    __device__ static __forceinline__ int ob(int q) { return kTok == 64 ? 0 : 8 * (q & 1); }
};

template <int kEB, int TOK>
struct ChunkRegs {
    using G = Geo<kEB, TOK>;
    uint4 k[G::kNS][G::kKVec];
    typename G::VReg v[8];
    float ksc, vsc;  // INT8 pools: scales of the lane's V block, fetched with its V
};

// Block ids of one chunk as this lane uses them: k = the block of its K rows, v = the
// block of its V columns and P run (-1: no block: past the keys, past the piece, or an
// out-of-range table entry). The chunk's kNS ids are read with wave-uniform (scalar)
// loads, so waiting for them never waits on the vector loads of K/V in flight, and are
// narrowed to the lane's two right there, from registers: a later lane-dependent pick
// from a stored array would be folded into an indexed load and spill.
struct LaneBlocks {
    int k, v;
};

// What a piece needs to start streaming: its first chunk's K/V in flight and the block
// ids of its first two chunks (PieceIO::start).
template <gg_dtype_t DT, int TOK>
struct PieceIn {
    ChunkRegs<PoolTraits<DT>::kEB, TOK> cur;
    LaneBlocks bl_cur, bl_next;
};

// A piece: tokens [t0, t_end) of sequence b against kv head kvh, written to partition
// slot `part` / record `rec` (both < 0: the output). Wave-uniform.
struct PieceDesc {
    int b, kvh, t0, t_end, part, rec;
};

template <gg_dtype_t DT, int TOK>
struct PieceIO {
    static constexpr int kEB = PoolTraits<DT>::kEB;
    using Geom = Geo<kEB, TOK>;
    static constexpr int kNS = Geom::kNS;
    static constexpr int kTok = Geom::kTok;

    // Block ids of chunk `ch` of the piece [t0, t_end), in two steps: fetch_blocks issues
    // the kNS table reads together (wave-uniform scalar loads; indices are clamped to the
    // row, so they wait for neither the piece bounds nor the context length), and
    // lane_blocks, called as late as possible, applies the bounds and narrows the ids
    // to the lane's two.
    struct RawBlocks {
        int q[kNS];
        int t;  // first token of the chunk
    };
    __device__ static __forceinline__ RawBlocks fetch_blocks(const AttnArgs& a, int b, int t0, int ch) {
        const int32_t* bt = a.block_tables + (size_t)b * a.max_blocks;
        RawBlocks r;
        r.t = t0 + ch * kTok;
#pragma unroll
        for (int qb = 0; qb < kNS; ++qb) r.q[qb] = bt[min((r.t >> 4) + qb, a.max_blocks - 1)];
        return r;
    }
    __device__ static __forceinline__ LaneBlocks lane_blocks(const KVView& kv, const RawBlocks& r, int t_end) {
        int q[kNS];
#pragma unroll
        for (int qb = 0; qb < kNS; ++qb) {
            const int blk = r.q[qb];
            q[qb] = (r.t + 16 * qb < t_end && blk < kv.num_blocks) ? blk : -1;
        }
        const int lane = threadIdx.x & 63, c16 = lane & 15, g4 = lane >> 4;
        const int ik = Geom::bq(c16 >> 2), iv = Geom::bq(g4);
        LaneBlocks l{q[0], q[0]};
#pragma unroll
        for (int qb = 1; qb < kNS; ++qb) {
            l.k = ik == qb ? q[qb] : l.k;
            l.v = iv == qb ? q[qb] : l.v;
        }
        return l;
    }
    __device__ static __forceinline__ LaneBlocks chunk_blocks(const AttnArgs& a, const KVView& kv, int b, int t0,
                                                              int t_end, int ch) {
        return lane_blocks(kv, fetch_blocks(a, b, t0, ch), t_end);
    }
    // K rows: lane supplies M index c16 of every tile. Loads are unconditional (missing
    // blocks read block 0); such tokens are always masked in S.
    __device__ static __forceinline__ void load_k(const KVView& kv, const LaneBlocks bl, int kvh,
                                                  ChunkRegs<kEB, TOK>& rg) {
        const int lane = threadIdx.x & 63, c16 = lane & 15, g4 = lane >> 4, kq = c16 >> 2;
        const int blk = bl.k;
        const uint8_t* base =
            kv.kc + (((size_t)(blk < 0 ? 0 : blk) * kv.Hkv + kvh) * (size_t)(2 * kBS * kD) + 32 * g4) * kEB;
#pragma unroll
        for (int s = 0; s < kNS; ++s) {
            const int off = Geom::ob(kq) + 4 * s + (c16 & 3);
#pragma unroll
            for (int v = 0; v < Geom::kKVec; ++v) rg.k[s][v] = *(const uint4*)(base + (size_t)off * kD * kEB + 16 * v);
        }
    }
    // V: lane owns block bq(g4), dim dt*16 + c16, offsets ob(g4) .. ob(g4)+16/kEB-1 (zeroed
    // later when the block is missing or partly past the keys).
    __device__ static __forceinline__ void load_v(const KVView& kv, const LaneBlocks bl, int kvh,
                                                  ChunkRegs<kEB, TOK>& rg) {
        const int lane = threadIdx.x & 63, c16 = lane & 15, g4 = lane >> 4;
        const int blk = bl.v;
        if constexpr (DT == GG_DTYPE_INT8) {
            // Scales first: the softmax that needs them then waits for nothing behind them.
            const size_t si = (size_t)(blk < 0 ? 0 : blk) * kv.Hkv + kvh;
            rg.ksc = f16_bits_to_f32(kv.k_blk_scale[si]);
            rg.vsc = f16_bits_to_f32(kv.v_blk_scale[si]);
        }
        const uint8_t* base =
            kv.vc + (((size_t)(blk < 0 ? 0 : blk) * kv.Hkv + kvh) * (size_t)(2 * kBS * kD) + Geom::ob(g4)) * kEB;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const int d = dt * 16 + c16;
            rg.v[dt] = *(const typename Geom::VReg*)(base + (size_t)d * kBS * kEB);
        }
    }
    // Issue the first chunk of piece d (this wave's first chunk is chunk `wave`): the block
    // ids of its first two chunks, then the first chunk's K rows and V columns.
    __device__ static __forceinline__ void start(const AttnArgs& a, const KVView& kv, const PieceDesc& d,
                                                 PieceIn<DT, TOK>& in) {
        const int wave_u = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        in.bl_cur = chunk_blocks(a, kv, d.b, d.t0, d.t_end, wave_u);
        in.bl_next = chunk_blocks(a, kv, d.b, d.t0, d.t_end, wave_u + kWaves);
        load_k(kv, in.bl_cur, d.kvh, in.cur);
        load_v(kv, in.bl_cur, d.kvh, in.cur);
    }
};

// Draft rows a piece appends itself (gg_verify_append_attention_planned on the MFMA path):
// rows [j0, j1) of its sequence (none when j0 == j1), and this thread's work item of them.
struct DeferredRows {
    AppendItem it;
    int j0, j1;
};
// Most work items (rows x 16 dim groups) a piece stages in LDS: 8 draft rows.
constexpr int kAppMax = 128;

// Start piece d (PieceIO::start) and, when the call carries draft rows (a.k_new), take
// care of the rows whose key positions lie in the piece. A key position belongs to exactly
// one piece, and only that piece reads it, so no other workgroup waits for these stores;
// chunks are multiples of 16 tokens, so a block's tokens (its K rows and its V columns)
// are all read by one chunk, and so by one wave.
//   - Rows inside the first chunks that `start` issues (short pieces), more rows than
//     kAppMax, no `ap` (the stream-K loop over pieces, whose registers are full), or a
//     PER_BLOCK INT8 pool (a block's new rows re-scale the whole block; a block lies in one
//     piece, since pieces are whole chunks): appended here by the whole workgroup, then a
//     barrier orders the stores before the piece's loads (within a workgroup a barrier
//     orders global stores before loads: same CU, write-through L1; for INT8, with
//     workgroup-scope release and acquire fences around it).
//   - Otherwise (the usual case: the rows are the item's last positions) their loads are
//     issued here, after `start`, one work item per thread. attn_piece converts them into
//     LDS before its Q-staging barrier; the wave that reads the chunk holding them patches
//     its registers from LDS (the pool still holds stale bytes there) and writes that
//     block's V tile back whole, and the K rows are stored after the loop. No load waits
//     behind these stores (gfx950 counts stores in vmcnt, so a store issued ahead of a
//     chunk's loads would hold up the wait for that chunk).
template <gg_dtype_t DT, int TOK>
__device__ __forceinline__ void start_piece(const AttnArgs& a, const KVView& kv, const PieceDesc& d,
                                            PieceIn<DT, TOK>& in, DeferredRows* ap) {
    constexpr int kTok = TOK;
    // The in-register patch of the chunk holding the rows needs 16-byte V runs.
    constexpr bool kDefer = DT != GG_DTYPE_INT8 && Geo<PoolTraits<DT>::kEB, TOK>::kVBytes == 16;
    if (ap) ap->j0 = ap->j1 = 0;
    if (a.k_new) {
        const int ctx = seq_keys(a, d.b, kBS), nrows = seq_rows(a, d.b);
        const int first = ctx - nrows;
        const int j0 = max(0, d.t0 - first), j1 = min(nrows, d.t_end - first);
        if (nrows > 0 && nrows <= ctx && j0 < j1) {
            const int items = (j1 - j0) * (kD / 8);
            if (kDefer && ap && items <= kAppMax && first + j0 >= d.t0 + kWaves * kTok) {
                PieceIO<DT, TOK>::start(a, kv, d, in);
                ap->j0 = j0;
                ap->j1 = j1;
                ap->it.live = false;
                if ((int)threadIdx.x < items) ap->it = append_load(a, kv, d.b, d.kvh, ctx, nrows, j0, threadIdx.x);
            } else if (DT == GG_DTYPE_INT8) {
                // Re-quantised rows and the block scales are read back by other waves:
                // workgroup-scope release and acquire around the barrier. (Issuing the
                // piece's first chunks before the block update, when the rows lie past
                // them, was slower: 121.4 -> 130.7 µs per call at config 4. Loads retire
                // in order, so the update's small loads waited behind the chunks.)
                append_item_rows(a, kv, d.b, d.kvh, j0, j1);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __syncthreads();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                PieceIO<DT, TOK>::start(a, kv, d, in);
            } else {
                append_item_rows(a, kv, d.b, d.kvh, j0, j1);
                __syncthreads();
                PieceIO<DT, TOK>::start(a, kv, d, in);
            }
            return;
        }
    }
    PieceIO<DT, TOK>::start(a, kv, d, in);
}

// One piece of work: tokens [t0, t_end) of sequence b against kv head kvh. The result
// goes to the output (part < 0 && rec < 0), to partition slot `part` of the fixed
// partition grid, or to stream-K record `rec`. Must be reached by the whole workgroup.
//
// `in` holds the piece's first chunk, already issued (PieceIO::start).
// Partial records go through device-scope (agent) relaxed atomic stores and loads: they
// bypass the per-XCD caches' stale copies, so a workgroup on another XCD reads what was
// written. Ordering before the merge counter comes from waiting for the stores to
// complete (every record store of the workgroup) before the counter's atomic add.
__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <gg_dtype_t DT, int NT>
__device__ __forceinline__ void attn_piece(const AttnArgs& a, const KVView& kv, const PieceDesc pd,
                                           PieceIn<DT, attn_chunk_tokens(PoolTraits<DT>::kEB, NT)>& in,
                                           const DeferredRows* ap) {
    const int b = pd.b, kvh = pd.kvh, t0 = pd.t0, t_end = pd.t_end, part = pd.part, rec = pd.rec;
    using T = PoolTraits<DT>;
    constexpr bool kIsBf16 = T::kBf16;
    constexpr int kEB = T::kEB;
    constexpr int TOK = attn_chunk_tokens(kEB, NT);
    using Geom = Geo<kEB, TOK>;
    using Regs = ChunkRegs<kEB, TOK>;
    constexpr int kTok = Geom::kTok;
    constexpr int kNS = Geom::kNS;

    const int ctx = seq_keys(a, b, kBS);
    const int R = a.rows;
    const int nrows = seq_rows(a, b);
    if (nrows <= 0 || nrows > ctx) return;
    const int Hq = a.num_q_heads;
    const int G = Hq / kv.Hkv;
    const int nvalid_rows = G * nrows;
    const bool final_out = part < 0 && rec < 0;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;
    const int g4 = lane >> 4;

    const int nchunks = (t_end - t0 + kTok - 1) / kTok;
    const int first_masked = ctx - nrows;  // tokens >= this are causally masked for some row

    // Score multiplier (log2 domain) and P.V multiplier per pool type.
    float sscale = a.scale * kLog2e;
    float vfold = 1.f;
    if constexpr (DT == GG_DTYPE_FP8_E4M3) {
        sscale *= kv.k_head_scale[kvh];
        vfold = kv.v_head_scale[kvh];
    }

    // Draft rows loaded by start_piece: converted into LDS here (the Q-staging barrier
    // below publishes them). The chunk that holds them reads stale pool bytes at their
    // positions; the wave that owns that chunk patches its registers from LDS (see the
    // loop), and the rows go to the pool after the loop, where nothing waits for the
    // stores (on gfx950 stores count in vmcnt, so a store ahead of a chunk's loads would
    // hold up the wait for that chunk). s_app keeps each work item (row, 8 dims) in the
    // pool's format; s_vt the same V values by dim: element r of s_vt[d] is row r's V[d].
    __shared__ AppendBytes s_app[kAppMax];
    __shared__ uint4 s_vt[kD];
    int app_lo = 0, app_hi = 0;  // their key positions [app_lo, app_hi)
    if constexpr (DT != GG_DTYPE_INT8) {
        if (ap) {
            const int j0 = __builtin_amdgcn_readfirstlane(ap->j0), j1 = __builtin_amdgcn_readfirstlane(ap->j1);
            if (j0 < j1) {
                const int i = threadIdx.x;
                if (i < (j1 - j0) * (kD / 8)) {
                    const AppendBytes o = append_encode(a, kv, ap->it);
                    s_app[i] = o;
                    const int r = i / (kD / 8), d0 = (i % (kD / 8)) * 8;
                    if constexpr (kEB == 1) {
                        const uint32_t u[2] = {o.v[0].x, o.v[0].y};
#pragma unroll
                        for (int e = 0; e < 8; ++e) ((uint8_t*)&s_vt[d0 + e])[r] = (uint8_t)(u[e >> 2] >> (8 * (e & 3)));
                    } else {
                        const uint32_t u[4] = {o.v[0].x, o.v[0].y, o.v[0].z, o.v[0].w};
#pragma unroll
                        for (int e = 0; e < 8; ++e) ((uint16_t*)&s_vt[d0 + e])[r] = (uint16_t)(u[e >> 1] >> (16 * (e & 1)));
                    }
                }
                app_lo = first_masked + j0;
                app_hi = first_masked + j1;
            }
        }
    }

    // ---- Q operands: B[k = 8*g4+i][n = c16] <- Q[row rt*16+c16][32*g4 + 8*mm + i] ----
    // Staged once per piece in LDS (wave w converts dim group mm = w for every row tile)
    // and read back per chunk one mm at a time, so only NT operands are live in the loop.
    // Loads are issued unconditionally (invalid rows read row 0 and are zeroed).
    // BF16 pools take Q as bf16 hi + lo (two S MFMAs) unless Q already is bf16, so f32
    // and f16 queries keep ~16 bits instead of bf16's 8.
    __shared__ uint4 s_q[NT][4][64];                   // [rt][mm][lane]
    __shared__ uint4 s_qlo[kIsBf16 ? NT : 1][4][64];  // low parts (BF16 pools)
    const bool qsplit = kIsBf16 && a.q_dtype != GG_DTYPE_BF16;
    int row_pos[NT];  // last visible key position of the lane's S row (c16)
    {
        const int mm = wave;
        size_t qb[NT];
        bool qvalid[NT];
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            const int r = rt * 16 + c16;
            qvalid[rt] = r < nvalid_rows;
            const int j = qvalid[rt] ? r / G : 0;
            const int g = qvalid[rt] ? r % G : 0;
            row_pos[rt] = qvalid[rt] ? first_masked + j : ctx - 1;
            qb[rt] = (((size_t)b * R + j) * Hq + (size_t)kvh * G + g) * kD + 32 * g4 + 8 * mm;
        }
        // One uniform dtype branch around all row tiles, so their loads issue together.
        uint4 op[NT];
        // Eight values -> MFMA operand (and, for a split, the operand of the remainder).
        auto pack8 = [&](const float* f, uint4& hi, uint4& lo) {
            if constexpr (kIsBf16) {
                uint32_t h[4], l[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    h[k] = pack_bf16x2(f[2 * k], f[2 * k + 1]);
                    l[k] = pack_bf16x2(f[2 * k] - __uint_as_float(h[k] << 16),
                                       f[2 * k + 1] - __uint_as_float(h[k] & 0xffff0000u));
                }
                hi = make_uint4(h[0], h[1], h[2], h[3]);
                lo = make_uint4(l[0], l[1], l[2], l[3]);
            } else {
                hi = make_uint4(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]), pack_f16x2(f[4], f[5]),
                                pack_f16x2(f[6], f[7]));
                lo = zero4();
            }
        };
        uint4 opl[NT];
        // f16 operands (FP8 / INT8 / F16 pools) hold |q| < 65504. A bf16 or f32 query beyond
        // 2^15 is scaled by 2^-k for the piece (k from the rows' largest |q|) and the score
        // multiplier by 2^k: power-of-two scalings are exact, so in range nothing changes.
        constexpr bool kF16Op = !kIsBf16;
        __shared__ float s_qmax[4];
        auto piece_q_shift = [&](float local_max) -> int {
            for (int o = 32; o > 0; o >>= 1) local_max = fmaxf(local_max, __shfl_xor(local_max, o));
            if (lane == 0) s_qmax[wave] = local_max;
            __syncthreads();
            const float mx = fmaxf(fmaxf(s_qmax[0], s_qmax[1]), fmaxf(s_qmax[2], s_qmax[3]));
            int e = 0;
            (void)frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
            return (mx == mx && mx <= 3.402823466e38f && e > 15) ? e - 15 : 0;
        };
        if (a.q_dtype == GG_DTYPE_F32) {
            float4 raw[NT][2];
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                for (int h = 0; h < 2; ++h) raw[rt][h] = ((const float4*)((const float*)a.q + qb[rt]))[h];
            float qs = 1.f;
            if constexpr (kF16Op) {
                float lm = 0.f;
#pragma unroll
                for (int rt = 0; rt < NT; ++rt)
                    if (qvalid[rt])
#pragma unroll
                        for (int h = 0; h < 2; ++h)
                            lm = fmaxf(lm, fmaxf(fmaxf(fabsf(raw[rt][h].x), fabsf(raw[rt][h].y)),
                                                 fmaxf(fabsf(raw[rt][h].z), fabsf(raw[rt][h].w))));
                const int k = piece_q_shift(lm);
                qs = ldexpf(1.f, -k);
                sscale = ldexpf(sscale, k);
            }
#pragma unroll
            for (int rt = 0; rt < NT; ++rt) {
                const float f[8] = {raw[rt][0].x * qs, raw[rt][0].y * qs, raw[rt][0].z * qs, raw[rt][0].w * qs,
                                    raw[rt][1].x * qs, raw[rt][1].y * qs, raw[rt][1].z * qs, raw[rt][1].w * qs};
                pack8(f, op[rt], opl[rt]);
            }
        } else {
            const bool src_bf16 = a.q_dtype == GG_DTYPE_BF16;
#pragma unroll
            for (int rt = 0; rt < NT; ++rt) {
                op[rt] = *(const uint4*)((const uint16_t*)a.q + qb[rt]);
                opl[rt] = zero4();
            }
            // Convert when the Q type differs from the MFMA operand type.
            if (src_bf16 != kIsBf16) {
                float f[NT][8];
                float lm = 0.f;
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) {
                    const uint32_t w[4] = {op[rt].x, op[rt].y, op[rt].z, op[rt].w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint16_t lo = (uint16_t)w[k], hi = (uint16_t)(w[k] >> 16);
                        f[rt][2 * k] = src_bf16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
                        f[rt][2 * k + 1] = src_bf16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
                    }
                    if (qvalid[rt])
#pragma unroll
                        for (int k = 0; k < 8; ++k) lm = fmaxf(lm, fabsf(f[rt][k]));
                }
                if constexpr (kF16Op) {
                    const int k = piece_q_shift(lm);
                    if (k > 0) {
                        const float qs = ldexpf(1.f, -k);
#pragma unroll
                        for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                            for (int e = 0; e < 8; ++e) f[rt][e] *= qs;
                        sscale = ldexpf(sscale, k);
                    }
                }
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) pack8(f[rt], op[rt], opl[rt]);
            }
        }
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            s_q[rt][mm][lane] = qvalid[rt] ? op[rt] : zero4();
            if constexpr (kIsBf16) s_qlo[rt][mm][lane] = qvalid[rt] ? opl[rt] : zero4();
        }
        __syncthreads();
    }

    f32x4 o[NT][8];
    float m_run[NT], l_run[NT];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
        m_run[rt] = -1e30f;
        l_run[rt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    using IO = PieceIO<DT, TOK>;

    Regs& cur = in.cur;
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // Block ids run two chunks ahead and are requested after the softmax: the LDS
    // reads of Q at the top of the next chunk wait on every outstanding scalar load,
    // and by then these have had the whole P.V stage to arrive.
    LaneBlocks& bl_cur = in.bl_cur;
    LaneBlocks& bl_next = in.bl_next;

    for (int ch = wave_u; ch < nchunks; ch += kWaves) {
        const int blk_v = bl_cur.v;
        const int tc = t0 + ch * kTok;
        const int tlane = tc + 16 * Geom::bq(g4) + Geom::ob(g4);  // first token of the lane's P run
        // Valid offsets of the lane's V block (offsets counted from the block start).
        const int nvalid_v = blk_v < 0 ? 0 : ctx - (tc + 16 * Geom::bq(g4));

        // (A missing block reads block 0's scales; its tokens are masked either way.) A K
        // scale of 0 (a block never written, or one whose rows are all zero, so every K
        // byte is 0) is taken as 1: the scores it scales are 0 either way, and masked
        // scores must stay -inf rather than become -inf * 0 = NaN.
        const float kblk_scale = DT == GG_DTYPE_INT8 ? (cur.ksc > 0.f ? cur.ksc : 1.f) : 1.f;
        const float vblk_scale = DT == GG_DTYPE_INT8 ? cur.vsc : 1.f;

        // Draft rows in this chunk: their K rows replace the stale pool bytes just read.
        const bool app_here = DT != GG_DTYPE_INT8 && app_lo < app_hi && tc < app_hi && tc + kTok > app_lo;
        if constexpr (DT != GG_DTYPE_INT8) {
            if (app_here) {
                const int kq = c16 >> 2;
#pragma unroll
                for (int s = 0; s < kNS; ++s) {
                    const int r = tc + 16 * Geom::bq(kq) + Geom::ob(kq) + 4 * s + (c16 & 3) - app_lo;
                    if (r >= 0 && r < app_hi - app_lo) {
#pragma unroll
                        for (int v = 0; v < Geom::kKVec; ++v) {
                            if constexpr (kEB == 1) {
                                const int g = 4 * g4 + 2 * v;
                                const uint4 A = s_app[r * (kD / 8) + g].k[0], B = s_app[r * (kD / 8) + g + 1].k[0];
                                cur.k[s][v] = make_uint4(A.x, A.y, B.x, B.y);
                            } else {
                                cur.k[s][v] = s_app[r * (kD / 8) + 4 * g4 + v].k[0];
                            }
                        }
                    }
                }
            }
        }

        // ---- S^T = K . Q^T for kTok tokens x all row tiles; each K tile decoded once ----
        // The Q index is opaque to the optimiser so that the LDS reads stay in the loop
        // instead of being hoisted into registers for the whole piece.
        // (Non-volatile and without a memory clobber, the asm leaves the block-table
        // loads free to stay scalar; the chunk index input keeps it inside the loop.)
        int qlane;
        asm("" : "=v"(qlane) : "0"(lane), "s"(ch));
        f32x4 sacc[NT][kNS];
#pragma unroll
        for (int rt = 0; rt < NT; ++rt)
#pragma unroll
            for (int s = 0; s < kNS; ++s) sacc[rt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            uint4 qop[NT];
#pragma unroll
            for (int rt = 0; rt < NT; ++rt) qop[rt] = s_q[rt][mm][qlane];
#pragma unroll
            for (int s = 0; s < kNS; ++s) {
                uint4 kop;
                if constexpr (kEB == 2) {
                    kop = cur.k[s][mm];
                } else {
                    const uint4 r = cur.k[s][mm >> 1];
                    kop = (mm & 1) ? bytes8_to_f16x8<DT>(r.z, r.w) : bytes8_to_f16x8<DT>(r.x, r.y);
                }
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) sacc[rt][s] = mfma(kop, qop[rt], sacc[rt][s], kIsBf16);
            }
            if constexpr (kIsBf16) {
                if (qsplit) {
#pragma unroll
                    for (int rt = 0; rt < NT; ++rt) qop[rt] = s_qlo[rt][mm][qlane];
#pragma unroll
                    for (int s = 0; s < kNS; ++s)
#pragma unroll
                        for (int rt = 0; rt < NT; ++rt) sacc[rt][s] = mfma(cur.k[s][mm], qop[rt], sacc[rt][s], true);
                }
            }
        }
        // Next chunk's K rows stream in while this chunk finishes.
        IO::load_k(kv, bl_next, kvh, cur);
#ifdef GG_TRACE
        if (ch == wave_u && threadIdx.x == 0) g_trace[4 * blockIdx.x + 3] = wall_clock64();
#endif

        // ---- online softmax; P packed as MFMA A operands ----
        // Masked scores: causal (keys past the row's position, which covers keys past the
        // context) and every key of a missing block (its K was read from block 0). A
        // lane's scores all come from its V block, so a missing block masks whole lanes.
        const bool blk_missing = blk_v < 0;
        const bool need_mask = tc + kTok - 1 >= first_masked || __any(blk_missing);
        const float mult = DT == GG_DTYPE_INT8 ? sscale * kblk_scale : sscale;
        constexpr int kNP = 4 * kNS;  // P values per lane per row tile
        uint4 pop[NT][Geom::kNPV][kIsBf16 ? 2 : 1];
        // One wave-uniform branch around all the masking, so that chunks with nothing to
        // mask (most of them) skip it instead of running it as selects.
        if (__builtin_expect(need_mask, 0)) {
#pragma unroll
            for (int rt = 0; rt < NT; ++rt)
#pragma unroll
                for (int s = 0; s < kNS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        sacc[rt][s][i] = (!blk_missing && (tlane + 4 * s + i) <= row_pos[rt]) ? sacc[rt][s][i] : -INFINITY;
        }
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            // The multiplier is positive, so the scaled maximum is the maximum of the raw
            // scores times the lane's multiplier (rounding is monotonic); the scale then
            // folds into the exponent's FMA.
            float sc[kNP];
            float cmax = -INFINITY;
#pragma unroll
            for (int s = 0; s < kNS; ++s) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = sacc[rt][s][i];
                    sc[4 * s + i] = v;
                    cmax = fmaxf(cmax, v);
                }
            }
            cmax = max_over_rows(cmax * mult);
            const float m_new = fmaxf(m_run[rt], cmax);
            const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - m_new);
            m_run[rt] = m_new;
            float psum = 0.f;
#pragma unroll
            for (int k = 0; k < kNP; ++k) {
                sc[k] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[k], mult, -m_new));
                psum += sc[k];
            }
            l_run[rt] = l_run[rt] * alpha + psum;
            // Rescale O rows (4*g4 + i) by their rows' alpha; skipped by the whole wave
            // when no row max moved (the common case once the running max has settled).
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float al = __shfl(alpha, 4 * g4 + i);
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) o[rt][dt][i] *= al;
                }
            }
            if constexpr (DT == GG_DTYPE_INT8) {
#pragma unroll
                for (int k = 0; k < kNP; ++k) sc[k] *= vblk_scale;
            }
#pragma unroll
            for (int pv = 0; pv < Geom::kNPV; ++pv) {
                const float* pp = sc + 8 * pv;
                if constexpr (kIsBf16) {
                    // P = hi + lo, both bf16, so the probabilities keep ~16 bits.
                    uint32_t hw[4], lw[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        hw[k] = cvt_pk_bf16(pp[2 * k], pp[2 * k + 1]);
                        const float h0 = __uint_as_float(hw[k] << 16), h1 = __uint_as_float(hw[k] & 0xffff0000u);
                        lw[k] = cvt_pk_bf16(pp[2 * k] - h0, pp[2 * k + 1] - h1);
                    }
                    pop[rt][pv][0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                    pop[rt][pv][kIsBf16 ? 1 : 0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
                } else {
                    pop[rt][pv][0] = make_uint4(cvt_pk_f16(pp[0], pp[1]), cvt_pk_f16(pp[2], pp[3]),
                                                cvt_pk_f16(pp[4], pp[5]), cvt_pk_f16(pp[6], pp[7]));
                }
            }
        }

        const typename IO::RawBlocks raw_after = IO::fetch_blocks(a, b, t0, ch + 2 * kWaves);

        // ---- O += P . V; each V dim tile decoded once for all row tiles ----
        // Draft rows in this chunk: their V columns replace the stale pool bytes. The lane's
        // run is offsets ob(g4) .. of its block, rows base + offset of the staged rows.
        // Lanes whose block holds draft rows then write their runs back to the pool: the
        // runs of a block cover its whole dim-major V tile, so these are full-line stores
        // (the draft rows alone would be 1- or 2-byte pieces of every line, each a partial
        // write to memory); the other offsets are written back with the bytes just read.
        if constexpr (DT != GG_DTYPE_INT8 && Geom::kVBytes == 16) {
            if (app_here) {
                const int blk0 = tc + 16 * Geom::bq(g4) - app_lo;  // staged row of the block's offset 0
                const int base = blk0 + Geom::ob(g4);
                const int nr = app_hi - app_lo;
                constexpr int kE = 8 * kEB;  // bits per element
                constexpr int kRun = 16 / kEB;  // elements per 16-byte run
                if (base < nr && base + kRun > 0) {
                    // Element o of the run takes staged row base + o.
                    const int lo_bits = (nr - (base > 0 ? base : 0)) * kE;
                    u128 mask = lo_bits >= 128 ? ~(u128)0 : (((u128)1 << lo_bits) - 1);
                    if (base < 0) mask <<= (-base) * kE;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) {
                        const uint4 sv = s_vt[dt * 16 + c16];
                        u128 nv = ((u128)sv.w << 96) | ((u128)sv.z << 64) | ((u128)sv.y << 32) | sv.x;
                        if (kEB == 1) nv &= ((u128)1 << 64) - 1;  // 8 staged rows of one byte
                        nv = base < 0 ? nv << ((-base) * kE) : nv >> (base * kE);
                        const uint4 c = cur.v[dt];
                        u128 cv = ((u128)c.w << 96) | ((u128)c.z << 64) | ((u128)c.y << 32) | c.x;
                        cv = (cv & ~mask) | (nv & mask);
                        cur.v[dt] = make_uint4((uint32_t)cv, (uint32_t)(cv >> 32), (uint32_t)(cv >> 64),
                                               (uint32_t)(cv >> 96));
                    }
                }
                if (blk_v >= 0 && blk0 < nr && blk0 + kBS > 0) {
                    uint8_t* vbase = const_cast<uint8_t*>(kv.vc) +
                                     (((size_t)blk_v * kv.Hkv + kvh) * (size_t)(2 * kBS * kD) + Geom::ob(g4)) * kEB;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) *(uint4*)(vbase + (size_t)(dt * 16 + c16) * kBS * kEB) = cur.v[dt];
                }
            }
        }
        if (nvalid_v < kBS) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                if constexpr (kEB == 2) cur.v[dt] = mask_halves8(cur.v[dt], nvalid_v, Geom::ob(g4));
                else if constexpr (Geom::kVBytes == 16) cur.v[dt] = mask_bytes16(cur.v[dt], nvalid_v);
                else cur.v[dt] = mask_bytes8(cur.v[dt], nvalid_v, Geom::ob(g4));
            }
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
            for (int pv = 0; pv < Geom::kNPV; ++pv) {
                uint4 vop;
                if constexpr (kEB == 2) {
                    vop = cur.v[dt];
                } else if constexpr (Geom::kVBytes == 16) {
                    const uint4 r = cur.v[dt];
                    vop = pv ? bytes8_to_f16x8<DT>(r.z, r.w) : bytes8_to_f16x8<DT>(r.x, r.y);
                } else {
                    vop = bytes8_to_f16x8<DT>(cur.v[dt].x, cur.v[dt].y);
                }
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) {
                    o[rt][dt] = mfma(pop[rt][pv][0], vop, o[rt][dt], kIsBf16);
                    if constexpr (kIsBf16) o[rt][dt] = mfma(pop[rt][pv][1], vop, o[rt][dt], true);
                }
            }
        }
        // Next chunk's V columns.
        IO::load_v(kv, bl_next, kvh, cur);
        bl_cur = bl_next;
        bl_next = IO::lane_blocks(kv, raw_after, t_end);
    }

    // The draft rows' K to the pool (their V went back with the patched runs), now that no
    // load of this piece waits behind the stores.
    if constexpr (DT != GG_DTYPE_INT8) {
        if (app_lo < app_hi)
            for (int i = threadIdx.x; i < (app_hi - app_lo) * (kD / 8); i += blockDim.x) append_write_k(kv, s_app[i]);
    }

    // ---- merge the four waves' states through LDS ----
    __shared__ float s_m[kWaves][64];
    __shared__ float s_l[kWaves][64];
    __shared__ float s_o[kWaves][16][kD + 4];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
        float lt = l_run[rt];
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
        if (g4 == 0) {
            s_m[wave][rt * 16 + c16] = m_run[rt];
            s_l[wave][rt * 16 + c16] = lt;
        }
    }
    __syncthreads();

    const size_t zbase = (size_t)b * R;
    for (int rt = 0; rt < NT; ++rt) {
        // Each wave writes its O rows scaled to the common row max.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = 4 * g4 + i;
            const int r = rt * 16 + rr;
            float mx = s_m[0][r];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][r]);
            const float f = __builtin_amdgcn_exp2f(s_m[wave][r] - mx);
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) s_o[wave][rr][dt * 16 + c16] = o[rt][dt][i] * f;
        }
        __syncthreads();
        // 256 threads sum the 4 wave copies of 16 rows x 128 dims.
        for (int e = threadIdx.x; e < 16 * kD; e += 256) {
            const int rr = e / kD, d = e % kD;
            const int r = rt * 16 + rr;
            if (r >= nvalid_rows) continue;
            float mx = s_m[0][r];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][r]);
            float L = 0.f, acc = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                L += s_l[w][r] * __builtin_amdgcn_exp2f(s_m[w][r] - mx);
                acc += s_o[w][rr][d];
            }
            const int j = r / G, g = r % G;
            const size_t z = zbase + j;
            const int h = kvh * G + g;
            if (final_out) {
                const float val = L > 0.f ? acc * vfold / L : 0.f;
                store_from_f32(a.out, a.out_dtype, (z * Hq + h) * kD + d, val);
            } else {
                const size_t pidx = rec >= 0 ? (size_t)rec * (size_t)(G * R) + (size_t)r
                                             : (z * Hq + h) * a.max_parts + part;
                // Device-scope stores: they reach the point every XCD reads from, so the
                // last piece of an LPT item can merge the records in the same launch.
                store_agent(a.ws_acc + pidx * kD + d, acc * vfold);
                if (d == 0) {
                    store_agent(a.ws_ml + pidx * 2 + 0, mx > -1e29f ? mx * kLn2 : -1e30f);
                    store_agent(a.ws_ml + pidx * 2 + 1, L);
                }
            }
        }
        __syncthreads();
    }
}

// Fixed partition grid: workgroup (part, kvh, b) takes tokens [part*P, (part+1)*P).
template <gg_dtype_t DT, int NT>
__global__ void __launch_bounds__(256, attn_occupancy(PoolTraits<DT>::kEB, NT)) attn_mfma_kernel(AttnArgs a, KVView kv) {
    const int part = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int ctx = seq_keys(a, b, kBS);
    const int P = a.partition;
    const int nparts = (ctx + P - 1) / P;
    if (part >= nparts) return;
    const PieceDesc d{b, kvh, part * P, min(part * P + P, ctx), nparts == 1 ? -1 : part, -1};
    PieceIn<DT, attn_chunk_tokens(PoolTraits<DT>::kEB, NT)> in;
    DeferredRows ap;
    start_piece(a, kv, d, in, &ap);
    attn_piece<DT, NT>(a, kv, d, in, &ap);
}

// Chunks of work of sequence b (0 when it has nothing to compute).
__device__ __forceinline__ int seq_chunks(const AttnArgs& a, int b, int tok) {
    const int ctx = seq_keys(a, b, kBS);
    const int nrows = seq_rows(a, b);
    if (nrows <= 0 || nrows > ctx) return 0;
    return (ctx + tok - 1) / tok;
}

// Stream-K: the (sequence, kv head) items are laid end to end in chunk units; the grid
// of gridDim.x workgroups splits that total evenly (at least sk_min_chunks each). A
// workgroup's range is cut at item boundaries into pieces; a piece that is a whole item
// writes the output, any other piece writes record (workgroup + item), and
// attn_streamk_combine_kernel merges the records of split items.
template <gg_dtype_t DT, int NT>
__global__ void __launch_bounds__(256, attn_occupancy(PoolTraits<DT>::kEB, NT)) attn_mfma_streamk_kernel(AttnArgs a, KVView kv) {
    constexpr int kTok = attn_chunk_tokens(PoolTraits<DT>::kEB, NT);
    const int w = blockIdx.x;
    const int Hkv = kv.Hkv;
    __shared__ long long s_scan[256];
    __shared__ long long s_total;
    __shared__ int s_b0;
    __shared__ long long s_base0;
    // Per-thread slice of sequences, its work, and an exclusive scan over threads.
    const int B = a.num_seqs;
    const int per_t = (B + 255) / 256;
    const int b_lo = min(B, (int)threadIdx.x * per_t), b_hi = min(B, b_lo + per_t);
    long long mine = 0;
    for (int bb = b_lo; bb < b_hi; ++bb) mine += (long long)Hkv * seq_chunks(a, bb, kTok);
    s_scan[threadIdx.x] = mine;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long c = 0;
        for (int t = 0; t < 256; ++t) {
            const long long v = s_scan[t];
            s_scan[t] = c;
            c += v;
        }
        s_total = c;
        s_b0 = B;
        s_base0 = c;
    }
    __syncthreads();
    const long long C = s_total;
    const long long per = max((C + gridDim.x - 1) / gridDim.x, (long long)a.sk_min_chunks);
    const long long g0 = (long long)w * per;
    if (g0 >= C) return;
    const long long g1 = min(g0 + per, C);
    // The thread whose slice holds chunk g0 finds the sequence.
    {
        long long gb = s_scan[threadIdx.x];
        if (gb <= g0 && g0 < gb + mine) {
            for (int bb = b_lo; bb < b_hi; ++bb) {
                const long long wk = (long long)Hkv * seq_chunks(a, bb, kTok);
                if (g0 < gb + wk) {
                    s_b0 = bb;
                    s_base0 = gb;
                    break;
                }
                gb += wk;
            }
        }
    }
    __syncthreads();
    // Loop state is wave-uniform 32-bit (chunk totals stay far below 2^31) and kept in
    // scalar registers.
    int b = __builtin_amdgcn_readfirstlane(s_b0);
    int gb = __builtin_amdgcn_readfirstlane((int)s_base0);  // chunk index where sequence b starts
    int g = __builtin_amdgcn_readfirstlane((int)g0);
    const int ge = __builtin_amdgcn_readfirstlane((int)g1);
    // The next piece of [g, ge): advances (g, b, gb); false when the range is done.
    auto next_piece = [&](PieceDesc& d) -> bool {
        while (g < ge && b < B) {
            const int nch = __builtin_amdgcn_readfirstlane(seq_chunks(a, b, kTok));
            const int wk = Hkv * nch;
            if (nch == 0 || g >= gb + wk) {
                gb += wk;
                ++b;
                continue;
            }
            const int off = g - gb;
            const int kvh = off / nch;
            const int c0 = off % nch;
            const int c1 = min(nch, c0 + (ge - g));
            const int item = b * Hkv + kvh;
            const bool whole = c0 == 0 && c1 == nch;
            const int ctx = __builtin_amdgcn_readfirstlane(seq_keys(a, b, kBS));
            d = PieceDesc{b, kvh, c0 * kTok, min(c1 * kTok, ctx), -1, whole ? -1 : w + item};
            g = __builtin_amdgcn_readfirstlane(g + (c1 - c0));
            return true;
        }
        return false;
    };
    PieceDesc d;
    while (next_piece(d)) {
        PieceIn<DT, attn_chunk_tokens(PoolTraits<DT>::kEB, NT)> in;
        start_piece(a, kv, d, in, nullptr);
        attn_piece<DT, NT>(a, kv, d, in, nullptr);
    }
}

// ---- LPT schedule: pieces of a few mean slot loads at most, longest first ----
//
// Items longer than T = ceil(f * total chunks / resident slots) are cut: while the items
// fill the slots, into pieces of T chunks and a shorter last piece; with fewer items, into
// equal pieces of at most T chunks. attn_lpt_plan_kernel orders the pieces by size,
// descending (ties: sequence, then piece, then kv head), and the main launch runs them in
// that order (with
// few items the first round pairs long and shorter pieces per CU, lpt_slot): dispatched in
// order, the longest pieces start first and the shortest fill the tail.
// The last piece of a split item to finish merges the item's partial records
// (lpt_merge_if_last), so the schedule is one launch. Its records are written and read
// with device-scope stores and loads; a device-scope fence instead would write back or
// invalidate a whole L2 here, which costs more than a separate merge launch.
//
// Plan layout (ints, in the workspace after the records), R = record bound, B = sequences:
//   [0]                       number of pieces
//   [1]                       1: T-chunk pieces and a remainder, 0: equal pieces
//   [2]                       T (with remainder pieces)
//   [16 + 4p ..]              piece p: (sequence, kv head | pieces per kv head << 16,
//                             first token, end token); sequence -1 past the last piece
//   [16 + 4R + 2b ..]         sequence b: (first record, pieces per kv head)
//   [16 + 4R + 2B + b*Hkv + h]  merge counter of (sequence b, kv head h)
// The records of sequence b are first + j*Hkv + kvh for its piece j: with equal pieces the
// records follow the ranks (a sequence's pieces have consecutive ranks); with remainder
// pieces (whose ranks are not consecutive) the plan numbers them by sequence.
__device__ __forceinline__ int* lpt_table(int* plan) { return plan + 16; }
// Workgroup of the piece of rank r (and, as an involution, rank of workgroup r). While the
// (sequence, kv head) items do not outnumber the S slots: over the first W = min(S,
// pieces) ranks, the groups of eight ranks in [H, W), H = W/2, are taken in reverse order,
// so workgroup w + H gets a rank near W - 1 - w. Dispatched round-robin, workgroups w and
// w + H land on one CU as its first two slots, which then hold a long and a shorter piece
// instead of two long ones. Measured, same box (with the ranks of [H, W) reversed one by
// one): config 2 (items = S/2) 73.3 -> 71.1 µs; over eight seeded config-3 layouts (items =
// S) the mean 127.2 -> 126.1 µs and the worst layout 136.8 -> 129.4 µs; config 5 (items =
// 2S) 128.3 -> 129.2 µs, so more items than slots keep the plain order. Records stay
// indexed by rank.
// Reversing whole groups of eight keeps every workgroup's index congruent to its rank
// modulo 8, and workgroup w runs on XCD w mod 8. A sequence's kv-head items have
// consecutive ranks from a multiple of Hkv, so with Hkv = 8 item (b, h) runs on XCD
// (first rank of b + h) mod 8 = h mod 8 whether b's items are long or short, and two
// sequences that share prefix blocks read each shared block of a head on one XCD, the
// second read mostly from that XCD's L2. (Reversed one by one, a short sequence's head h
// ran on XCD 7 - h, and a shared block's second read went to another XCD's L2.) Config 3
// (20 % of the blocks shared by pairs of sequences), same box: attention reads 291,491 ->
// 282,994 KiB per call (FETCH_SIZE; 597.0 -> 579.6 MB, the unique pool bytes are 579.2 MB),
// 117.5 -> 116.9 µs per call; configs 2 and 5 unchanged.
__device__ __forceinline__ int lpt_slot(int r, int S, int total, bool pair) {
    const int W = min(S, total);
    const int H = W / 2;
    if (pair && r >= H && r < W) {
        const int q = r - H, G = (W - H) / 8;
        return q < 8 * G ? H + 8 * (G - 1 - q / 8) + (q & 7) : r;
    }
    return r;
}
__device__ __forceinline__ int* lpt_seq(int* plan, int recs) { return plan + 16 + 4 * recs; }
// Merge counters, one per (sequence, kv head): pieces of a split item that have written
// their records. The plan clears them; the piece that merges an item clears its counter.
__device__ __forceinline__ int* lpt_count(int* plan, int recs, int B) { return lpt_seq(plan, recs) + 2 * B; }

// Sum over a 1024-thread workgroup (wave sums, then the 16 wave totals).
__device__ __forceinline__ long long block_sum_1024(long long v, long long* s_w) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = v;
    __syncthreads();
    long long t = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) t += s_w[w];
    return t;
}

// Exclusive prefix sum over a 1024-thread workgroup, and the total.
__device__ __forceinline__ int block_excl_scan_1024(int v, int* s_w, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    __syncthreads();
    if (lane == 63) s_w[w] = inc;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        before += i < w ? s_w[i] : 0;
        all += s_w[i];
    }
    *total = all;
    return before + inc - v;
}

// One 1024-thread workgroup (one sequence per thread): sizes, ranks and lays out the
// pieces.
__global__ void __launch_bounds__(1024) attn_lpt_plan_kernel(AttnArgs a, int Hkv, int tok, int slots, int recs) {
    __shared__ __align__(16) int s_key[kLptMaxSeqs];  // piece size in chunks (0: no work)
    __shared__ __align__(16) int s_cnt[kLptMaxSeqs];  // pieces of the sequence over all kv heads
    __shared__ long long s_w[16];
    __shared__ int s_wi[16];
    const int B = a.num_seqs;
    const int b = threadIdx.x;
    const int nch = b < B ? seq_chunks(a, b, tok) : 0;
    const int ctx = b < B ? seq_keys(a, b, kBS) : 0;
    const long long C = block_sum_1024((long long)Hkv * nch, s_w);
    const bool few = lpt_few_items(slots, B, Hkv);
    const long long den = (long long)slots * (few ? kLptPieceDenFew : kLptPieceDen);
    const long long num = few ? kLptPieceNumFew : kLptPieceNum;
    const int T = (int)max((C * num + den - 1) / den, (long long)kStreamKMinChunks);
    if (!few) {
        // Items that fill the slots: pieces of T chunks and the remainder last. The full
        // pieces come first (by sequence), then the last pieces by size, descending (ties:
        // sequence). Records by (sequence, piece, kv head): a sequence's first record is the
        // count of the pieces of the sequences before it.
        const int np = nch ? (nch + T - 1) / T : 0;
        const int rem = np ? nch - (np - 1) * T : 0;
        const int nfull = np > 1 ? (np - 1) * Hkv : 0;
        const int cnt = np * Hkv;
        if (b < ((B + 7) & ~7)) {
            s_key[b] = b < B ? rem : 0;
            s_cnt[b] = (b < B && np) ? Hkv : 0;
        }
        int F, total;
        const int full_pos = block_excl_scan_1024(nfull, s_wi, &F);
        const int rec_first = block_excl_scan_1024(cnt, s_wi, &total);  // (barriers publish s_key)
        int* plan = a.plan;
        if (b == 0) {
            plan[0] = total;
            plan[1] = 1;
            plan[2] = T;
        }
        if (b >= B) return;
        int pos = F;
        for (int t0 = 0; t0 < B; t0 += 8) {
            const int4 k0 = *(const int4*)&s_key[t0], k1 = *(const int4*)&s_key[t0 + 4];
            const int4 n0 = *(const int4*)&s_cnt[t0], n1 = *(const int4*)&s_cnt[t0 + 4];
            const int kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            const int nn[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int t = t0 + e;
                pos += (kk[e] > rem || (kk[e] == rem && t < b)) ? nn[e] : 0;
            }
        }
        int* seq = lpt_seq(plan, recs) + 2 * b;
        seq[0] = rec_first;
        seq[1] = np;
        for (int h = 0; h < Hkv; ++h) lpt_count(plan, recs, B)[b * Hkv + h] = 0;
        int4* table = (int4*)lpt_table(plan);
        for (int j = 0; j < np; ++j) {
            const int c0 = j * T, c1 = j == np - 1 ? nch : (j + 1) * T;
            const int t0 = c0 * tok, t1 = min(c1 * tok, ctx);
            for (int h = 0; h < Hkv; ++h) {
                const int r = j < np - 1 ? full_pos + j * Hkv + h : pos + h;
                table[lpt_slot(r, slots, total, B * Hkv <= slots)] = make_int4(b, h | (np << 16), t0, t1);
            }
        }
        for (int q = total + b; q < recs; q += B) table[q] = make_int4(-1, 0, 0, 0);
        return;
    }
    // Fewer items than slots: every long item has to be cut to fill the slots, and equal
    // pieces balance them. Records by rank.
    const int np = nch ? (nch + T - 1) / T : 0;
    const int key = np ? (nch + np - 1) / np : 0;
    const int cnt = np * Hkv;
    // (Entries past B, up to a multiple of 8, read as empty.)
    if (b < ((B + 7) & ~7)) {
        s_key[b] = b < B ? key : 0;
        s_cnt[b] = b < B ? cnt : 0;
    }
    const long long total = block_sum_1024(cnt, s_w);  // (its barriers also publish s_key / s_cnt)
    int* plan = a.plan;
    if (b == 0) {
        plan[0] = (int)total;
        plan[1] = 0;
    }
    if (b >= B) return;
    // Pieces ahead of this sequence's: larger pieces, then equal pieces of lower sequences.
    // Eight sequences per step from 16-byte LDS reads (independent adds, no serial chain).
    int pos = 0;
    for (int t0 = 0; t0 < B; t0 += 8) {
        const int4 k0 = *(const int4*)&s_key[t0], k1 = *(const int4*)&s_key[t0 + 4];
        const int4 n0 = *(const int4*)&s_cnt[t0], n1 = *(const int4*)&s_cnt[t0 + 4];
        const int kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const int nn[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = t0 + e;
            pos += (kk[e] > key || (kk[e] == key && t < b)) ? nn[e] : 0;
        }
    }
    int* seq = lpt_seq(plan, recs) + 2 * b;
    seq[0] = pos;
    seq[1] = np;
    for (int h = 0; h < Hkv; ++h) lpt_count(plan, recs, B)[b * Hkv + h] = 0;
    int4* table = (int4*)lpt_table(plan);
    for (int j = 0; j < np; ++j) {
        const int c0 = (int)((long long)j * nch / np), c1 = (int)((long long)(j + 1) * nch / np);
        const int t0 = c0 * tok, t1 = min(c1 * tok, ctx);
        for (int h = 0; h < Hkv; ++h)
            table[lpt_slot(pos + j * Hkv + h, slots, (int)total, B * Hkv <= slots)] =
                make_int4(b, h | (np << 16), t0, t1);
    }
    // Entries past the last piece tell their workgroups to exit.
    for (int q = (int)total + b; q < recs; q += B) table[q] = make_int4(-1, 0, 0, 0);
}

// The piece of a split item that finishes last merges the item's records: the online
// log-sum-exp over its pieces in piece order, as a merge launch of its own would. Each
// piece waits until its record stores have completed, then counts itself in the item's
// counter (a device-scope atomic, no fence: the records were written with device-scope
// stores, and the merging workgroup reads them with device-scope loads). No workgroup
// waits for another, so there is no spinning; the merge costs the last piece a read of
// the item's records.
// Ordering, on gfx950 (gg_kv_create refuses other devices): a device-scope relaxed store
// is issued with the system-coherent bit, so it is written through the XCD's L2 to the
// coherence point, and it counts in vmcnt until that write is acknowledged;
// `s_waitcnt vmcnt(0)` therefore returns only once every record store of the thread is
// visible at the coherence point. The barrier orders all threads' waits before thread 0's
// counter add, which is performed at the coherence point. The merging piece sees the final
// count in the add's return value and only then issues its record loads, which are
// device-scope (system-coherent bit: served from the coherence point, never from a stale
// line of its own XCD's L2). So every record load follows, in time, the completion of the
// record's store. The language-level way (a release add and an acquire read) writes back
// and invalidates the whole XCD L2 on this device and costs config 3 about 4 % (measured).
__device__ void lpt_merge_if_last(const AttnArgs& a, int Hkv, int b, int kvh, int np) {
    __shared__ int s_last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's record stores are done
    __syncthreads();
    const int recs = lpt_records(a.sk_grid, a.num_seqs, Hkv);
    int* cnt = lpt_count(a.plan, recs, a.num_seqs) + b * Hkv + kvh;
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
    __syncthreads();
    if (!s_last) return;
    const int first = lpt_seq(a.plan, recs)[2 * b];
    const int G = a.num_q_heads / Hkv;
    const int RW = G * a.rows;
    const int nrows = seq_rows(a, b), ctx = seq_keys(a, b, kBS);
    if (nrows > 0 && nrows <= ctx) {
        // Thread pairs (row, 4 dims): 32 threads per row.
        for (int e = threadIdx.x; e < G * nrows * (kD / 4); e += blockDim.x) {
            const int r = e / (kD / 4), d4 = e % (kD / 4);
            float M = -1e30f, L = 0.f;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int j = 0; j < np; ++j) {
                const size_t q = (size_t)(first + j * Hkv + kvh) * RW + r;
                const float mx = load_agent(a.ws_ml + q * 2), ly = load_agent(a.ws_ml + q * 2 + 1);
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = load_agent(a.ws_acc + q * kD + 4 * d4 + i);
                const float mn = fmaxf(M, mx);
                const float fo = __expf(M - mn), fn = __expf(mx - mn);
                M = mn;
                L = L * fo + ly * fn;
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = acc[i] * fo + v[i] * fn;
            }
            const float inv = L > 0.f ? 1.f / L : 0.f;
            const int j = r / G, g = r % G;
            const size_t obase = (((size_t)b * a.rows + j) * a.num_q_heads + (size_t)kvh * G + g) * kD + 4 * d4;
#pragma unroll
            for (int i = 0; i < 4; ++i) store_from_f32(a.out, a.out_dtype, obase + i, acc[i] * inv);
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next layer
}

// Workgroup p computes the piece at table entry p (exits past the last piece); the last
// piece of a split item to finish merges it.
template <gg_dtype_t DT, int NT>
__global__ void __launch_bounds__(256, attn_occupancy(PoolTraits<DT>::kEB, NT)) attn_mfma_lpt_kernel(AttnArgs a, KVView kv) {
    const int p = blockIdx.x;
#ifdef GG_TRACE
    const long long tr_t0 = wall_clock64();
#endif
    // One load tells the workgroup everything about its piece.
    const int4 e = ((const int4*)lpt_table(a.plan))[p];
    const int b = e.x;
    if (b < 0) return;  // past the last piece
    const int kvh = e.y & 0xffff, np = e.y >> 16;
    // The piece's record: with remainder pieces (plan[1]) the sequence's first record plus
    // (piece j = first chunk / T) * Hkv + kv head; with equal pieces its rank.
    int rec = -1;
    if (np > 1) {
        constexpr int kTokC = attn_chunk_tokens(PoolTraits<DT>::kEB, NT);
        rec = a.plan[1] ? lpt_seq(a.plan, lpt_records(a.sk_grid, a.num_seqs, kv.Hkv))[2 * b] +
                              (e.z / kTokC / a.plan[2]) * kv.Hkv + kvh
                        : lpt_slot(p, a.sk_grid, a.plan[0], a.num_seqs * kv.Hkv <= a.sk_grid);
    }
    const PieceDesc d{b, kvh, e.z, e.w, -1, rec};
    PieceIn<DT, attn_chunk_tokens(PoolTraits<DT>::kEB, NT)> in;
    DeferredRows ap;
    start_piece(a, kv, d, in, &ap);
    attn_piece<DT, NT>(a, kv, d, in, &ap);
    if (np > 1) lpt_merge_if_last(a, kv.Hkv, b, kvh, np);
#ifdef GG_TRACE
    if (threadIdx.x == 0) {
        g_trace[4 * p + 0] = tr_t0;
        g_trace[4 * p + 1] = wall_clock64();
        // CU id, a valid bit, the XCC (hardware register XCC_ID) and the piece's key count
        const long long xcc = (long long)(__builtin_amdgcn_s_getreg(20 | (15 << 11)) & 0xf);
        g_trace[4 * p + 2] = (long long)__smid() | (1LL << 32) | (xcc << 40) | ((long long)(e.w - e.z) << 44);
    }
#endif
}

template <gg_dtype_t DT>
gg_status_t launch_dt(const AttnArgs& a, const KVView& kv, int nt, hipStream_t s) {
    if (a.sched == ATTN_SCHED_LPT) {
        const int recs = lpt_records(a.sk_grid, a.num_seqs, kv.Hkv);
        switch (nt) {
            case 1: attn_mfma_lpt_kernel<DT, 1><<<recs, 256, 0, s>>>(a, kv); break;
            case 2: attn_mfma_lpt_kernel<DT, 2><<<recs, 256, 0, s>>>(a, kv); break;
            case 3: attn_mfma_lpt_kernel<DT, 3><<<recs, 256, 0, s>>>(a, kv); break;
            case 4: attn_mfma_lpt_kernel<DT, 4><<<recs, 256, 0, s>>>(a, kv); break;
            default: return fail(GG_ERR_INVALID, "attention: too many rows per kv head for the MFMA path");
        }
        return GG_OK;
    }
    if (a.sched == ATTN_SCHED_STREAMK) {
        const int grid = a.sk_grid;
        switch (nt) {
            case 1: attn_mfma_streamk_kernel<DT, 1><<<grid, 256, 0, s>>>(a, kv); break;
            case 2: attn_mfma_streamk_kernel<DT, 2><<<grid, 256, 0, s>>>(a, kv); break;
            case 3: attn_mfma_streamk_kernel<DT, 3><<<grid, 256, 0, s>>>(a, kv); break;
            case 4: attn_mfma_streamk_kernel<DT, 4><<<grid, 256, 0, s>>>(a, kv); break;
            default: return fail(GG_ERR_INVALID, "attention: too many rows per kv head for the MFMA path");
        }
        return GG_OK;
    }
    dim3 grid(a.max_parts, kv.Hkv, a.num_seqs);
    switch (nt) {
        case 1: attn_mfma_kernel<DT, 1><<<grid, 256, 0, s>>>(a, kv); break;
        case 2: attn_mfma_kernel<DT, 2><<<grid, 256, 0, s>>>(a, kv); break;
        case 3: attn_mfma_kernel<DT, 3><<<grid, 256, 0, s>>>(a, kv); break;
        case 4: attn_mfma_kernel<DT, 4><<<grid, 256, 0, s>>>(a, kv); break;
        default: return fail(GG_ERR_INVALID, "attention: too many rows per kv head for the MFMA path");
    }
    return GG_OK;
}

// Merge the stream-K records of one (sequence, kv head) item that was split over
// several workgroups. Workgroup (item, y) takes rows 4y .. 4y+3 of the item; each thread
// one row and four dims, merged in one online pass whose record loads are independent.
__global__ void __launch_bounds__(128) attn_streamk_combine_kernel(AttnArgs a, int Hkv, int tok, int grid) {
    const int item = blockIdx.x;
    const int b = item / Hkv, kvh = item % Hkv;
    const int G = a.num_q_heads / Hkv;
    const int nrows = seq_rows(a, b);
    const int r = blockIdx.y * 4 + (threadIdx.x >> 5);
    const int d4 = threadIdx.x & 31;
    const int nch = seq_chunks(a, b, tok);
    if (nch == 0 || (int)blockIdx.y * 4 >= G * nrows) return;
    // Chunks before sequence b and in total (same arithmetic as the producer).
    __shared__ long long s_before[128], s_total[128];
    long long before = 0, total = 0;
    for (int bb = threadIdx.x; bb < a.num_seqs; bb += 128) {
        const long long wk = (long long)Hkv * seq_chunks(a, bb, tok);
        total += wk;
        if (bb < b) before += wk;
    }
    s_before[threadIdx.x] = before;
    s_total[threadIdx.x] = total;
    __syncthreads();
    for (int o = 64; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            s_before[threadIdx.x] += s_before[threadIdx.x + o];
            s_total[threadIdx.x] += s_total[threadIdx.x + o];
        }
        __syncthreads();
    }
    before = s_before[0];
    total = s_total[0];
    const long long per = max((total + grid - 1) / grid, (long long)a.sk_min_chunks);
    const long long gi0 = before + (long long)kvh * nch, gi1 = gi0 + nch;
    const int w0 = (int)(gi0 / per), w1 = (int)((gi1 - 1) / per);
    if (w0 == w1 || r >= G * nrows) return;  // one piece: the producer wrote the output
    const int RW = G * a.rows;
    float M = -1e30f, L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int w = w0; w <= w1; ++w) {
        const size_t p = (size_t)(w + item) * RW + r;
        const float2 ml = *(const float2*)(a.ws_ml + p * 2);
        const float4 v = ((const float4*)(a.ws_acc + p * kD))[d4];
        const float mn = fmaxf(M, ml.x);
        const float fo = __expf(M - mn), fn = __expf(ml.x - mn);
        M = mn;
        L = L * fo + ml.y * fn;
        acc.x = acc.x * fo + v.x * fn;
        acc.y = acc.y * fo + v.y * fn;
        acc.z = acc.z * fo + v.z * fn;
        acc.w = acc.w * fo + v.w * fn;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int j = r / G, g = r % G;
    const size_t obase = (((size_t)b * a.rows + j) * a.num_q_heads + (size_t)kvh * G + g) * kD + 4 * d4;
    store_from_f32(a.out, a.out_dtype, obase + 0, acc.x * inv);
    store_from_f32(a.out, a.out_dtype, obase + 1, acc.y * inv);
    store_from_f32(a.out, a.out_dtype, obase + 2, acc.z * inv);
    store_from_f32(a.out, a.out_dtype, obase + 3, acc.w * inv);
}

}  // namespace

gg_status_t launch_attn_mfma(const AttnArgs& a, const KVView& kv, hipStream_t s) {
    const int G = a.num_q_heads / kv.Hkv;
    const int nt = (G * a.rows + 15) / 16;
    const int tok = attn_chunk_tokens(dtype_bytes(kv.dt), nt);
    if (a.sched == ATTN_SCHED_LPT && !a.plan_ready) {
        const gg_status_t st = launch_attn_plan(a, s);
        if (st != GG_OK) return st;
    }
    gg_status_t st;
    switch (kv.dt) {
        case GG_DTYPE_BF16: st = launch_dt<GG_DTYPE_BF16>(a, kv, nt, s); break;
        case GG_DTYPE_F16: st = launch_dt<GG_DTYPE_F16>(a, kv, nt, s); break;
        case GG_DTYPE_FP8_E4M3: st = launch_dt<GG_DTYPE_FP8_E4M3>(a, kv, nt, s); break;
        case GG_DTYPE_INT8: st = launch_dt<GG_DTYPE_INT8>(a, kv, nt, s); break;
        default: return fail(GG_ERR_INVALID, "attention: pool dtype not on the MFMA path");
    }
    if (st != GG_OK) return st;
    const dim3 cgrid(a.num_seqs * kv.Hkv, (G * a.rows + 3) / 4);
    if (a.sched == ATTN_SCHED_STREAMK) attn_streamk_combine_kernel<<<cgrid, 128, 0, s>>>(a, kv.Hkv, tok, a.sk_grid);
    // (LPT: the split items are merged inside the main launch, lpt_merge_if_last.)
    return GG_OK;
}

gg_status_t launch_attn_plan(const AttnArgs& a, hipStream_t s) {
    if (a.sched != ATTN_SCHED_LPT) return GG_OK;
    if (a.num_seqs > kLptMaxSeqs) return fail(GG_ERR_INTERNAL, "attention: LPT plan over too many sequences");
    const KV* kv = a.kv;
    const int Hkv = kv->num_kv_heads;
    const int tok = attn_chunk_tokens(dtype_bytes(kv->dtype), (a.num_q_heads / Hkv * a.rows + 15) / 16);
    attn_lpt_plan_kernel<<<1, 1024, 0, s>>>(a, Hkv, tok, a.sk_grid, lpt_records(a.sk_grid, a.num_seqs, Hkv));
    return check_hip(hipGetLastError(), "verify_attention plan launch");
}

int attn_streamk_grid(const KV* kv, int rows, int num_q_heads) {
    const int G = num_q_heads / kv->num_kv_heads;
    const int nt = (G * rows + 15) / 16;
    // One resident wave of workgroups: each CU holds attn_occupancy of them.
    return device_cu_count() * attn_occupancy((int)dtype_bytes(kv->dtype), nt);
}

size_t attn_streamk_workspace_bytes(const KV* kv, int num_seqs, int rows, int num_q_heads, size_t* ml_elems,
                                    size_t* acc_elems) {
    // Records for LPT pieces or for stream-K's grid + items, whichever bound is larger.
    const int grid = attn_streamk_grid(kv, rows, num_q_heads);
    const size_t items = (size_t)num_seqs * kv->num_kv_heads;
    const size_t records = std::max((size_t)lpt_records(grid, num_seqs, kv->num_kv_heads), (size_t)grid + items);
    const size_t rw = (size_t)(num_q_heads / kv->num_kv_heads) * rows;
    const size_t n_ml = records * rw * 2;
    const size_t n_acc = records * rw * kD;
    const size_t plan_ints = 16 + 4 * records + 2 * (size_t)num_seqs + items;  // (items: merge counters)
    if (ml_elems) *ml_elems = n_ml;
    if (acc_elems) *acc_elems = n_acc;
    return (((n_ml + 63) / 64) * 64 + n_acc) * sizeof(float) + plan_ints * sizeof(int);
}

#ifdef GG_TRACE
extern "C" __attribute__((visibility("default"))) void* gg_debug_trace_ptr() {
    void* p = nullptr;
    (void)hipGetSymbolAddress(&p, HIP_SYMBOL(g_trace));
    return p;
}
#endif

}  // namespace gg
