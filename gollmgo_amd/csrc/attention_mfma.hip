// attention_mfma.hip — gfx950 MFMA phase-1 kernel of the verify attention.
//
// One 256-thread workgroup per (sequence, kv head, partition). Its G*R query rows
// (G query heads of the kv head x R verify rows, row r = j*G + g) form NT tiles of
// 16 rows; K/V of each 64-token chunk (four 16-token blocks) are read ONCE with
// 16-byte loads and shared by every row — the GQA x draft reuse that turns
// a bandwidth-bound decode into MFMA-friendly tiles. The four waves stream
// disjoint chunks and merge their (max, sum, P.V) states through LDS at the end.
//
// Per chunk and row tile, with lane = 16*g4 + c:
//   S^T = K . Q^T   v_mfma_f32_16x16x32_{bf16,f16}: A = K (16 tokens x 32 dims),
//                   B = Q^T. Token m = 4q+i of tile s is (block q, offset 4s+i), so
//                   the output gives lane (g4, c) row c and block g4's offsets 4s..4s+3.
//   P = softmax     online, per row, base-2 exponent; row max via xor-shuffles 16/32.
//   O += P . V      A = P (row c, k = 8*g4+i -> block g4 offset 8*pv+i),
//                   B = V from the dim-major V block: one 16-byte load gives a lane
//                   all 16 offsets of one dim.
// Head dims are permuted consistently in K and Q (lane group g4 owns dims
// 32*g4..32*g4+31), so every K load is a contiguous 32- or 64-byte run.
//
// Pool types: BF16 (bf16 MFMA; P split into bf16 hi+lo for two MFMAs so the
// probabilities keep ~16 bits), F16 (f16 MFMA), FP8-E4M3 and INT8 (decoded in
// registers to exact f16 values: E4M3 bits shifted into an f16 at 2^-8 scale, int8
// via the 0x6400 magic; the per-head / per-block scales are applied to the fp32
// scores and to P, never to the operands).
#include "gg_common.h"
#include "attention_common.h"

namespace gg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// Two E4M3 bytes (bits 0-7 and 16-23 of x) -> two f16 equal to value * 2^-8 (exact).
__device__ __forceinline__ uint32_t e4m3x2_to_f16x2(uint32_t x) {
    return ((x & 0x00800080u) << 8) | ((x & 0x007F007Fu) << 7);
}
// Four E4M3 bytes -> four f16 (value * 2^-8), as two dwords.
__device__ __forceinline__ uint2 e4m3x4_to_f16x4(uint32_t w) {
    uint32_t lo = (w & 0xFFu) | ((w & 0xFF00u) << 8);
    uint32_t hi = ((w >> 16) & 0xFFu) | ((w >> 8) & 0xFF0000u);
    return make_uint2(e4m3x2_to_f16x2(lo), e4m3x2_to_f16x2(hi));
}
// Four int8 -> four f16 (exact): (0x6400 | (b ^ 0x80)) is 1024 + b + 128.
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t w) {
    w ^= 0x80808080u;
    uint32_t lo = (w & 0xFFu) | ((w & 0xFF00u) << 8) | 0x64006400u;
    uint32_t hi = ((w >> 16) & 0xFFu) | ((w >> 8) & 0xFF0000u) | 0x64006400u;
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

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

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

template <gg_dtype_t DT, int NT>
__global__ void __launch_bounds__(256, (NT <= 2 ? 2 : 1))
    attn_mfma_kernel(AttnArgs a, KVView kv) {
    using T = PoolTraits<DT>;
    constexpr bool kIsBf16 = T::kBf16;
    constexpr int kEB = T::kEB;
    constexpr int kRows = NT * 16;

    const int part = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int ctx = seq_keys(a, b, kBS);
    const int P = a.partition;
    const int nparts = (ctx + P - 1) / P;
    if (part >= nparts) return;
    const int R = a.rows;
    const int nrows = a.row_counts ? a.row_counts[b] : R;
    if (nrows <= 0 || nrows > ctx) return;
    const int Hq = a.num_q_heads;
    const int G = Hq / kv.Hkv;
    const int nvalid_rows = G * nrows;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int c16 = lane & 15;
    const int g4 = lane >> 4;

    const int t0 = part * P;
    const int t_end = min(t0 + P, ctx);
    const int nchunks = (t_end - t0 + kChunk - 1) / kChunk;
    const int first_masked = ctx - nrows;  // tokens >= this are causally masked for some row

    // Score multiplier (log2 domain) and P.V multiplier per pool type.
    float sscale = a.scale * kLog2e;
    float vfold = 1.f;
    if constexpr (DT == GG_DTYPE_FP8_E4M3) {
        sscale *= kv.k_head_scale[kvh] * 256.f;
        vfold = kv.v_head_scale[kvh] * 256.f;
    }

    // ---- Q operands: B[k = 8*g4+i][n = c16] <- Q[row rt*16+c16][32*g4 + 8*mm + i] ----
    uint4 qop[NT][4];
    int row_pos[NT];  // last visible key position of the lane's S row (c16)
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
        const int r = rt * 16 + c16;
        const bool valid = r < nvalid_rows;
        const int j = valid ? r / G : 0;
        const int g = valid ? r % G : 0;
        row_pos[rt] = valid ? first_masked + j : ctx - 1;
        const size_t qb = (((size_t)b * R + j) * Hq + (size_t)kvh * G + g) * kD + 32 * g4;
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            float f[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) f[i] = valid ? load_as_f32(a.q, a.q_dtype, qb + 8 * mm + i) : 0.f;
            if constexpr (kIsBf16)
                qop[rt][mm] = make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                         pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
            else
                qop[rt][mm] = make_uint4(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]),
                                         pack_f16x2(f[4], f[5]), pack_f16x2(f[6], f[7]));
        }
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

    const int32_t* bt = a.block_tables + (size_t)b * a.max_blocks;
    const size_t head_stride_k = (size_t)kBS * kD;  // elements per (block, head) tile

    for (int ch = wave; ch < nchunks; ch += kWaves) {
        const int tc = t0 + ch * kChunk;
        // K rows: lane supplies token (block c16/4, offset 4s + c16%4) for tile s.
        const int tk = tc + 16 * (c16 >> 2);
        int blk_k = tk < ctx ? bt[tk >> 4] : -1;
        if (blk_k >= kv.num_blocks) blk_k = -1;
        // V columns / P rows: lane owns block g4 of the chunk.
        const int tv = tc + 16 * g4;
        int blk_v = tv < ctx ? bt[tv >> 4] : -1;
        if (blk_v >= kv.num_blocks) blk_v = -1;
        const int nvalid_v = ctx - tv;

        // ---- loads ----
        constexpr int kKVec = 32 * kEB / 16;  // 16-byte loads per lane per K tile
        uint4 kraw[4][kKVec];
        {
            const uint8_t* kbase = kv.kc + (((size_t)(blk_k < 0 ? 0 : blk_k) * kv.Hkv + kvh) * head_stride_k +
                                            32 * g4) * kEB;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int off = 4 * s + (c16 & 3);
#pragma unroll
                for (int v = 0; v < kKVec; ++v)
                    kraw[s][v] = blk_k >= 0 ? *(const uint4*)(kbase + (size_t)off * kD * kEB + 16 * v) : zero4();
            }
        }
        constexpr int kVVec = 16 * kEB / 16;  // 16-byte loads per lane per V dim-tile
        uint4 vraw[8][kVVec];
        {
            const uint8_t* vbase = kv.vc + (((size_t)(blk_v < 0 ? 0 : blk_v) * kv.Hkv + kvh) * kD) * kBS * kEB;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const int d = dt * 16 + c16;
#pragma unroll
                for (int v = 0; v < kVVec; ++v)
                    vraw[dt][v] = blk_v >= 0 ? *(const uint4*)(vbase + (size_t)d * kBS * kEB + 16 * v) : zero4();
            }
        }
        if (blk_v >= 0 && nvalid_v < kBS) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                if constexpr (kEB == 1) vraw[dt][0] = mask_bytes16(vraw[dt][0], nvalid_v);
                else {
                    vraw[dt][0] = mask_halves8(vraw[dt][0], nvalid_v, 0);
                    vraw[dt][1] = mask_halves8(vraw[dt][1], nvalid_v, 8);
                }
            }
        }

        float kblk_scale = 1.f, vblk_scale = 1.f;
        if constexpr (DT == GG_DTYPE_INT8) {
            if (blk_v >= 0) {
                kblk_scale = f16_bits_to_f32(kv.k_blk_scale[(size_t)blk_v * kv.Hkv + kvh]);
                vblk_scale = f16_bits_to_f32(kv.v_blk_scale[(size_t)blk_v * kv.Hkv + kvh]);
            }
        }

        // K operands per (tile s, dim group mm)
        uint4 kop[4][4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                if constexpr (kEB == 2) {
                    kop[s][mm] = kraw[s][mm];
                } else {
                    const uint4 r = kraw[s][mm >> 1];
                    const uint32_t w0 = (mm & 1) ? r.z : r.x;
                    const uint32_t w1 = (mm & 1) ? r.w : r.y;
                    kop[s][mm] = bytes8_to_f16x8<DT>(w0, w1);
                }
            }
        }

        const bool need_mask = tc + kChunk - 1 >= first_masked;
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            // ---- scores for 64 tokens x 16 rows ----
            f32x4 sacc[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                sacc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int mm = 0; mm < 4; ++mm) sacc[s] = mfma(kop[s][mm], qop[rt][mm], sacc[s], kIsBf16);
            }
            float sc[16];
            float cmax = -INFINITY;
            const float mult = DT == GG_DTYPE_INT8 ? sscale * kblk_scale : sscale;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = sacc[s][i] * mult;
                    if (need_mask) {
                        const int t = tv + 4 * s + i;
                        v = t <= row_pos[rt] ? v : -INFINITY;
                    }
                    sc[4 * s + i] = v;
                    cmax = fmaxf(cmax, v);
                }
            }
            cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
            cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
            const float m_new = fmaxf(m_run[rt], cmax);
            const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - m_new);
            m_run[rt] = m_new;
            float psum = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                sc[k] = __builtin_amdgcn_exp2f(sc[k] - m_new);
                psum += sc[k];
            }
            l_run[rt] = l_run[rt] * alpha + psum;
            // Rescale O rows (4*g4 + i) with their rows' alpha.
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float al = __shfl(alpha, 4 * g4 + i);
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) o[rt][dt][i] *= al;
            }
            // ---- O += P . V ----
            if constexpr (DT == GG_DTYPE_INT8) {
#pragma unroll
                for (int k = 0; k < 16; ++k) sc[k] *= vblk_scale;
            }
#pragma unroll
            for (int pv = 0; pv < 2; ++pv) {
                const float* pp = sc + 8 * pv;
                if constexpr (kIsBf16) {
                    float hi[8], lo[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        hi[k] = bf16_bits_to_f32(f32_to_bf16_bits(pp[k]));
                        lo[k] = pp[k] - hi[k];
                    }
                    const uint4 ph = make_uint4(pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3]),
                                                pack_bf16x2(hi[4], hi[5]), pack_bf16x2(hi[6], hi[7]));
                    const uint4 pl = make_uint4(pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]),
                                                pack_bf16x2(lo[4], lo[5]), pack_bf16x2(lo[6], lo[7]));
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) {
                        o[rt][dt] = mfma(ph, vraw[dt][pv], o[rt][dt], true);
                        o[rt][dt] = mfma(pl, vraw[dt][pv], o[rt][dt], true);
                    }
                } else {
                    const uint4 ph = make_uint4(pack_f16x2(pp[0], pp[1]), pack_f16x2(pp[2], pp[3]),
                                                pack_f16x2(pp[4], pp[5]), pack_f16x2(pp[6], pp[7]));
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) {
                        uint4 vop;
                        if constexpr (kEB == 2) {
                            vop = vraw[dt][pv];
                        } else {
                            const uint4 r = vraw[dt][0];
                            vop = pv ? bytes8_to_f16x8<DT>(r.z, r.w) : bytes8_to_f16x8<DT>(r.x, r.y);
                        }
                        o[rt][dt] = mfma(ph, vop, o[rt][dt], false);
                    }
                }
            }
        }
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
            if (nparts == 1) {
                const float val = L > 0.f ? acc * vfold / L : 0.f;
                store_from_f32(a.out, a.out_dtype, (z * Hq + h) * kD + d, val);
            } else {
                const size_t pidx = (z * Hq + h) * a.max_parts + part;
                a.ws_acc[pidx * kD + d] = acc * vfold;
                if (d == 0) {
                    a.ws_ml[pidx * 2 + 0] = mx > -1e29f ? mx * kLn2 : -1e30f;
                    a.ws_ml[pidx * 2 + 1] = L;
                }
            }
        }
        __syncthreads();
    }
}

template <gg_dtype_t DT>
gg_status_t launch_dt(const AttnArgs& a, const KVView& kv, int nt, hipStream_t s) {
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

}  // namespace

gg_status_t launch_attn_mfma(const AttnArgs& a, const KVView& kv, hipStream_t s) {
    const int G = a.num_q_heads / kv.Hkv;
    const int nt = (G * a.rows + 15) / 16;
    switch (kv.dt) {
        case GG_DTYPE_BF16: return launch_dt<GG_DTYPE_BF16>(a, kv, nt, s);
        case GG_DTYPE_F16: return launch_dt<GG_DTYPE_F16>(a, kv, nt, s);
        case GG_DTYPE_FP8_E4M3: return launch_dt<GG_DTYPE_FP8_E4M3>(a, kv, nt, s);
        case GG_DTYPE_INT8: return launch_dt<GG_DTYPE_INT8>(a, kv, nt, s);
        default: return fail(GG_ERR_INVALID, "attention: pool dtype not on the MFMA path");
    }
}

}  // namespace gg
