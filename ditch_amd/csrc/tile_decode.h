// tile_decode.h — the tiled products' per-format weight decode from a
// tile word and the tensor's per-row side words (TileView::side, built at
// upload for tensors the conversion instructions decode exactly, `fast`),
// shared by the tiled GEMM (gemm_tile.hip) and the edit's W^T y products
// (edit_batch.hip).
#pragma once
#include <type_traits>

#include "gemm_common.h"

namespace ditch {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// per-format weight stages (64 k = two 32-wide MFMA tiles per lane)

__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    bf16x2_t v;
    v.x = (__bf16)a;  // v_cvt_pk_bf16_f32: round to nearest even
    v.y = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
}

// Per-format pipeline geometry: TPS k tiles (32 wide) per stage, NU weight
// units (1 KiB per 16-row group) and NS side words per row per stage.
template <int TF> struct TileCfg;
template <> struct TileCfg<TF_BF16> { static constexpr int TPS = 2, NU = 2, NS = 0; };  // units 2s, 2s+1
template <> struct TileCfg<TF_FP8> { static constexpr int TPS = 2, NU = 1, NS = 1; };   // unit s; f32 scale
template <> struct TileCfg<TF_MX4> { static constexpr int TPS = 4, NU = 1, NS = 1; };   // unit s; 4 E8M0 bytes
template <> struct TileCfg<TF_INT4> { static constexpr int TPS = 4, NU = 1, NS = 2; };  // unit s; two 64-col groups
template <> struct TileCfg<TF_Q8> { static constexpr int TPS = 2, NU = 1, NS = 1; };    // unit s; two f16 block scales

// Side word of stage s, entry j, for a row whose side row starts at `base`.
// Calls f(std::integral_constant<int, j>) for j = 0 .. N-1 (instruction
// immediates must be constant expressions).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// FP8 and INT4 index their scale column by 64-column steps: stage s entry j
// is step s (FP8) or 2 s + j (INT4) over `per` = block_cols / 64 or
// group / 64 steps a column; `sh` = log2(per) when per is a power of two,
// else -1 (a 32-bit division: this runs once per copy and stage)
struct SideStep {
    uint32_t per;
    int sh;
};
template <int TF>
__device__ __forceinline__ SideStep side_step(const TileView &w) {
    const uint32_t per = TF == TF_FP8 ? (uint32_t)(w.block_cols / 64) : TF == TF_INT4 ? (uint32_t)(w.group / 64) : 1u;
    return SideStep{per, (per & (per - 1)) == 0 ? __builtin_ctz(per) : -1};
}
template <int TF>
__device__ __forceinline__ const uint32_t *side_word(const SideStep &st, const uint32_t *side, int64_t s, int j) {
    if constexpr (TF == TF_MX4) return side + s;
    else if constexpr (TF == TF_Q8) return side + s * 16;  // [group][unit][row % 16]
    else {
        const uint32_t u = TF == TF_FP8 ? (uint32_t)s : (uint32_t)(2 * s + j);
        return side + (st.sh >= 0 ? u >> st.sh : u / st.per);
    }
}

// Side row of this lane's weight row (FP8: its row of the scale grid).
__device__ __forceinline__ int64_t side_row(const TileView &w, int64_t g, int lane) {
    if (w.tf == TF_Q8) return g * w.units_k * 16 + (lane & 15);
    int64_t r = g * 16 + (lane & 15);
    r = r < w.rows ? r : w.rows - 1;
    if (w.tf == TF_FP8) {
        if (w.row_shard == 0) r = r / w.block_rows;
        else {
            int64_t per_shard = (w.row_shard + w.block_rows - 1) / w.block_rows;
            r = r / w.row_shard * per_shard + (r % w.row_shard) / w.block_rows;
        }
    }
    return r * w.side_cols;
}

// B fragment of k tile t of a stage from its codes (NU x 16 bytes) and side
// words. `second` is false when a bf16 stage's second unit lies past the
// matrix (its codes are a repeat of the first and must read as zero).
template <int TF>
__device__ __forceinline__ u32x4 decode_tile_lds(const TileView &w, const u32x4 (&c)[TileCfg<TF>::NU],
                                                 const uint32_t *sd, int t, bool second) {
    u32x4 f;
    if constexpr (TF == TF_BF16) {
        f = t == 0 ? c[0] : (second ? c[1] : u32x4{0, 0, 0, 0});
    } else if constexpr (TF == TF_MX4) {
        const uint32_t wd = c[0][t];
        const uint32_t sb = (sd[0] >> (8 * t)) & 0xffu;
        const float sc = u2f(sb ? (sb << 23) : 0x00400000u);  // 2^(b-127); byte 0 is the subnormal 2^-127
        f[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 0));
        f[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 1));
        f[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 2));
        f[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 3));
    } else if constexpr (TF == TF_FP8) {
        const float sc = u2f(sd[0]);
        const uint32_t w0 = c[0][2 * t], w1 = c[0][2 * t + 1];
        floatx2 p0 = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false), p1 = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
        floatx2 p2 = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false), p3 = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
        f[0] = cvt_pk_bf16(__fmul_rn(p0.x, sc), __fmul_rn(p0.y, sc));
        f[1] = cvt_pk_bf16(__fmul_rn(p1.x, sc), __fmul_rn(p1.y, sc));
        f[2] = cvt_pk_bf16(__fmul_rn(p2.x, sc), __fmul_rn(p2.y, sc));
        f[3] = cvt_pk_bf16(__fmul_rn(p3.x, sc), __fmul_rn(p3.y, sc));
    } else if constexpr (TF == TF_Q8) {
        // the int8 codes, exact in bf16; the block scale multiplies the tile's partial sums
        const uint32_t w0 = c[0][2 * t], w1 = c[0][2 * t + 1];
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = (float)(int8_t)((w0 >> (8 * j)) & 0xffu);
            v[4 + j] = (float)(int8_t)((w1 >> (8 * j)) & 0xffu);
        }
        f = u32x4{pack_hi(v[0], v[1]), pack_hi(v[2], v[3]), pack_hi(v[4], v[5]), pack_hi(v[6], v[7])};
    } else if constexpr (TF == TF_INT4) {
        const uint32_t word = sd[t >> 1];
        const uint32_t bits = word & 0xffffu;
        // the scale's own dtype, widened exactly (both widenings, then a
        // select: no branch inside the product loop)
        const float sc_bf = u2f(bits << 16), sc_h = (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
        const float sc = w.scale_type == SC_BF16 ? sc_bf : sc_h;
        // (q - z) s as q s - z s in one fused multiply-add: q s and z s are
        // exact (4-bit integers times a 16-bit scale; upload keeps a bf16
        // scale's magnitude under 2^120, so 15 s stays finite), their
        // difference is (q - z) s, exact in f32, so the fused operation
        // returns it unrounded (a zero weight, q = z, comes out +0 where the
        // reference's product gives -0 under a negative scale: a product
        // differs only in the sign of an all-zero sum); the nibbles are
        // spread into bytes and converted by byte lane
        const float zs = __fmul_rn((float)(int32_t)(word >> 16), sc);
        const uint32_t wd = c[0][t];
        // (the masks as instructions the compiler cannot see through: it
        // would fold each byte's mask and shift into a bit-field extract,
        // one instruction per nibble ahead of its conversion)
        uint32_t lo, hi;
        asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(wd));
        asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(wd >> 4));
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = __builtin_fmaf((float)((lo >> (8 * j)) & 0xffu), sc, -zs);
            v[2 * j + 1] = __builtin_fmaf((float)((hi >> (8 * j)) & 0xffu), sc, -zs);
        }
        f = u32x4{cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]), cvt_pk_bf16(v[4], v[5]), cvt_pk_bf16(v[6], v[7])};
    }
    return f;
}

}  // namespace ditch
