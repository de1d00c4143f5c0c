// gemm_common.h — MFMA fragments, activation splitting and per-format weight
// decoding shared by the product kernels (gemm.hip, gemm_tile.hip).
//
// out[n][rows] = x[n][cols] @ W^T, the product of tensor.matmulT
// (tensor.zig:1023-1045) with the weight decoded inside the kernel.
//
// Numerics. The reference widens every weight to f32 (its virtual bf16
// tensors are exact in bf16) and accumulates in f32 (tensor.zig:889-913).
// Here the weight fragment is the exact decoded bf16 value (FP8, MXFP4,
// INT4 and bf16 weights), or the exact small integer of a Q8_0 code with the
// block scale applied to the per-block partial sum, or an exact hi/lo bf16
// split (f16, f32). The f32 activation is split into hi = bf16_rne(x) and
// lo = bf16_rne(x - hi), so x - hi - lo is below 2^-17 |x|. Each bf16 x bf16
// product is exact in the f32 accumulator of v_mfma_f32_16x16x32_bf16; the
// difference to the CPU is the order of f32 additions and that 2^-17
// residual.
//
// Fragment layout (v_mfma_f32_16x16x32_bf16, A = activations, B = W^T):
//   A: lane l holds x[token l%16][k 8*(l/16) .. +8]
//   B: lane l holds W[row   l%16][k 8*(l/16) .. +8]   (one 16 B tile word)
//   D: lane l holds out[token 4*(l/16) + r][row l%16], r = 0..3
#pragma once
#include "decode.h"
#include "internal.h"

namespace ditch {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma_bf16(u32x4 a, u32x4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ floatx4 mfma_f32(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// high halves of two f32 -> one packed bf16 pair (exact when the values are)
__device__ __forceinline__ uint32_t pack_hi(float lo, float hi) {
    return __builtin_amdgcn_perm(f2u(hi), f2u(lo), 0x07060302u);
}
// round-to-nearest-even bf16 of finite values, as 16 high bits of a f32
__device__ __forceinline__ uint32_t rne_bits(float v) {
    uint32_t b = f2u(v);
    return (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
}
__device__ __forceinline__ uint32_t pack_rne(float a, float b) {
    return (rne_bits(a) >> 16) | rne_bits(b);
}

// x (8 consecutive f32) -> hi and lo bf16 fragments
__device__ __forceinline__ void split8(const float (&v)[8], u32x4 &hi, u32x4 &lo) {
    float h[8], l[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        h[j] = u2f(rne_bits(v[j]));
        l[j] = __fsub_rn(v[j], h[j]);
    }
    hi = u32x4{pack_hi(h[0], h[1]), pack_hi(h[2], h[3]), pack_hi(h[4], h[5]), pack_hi(h[6], h[7])};
    lo = u32x4{pack_rne(l[0], l[1]), pack_rne(l[2], l[3]), pack_rne(l[4], l[5]), pack_rne(l[6], l[7])};
}

// The A operand words of 8 activations: XT bf16 terms x = t0 + t1 (+ t2),
// each the round-to-nearest-even bf16 of the remainder of the previous
// ones (remainder below 2^-18 |x| for two terms, 2^-27 |x| for three), or
// for the fp32 MFMA the f32 values themselves in t[0] (0..3) and t[1] (4..7).
template <bool FP32, int XT>
__device__ __forceinline__ void a_words(const float (&v)[8], u32x4 (&t)[XT]) {
    if constexpr (FP32) {
        t[0] = u32x4{f2u(v[0]), f2u(v[1]), f2u(v[2]), f2u(v[3])};
        t[1] = u32x4{f2u(v[4]), f2u(v[5]), f2u(v[6]), f2u(v[7])};
    } else {
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) r[j] = v[j];
#pragma unroll
        for (int e = 0; e < XT; e++) {
            float h[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                h[j] = u2f(rne_bits(r[j]));
                r[j] = __fsub_rn(r[j], h[j]);
            }
            t[e] = u32x4{pack_hi(h[0], h[1]), pack_hi(h[2], h[3]), pack_hi(h[4], h[5]), pack_hi(h[6], h[7])};
        }
    }
}

// a_words for bf16 terms with the hardware's round-to-nearest-even
// conversion (v_cvt_pk_bf16_f32, two values per instruction): the same
// terms as a_words for finite values.
template <int XT>
__device__ __forceinline__ void a_words_cvt(const float (&v)[8], u32x4 (&t)[XT]) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; j++) r[j] = v[j];
#pragma unroll
    for (int e = 0; e < XT; e++) {
        uint32_t wd[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            wd[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{r[2 * q], r[2 * q + 1]}, bf16x2_t));
            if (e + 1 < XT) {
                r[2 * q] = __fsub_rn(r[2 * q], u2f(wd[q] << 16));
                r[2 * q + 1] = __fsub_rn(r[2 * q + 1], u2f(wd[q] & 0xffff0000u));
            }
        }
        t[e] = u32x4{wd[0], wd[1], wd[2], wd[3]};
    }
}

struct GemmParams {
    TileView w;
    float *out;
    const float *x;
    int64_t n;          // tokens (rows of x)
    int64_t ldx;        // row stride of x (== cols)
    const int32_t *row_index;  // optional gather of x rows
    const float *bias;
    int accumulate;
    const float *delta_b;
    const float *delta_xa;
    int delta_rank;
    int delta_stride;  // row stride of delta_xa (>= delta_rank)
    // grouped (routed experts): segment z = blockIdx.z has its own weight,
    // rows [seg[z].off, seg[z].off + seg[z].cnt) of x/out and delta
    const GroupSeg *segs;
    // GEMV activation fragments (gv_split_kernel): 16-byte words
    // [k tile][term][k quarter][xn tokens], segment z at xf + z * xf_seg
    const uint8_t *xf;
    int64_t xn, xf_seg;
};

// The GEMV regime (gemv.hip): n <= 16 tokens, or segments of at most 16.
void launch_gemv(GemmParams &p, int tf, int64_t rows, int64_t cols, bool exact, unsigned nseg, DevBuf *ws,
                 hipStream_t s);

// ---------------------------------------------------------------------------
// Per-format B fragments of k tile `t` of a 16-byte (32 for f32) tile word.

struct Raw {
    uint4 a, b;  // b only for TF_F32
};

template <int TF>
__device__ __forceinline__ Raw load_raw(const TileView &w, int64_t group, int64_t unit, int lane) {
    Raw r;
    const uint8_t *base = w.codes + (group * w.units_k + unit) * (int64_t)unit_bytes_of(TF);
    r.a = *(const uint4 *)(base + lane * 16);
    if constexpr (TF == TF_F32) r.b = *(const uint4 *)(base + 1024 + lane * 16);
    else r.b = make_uint4(0, 0, 0, 0);
    return r;
}

__device__ __forceinline__ uint32_t word_of(const uint4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Number of k tiles per unit and MFMA terms.
template <int TF> struct Fmt {
    static constexpr int tiles = TF == TF_Q8 || TF == TF_FP8 ? 2 : (TF == TF_MX4 || TF == TF_INT4) ? 4 : 1;
    // f16 and f32 weights run on the fp32 MFMA with f32 activations: every
    // product is exact, as in the CPU's f32 fused multiply-adds
    static constexpr bool fp32 = TF == TF_F16 || TF == TF_F32;
    static constexpr bool acc_scale = TF == TF_Q8;  // block scale on the partial sum
};

// Per-unit side data (scales) loaded once per unit.
struct UnitSide {
    uint32_t word;   // Q8: two f16 scales; MX4: four e8m0 bytes
};

template <int TF>
__device__ __forceinline__ UnitSide load_side(const TileView &w, int64_t row, int64_t unit) {
    UnitSide s{0};
    int64_t r = row < w.rows ? row : w.rows - 1;
    if constexpr (TF == TF_Q8) {
        s.word = *(const uint32_t *)((const uint16_t *)w.scale + r * w.scale_cols + unit * 2);
    } else if constexpr (TF == TF_MX4) {
        s.word = *(const uint32_t *)((const uint8_t *)w.scale + r * w.scale_cols + unit * 4);
    }
    return s;
}

// The FP8 / INT4 scale (and INT4 zero point) of the k tile starting at k0 of
// `row`; k beyond the matrix (codes zero there) reads the last column block.
template <int TF>
__device__ __forceinline__ float tile_scale_of(const TileView &w, int64_t row, int64_t k0, int *zp_out = nullptr) {
    const int64_t r = row < w.rows ? row : w.rows - 1;
    if constexpr (TF == TF_FP8) {
        int64_t sr;
        if (w.row_shard == 0) sr = r / w.block_rows;
        else {
            int64_t per_shard = (w.row_shard + w.block_rows - 1) / w.block_rows;
            sr = r / w.row_shard * per_shard + (r % w.row_shard) / w.block_rows;
        }
        int64_t kb = k0 / w.block_cols;
        kb = kb < w.scale_cols ? kb : w.scale_cols - 1;
        return load_scale(w.scale, sr * w.scale_cols + kb, w.scale_type);
    } else {
        int64_t g = k0 / w.group;
        g = g < w.scale_cols ? g : w.scale_cols - 1;
        if (zp_out) *zp_out = w.zero ? (int)gload<uint8_t>(w.zero + r * w.scale_cols + g) - 8 : 0;
        return load_scale(w.scale, r * w.scale_cols + g, w.scale_type);
    }
}

// bf16_rne(e4m3/e5m2 code * s) for the 8 codes of tile t.
__device__ __forceinline__ void decode_fp8(const TileView &w, const Raw &raw, int t, float s, u32x4 &bh) {
    uint32_t w0 = word_of(raw.a, 2 * t), w1 = word_of(raw.a, 2 * t + 1);
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        f[j] = bf16_to_f32(f32_to_bf16(mul_x86(fp8_value((w0 >> (8 * j)) & 0xffu, w.e5m2), s)));
        f[4 + j] = bf16_to_f32(f32_to_bf16(mul_x86(fp8_value((w1 >> (8 * j)) & 0xffu, w.e5m2), s)));
    }
    bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
}

// bf16_rne(e2m1 code * 2^e) for the 8 codes of tile t; byte t of `word` is e.
// e2m1 * 2^e has at most two significant bits, so the f32 product is the
// exact bf16 value. E8M0 255 (NaN) multiplies by infinity: every code gives
// an infinity or a NaN, and every product reading it a NaN or infinity, as
// with the reference's NaN weights (payloads aside).
__device__ __forceinline__ void decode_mx4(const Raw &raw, uint32_t word, int t, u32x4 &bh) {
    const uint32_t wd = word_of(raw.a, t);
    const float sc = e8m0_scale((word >> (8 * t)) & 0xffu);
    float f[8];
#pragma unroll
    for (int j = 0; j < 8; j++) f[j] = __fmul_rn(e2m1_value((wd >> (4 * j)) & 0xfu), sc);
    bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
}

// bf16_rne((q - zp) * s) for the 8 codes of tile t.
__device__ __forceinline__ void decode_int4(const Raw &raw, int t, float s, int zp, u32x4 &bh) {
    uint32_t wd = word_of(raw.a, t);
    float f[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int q = (int)((wd >> (4 * j)) & 0xfu) - 8;
        f[j] = bf16_to_f32(f32_to_bf16(mul_x86((float)(q - zp), s)));
    }
    bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
}

// B fragment (hi; lo for split formats) of tile t.
template <int TF>
__device__ __forceinline__ void decode_tile(const TileView &w, const Raw &raw, const UnitSide &side, int t,
                                            int64_t row, int64_t k0, u32x4 &bh, u32x4 &bl, float &tile_scale) {
    if constexpr (TF == TF_BF16) {
        bh = u32x4{raw.a.x, raw.a.y, raw.a.z, raw.a.w};
    } else if constexpr (TF == TF_F16 || TF == TF_F32) {
        // the 8 f32 weights, as bit patterns: bh = values 0..3, bl = 4..7
        if constexpr (TF == TF_F16) {
            float f[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t wd = word_of(raw.a, j / 2);
                f[j] = f16_to_f32((uint16_t)((j & 1) ? (wd >> 16) : (wd & 0xffffu)));
            }
            bh = u32x4{f2u(f[0]), f2u(f[1]), f2u(f[2]), f2u(f[3])};
            bl = u32x4{f2u(f[4]), f2u(f[5]), f2u(f[6]), f2u(f[7])};
        } else {
            bh = u32x4{raw.a.x, raw.a.y, raw.a.z, raw.a.w};
            bl = u32x4{raw.b.x, raw.b.y, raw.b.z, raw.b.w};
        }
    } else if constexpr (TF == TF_Q8) {
        uint32_t w0 = word_of(raw.a, 2 * t), w1 = word_of(raw.a, 2 * t + 1);
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            f[j] = (float)(int8_t)((w0 >> (8 * j)) & 0xffu);
            f[4 + j] = (float)(int8_t)((w1 >> (8 * j)) & 0xffu);
        }
        bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
        uint16_t sb = (uint16_t)((side.word >> (16 * t)) & 0xffffu);
        tile_scale = f16_to_f32_hw(sb);
    } else if constexpr (TF == TF_FP8) {
        decode_fp8(w, raw, t, tile_scale_of<TF>(w, row, k0), bh);
    } else if constexpr (TF == TF_MX4) {
        decode_mx4(raw, side.word, t, bh);
    } else if constexpr (TF == TF_INT4) {
        int zp;
        const float s = tile_scale_of<TF>(w, row, k0, &zp);
        decode_int4(raw, t, s, zp, bh);
    }
}

// acc += (sum of the activation terms) . B, with the format's structure
// (NR < 4: only the first NR of the lane's four tokens are used, so the
// block-scale multiply-adds of the others are skipped)
template <int TF, int XT, int NR = 4>
__device__ __forceinline__ void mac(floatx4 &acc, const u32x4 (&x)[XT], const u32x4 &bh, const u32x4 &bl,
                                    float tile_scale) {
    if constexpr (Fmt<TF>::acc_scale) {
        floatx4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < XT; e++) t = mfma_bf16(x[e], bh, t);
#pragma unroll
        for (int r = 0; r < NR; r++) acc[r] = __builtin_fmaf(tile_scale, t[r], acc[r]);
    } else if constexpr (Fmt<TF>::fp32) {
        // 8 rank-4 steps over k = 8 * (lane / 16) + s: A and B hold the same
        // k in the same register, so the 32 products of the tile are summed
#pragma unroll
        for (int s = 0; s < 4; s++) acc = mfma_f32(u2f(x[0][s]), u2f(bh[s]), acc);
#pragma unroll
        for (int s = 0; s < 4; s++) acc = mfma_f32(u2f(x[1][s]), u2f(bl[s]), acc);
    } else {
#pragma unroll
        for (int e = 0; e < XT; e++) acc = mfma_bf16(x[e], bh, acc);
    }
}

// Loads the A fragment (8 activations of token `tok`, k0..k0+8) from global.
__device__ __forceinline__ void load_x8(const GemmParams &p, int64_t tok, int64_t k0, float (&v)[8], bool vec_ok) {
    int64_t K = p.w.cols;
    if (tok >= p.n) {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = 0.f;
        return;
    }
    int64_t src = p.row_index ? (int64_t)p.row_index[tok] : tok;
    const float *xr = p.x + src * p.ldx;
    if (vec_ok && k0 + 8 <= K) {
        float4 a = *(const float4 *)(xr + k0), b = *(const float4 *)(xr + k0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = (k0 + j < K) ? xr[k0 + j] : 0.f;
    }
}

// Epilogue of a lane's tile (tokens tb[m] + r, rows rw[i]): out = acc + delta
// (the rank-k sum from 0 in j order) + bias (+ the old output), one 16-token
// block at a time. The block's operands (delta factors, bias, old outputs)
// are all read before its first store, so their loads are in flight
// together (element by element, each read of an output would wait for the
// possibly aliasing store before it).
template <int NM, int NI>
__device__ __forceinline__ void store_block(const GemmParams &p, const int64_t (&tb)[NM], const int64_t (&rw)[NI],
                                            const floatx4 (&acc)[NM][NI]) {
    bool rin[NI];
    float bias[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        rin[i] = rw[i] < p.w.rows;
        bias[i] = p.bias && rin[i] ? p.bias[rw[i]] : 0.f;
    }
#pragma unroll
    for (int m = 0; m < NM; m++) {
        bool tin[4];
#pragma unroll
        for (int r = 0; r < 4; r++) tin[r] = tb[m] + r < p.n;
        floatx4 v[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) v[i] = acc[m][i];
        if (p.delta_rank > 0) {
            floatx4 d[NI];
#pragma unroll
            for (int i = 0; i < NI; i++) d[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            for (int j = 0; j < p.delta_rank; j++) {
                float bj[NI], xj[4];
#pragma unroll
                for (int i = 0; i < NI; i++) bj[i] = rin[i] ? p.delta_b[rw[i] * p.delta_rank + j] : 0.f;
#pragma unroll
                for (int r = 0; r < 4; r++) xj[r] = tin[r] ? p.delta_xa[(tb[m] + r) * p.delta_stride + j] : 0.f;
#pragma unroll
                for (int i = 0; i < NI; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) d[i][r] = __fadd_rn(d[i][r], __fmul_rn(bj[i], xj[r]));
            }
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) v[i][r] = __fadd_rn(v[i][r], d[i][r]);
        }
        if (p.bias) {
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) v[i][r] = __fadd_rn(v[i][r], bias[i]);
        }
        if (p.accumulate) {
            floatx4 old[NI];
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) old[i][r] = rin[i] && tin[r] ? p.out[(tb[m] + r) * p.w.rows + rw[i]] : 0.f;
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) v[i][r] = __fadd_rn(old[i][r], v[i][r]);
        }
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (rin[i] && tin[r]) p.out[(tb[m] + r) * p.w.rows + rw[i]] = v[i][r];
    }
}

// Rebases the parameters on segment blockIdx.z of a grouped product: the
// segment's weight, its row window of x/out (tokens are local to the window)
// and its delta. Returns false when the block has no rows to do.
__device__ __forceinline__ bool select_segment(GemmParams &p, int64_t m0) {
    if (!p.segs) return m0 < p.n;
    const GroupSeg &s = p.segs[blockIdx.z];
    if (m0 >= s.cnt) return false;
    p.w = s.w;
    p.n = s.cnt;
    p.out += (int64_t)s.off * s.w.rows;
    if (p.row_index) p.row_index += s.off;
    else p.x += (int64_t)s.off * p.ldx;
    p.ldx = s.w.cols;
    p.delta_rank = s.delta_rank;
    p.delta_b = s.delta_b;
    p.delta_xa = s.delta_rank ? p.delta_xa + (int64_t)s.off * p.delta_stride : nullptr;
    if (p.xf) p.xf += (int64_t)blockIdx.z * p.xf_seg;
    return true;
}


// ---------------------------------------------------------------------------
// MX (scaled-MFMA) activation fragments

// Activation fragments: per 16-token block and 128-k stage a 6400-byte block
// (lane l: token 16 m16 + l % 16, k = 128 stage + 32 (l / 16) .. +32; the
// 32 fp6 codes of a term are 6 dwords, code j at bits 6j..6j+5):
//     [term][lane] 16 B   dwords 0..3 of each term       4 x 1 KiB
//     [term][lane] 8 B    dwords 4..5                    4 x 512 B
//     [lane] 4 B          E8M0 byte of term e in byte e  256 B
// so that every part is read with one conflict-free LDS load per lane and
// copied in whole KiB (the last 256 B apart).

constexpr int MX_TERMS = 4;
constexpr int MX_BLOCK = 6400;  // bytes per 16 tokens x 128 k

// Writes the MX_TERMS fp6 terms of the 32 values r (one E8M0 block) into lane
// slot `slot` of a fragment block (slot = token % 16 + 16 * block within the
// stage); r is left holding the remainder. A NaN or infinity among the 32
// values gives the slot E8M0 255 (NaN) in every term, so that every product
// reading it is NaN. SLOTS: the slots of the block (64 in a fragment block;
// fewer for a staging copy that holds part of the slots in the same order).
template <int SLOTS = 64>
__device__ __forceinline__ void mx_write_slot(float (&r)[32], uint8_t *blk, int slot) {
    typedef float v16f_t __attribute__((ext_vector_type(16)));
    u32x4 *lo = (u32x4 *)blk + slot;                                        // + SLOTS e
    uint2 *hi = (uint2 *)(blk + 16 * MX_TERMS * SLOTS) + slot;              // + SLOTS e
    uint32_t *scw = (uint32_t *)(blk + 24 * MX_TERMS * SLOTS) + slot;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < 32; j++) finite = finite && __builtin_isfinite(r[j]);
    if (!finite) {
#pragma unroll
        for (int e = 0; e < MX_TERMS; e++) {
            lo[SLOTS * e] = u32x4{0, 0, 0, 0};
            hi[SLOTS * e] = make_uint2(0, 0);
        }
        *scw = 0xffffffffu;
        return;
    }
    uint32_t scales = 0;
#pragma unroll
    for (int e = 0; e < MX_TERMS; e++) {
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++) m = fmaxf(m, fabsf(r[j]));
        // scale 2^x with m / 2^x in (3.75, 7.5]: m = f 2^E, f in [1, 2)
        const uint32_t mb = __builtin_bit_cast(uint32_t, m);
        int x = (int)(mb >> 23) - 129 + ((mb & 0x7fffffu) > 0x700000u ? 1 : 0);  // E - 2 (+1 when f > 1.875)
        const bool live = m > 0.f && x >= -126;  // remainders under 7.5 * 2^-127 stay in r: codes 0
        x = live ? x : -127;
        scales |= (uint32_t)(x + 127) << (8 * e);
        const float sc = __builtin_bit_cast(float, (uint32_t)(live ? x + 127 : 127) << 23);
        // v_cvt_scalef32_2xpk16_fp6_f32: round-to-nearest-even e2m3 of v / sc,
        // code 2j from the first operand's element j and 2j + 1 from the
        // second's; the reverse conversion gives code * sc exactly, so the
        // subtraction below is exact (the value and its rounding are within
        // a factor of two, or the code is zero)
        v16f_t ev, od;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            ev[j] = live ? r[2 * j] : 0.f;
            od[j] = live ? r[2 * j + 1] : 0.f;
        }
        const auto d = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(ev, od, sc);
        const auto back = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(d, sc);
#pragma unroll
        for (int j = 0; j < 32; j++) r[j] = __fsub_rn(r[j], back[j]);
        lo[SLOTS * e] = u32x4{(uint32_t)d[0], (uint32_t)d[1], (uint32_t)d[2], (uint32_t)d[3]};
        hi[SLOTS * e] = make_uint2((uint32_t)d[4], (uint32_t)d[5]);
    }
    *scw = scales;
}

// Sum over the 16 lanes of a DPP row (lanes 16 r .. 16 r + 15): quad swaps,
// then the half-row and row mirrors; every lane of the row holds the total.
__device__ __forceinline__ float row16_sum(float v) {
    v = __fadd_rn(v, u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0xB1, 0xf, 0xf, false)));
    v = __fadd_rn(v, u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0x4E, 0xf, 0xf, false)));
    v = __fadd_rn(v, u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0x141, 0xf, 0xf, false)));
    v = __fadd_rn(v, u2f((uint32_t)__builtin_amdgcn_mov_dpp((int)f2u(v), 0x140, 0xf, 0xf, false)));
    return v;
}

}  // namespace ditch
