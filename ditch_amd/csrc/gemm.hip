// gemm.hip — dequant-fused matrix products on MFMA (gfx950).
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
};

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
        tile_scale = f16_to_f32(sb);
    } else if constexpr (TF == TF_FP8) {
        int64_t r = row < w.rows ? row : w.rows - 1;
        int64_t sr;
        if (w.row_shard == 0) sr = r / w.block_rows;
        else {
            int64_t per_shard = (w.row_shard + w.block_rows - 1) / w.block_rows;
            sr = r / w.row_shard * per_shard + (r % w.row_shard) / w.block_rows;
        }
        float s = load_scale(w.scale, sr * w.scale_cols + k0 / w.block_cols, w.scale_type);
        uint32_t w0 = word_of(raw.a, 2 * t), w1 = word_of(raw.a, 2 * t + 1);
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            f[j] = bf16_to_f32(f32_to_bf16(mul_x86(fp8_value((w0 >> (8 * j)) & 0xffu, w.e5m2), s)));
            f[4 + j] = bf16_to_f32(f32_to_bf16(mul_x86(fp8_value((w1 >> (8 * j)) & 0xffu, w.e5m2), s)));
        }
        bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
    } else if constexpr (TF == TF_MX4) {
        uint32_t wd = word_of(raw.a, t);
        uint32_t sb = (side.word >> (8 * t)) & 0xffu;
        float sc = e8m0_scale(sb);
        float f[8];
        if (sb != 255u) {
            // e2m1 * 2^e has at most two significant bits: the product is the
            // exact bf16 value, so its high half is the rounded result.
#pragma unroll
            for (int j = 0; j < 8; j++) f[j] = __fmul_rn(e2m1_value((wd >> (4 * j)) & 0xfu), sc);
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) f[j] = bf16_to_f32(f32_to_bf16(mul_x86(e2m1_value((wd >> (4 * j)) & 0xfu), sc)));
        }
        bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
    } else if constexpr (TF == TF_INT4) {
        int64_t r = row < w.rows ? row : w.rows - 1;
        int64_t g = k0 / w.group;
        float s = load_scale(w.scale, r * w.scale_cols + g, w.scale_type);
        int zp = w.zero ? (int)w.zero[r * w.scale_cols + g] - 8 : 0;
        uint32_t wd = word_of(raw.a, t);
        float f[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int q = (int)((wd >> (4 * j)) & 0xfu) - 8;
            f[j] = bf16_to_f32(f32_to_bf16(mul_x86((float)(q - zp), s)));
        }
        bh = u32x4{pack_hi(f[0], f[1]), pack_hi(f[2], f[3]), pack_hi(f[4], f[5]), pack_hi(f[6], f[7])};
    }
}

// acc += (sum of the activation terms) . B, with the format's structure
template <int TF, int XT>
__device__ __forceinline__ void mac(floatx4 &acc, const u32x4 (&x)[XT], const u32x4 &bh, const u32x4 &bl,
                                    float tile_scale) {
    if constexpr (Fmt<TF>::acc_scale) {
        floatx4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < XT; e++) t = mfma_bf16(x[e], bh, t);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(tile_scale, t[r], acc[r]);
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

// Epilogue for one output element.
__device__ __forceinline__ void store_out(const GemmParams &p, int64_t tok, int64_t row, float v) {
    if (tok >= p.n || row >= p.w.rows) return;
    if (p.delta_rank > 0) {
        float d = 0.f;
        for (int j = 0; j < p.delta_rank; j++)
            d = __fadd_rn(d, __fmul_rn(p.delta_b[row * p.delta_rank + j], p.delta_xa[tok * p.delta_stride + j]));
        v = __fadd_rn(v, d);
    }
    if (p.bias) v = __fadd_rn(v, p.bias[row]);
    float *o = p.out + tok * p.w.rows + row;
    if (p.accumulate) v = __fadd_rn(*o, v);
    *o = v;
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
    return true;
}

// ---------------------------------------------------------------------------
// GEMV regime (n <= 16): one 16-token fragment, NT 16-row groups per block,
// K split over the 4 waves and reduced through LDS.

template <int TF, int NT, int XT>
__global__ __launch_bounds__(256) void gemv_kernel(GemmParams p) {
    if (!select_segment(p, 0)) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t groups = (p.w.rows + 15) / 16;
    const int64_t g0 = (int64_t)blockIdx.x * NT;
    if (g0 >= groups) return;
    const int64_t units = p.w.units_k;
    const int64_t per = (units + 3) / 4;
    const int64_t u0 = wave * per;
    const int64_t u1 = u0 + per < units ? u0 + per : units;
    const int UK = unit_k_of(TF);
    const bool vec_ok = (p.ldx % 4 == 0) && (((uintptr_t)p.x & 15) == 0);
    const int64_t tok = lane % 16;
    const int kq = lane / 16;

    floatx4 acc[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int64_t u = u0; u < u1; u++) {
        Raw raw[NT];
        UnitSide side[NT];
#pragma unroll
        for (int i = 0; i < NT; i++) {
            int64_t g = g0 + i < groups ? g0 + i : groups - 1;
            raw[i] = load_raw<TF>(p.w, g, u, lane);
            side[i] = load_side<TF>(p.w, g * 16 + lane % 16, u);
        }
#pragma unroll
        for (int t = 0; t < Fmt<TF>::tiles; t++) {
            int64_t k0 = u * UK + 32 * t + 8 * kq;
            float xv[8];
            load_x8(p, tok, k0, xv, vec_ok);
            u32x4 xt[XT];
            a_words<Fmt<TF>::fp32, XT>(xv, xt);
#pragma unroll
            for (int i = 0; i < NT; i++) {
                u32x4 bh, bl = u32x4{0, 0, 0, 0};
                float ts = 1.f;
                decode_tile<TF>(p.w, raw[i], side[i], t, (g0 + i) * 16 + lane % 16, k0, bh, bl, ts);
                mac<TF, XT>(acc[i], xt, bh, bl, ts);
            }
        }
    }
    // reduce the four K slices
    __shared__ floatx4 red[3][NT][64];
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < NT; i++) red[wave - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < NT; i++) {
            floatx4 a = acc[i];
#pragma unroll
            for (int w = 0; w < 3; w++) {
                floatx4 b = red[w][i][lane];
                a[0] += b[0]; a[1] += b[1]; a[2] += b[2]; a[3] += b[3];
            }
            int64_t row = (g0 + i) * 16 + lane % 16;
#pragma unroll
            for (int r = 0; r < 4; r++) store_out(p, 4 * kq + r, row, a[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// GEMM regime: block tile 16*MT tokens x 64*NT rows; the activation tile of
// one unit is staged in LDS as hi/lo fragments, each wave streams its own
// 16*NT weight rows straight from HBM into registers.

template <int TF, int MT, int NT, int XT>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    constexpr int UK = TF == TF_Q8 || TF == TF_FP8 ? 64 : (TF == TF_MX4 || TF == TF_INT4) ? 128 : 32;
    constexpr int TILES = UK / 32;
    constexpr int BM = 16 * MT;
    // [mt][t][term][lane] 16-byte words
    __shared__ u32x4 xs[MT][TILES][XT][64];

    const int64_t m0 = (int64_t)blockIdx.y * BM;
    if (!select_segment(p, m0)) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t groups = (p.w.rows + 15) / 16;
    const int64_t g0 = (int64_t)blockIdx.x * (4 * NT) + wave * NT;
    if (g0 - wave * NT >= groups) return;
    const int64_t units = p.w.units_k;
    const bool vec_ok = (p.ldx % 4 == 0) && (((uintptr_t)p.x & 15) == 0);
    const int kq = lane / 16;

    floatx4 acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int i = 0; i < NT; i++) acc[m][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int64_t u = 0; u < units; u++) {
        Raw raw[NT];
        UnitSide side[NT];
#pragma unroll
        for (int i = 0; i < NT; i++) {
            int64_t g = g0 + i < groups ? g0 + i : groups - 1;
            raw[i] = load_raw<TF>(p.w, g, u, lane);
            side[i] = load_side<TF>(p.w, g * 16 + lane % 16, u);
        }
        __syncthreads();
        // stage BM x UK activations: BM * UK / 8 groups of 8 over 256 threads
        constexpr int NG = BM * UK / 8;
#pragma unroll
        for (int q0 = 0; q0 < NG; q0 += 256) {
            int q = q0 + threadIdx.x;
            if (q < NG) {
                int i = q % BM, g8 = q / BM;
                float xv[8];
                load_x8(p, m0 + i, u * UK + 8 * g8, xv, vec_ok);
                u32x4 xt[XT];
                a_words<Fmt<TF>::fp32, XT>(xv, xt);
                int t = g8 / 4, sl = (i % 16) + 16 * (g8 % 4);
#pragma unroll
                for (int e = 0; e < XT; e++) xs[i / 16][t][e][sl] = xt[e];
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TILES; t++) {
            int64_t k0 = u * UK + 32 * t + 8 * kq;
            u32x4 bh[NT], bl[NT];
            float ts[NT];
#pragma unroll
            for (int i = 0; i < NT; i++) {
                bl[i] = u32x4{0, 0, 0, 0};
                ts[i] = 1.f;
                decode_tile<TF>(p.w, raw[i], side[i], t, (g0 + i) * 16 + lane % 16, k0, bh[i], bl[i], ts[i]);
            }
#pragma unroll
            for (int m = 0; m < MT; m++) {
                u32x4 xt[XT];
#pragma unroll
                for (int e = 0; e < XT; e++) xt[e] = xs[m][t][e][lane];
#pragma unroll
                for (int i = 0; i < NT; i++) mac<TF, XT>(acc[m][i], xt, bh[i], bl[i], ts[i]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int i = 0; i < NT; i++) {
            int64_t row = (g0 + i) * 16 + lane % 16;
#pragma unroll
            for (int r = 0; r < 4; r++) store_out(p, m0 + 16 * m + 4 * kq + r, row, acc[m][i][r]);
        }
}

// ---------------------------------------------------------------------------

template <int TF, int XT>
static void dispatch(const GemmParams &p, int64_t max_rows, int64_t n_for_shape, unsigned nseg, hipStream_t s) {
    int64_t groups = (max_rows + 15) / 16;
    if (n_for_shape <= 16) {
        constexpr int NT = 1;
        dim3 grid((unsigned)((groups + NT - 1) / NT), 1, nseg);
        hipLaunchKernelGGL((gemv_kernel<TF, NT, XT>), grid, dim3(256), 0, s, p);
    } else if (n_for_shape <= 64 || XT > 2) {
        constexpr int MT = 4, NT = 2;
        dim3 grid((unsigned)((groups + 4 * NT - 1) / (4 * NT)), (unsigned)((n_for_shape + 16 * MT - 1) / (16 * MT)), nseg);
        hipLaunchKernelGGL((gemm_kernel<TF, MT, NT, XT>), grid, dim3(256), 0, s, p);
    } else {
        constexpr int MT = 8, NT = 2;
        dim3 grid((unsigned)((groups + 4 * NT - 1) / (4 * NT)), (unsigned)((n_for_shape + 16 * MT - 1) / (16 * MT)), nseg);
        hipLaunchKernelGGL((gemm_kernel<TF, MT, NT, XT>), grid, dim3(256), 0, s, p);
    }
}

template <int TF>
static void dispatch_xt(const GemmParams &p, int64_t max_rows, int64_t n_for_shape, unsigned nseg, bool exact,
                        hipStream_t s) {
    if (Fmt<TF>::fp32) dispatch<TF, 2>(p, max_rows, n_for_shape, nseg, s);  // f32 activations, exact products
    else if (exact) dispatch<TF, 3>(p, max_rows, n_for_shape, nseg, s);
    else dispatch<TF, 2>(p, max_rows, n_for_shape, nseg, s);
}

static void dispatch_tf(int tf, const GemmParams &p, int64_t max_rows, int64_t n_for_shape, unsigned nseg, bool exact,
                        hipStream_t s) {
    switch (tf) {
    case TF_BF16: dispatch_xt<TF_BF16>(p, max_rows, n_for_shape, nseg, exact, s); break;
    case TF_F16: dispatch_xt<TF_F16>(p, max_rows, n_for_shape, nseg, exact, s); break;
    case TF_F32: dispatch_xt<TF_F32>(p, max_rows, n_for_shape, nseg, exact, s); break;
    case TF_Q8: dispatch_xt<TF_Q8>(p, max_rows, n_for_shape, nseg, exact, s); break;
    case TF_FP8: dispatch_xt<TF_FP8>(p, max_rows, n_for_shape, nseg, exact, s); break;
    case TF_MX4: dispatch_xt<TF_MX4>(p, max_rows, n_for_shape, nseg, exact, s); break;
    case TF_INT4: dispatch_xt<TF_INT4>(p, max_rows, n_for_shape, nseg, exact, s); break;
    default: throw Error{DITCH_UNSUPPORTED, "tile format"};
    }
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_matmul(const TileView &w, float *out, const float *x, int64_t n, const MatmulEpilogue &ep, hipStream_t s,
                   const int32_t *row_index) {
    if (n <= 0 || w.rows <= 0) return;
    GemmParams p{};
    p.w = w;
    p.out = out;
    p.x = x;
    p.n = n;
    p.ldx = w.cols;
    p.row_index = row_index;
    p.bias = ep.bias;
    p.accumulate = ep.accumulate;
    p.delta_b = ep.delta_b;
    p.delta_xa = ep.delta_xa;
    p.delta_rank = ep.delta_rank;
    p.delta_stride = ep.delta_rank;
    p.segs = nullptr;
    dispatch_tf(w.tf, p, w.rows, n, 1, ep.exact != 0, s);
}

void launch_matmul_grouped(const GroupSeg *d_segs, unsigned nseg, int tf, int64_t rows, int64_t cols, int64_t max_cnt,
                           float *out, const float *x, const int32_t *row_index, const float *delta_xa,
                           int delta_stride, hipStream_t s) {
    if (nseg == 0 || max_cnt <= 0) return;
    GemmParams p{};
    p.out = out;
    p.x = x;
    p.n = max_cnt;
    p.ldx = cols;
    p.row_index = row_index;
    p.delta_xa = delta_xa;
    p.delta_stride = delta_stride;
    p.segs = d_segs;
    p.w.rows = rows;
    p.w.cols = cols;
    dispatch_tf(tf, p, rows, max_cnt, nseg, false, s);
}

}  // namespace ditch
