// gemm_tile.hip — the large-batch product (prompt forward, n >= 128 tokens).
//
// out[n][rows] = x[n][cols] @ W^T (tensor.matmulT, tensor.zig:1023-1045) for
// weights whose decode the gfx950 conversion instructions do exactly
// (TileView::fast): bf16, MXFP4, FP8, INT4, Q8_0.
//
// Two kernels:
//
// split_kernel writes the activations once as bf16 MFMA A fragments, XT
// terms per value (x = t0 + t1 (+ t2), each the round-to-nearest-even bf16
// of the remainder), in the order the product reads them:
//     xs[m16][kt][term][lane] (16 B each), lane l = token 16*m16 + l%16,
//     k = 32*kt + 8*(l/16) .. +8
// so every A fragment is one contiguous KiB. k tiles past the matrix are
// zero up to an even count.
//
// tile_gemm_kernel: a workgroup of WAVES waves computes BM = 16*WM tokens x
// BN = 16*WN*WAVES weight rows. The A fragments of a 64-wide k stage are
// staged in LDS (double buffered, each wave copies whole fragments with
// 16-byte loads) and read by every wave; each wave owns WN row groups of
// the weight and streams their tiles from HBM straight into registers two
// stages ahead, decoding them with v_cvt_scalef32_pk_bf16_fp4 (MXFP4),
// v_cvt_pk_f32_fp8 + f32 scale + v_cvt_pk_bf16_f32 (FP8), or integer
// unpacking (INT4, Q8_0). The block index is remapped so that the
// workgroups an XCD runs at the same time cover an 8 x (few) patch of output
// tiles: they share A and W tiles in that XCD's L2.
#include "gemm_common.h"

namespace ditch {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// activation fragments

struct SplitParams {
    u32x4 *xs;
    const float *x;
    const int32_t *row_index;  // optional gather of x rows
    int64_t n, ldx, K;
    int64_t kt_total;  // k tiles per 16-token block (even)
    int64_t m16;       // 16-token blocks
};

template <int XT>
__global__ __launch_bounds__(256) void split_kernel(SplitParams p) {
    int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.m16 * p.kt_total * 64) return;
    const int lane = (int)(t & 63);
    const int64_t f = t >> 6;  // fragment = m16 * kt_total + kt
    const int64_t kt = f % p.kt_total, mb = f / p.kt_total;
    const int64_t tok = mb * 16 + (lane & 15);
    const int64_t k0 = kt * 32 + 8 * (lane >> 4);
    float v[8];
    if (tok < p.n) {
        int64_t src = p.row_index ? (int64_t)p.row_index[tok] : tok;
        const float *xr = p.x + src * p.ldx;
        if (k0 + 8 <= p.K && ((((uintptr_t)(xr + k0)) & 15) == 0)) {
            float4 a = *(const float4 *)(xr + k0), b = *(const float4 *)(xr + k0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (k0 + j < p.K) ? xr[k0 + j] : 0.f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = 0.f;
    }
    u32x4 w[XT];
    a_words<false, XT>(v, w);
#pragma unroll
    for (int e = 0; e < XT; e++) p.xs[(f * XT + e) * 64 + lane] = w[e];
}

// ---------------------------------------------------------------------------
// per-format weight stages (64 k = two 32-wide MFMA tiles per lane)

__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    bf16x2_t v;
    v.x = (__bf16)a;  // v_cvt_pk_bf16_f32: round to nearest even
    v.y = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
}

template <int TF> struct BSt;
template <> struct BSt<TF_BF16> { uint4 a, b; };
template <> struct BSt<TF_MX4> { uint2 c; uint32_t sw; };
template <> struct BSt<TF_FP8> { uint4 c; float sc; };
template <> struct BSt<TF_INT4> { uint2 c; float sc; int32_t zf; };
template <> struct BSt<TF_Q8> { uint4 c; uint32_t sw; };

// Per-lane constants of one row group.
struct RowCtx {
    int64_t g;    // row group (clamped to the matrix)
    int64_t row;  // weight row of this lane (clamped)
    int64_t srow; // FP8: row of the scale grid
};

__device__ __forceinline__ RowCtx row_ctx(const TileView &w, int64_t g, int lane) {
    RowCtx c;
    c.g = g;
    int64_t r = g * 16 + (lane & 15);
    c.row = r < w.rows ? r : w.rows - 1;
    c.srow = 0;
    if (w.tf == TF_FP8) {
        if (w.row_shard == 0) c.srow = c.row / w.block_rows;
        else {
            int64_t per_shard = (w.row_shard + w.block_rows - 1) / w.block_rows;
            c.srow = c.row / w.row_shard * per_shard + (c.row % w.row_shard) / w.block_rows;
        }
    }
    return c;
}

template <int TF>
__device__ __forceinline__ void load_stage(const TileView &w, const RowCtx &rc, int64_t s, int lane, BSt<TF> &b) {
    const uint8_t *grp = w.codes + rc.g * w.units_k * 1024;
    if constexpr (TF == TF_BF16) {
        // units 2s and 2s + 1 (the second is absent past an odd unit count)
        b.a = *(const uint4 *)(grp + (2 * s) * 1024 + lane * 16);
        if (2 * s + 1 < w.units_k) b.b = *(const uint4 *)(grp + (2 * s + 1) * 1024 + lane * 16);
        else b.b = make_uint4(0, 0, 0, 0);
    } else if constexpr (TF == TF_MX4) {
        int64_t u = s >> 1;
        b.c = *(const uint2 *)(grp + u * 1024 + lane * 16 + 8 * (s & 1));
        b.sw = *(const uint32_t *)((const uint8_t *)w.scale + rc.row * w.scale_cols + u * 4);
    } else if constexpr (TF == TF_FP8) {
        b.c = *(const uint4 *)(grp + s * 1024 + lane * 16);
        b.sc = load_scale(w.scale, rc.srow * w.scale_cols + (s * 64) / w.block_cols, w.scale_type);
    } else if constexpr (TF == TF_INT4) {
        int64_t u = s >> 1;
        b.c = *(const uint2 *)(grp + u * 1024 + lane * 16 + 8 * (s & 1));
        int64_t gi = rc.row * w.scale_cols + (s * 64) / w.group;
        b.sc = load_scale(w.scale, gi, w.scale_type);
        b.zf = w.zero ? (int32_t)w.zero[gi] : 8;
    } else if constexpr (TF == TF_Q8) {
        b.c = *(const uint4 *)(grp + s * 1024 + lane * 16);
        b.sw = *(const uint32_t *)((const uint16_t *)w.scale + rc.row * w.scale_cols + 2 * s);
    }
}

// B fragment of tile t (0, 1) of stage s; `ts` is the partial-sum scale (Q8_0).
template <int TF>
__device__ __forceinline__ void decode_stage(const BSt<TF> &b, int64_t s, int t, u32x4 &f, float &ts) {
    ts = 1.f;
    if constexpr (TF == TF_BF16) {
        const uint4 &v = t ? b.b : b.a;
        f = u32x4{v.x, v.y, v.z, v.w};
    } else if constexpr (TF == TF_MX4) {
        uint32_t wd = t ? b.c.y : b.c.x;
        uint32_t sb = (b.sw >> (8 * (2 * (uint32_t)(s & 1) + t))) & 0xffu;
        float sc = u2f(sb ? (sb << 23) : 0x00400000u);  // 2^(b-127); byte 0 is the subnormal 2^-127
        f[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 0));
        f[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 1));
        f[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 2));
        f[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, sc, 3));
    } else if constexpr (TF == TF_FP8) {
        uint32_t w0 = t ? b.c.z : b.c.x, w1 = t ? b.c.w : b.c.y;
        floatx2 p0 = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false), p1 = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
        floatx2 p2 = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false), p3 = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
        f[0] = cvt_pk_bf16(__fmul_rn(p0.x, b.sc), __fmul_rn(p0.y, b.sc));
        f[1] = cvt_pk_bf16(__fmul_rn(p1.x, b.sc), __fmul_rn(p1.y, b.sc));
        f[2] = cvt_pk_bf16(__fmul_rn(p2.x, b.sc), __fmul_rn(p2.y, b.sc));
        f[3] = cvt_pk_bf16(__fmul_rn(p3.x, b.sc), __fmul_rn(p3.y, b.sc));
    } else if constexpr (TF == TF_INT4) {
        uint32_t wd = t ? b.c.y : b.c.x;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = __fmul_rn((float)((int32_t)((wd >> (4 * j)) & 0xfu) - b.zf), b.sc);
        f = u32x4{cvt_pk_bf16(v[0], v[1]), cvt_pk_bf16(v[2], v[3]), cvt_pk_bf16(v[4], v[5]), cvt_pk_bf16(v[6], v[7])};
    } else if constexpr (TF == TF_Q8) {
        uint32_t w0 = t ? b.c.z : b.c.x, w1 = t ? b.c.w : b.c.y;
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = (float)(int8_t)((w0 >> (8 * j)) & 0xffu);
            v[4 + j] = (float)(int8_t)((w1 >> (8 * j)) & 0xffu);
        }
        f = u32x4{pack_hi(v[0], v[1]), pack_hi(v[2], v[3]), pack_hi(v[4], v[5]), pack_hi(v[6], v[7])};
        ts = f16_to_f32((uint16_t)((b.sw >> (16 * t)) & 0xffffu));
    }
}

// ---------------------------------------------------------------------------

struct TileGemmParams {
    TileView w;
    const u32x4 *xs;
    int64_t kt_total;
    float *out;
    int64_t ldo;
    int64_t n;
    const float *bias;
    int accumulate;
    const float *delta_b;
    const float *delta_xa;
    int delta_rank;
    int delta_stride;
    int tiles_m, tiles_n;
};

// Block -> output tile. Consecutive blocks are dispatched round robin over
// the 8 XCDs; renumber them so that each XCD receives a contiguous run of
// tiles, and walk tiles in groups of 8 m-tiles per n-tile so that the
// blocks resident on one XCD at a time share their A and W tiles in L2.
__device__ __forceinline__ void map_tile(int g, int G, int tm, int tn, int &mt, int &nt) {
    int xcd = g & 7, j = g >> 3;
    int per = G >> 3, rem = G & 7;
    int t = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + j;
    const int GM = 8;
    int width = GM * tn;
    int grp = t / width, first = grp * GM;
    int gs = tm - first < GM ? tm - first : GM;
    int r = t - grp * width;
    mt = first + r % gs;
    nt = r / gs;
}

__device__ __forceinline__ void tile_store(const TileGemmParams &p, int64_t tok, int64_t row, float v) {
    if (tok >= p.n || row >= p.w.rows) return;
    if (p.delta_rank > 0) {
        float d = 0.f;
        for (int j = 0; j < p.delta_rank; j++)
            d = __fadd_rn(d, __fmul_rn(p.delta_b[row * p.delta_rank + j], p.delta_xa[tok * p.delta_stride + j]));
        v = __fadd_rn(v, d);
    }
    if (p.bias) v = __fadd_rn(v, p.bias[row]);
    float *o = p.out + tok * p.ldo + row;
    if (p.accumulate) v = __fadd_rn(*o, v);
    *o = v;
}

template <int TF, int XT, int WAVES, int WN, int WM>
__global__ __launch_bounds__(WAVES * 64) void tile_gemm_kernel(TileGemmParams p) {
    constexpr int FR = WM * 2 * XT;   // A fragments per stage: [m][t][term]
    constexpr int PER = FR / WAVES;   // fragments each wave copies per stage
    static_assert(FR % WAVES == 0, "stage fragments must split evenly over the waves");
    __shared__ u32x4 As[2][FR][64];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int mt, nt;
    map_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, mt, nt);
    const int64_t groups = (p.w.rows + 15) / 16;
    const int64_t g0 = (int64_t)nt * (WN * WAVES) + wave * WN;
    const int64_t m16_0 = (int64_t)mt * WM, m16_n = (p.n + 15) / 16;
    const int64_t S = p.kt_total / 2;

    RowCtx rc[WN];
#pragma unroll
    for (int i = 0; i < WN; i++) rc[i] = row_ctx(p.w, g0 + i < groups ? g0 + i : groups - 1, lane);

    u32x4 ar[PER];
    auto load_a = [&](int64_t s) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int f = wave + WAVES * j;
            const int m = f / (2 * XT), t = (f / XT) % 2, e = f % XT;
            int64_t mb = m16_0 + m;
            mb = mb < m16_n ? mb : m16_n - 1;
            ar[j] = p.xs[((mb * p.kt_total + 2 * s + t) * XT + e) * 64 + lane];
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int j = 0; j < PER; j++) As[buf][wave + WAVES * j][lane] = ar[j];
    };

    floatx4 acc[WM][WN];
#pragma unroll
    for (int m = 0; m < WM; m++)
#pragma unroll
        for (int i = 0; i < WN; i++) acc[m][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    BSt<TF> bs[2][WN];
    auto load_b = [&](int slot, int64_t s) {
#pragma unroll
        for (int i = 0; i < WN; i++) load_stage<TF>(p.w, rc[i], s, lane, bs[slot][i]);
    };
    auto compute = [&](int buf, int slot, int64_t s) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            u32x4 bf[WN];
            float ts[WN];
#pragma unroll
            for (int i = 0; i < WN; i++) decode_stage<TF>(bs[slot][i], s, t, bf[i], ts[i]);
#pragma unroll
            for (int m = 0; m < WM; m++) {
                u32x4 a[XT];
#pragma unroll
                for (int e = 0; e < XT; e++) a[e] = As[buf][(m * 2 + t) * XT + e][lane];
#pragma unroll
                for (int i = 0; i < WN; i++) mac<TF, XT>(acc[m][i], a, bf[i], bf[i], ts[i]);
            }
        }
    };

    load_a(0);
    load_b(0, 0);
    store_a(0);
    if (S > 1) {
        load_a(1);
        load_b(1, 1);
    }
    __syncthreads();
    for (int64_t s = 0; s < S; s += 2) {
        compute(0, 0, s);
        if (s + 1 < S) store_a(1);
        if (s + 2 < S) {
            load_a(s + 2);
            load_b(0, s + 2);
        }
        __syncthreads();
        if (s + 1 < S) {
            compute(1, 1, s + 1);
            if (s + 2 < S) store_a(0);
            if (s + 3 < S) {
                load_a(s + 3);
                load_b(1, s + 3);
            }
            __syncthreads();
        }
    }

    const int kq = lane >> 4;
#pragma unroll
    for (int m = 0; m < WM; m++)
#pragma unroll
        for (int i = 0; i < WN; i++) {
            int64_t row = (g0 + i) * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) tile_store(p, (m16_0 + m) * 16 + 4 * kq + r, row, acc[m][i][r]);
        }
}

// ---------------------------------------------------------------------------

int64_t split_k_tiles(const TileView &w) {
    int64_t kt = w.units_k * (unit_k_of(w.tf) / 32);
    return (kt + 1) & ~(int64_t)1;
}

bool tile_gemm_takes(const TileView &w, int64_t n) {
    if (!w.fast || n < 128) return false;
    return w.tf == TF_BF16 || w.tf == TF_MX4 || w.tf == TF_FP8 || w.tf == TF_INT4;
}

size_t split_bytes(const TileView &w, int64_t n, int xt) {
    return (size_t)((n + 15) / 16) * split_k_tiles(w) * xt * 1024;
}

void launch_split(void *xs, const float *x, const int32_t *row_index, int64_t n, int64_t ldx, int64_t K,
                  int64_t kt_total, int xt, hipStream_t s) {
    SplitParams sp{(u32x4 *)xs, x, row_index, n, ldx, K, kt_total, (n + 15) / 16};
    int64_t total = sp.m16 * kt_total * 64;
    dim3 grid((unsigned)((total + 255) / 256));
    if (xt == 3) hipLaunchKernelGGL(split_kernel<3>, grid, dim3(256), 0, s, sp);
    else hipLaunchKernelGGL(split_kernel<2>, grid, dim3(256), 0, s, sp);
    DITCH_TRY_HIP(hipGetLastError());
}

template <int TF, int XT, int WAVES, int WN, int WM>
static void launch_tile(TileGemmParams &p, hipStream_t s) {
    constexpr int BM = 16 * WM, BN = 16 * WN * WAVES;
    p.tiles_m = (int)((p.n + BM - 1) / BM);
    p.tiles_n = (int)((p.w.rows + BN - 1) / BN);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n));
    hipLaunchKernelGGL((tile_gemm_kernel<TF, XT, WAVES, WN, WM>), grid, dim3(WAVES * 64), 0, s, p);
}

template <int TF, int XT>
static void launch_tile_tf(TileGemmParams &p, hipStream_t s) {
    launch_tile<TF, XT, 4, 4, 8>(p, s);
}

void launch_tile_gemm(const TileView &w, float *out, int64_t ldo, const void *xs, int64_t n, int xt,
                      const MatmulEpilogue &ep, hipStream_t s) {
    TileGemmParams p{};
    p.w = w;
    p.xs = (const u32x4 *)xs;
    p.kt_total = split_k_tiles(w);
    p.out = out;
    p.ldo = ldo;
    p.n = n;
    p.bias = ep.bias;
    p.accumulate = ep.accumulate;
    p.delta_b = ep.delta_b;
    p.delta_xa = ep.delta_xa;
    p.delta_rank = ep.delta_rank;
    p.delta_stride = ep.delta_rank;
    const bool x3 = xt == 3;
    switch (w.tf) {
    case TF_BF16: x3 ? launch_tile_tf<TF_BF16, 3>(p, s) : launch_tile_tf<TF_BF16, 2>(p, s); break;
    case TF_MX4: x3 ? launch_tile_tf<TF_MX4, 3>(p, s) : launch_tile_tf<TF_MX4, 2>(p, s); break;
    case TF_FP8: x3 ? launch_tile_tf<TF_FP8, 3>(p, s) : launch_tile_tf<TF_FP8, 2>(p, s); break;
    case TF_INT4: x3 ? launch_tile_tf<TF_INT4, 3>(p, s) : launch_tile_tf<TF_INT4, 2>(p, s); break;
    default: throw Error{DITCH_UNSUPPORTED, "tiled GEMM: tile format"};
    }
    DITCH_TRY_HIP(hipGetLastError());
}

}  // namespace ditch
