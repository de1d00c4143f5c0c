// gemv.hip — the dequant-fused product in the GEMV regime (n <= 16 tokens,
// or routed-expert segments of at most 16): out[n][rows] = x[n][cols] . W^T
// with W decoded in registers (tensor.matmulT, tensor.zig:1023-1045; the
// M <= 16 rows of the decode-shaped calls, tensor.zig:1001-1020).
//
// One 16-token MFMA fragment; NT 16-row groups per workgroup; K split over
// its W waves and reduced through LDS. Each wave keeps D units (16 rows x
// UK columns of codes, 1 KiB) in flight in a register ring: the codes, scale
// words and activations of unit u + D are requested as soon as unit u has
// been multiplied, in the order they are consumed, so the in-order
// completion count never waits on a later unit.
//
// The activations reach the MFMA as bf16 terms (gemm_common.h), taken one of
// two ways:
//   - n <= 8: each wave loads the f32 rows of its unit (column pairs spread
//     over the lanes, one pass per 128 values), splits them and writes the
//     words into its own LDS slot in fragment order; the A operands come
//     back with one 16-byte LDS read per term and k tile. The split costs
//     a few instructions per unit instead of one per activation and lane.
//   - 8 < n <= 16: gv_split_kernel writes the terms once per call in the
//     order the lanes read them ([k tile][term][k quarter][token]), and the
//     GEMV loads them with its codes.
#include "gemm_common.h"

namespace ditch {

#ifndef GEMV_NT
#define GEMV_NT 2
#endif
#ifndef GEMV_W
#define GEMV_W 4
#endif
#ifndef GEMV_D
#define GEMV_D 8
#endif

constexpr int GV_XN = 8;  // tokens the in-kernel split takes

// Per-lane side data of one unit: the Q8 / MXFP4 scale word, or the FP8 /
// INT4 scale (and zero point) of each of the lane's k tiles.
template <int TF> struct GvSide {
    uint32_t word;
    float s[Fmt<TF>::tiles];
    int zp[Fmt<TF>::tiles];
};

template <int TF>
__device__ __forceinline__ void gv_side(const TileView &w, int64_t row, int64_t unit, int kq, GvSide<TF> &sd) {
    constexpr int UK = TF == TF_Q8 || TF == TF_FP8 ? 64 : (TF == TF_MX4 || TF == TF_INT4) ? 128 : 32;
    if constexpr (TF == TF_FP8 || TF == TF_INT4) {
        // one scale block covers the unit when it spans a multiple of UK columns
        const int64_t span = TF == TF_FP8 ? w.block_cols : w.group;
        if (span % UK == 0) {
            int zp = 0;
            const float s = tile_scale_of<TF>(w, row, unit * UK, &zp);
#pragma unroll
            for (int t = 0; t < Fmt<TF>::tiles; t++) {
                sd.s[t] = s;
                sd.zp[t] = zp;
            }
        } else {
#pragma unroll
            for (int t = 0; t < Fmt<TF>::tiles; t++) {
                sd.zp[t] = 0;
                sd.s[t] = tile_scale_of<TF>(w, row, unit * UK + 32 * t + 8 * kq, &sd.zp[t]);
            }
        }
    }
}

template <int TF>
__device__ __forceinline__ void gv_decode(const TileView &w, const Raw &raw, const GvSide<TF> &sd, int t, u32x4 &bh,
                                          u32x4 &bl, float &ts) {
    if constexpr (TF == TF_FP8) decode_fp8(w, raw, t, sd.s[t], bh);
    else if constexpr (TF == TF_INT4) decode_int4(raw, t, sd.s[t], sd.zp[t], bh);
    else decode_tile<TF>(w, raw, UnitSide{sd.word}, t, 0, 0, bh, bl, ts);  // no loads for the other formats
}

// ---------------------------------------------------------------------------
// 8 < n <= 16: the terms written once per call

struct GvSplitParams {
    uint8_t *xf;
    const float *x;
    const int32_t *row_index;
    const GroupSeg *segs;
    int64_t n, ldx, K, tiles, xn, xf_seg;
};

// One thread per (k tile, k quarter, token) of segment blockIdx.y: the XT
// words of its 8 activations (columns past K are 0). Tokens past the
// segment's count are not written; the GEMV never reads them.
template <bool FP32, int XT>
__global__ __launch_bounds__(256) void gv_split_kernel(GvSplitParams q) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= q.tiles * 4 * q.xn) return;
    const int64_t tok = i % q.xn, kq = (i / q.xn) % 4, tile = i / (4 * q.xn);
    int64_t cnt = q.n, off = 0;
    if (q.segs) {
        cnt = q.segs[blockIdx.y].cnt;
        off = q.segs[blockIdx.y].off;
    }
    if (tok >= cnt) return;
    const int64_t src = q.row_index ? (int64_t)q.row_index[off + tok] : off + tok;
    const float *xr = q.x + src * q.ldx;
    const int64_t k0 = tile * 32 + 8 * kq;
    float v[8];
    if (k0 + 8 <= q.K && ((uintptr_t)(xr + k0) & 15) == 0) {
        const float4 a = *(const float4 *)(xr + k0), b = *(const float4 *)(xr + k0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = k0 + j < q.K ? xr[k0 + j] : 0.f;
    }
    u32x4 t[XT];
    if constexpr (FP32) a_words<true, XT>(v, t);
    else a_words_cvt<XT>(v, t);
    uint8_t *dst = q.xf + (int64_t)blockIdx.y * q.xf_seg + ((tile * XT * 4 + kq) * q.xn + tok) * 16;
#pragma unroll
    for (int e = 0; e < XT; e++) *(u32x4 *)(dst + e * 4 * q.xn * 16) = t[e];
}

// ---------------------------------------------------------------------------

// LX: the activations are f32 rows split in the kernel (n <= GV_XN), else
// fragments from gv_split_kernel. PPC > 0 (LX): the column-pair passes are
// known at compile time and every unit lies inside K with 8-byte aligned
// rows, so the activation loads carry no per-pass or per-unit conditions.
// NR < 4: n = NR tokens (the lanes' other accumulator rows are not stored).
template <int TF, int NT, int XT, int D, int W, bool LX, int PPC = 0, int NR = 4>
__global__ __launch_bounds__(64 * W) void gemv_kernel(GemmParams p) {
    if (!select_segment(p, 0)) return;
    constexpr int TL = Fmt<TF>::tiles;
    constexpr bool FP32 = Fmt<TF>::fp32;
    constexpr int UK = TF == TF_Q8 || TF == TF_FP8 ? 64 : (TF == TF_MX4 || TF == TF_INT4) ? 128 : 32;
    constexpr int UB = TF == TF_F32 ? 2048 : 1024;  // bytes of a unit's codes
    // LX: column pairs of a unit per lane for GV_XN tokens (fewer passes run for smaller n)
    constexpr int PP = LX ? (GV_XN * UK / 2 + 63) / 64 : 1;
    constexpr int XS = TL * XT * 4 * GV_XN * 16;  // bytes of a wave's LDS slot
    __shared__ u32x4 xl[LX ? W * XS / 16 : 1];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t groups = (p.w.rows + 15) / 16;
    const int64_t g0 = (int64_t)blockIdx.x * NT;
    if (g0 >= groups) return;
    const int64_t units = p.w.units_k, K = p.w.cols;
    const int64_t per = (units + W - 1) / W;
    const int64_t u0 = wave * per < units ? wave * per : units;
    const int64_t u1 = u0 + per < units ? u0 + per : units;
    const int tok = lane % 16, kq = lane / 16;
    // the lane's activation words: tokens past n read token n - 1 (their
    // outputs are not stored; each output row of the MFMA depends on its own
    // token only)
    const int64_t tc = tok < p.n ? tok : p.n - 1;
    const uint32_t xoff = LX ? (uint32_t)((kq * GV_XN + tc) * 16) : (uint32_t)((kq * p.xn + tc) * 16);
    const int64_t xterm = LX ? 4 * GV_XN * 16 : 4 * p.xn * 16;  // bytes between consecutive terms' words
    // LX: the lane's column pairs: pass m takes pair lane + 64 m of the unit's
    // n x UK / 2 (token-major); passes past n tokens are skipped, lanes past
    // them repeat token n - 1
    const int pp = PPC ? PPC : LX ? (int)((p.n * UK / 2 + 63) / 64) : 0;
    const float *xrow[PP];
    uint32_t xo[PP];  // PPC: byte offset of the lane's pair in unit 0 (activations under 4 GiB)
    uint32_t lofs[PP];  // LDS byte offset of the pair's first term word in the wave's slot
    int kl[PP];         // column of the pair in the unit
#pragma unroll
    for (int m = 0; m < PP; m++) {
        const int P = lane + 64 * m;
        const int64_t pt = P / (UK / 2) < p.n ? P / (UK / 2) : p.n - 1;
        const int k = 2 * (P % (UK / 2));
        kl[m] = k;
        xrow[m] = LX ? p.x + (p.row_index ? (int64_t)p.row_index[pt] : pt) * p.ldx : nullptr;
        xo[m] = LX ? (uint32_t)(((p.row_index ? (int64_t)p.row_index[pt] : pt) * p.ldx + k) * 4) : 0u;
        if constexpr (FP32) lofs[m] = (uint32_t)(((((k / 32) * XT + (k % 8) / 4) * 4 + (k % 32) / 8) * GV_XN + pt) * 16 + (k % 4) * 4);
        else lofs[m] = (uint32_t)(((((k / 32) * XT) * 4 + (k % 32) / 8) * GV_XN + pt) * 16 + ((k % 8) / 2) * 4);
    }
    const bool x_pairs = ((p.ldx & 1) == 0) && (((uintptr_t)p.x & 7) == 0);  // 8-byte pair loads
    char *slot = (char *)xl + wave * XS;
    // per-lane byte offsets of the codes and the MXFP4 scale words
    const uint32_t woff = (uint32_t)lane * 16;
    uint32_t soff[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) {
        const int64_t g = g0 + i < groups ? g0 + i : groups - 1;
        const int64_t r = g * 16 + lane % 16 < p.w.rows ? g * 16 + lane % 16 : p.w.rows - 1;
        soff[i] = (uint32_t)(r * p.w.scale_cols);
    }

    floatx4 acc[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

    Raw raw[D][NT];
    GvSide<TF> sd[D][NT];
    u32x4 xw[LX ? 1 : D][TL][XT];  // fragments from global
    float2 xp[LX ? D : 1][PP];     // f32 column pairs (LX)
    auto fetch = [&](int j, int64_t u) __attribute__((always_inline)) {
        // LX: the activations first, so that the split of unit u (done while
        // unit u - 1 is multiplied) waits on them and not on u's codes
        if constexpr (LX) {
            const int64_t kb = u * UK;
            if (PPC > 0) {
#pragma unroll
                for (int m = 0; m < PPC; m++) xp[j][m] = gload<float2>((const char *)(p.x + kb) + xo[m]);
            } else if (x_pairs && kb + UK <= K) {
#pragma unroll
                for (int m = 0; m < PP; m++)
                    if (m < pp) xp[j][m] = gload<float2>(xrow[m] + kb + kl[m]);
            } else {
                // the matrix's last columns, or unaligned rows: values past K are 0
#pragma unroll
                for (int m = 0; m < PP; m++)
                    if (m < pp) {
                        const int64_t k = kb + kl[m];
                        xp[j][m].x = k < K ? xrow[m][k] : 0.f;
                        xp[j][m].y = k + 1 < K ? xrow[m][k + 1] : 0.f;
                    }
            }
        }
#pragma unroll
        for (int i = 0; i < NT; i++) {
            const int64_t g = g0 + i < groups ? g0 + i : groups - 1;
            const char *wb = (const char *)p.w.codes + (g * units + u) * UB;
            raw[j][i].a = gload<uint4>(wb + woff);
            if constexpr (TF == TF_F32) raw[j][i].b = gload<uint4>(wb + 1024 + woff);
            if constexpr (TF == TF_Q8)  // the group's 16 scale words of the unit: 64 contiguous bytes
                sd[j][i].word = gload<uint32_t>((const char *)p.w.side + (g * units + u) * 64 + (lane % 16) * 4);
            else if constexpr (TF == TF_MX4)
                sd[j][i].word = gload<uint32_t>((const char *)p.w.scale + u * 4 + soff[i]);
            else gv_side<TF>(p.w, g * 16 + lane % 16, u, kq, sd[j][i]);
        }
        if constexpr (!LX) {
            const char *xb = (const char *)p.xf + u * TL * XT * xterm;
#pragma unroll
            for (int t = 0; t < TL; t++)
#pragma unroll
                for (int e = 0; e < XT; e++) xw[j][t][e] = gload<u32x4>(xb + (t * XT + e) * xterm + xoff);
        }
        // keep each unit's loads together, in issue order: merged with the
        // next units' scale words, a load would be issued with the last unit
        asm volatile("" ::: "memory");
    };
    // LX: split ring slot j's pairs into the wave's LDS slot
    auto split = [&](int j) __attribute__((always_inline)) {
        if constexpr (LX) {
#pragma unroll
            for (int m = 0; m < PP; m++)
                if (PPC > 0 ? m < PPC : m < pp) {
                    if constexpr (FP32) {
                        *(uint2 *)(slot + lofs[m]) = make_uint2(f2u(xp[j][m].x), f2u(xp[j][m].y));
                    } else {
                        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
                        typedef float f2_t __attribute__((ext_vector_type(2)));
                        float r0 = xp[j][m].x, r1 = xp[j][m].y;
#pragma unroll
                        for (int e = 0; e < XT; e++) {
                            const uint32_t wd =
                                __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{r0, r1}, bf16x2_t));
                            *(uint32_t *)(slot + lofs[m] + e * xterm) = wd;
                            if (e + 1 < XT) {
                                r0 = __fsub_rn(r0, u2f(wd << 16));
                                r1 = __fsub_rn(r1, u2f(wd & 0xffff0000u));
                            }
                        }
                    }
                }
        }
    };
    // unit j of the ring; nxt: the next unit (ring slot j + 1) exists, and
    // its split is written into the LDS slot once unit j's words are read
    // (the wave's LDS accesses complete in order)
    auto compute = [&](int j, bool nxt) __attribute__((always_inline)) {
        u32x4 xa[TL][XT];
        if constexpr (LX) {
#pragma unroll
            for (int t = 0; t < TL; t++)
#pragma unroll
                for (int e = 0; e < XT; e++) xa[t][e] = *(const u32x4 *)(slot + (t * XT + e) * xterm + xoff);
            if (nxt) split((j + 1) % D);
        } else {
#pragma unroll
            for (int t = 0; t < TL; t++)
#pragma unroll
                for (int e = 0; e < XT; e++) xa[t][e] = xw[j][t][e];
        }
#pragma unroll
        for (int t = 0; t < TL; t++) {
#pragma unroll
            for (int i = 0; i < NT; i++) {
                u32x4 bh, bl = u32x4{0, 0, 0, 0};
                float ts = 1.f;
                gv_decode<TF>(p.w, raw[j][i], sd[j][i], t, bh, bl, ts);
                mac<TF, XT, NR>(acc[i], xa[t], bh, bl, ts);
            }
        }
    };
    if (u1 - u0 >= 2 * D) {
        // steady state: the ring is filled unconditionally and every slot
        // refilled, so the wait before each unit is a fixed count of the
        // later units' loads
#pragma unroll
        for (int j = 0; j < D; j++) fetch(j, u0 + j);
        split(0);
        int64_t b = u0;
        do {
#pragma unroll
            for (int j = 0; j < D; j++) {
                compute(j, true);
                fetch(j, b + D + j);
            }
            b += D;
        } while (b + 2 * D <= u1);
        // b + D <= u1 < b + 2 D: the ring holds units b .. b + D - 1
#pragma unroll
        for (int j = 0; j < D; j++) {
            compute(j, b + j + 1 < u1);
            if (b + D + j < u1) fetch(j, b + D + j);
        }
#pragma unroll
        for (int j = 0; j < D; j++)
            if (b + D + j < u1) compute(j, b + D + j + 1 < u1);
    } else if (u0 < u1) {
#pragma unroll
        for (int j = 0; j < D; j++)
            if (u0 + j < u1) fetch(j, u0 + j);
        split(0);
#pragma unroll
        for (int j = 0; j < D; j++) {
            if (u0 + j < u1) {
                compute(j, u0 + j + 1 < u1);
                if (u0 + D + j < u1) fetch(j, u0 + D + j);
            }
        }
#pragma unroll
        for (int j = 0; j < D; j++)
            if (u0 + D + j < u1) compute(j, u0 + D + j + 1 < u1);
    }
    // reduce the W K slices
    __shared__ floatx4 red[W - 1][NT][64];
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < NT; i++) red[wave - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wave == 0) {
        floatx4 a[1][NT];
        int64_t rw[NT];
        const int64_t tb[1] = {4 * kq};
#pragma unroll
        for (int i = 0; i < NT; i++) {
            a[0][i] = acc[i];
#pragma unroll
            for (int w = 0; w < W - 1; w++) {
                floatx4 b = red[w][i][lane];
                a[0][i][0] += b[0]; a[0][i][1] += b[1]; a[0][i][2] += b[2]; a[0][i][3] += b[3];
            }
            rw[i] = (g0 + i) * 16 + lane % 16;
        }
        store_block(p, tb, rw, a);
    }
}

// ---------------------------------------------------------------------------

template <int TF, int XT>
static void gemv_launch(const GemmParams &p, int64_t rows, unsigned nseg, bool lx, hipStream_t s) {
    // units in flight per wave: GEMV_D k tiles of 32
    constexpr int NT = GEMV_NT, D = GEMV_D / Fmt<TF>::tiles > 1 ? GEMV_D / Fmt<TF>::tiles : 1, W = GEMV_W;
    const int64_t groups = (rows + 15) / 16;
    const dim3 grid((unsigned)((groups + NT - 1) / NT), 1, nseg);
    if (lx) {
        // every unit inside K, rows 8-byte aligned: the passes as a constant
        constexpr int UK = TF == TF_Q8 || TF == TF_FP8 ? 64 : (TF == TF_MX4 || TF == TF_INT4) ? 128 : 32;
        const int pp = (int)((p.n * UK / 2 + 63) / 64);
        const bool full = p.w.cols % UK == 0 && (p.ldx & 1) == 0 && ((uintptr_t)p.x & 7) == 0 && nseg == 1 &&
                          !p.row_index && (uint64_t)p.n * p.ldx * 4 < (1ull << 32);
        if (XT == 2 && full && pp == 1 && p.n == 1)
            hipLaunchKernelGGL((gemv_kernel<TF, NT, XT, D, W, true, 1, 1>), grid, dim3(64 * W), 0, s, p);
        else if (XT == 2 && full && pp == 1)
            hipLaunchKernelGGL((gemv_kernel<TF, NT, XT, D, W, true, 1>), grid, dim3(64 * W), 0, s, p);
        else if (XT == 2 && full && pp == 2)
            hipLaunchKernelGGL((gemv_kernel<TF, NT, XT, D, W, true, 2>), grid, dim3(64 * W), 0, s, p);
        else hipLaunchKernelGGL((gemv_kernel<TF, NT, XT, D, W, true>), grid, dim3(64 * W), 0, s, p);
    } else hipLaunchKernelGGL((gemv_kernel<TF, NT, XT, D, W, false>), grid, dim3(64 * W), 0, s, p);
}

// The build compiles this file once per tile format and activation term
// count with GEMV_TF and GEMV_XT set (each object holds those kernels: the
// fully unrolled register rings make every format a long compile, and the
// objects build in parallel) and once without them (the split kernel and
// the dispatch). f16 and f32 weights take two f32 terms only.
#define GEMV_ENTRY_NAME(tf, xt) gemv_launch_tf##tf##_x##xt
#define GEMV_ENTRY(tf, xt) GEMV_ENTRY_NAME(tf, xt)
#define GEMV_ENTRY_ARGS const GemmParams &p, int64_t rows, unsigned nseg, bool lx, hipStream_t s

#ifdef GEMV_TF
void GEMV_ENTRY(GEMV_TF, GEMV_XT)(GEMV_ENTRY_ARGS) { gemv_launch<GEMV_TF, GEMV_XT>(p, rows, nseg, lx, s); }
#else
#define GEMV_DECLARE(tf) void GEMV_ENTRY(tf, 2)(GEMV_ENTRY_ARGS); void GEMV_ENTRY(tf, 3)(GEMV_ENTRY_ARGS);
GEMV_DECLARE(0)
GEMV_DECLARE(3)
GEMV_DECLARE(4)
GEMV_DECLARE(5)
GEMV_DECLARE(6)
void GEMV_ENTRY(1, 2)(GEMV_ENTRY_ARGS);
void GEMV_ENTRY(2, 2)(GEMV_ENTRY_ARGS);
static_assert(TF_BF16 == 0 && TF_F16 == 1 && TF_F32 == 2 && TF_Q8 == 3 && TF_FP8 == 4 && TF_MX4 == 5 && TF_INT4 == 6,
              "one GEMV object per tile format 0..6");

void launch_gemv(GemmParams &p, int tf, int64_t rows, int64_t cols, bool exact, unsigned nseg, DevBuf *ws,
                 hipStream_t s) {
    const bool fp32 = tf == TF_F16 || tf == TF_F32;
    const int xt = fp32 ? 2 : exact ? 3 : 2;
    const bool lx = p.n <= GV_XN;  // p.n: the tokens, or the largest segment
    if (!lx) {
        DITCH_CHECK(ws != nullptr, DITCH_INVALID_ARGUMENT, "GEMV needs a workspace");
        const int64_t uk = unit_k_of(tf);
        GvSplitParams q{};
        q.x = p.x;
        q.row_index = p.row_index;
        q.segs = p.segs;
        q.n = p.n;
        q.ldx = p.ldx;
        q.K = cols;
        q.tiles = (cols + uk - 1) / uk * uk / 32;
        q.xn = p.segs ? 16 : p.n;
        q.xf_seg = q.tiles * xt * 4 * q.xn * 16;
        q.xf = ws->get<uint8_t>((size_t)(q.xf_seg * nseg));
        const dim3 grid((unsigned)((q.tiles * 4 * q.xn + 255) / 256), nseg);
        if (fp32) hipLaunchKernelGGL((gv_split_kernel<true, 2>), grid, dim3(256), 0, s, q);
        else if (xt == 3) hipLaunchKernelGGL((gv_split_kernel<false, 3>), grid, dim3(256), 0, s, q);
        else hipLaunchKernelGGL((gv_split_kernel<false, 2>), grid, dim3(256), 0, s, q);
        DITCH_TRY_HIP(hipGetLastError());
        p.xf = q.xf;
        p.xn = q.xn;
        p.xf_seg = q.xf_seg;
    }
    const bool x3 = xt == 3;
    switch (tf) {
    case TF_BF16: x3 ? GEMV_ENTRY(0, 3)(p, rows, nseg, lx, s) : GEMV_ENTRY(0, 2)(p, rows, nseg, lx, s); break;
    case TF_F16: GEMV_ENTRY(1, 2)(p, rows, nseg, lx, s); break;
    case TF_F32: GEMV_ENTRY(2, 2)(p, rows, nseg, lx, s); break;
    case TF_Q8: x3 ? GEMV_ENTRY(3, 3)(p, rows, nseg, lx, s) : GEMV_ENTRY(3, 2)(p, rows, nseg, lx, s); break;
    case TF_FP8: x3 ? GEMV_ENTRY(4, 3)(p, rows, nseg, lx, s) : GEMV_ENTRY(4, 2)(p, rows, nseg, lx, s); break;
    case TF_MX4: x3 ? GEMV_ENTRY(5, 3)(p, rows, nseg, lx, s) : GEMV_ENTRY(5, 2)(p, rows, nseg, lx, s); break;
    case TF_INT4: x3 ? GEMV_ENTRY(6, 3)(p, rows, nseg, lx, s) : GEMV_ENTRY(6, 2)(p, rows, nseg, lx, s); break;
    default: throw Error{DITCH_UNSUPPORTED, "tile format"};
    }
    DITCH_TRY_HIP(hipGetLastError());
}
#endif

}  // namespace ditch
