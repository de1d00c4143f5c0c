// gemm_f32.hip — products on f32 and f16 weights for n > 16 tokens
// (tensor.matmulT, tensor.zig:1023-1045, with the reference's f32 fused
// multiply-adds: every product x * w exact, sums in f32).
//
// The products run on the fp32 MFMA (v_mfma_f32_16x16x4_f32), which forms
// every product exactly; it issues a 16 x 16 x 4 step in 32 cycles, so the
// product is MFMA-bound and what matters is keeping every SIMD busy:
//
//   - a wave owns 64 tokens x 32 rows (4 x 2 tiles, 32 accumulator VGPRs),
//     and takes its operands straight from memory into registers: per
//     32-column unit the lane's 8 weights of each row group (the tile layout:
//     row l % 16, columns 8 (l / 16) .. +8) and the same 8 columns of each
//     of its tokens' activation rows; eight rank-4 steps per tile and unit
//     pair register s of A with register s of B (k = 8 (l / 16) + s);
//   - the next unit's operands are requested before a unit's products (two
//     register sets, alternating);
//   - a workgroup is 4 waves: 4 / KS tiles, each over KS k slices whose sums
//     are added in slice order through LDS; KS grows until the grid gives
//     every SIMD four waves (the attention and small projections of a 0.5B
//     model have only a few hundred 64 x 32 tiles).
#include "gemm_f32.h"

namespace ditch {

namespace {

constexpr int FM = 4, FN = 2;  // token tiles x row groups per wave

template <int TF>
__device__ __forceinline__ void f32_weights(const uint8_t *unit, int lane, float (&b)[8]) {
    if constexpr (TF == TF_F32) {
        const float4 lo = *((const float4 *)unit + lane), hi = *((const float4 *)(unit + 1024) + lane);
        b[0] = lo.x; b[1] = lo.y; b[2] = lo.z; b[3] = lo.w;
        b[4] = hi.x; b[5] = hi.y; b[6] = hi.z; b[7] = hi.w;
    } else {
        const uint4 h = *((const uint4 *)unit + lane);
        const uint32_t wd[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            b[2 * j] = f16_to_f32((uint16_t)(wd[j] & 0xffffu));
            b[2 * j + 1] = f16_to_f32((uint16_t)(wd[j] >> 16));
        }
    }
}

// VEC: K a multiple of 32 and rows 16-byte aligned: every activation load is
// two unguarded float4 (no branch in the loop, so the next unit's loads stay
// in flight across the current unit's products)
template <int TF, int KS, bool VEC>
__global__ __launch_bounds__(256) void f32_gemm_kernel(GemmParams p, int tiles_m, int tiles) {
    constexpr int TW = 4 / KS;  // tiles per workgroup
    constexpr int UB = TF == TF_F32 ? 2048 : 1024;
    __shared__ floatx4 red[KS > 1 ? 4 * FM * FN * 64 : 1];  // [wave][tile][lane]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = wave % KS, tw = wave / KS;
    int tile = (int)blockIdx.x * TW + tw;
    const bool live = tile < tiles;
    tile = live ? tile : tiles - 1;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const TileView &w = p.w;
    const int64_t U = w.units_k, K = w.cols;
    const int64_t groups = (w.rows + 15) / 16;
    const int64_t u0 = U * ks / KS, u1 = U * (ks + 1) / KS;
    const int q = lane >> 4;

    const uint8_t *wb[FN];
#pragma unroll
    for (int i = 0; i < FN; i++) {
        int64_t g = (int64_t)tn * FN + i;
        g = g < groups ? g : groups - 1;
        wb[i] = w.codes + g * U * UB;
    }
    // tokens past n read the last token's row: their outputs are not stored
    const float *xr[FM];
#pragma unroll
    for (int m = 0; m < FM; m++) {
        int64_t tok = (int64_t)tm * 64 + 16 * m + (lane & 15);
        tok = tok < p.n ? tok : p.n - 1;
        xr[m] = p.x + (p.row_index ? (int64_t)p.row_index[tok] : tok) * p.ldx;
    }

    auto load_a = [&](int64_t u, float (&a)[FM][8]) {
        const int64_t k0 = u * 32 + 8 * q;
#pragma unroll
        for (int m = 0; m < FM; m++) {
            if constexpr (VEC) {
                const float4 lo = *(const float4 *)(xr[m] + k0), hi = *(const float4 *)(xr[m] + k0 + 4);
                a[m][0] = lo.x; a[m][1] = lo.y; a[m][2] = lo.z; a[m][3] = lo.w;
                a[m][4] = hi.x; a[m][5] = hi.y; a[m][6] = hi.z; a[m][7] = hi.w;
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) a[m][j] = k0 + j < K ? xr[m][k0 + j] : 0.f;
            }
        }
    };

    floatx4 acc[FM][FN];
#pragma unroll
    for (int m = 0; m < FM; m++)
#pragma unroll
        for (int i = 0; i < FN; i++) acc[m][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (u0 < u1) {
        // two operand sets: the loads of one unit are issued before the
        // products of the other
        float a0[FM][8], b0[FN][8], a1[FM][8], b1[FN][8];
        auto load = [&](int64_t u, float (&a)[FM][8], float (&b)[FN][8]) {
            u = u < u1 ? u : u1 - 1;
            load_a(u, a);
#pragma unroll
            for (int i = 0; i < FN; i++) f32_weights<TF>(wb[i] + u * UB, lane, b[i]);
        };
        auto products = [&](const float (&a)[FM][8], const float (&b)[FN][8]) {
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int m = 0; m < FM; m++)
#pragma unroll
                    for (int i = 0; i < FN; i++) acc[m][i] = mfma_f32(a[m][s], b[i][s], acc[m][i]);
        };
        load(u0, a0, b0);
        int64_t u = u0;
        // no branch inside the loop: every wait is a fixed count of loads
        // (pinning each set's loads ahead of the other set's products with
        // scheduling barriers measured 30-40 % slower)
        for (; u + 1 < u1; u += 2) {
            load(u + 1, a1, b1);
            products(a0, b0);
            load(u + 2, a0, b0);
            products(a1, b1);
        }
        if (u < u1) products(a0, b0);
    }

    if constexpr (KS > 1) {
#pragma unroll
        for (int m = 0; m < FM; m++)
#pragma unroll
            for (int i = 0; i < FN; i++) red[(wave * FM * FN + m * FN + i) * 64 + lane] = acc[m][i];
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int k = 1; k < KS; k++)
#pragma unroll
            for (int m = 0; m < FM; m++)
#pragma unroll
                for (int i = 0; i < FN; i++) {
                    const floatx4 o = red[((wave + k) * FM * FN + m * FN + i) * 64 + lane];
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[m][i][r] = __fadd_rn(acc[m][i][r], o[r]);
                }
    }
    if (!live) return;
    int64_t tb[FM], rw[FN];
#pragma unroll
    for (int m = 0; m < FM; m++) tb[m] = (int64_t)tm * 64 + 16 * m + 4 * q;
#pragma unroll
    for (int i = 0; i < FN; i++) rw[i] = ((int64_t)tn * FN + i) * 16 + (lane & 15);
    store_block(p, tb, rw, acc);
}

template <int TF, bool VEC>
void launch_tf(const GemmParams &p, hipStream_t s) {
    const int64_t groups = (p.w.rows + 15) / 16;
    const int tiles_m = (int)((p.n + 63) / 64), tiles = tiles_m * (int)((groups + FN - 1) / FN);
    // k slices until the grid gives every SIMD four waves (at least 2 units
    // each; two waves a SIMD measured 7 % slower on C1, eight 1 % slower)
    int ks = 1;
    while (ks < 4 && (int64_t)tiles * ks < 4096 && p.w.units_k / (2 * ks) >= 2) ks *= 2;
    const dim3 grid((unsigned)((tiles + 4 / ks - 1) / (4 / ks)));
    if (ks == 1) hipLaunchKernelGGL((f32_gemm_kernel<TF, 1, VEC>), grid, dim3(256), 0, s, p, tiles_m, tiles);
    else if (ks == 2) hipLaunchKernelGGL((f32_gemm_kernel<TF, 2, VEC>), grid, dim3(256), 0, s, p, tiles_m, tiles);
    else hipLaunchKernelGGL((f32_gemm_kernel<TF, 4, VEC>), grid, dim3(256), 0, s, p, tiles_m, tiles);
}

}  // namespace

bool f32_gemm_takes(const TileView &w, int64_t n) { return (w.tf == TF_F32 || w.tf == TF_F16) && n > 16; }

void launch_f32_gemm(const GemmParams &p, hipStream_t s) {
    DITCH_CHECK(f32_gemm_takes(p.w, p.n) && !p.segs, DITCH_INVALID_ARGUMENT, "f32 product: weight or batch not taken");
    const bool vec = p.w.cols % 32 == 0 && p.ldx % 4 == 0 && ((uintptr_t)p.x & 15) == 0;
    if (p.w.tf == TF_F32) vec ? launch_tf<TF_F32, true>(p, s) : launch_tf<TF_F32, false>(p, s);
    else vec ? launch_tf<TF_F16, true>(p, s) : launch_tf<TF_F16, false>(p, s);
    DITCH_TRY_HIP(hipGetLastError());
}

}  // namespace ditch
