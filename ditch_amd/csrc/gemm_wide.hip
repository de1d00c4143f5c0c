// gemm_wide.hip — the Q8_0 product for 32 <= n <= 256 tokens
// (tensor.matmulT, tensor.zig:1023-1045, on GGUF Q8_0 weights: quant.zig
// block_q8_0, 32 int8 codes and one f16 scale per row and 32 columns).
//
// At these batch sizes the weight stream (1.0625 B per weight) still
// dominates HBM traffic, and the product is too small to give every CU a
// tile of the 64 x 512 tiled product without splitting K through partial
// sums in HBM. Here a workgroup owns 64 weight rows (four 16-row groups) and
// every token, so each weight is read from HBM exactly once and nothing but
// the outputs is written:
//
//   - every multiplying wave owns a 64-token x 64-row tile (16 accumulator
//     tiles of v_mfma_f32_16x16x32_bf16) over a slice of the 64-column units;
//     the workgroup's slices are added in slice order in LDS at the end, then
//     delta, bias and accumulate are applied as everywhere else;
//   - the weight codes are the MFMA's B operand as laid out in HBM (one
//     16-byte load per lane and row group covers two 32-column k tiles),
//     widened to bf16 (exact for int8), and every 32-column partial sum is
//     scaled by its f16 block scale with one multiply-add per output
//     (acc += s * sum), as in the tiled product;
//   - the A fragments (two bf16 terms per activation, split_kernel layout)
//     come from L2: all workgroups read the same few MiB.
//
// Two kernels:
//   - wide_q8_direct_kernel (n <= 64): 8 waves, each its own eighth of the
//     units; a wave loads its codes and A fragments itself, one unit ahead;
//   - wide_q8_kernel<KS> (64 < n <= 256): 4 multiplying waves (KS k slices x
//     4 / KS token parts) fed by 4 producer waves, which load the codes
//     several units ahead and write bf16 B fragments and scale words into a
//     two-stage LDS ring.
#include "gemm_wide.h"

namespace ditch {

namespace {

constexpr int WXT = 2;  // activation terms

struct WideParams {
    TileView w;
    const u32x4 *xs;
    int64_t ldk;  // k tiles per 16-token block of xs
    int64_t m16;  // 16-token blocks in xs
    float *out;
    int64_t ldo, n;
    const float *bias;
    int accumulate;
    const float *delta_b, *delta_xa;
    int delta_rank, delta_stride;
};

// int8 codes of one 32-column k tile (two words: 8 codes) -> bf16 pairs
__device__ __forceinline__ u32x4 q8_bf16(uint32_t w0, uint32_t w1) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        v[j] = (float)(int8_t)((w0 >> (8 * j)) & 0xffu);
        v[4 + j] = (float)(int8_t)((w1 >> (8 * j)) & 0xffu);
    }
    return u32x4{pack_hi(v[0], v[1]), pack_hi(v[2], v[3]), pack_hi(v[4], v[5]), pack_hi(v[6], v[7])};
}

// f(std::integral_constant<int, j>) for j = 0 .. N-1 (register ring slots
// must be compile-time indices)
template <int N, int I = 0, typename F>
__device__ __forceinline__ void wide_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        wide_for<N, I + 1>(f);
    }
}

// The partial tiles red[part * KS + slice][tile][lane] of the TH token parts
// (64 tokens x 64 rows each), added in slice order, then delta, bias and
// accumulate as in every other product; all 512 threads take outputs.
template <int KS, int TH>
__device__ __forceinline__ void wide_finish(const WideParams &p, const floatx4 *red, int64_t g0) {
    const float *rf = (const float *)red;
    for (int idx = threadIdx.x; idx < TH * 4096; idx += 512) {
        const int pth = idx >> 12, rem = idx & 4095;
        const int tl = rem >> 6, rl = rem & 63;  // token and row within the part's 64 x 64
        const int i = tl >> 4, q = tl & 3, r = rl >> 4, ln = (rl & 15) + 16 * ((tl & 15) >> 2);
        const int64_t tok = (int64_t)pth * 64 + tl, row = g0 * 16 + rl;
        if (tok >= p.n || row >= p.w.rows) continue;
        float v = rf[(((pth * KS) * 16 + i * 4 + r) * 64 + ln) * 4 + q];
#pragma unroll
        for (int k = 1; k < KS; k++) v = __fadd_rn(v, rf[(((pth * KS + k) * 16 + i * 4 + r) * 64 + ln) * 4 + q]);
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
}

// Up to 64 tokens: all 8 waves multiply (two a SIMD), each over its own
// slice of the units (KS = 8), and load their own codes: a unit's codes are
// widened to bf16 as soon as it starts and the next unit's codes requested
// into the same registers, then its A fragments are replaced by the next
// unit's one by one as they are multiplied (every load one unit ahead, in
// the order the products use them).
__global__ __launch_bounds__(512) void wide_q8_direct_kernel(WideParams p) {
    constexpr int KS = 8, TH = 1;
    __shared__ floatx4 red[8 * 16 * 64];  // [wave][tile][lane]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = wave;
    const TileView &w = p.w;
    const int64_t U = w.units_k;
    const int64_t groups = (w.rows + 15) / 16;
    const int64_t g0 = (int64_t)blockIdx.x * 4;
    const int64_t u0 = U * ks / KS, u1 = U * (ks + 1) / KS;
    const int lrow = lane & 15;
    const uint8_t *cbase[4];
    const uint32_t *sbase[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t g = g0 + r < groups ? g0 + r : groups - 1;
        cbase[r] = w.codes + g * U * 1024;
        sbase[r] = w.side + g * U * 16;
    }
    const u32x4 *abase[4];
#pragma unroll
    for (int i = 0; i < 4; i++) abase[i] = p.xs + (i < p.m16 ? i : p.m16 - 1) * p.ldk * (WXT * 64);
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][r] = floatx4{0.f, 0.f, 0.f, 0.f};
    uint4 bc[4];
    uint32_t sw[4];
    u32x4 a[2][4][WXT];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        bc[r] = *((const uint4 *)(cbase[r] + u0 * 1024) + lane);
        sw[r] = sbase[r][u0 * 16 + lrow];
    }
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < WXT; e++) a[t][i][e] = abase[i][((2 * u0 + t) * WXT + e) * 64 + lane];
    for (int64_t u = u0; u < u1; u++) {
        const int64_t un = u + 1 < u1 ? u + 1 : u1 - 1;
        u32x4 bh[2][4];
        uint32_t swc[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            bh[0][r] = q8_bf16(bc[r].x, bc[r].y);
            bh[1][r] = q8_bf16(bc[r].z, bc[r].w);
            swc[r] = sw[r];
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            bc[r] = *((const uint4 *)(cbase[r] + un * 1024) + lane);
            sw[r] = sbase[r][un * 16 + lrow];
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; r++) sc[r] = f16_to_f32_hw((uint16_t)(t ? swc[r] >> 16 : swc[r] & 0xffffu));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                floatx4 part[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    part[r] = mfma_bf16(a[t][i][0], bh[t][r], floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int e = 1; e < WXT; e++) part[r] = mfma_bf16(a[t][i][e], bh[t][r], part[r]);
                }
#pragma unroll
                for (int e = 0; e < WXT; e++) a[t][i][e] = abase[i][((2 * un + t) * WXT + e) * 64 + lane];
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int q = 0; q < 4; q++) acc[i][r][q] = __builtin_fmaf(sc[r], part[r][q], acc[i][r][q]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[(wave * 16 + i * 4 + r) * 64 + lane] = acc[i][r];
    __syncthreads();
    wide_finish<KS, TH>(p, red, g0);
}

// Waves 0-3 multiply (one a SIMD), waves 4-7 feed them: producer p loads the
// codes and side words of its share of the next units (D units ahead, in
// registers), widens the codes to bf16 B fragments and writes them with the
// side words into the LDS stage the products read next; one barrier a unit.
// The producers' loads are the only ones in their waves' queues, and the
// consumers' A loads the only ones in theirs, so neither stream waits for
// the other's latency.
template <int KS>
__global__ __launch_bounds__(512) void wide_q8_kernel(WideParams p) {
    constexpr int TH = 4 / KS;  // token parts
    constexpr int D = KS == 1 ? 4 : 3;  // units a producer has in flight
    __shared__ u32x4 Bs[2][KS * 4 * 2 * 64];   // [stage][slice][group][k tile][lane]
    __shared__ uint32_t Ss[2][KS * 4 * 16];    // [stage][slice][group][row]
    __shared__ floatx4 red[4 * 16 * 64];       // [consumer][tile][lane]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const TileView &w = p.w;
    const int64_t U = w.units_k;
    const int64_t groups = (w.rows + 15) / 16;
    const int64_t g0 = (int64_t)blockIdx.x * 4;
    const int64_t S = (U + KS - 1) / KS;  // steps: units of the longest slice
    const int lrow = lane & 15;

    if (wave >= 4) {
        // producer: pieces (slice, group) j = pr * KS .. + KS
        const int pr = wave - 4;
        const uint8_t *cb[KS];
        const uint32_t *sb[KS];
        int64_t pu0[KS], pu1[KS];
        int dst[KS];
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const int piece = pr * KS + j, ks = piece / 4, r = piece % 4;
            int64_t g = g0 + r;
            g = g < groups ? g : groups - 1;
            cb[j] = w.codes + g * U * 1024;
            sb[j] = w.side + g * U * 16;
            pu0[j] = U * ks / KS;
            pu1[j] = U * (ks + 1) / KS;
            dst[j] = ks * 4 + r;
        }
        uint4 rc[D][KS];
        uint32_t rs[D][KS];
        auto load = [&](int64_t step, auto slot) {
            constexpr int q = decltype(slot)::value;
#pragma unroll
            for (int j = 0; j < KS; j++) {
                int64_t un = pu0[j] + step;
                un = un < pu1[j] ? un : pu1[j] - 1;
                rc[q][j] = *((const uint4 *)(cb[j] + un * 1024) + lane);
                rs[q][j] = sb[j][un * 16 + lrow];
            }
        };
        auto put = [&](int st, auto slot) {
            constexpr int q = decltype(slot)::value;
#pragma unroll
            for (int j = 0; j < KS; j++) {
                Bs[st][(dst[j] * 2 + 0) * 64 + lane] = q8_bf16(rc[q][j].x, rc[q][j].y);
                Bs[st][(dst[j] * 2 + 1) * 64 + lane] = q8_bf16(rc[q][j].z, rc[q][j].w);
                if (lane < 16) Ss[st][dst[j] * 16 + lane] = rs[q][j];
            }
        };
        wide_for<D>([&](auto q) { load(decltype(q)::value, q); });
        put(0, std::integral_constant<int, 0>{});
        load(D, std::integral_constant<int, 0>{});
        __syncthreads();
        // step u: stage (u + 1) % 2 <- ring slot (u + 1) % D, then that slot
        // loads step u + 1 + D
        for (int64_t u = 0; u < S; u += D) {
            wide_for<D>([&](auto jq) {
                constexpr int j = decltype(jq)::value, q = (j + 1) % D;
                if (u + j < S) {
                    if (u + j + 1 < S) {
                        put((int)((u + j + 1) & 1), std::integral_constant<int, q>{});
                        load(u + j + 1 + D, std::integral_constant<int, q>{});
                    }
                    __syncthreads();
                }
            });
        }
    } else {
        // consumer: 64 tokens x 64 rows over the units of slice ks
        const int ks = wave % KS, th = wave / KS;
        const int64_t u0 = U * ks / KS, u1 = U * (ks + 1) / KS;
        const u32x4 *abase[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int64_t mb = 4 * th + i;
            mb = mb < p.m16 ? mb : p.m16 - 1;
            abase[i] = p.xs + mb * p.ldk * (WXT * 64);
        }
        floatx4 acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][r] = floatx4{0.f, 0.f, 0.f, 0.f};
        u32x4 a[2][4][WXT];  // [k tile][token tile][term] of the current unit
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < WXT; e++) a[t][i][e] = abase[i][((2 * u0 + t) * WXT + e) * 64 + lane];
        __syncthreads();
        for (int64_t u = 0; u < S; u++) {
            if (u0 + u < u1) {
                const int st = (int)(u & 1);
                int64_t un = u0 + u + 1;
                un = un < u1 ? un : u1 - 1;
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    u32x4 bh[4];
                    float sc[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        bh[r] = Bs[st][((ks * 4 + r) * 2 + t) * 64 + lane];
                        const uint32_t sw = Ss[st][(ks * 4 + r) * 16 + lrow];
                        sc[r] = f16_to_f32_hw((uint16_t)(t ? sw >> 16 : sw & 0xffffu));
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        floatx4 part[4];
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            part[r] = mfma_bf16(a[t][i][0], bh[r], floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                            for (int e = 1; e < WXT; e++) part[r] = mfma_bf16(a[t][i][e], bh[r], part[r]);
                        }
#pragma unroll
                        for (int e = 0; e < WXT; e++) a[t][i][e] = abase[i][((2 * un + t) * WXT + e) * 64 + lane];
#pragma unroll
                        for (int r = 0; r < 4; r++)
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                acc[i][r][q] = __builtin_fmaf(sc[r], part[r][q], acc[i][r][q]);
                    }
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[(wave * 16 + i * 4 + r) * 64 + lane] = acc[i][r];
    }

    __syncthreads();
    wide_finish<KS, TH>(p, red, g0);
}

}  // namespace

bool wide_gemm_takes(const TileView &w, int64_t n, int xt, int64_t ldk) {
    return w.tf == TF_Q8 && w.fast && w.side && xt == WXT && n >= 32 && n <= 256 && w.units_k >= 8 &&
           ldk >= 2 * w.units_k;
}

void launch_wide_gemm(const TileView &w, float *out, int64_t ldo, const void *xs, int64_t ldk, int64_t n,
                      const MatmulEpilogue &ep, hipStream_t s) {
    DITCH_CHECK(wide_gemm_takes(w, n, WXT, ldk), DITCH_INVALID_ARGUMENT, "wide product: weight or batch not taken");
    WideParams p{};
    p.w = w;
    p.xs = (const u32x4 *)xs;
    p.ldk = ldk;
    p.m16 = (n + 15) / 16;
    p.out = out;
    p.ldo = ldo;
    p.n = n;
    p.bias = ep.bias;
    p.accumulate = ep.accumulate;
    p.delta_b = ep.delta_b;
    p.delta_xa = ep.delta_xa;
    p.delta_rank = ep.delta_rank;
    p.delta_stride = ep.delta_rank;
    const dim3 grid((unsigned)(((w.rows + 15) / 16 + 3) / 4));
    if (n <= 64) hipLaunchKernelGGL(wide_q8_direct_kernel, grid, dim3(512), 0, s, p);
    else if (n <= 128) hipLaunchKernelGGL(wide_q8_kernel<2>, grid, dim3(512), 0, s, p);
    else hipLaunchKernelGGL(wide_q8_kernel<1>, grid, dim3(512), 0, s, p);
    DITCH_TRY_HIP(hipGetLastError());
}

}  // namespace ditch
