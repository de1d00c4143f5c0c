// gemm.hip — dequant-fused products for the formats and shapes the tiled
// kernel (gemm_tile.hip) does not take, and the launchers of every product
// (the GEMV regime lives in gemv.hip).
#include "gemm_common.h"
#include "gemm_f32.h"

namespace ditch {

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
    int64_t tb[MT], rw[NT];
#pragma unroll
    for (int m = 0; m < MT; m++) tb[m] = m0 + 16 * m + 4 * kq;
#pragma unroll
    for (int i = 0; i < NT; i++) rw[i] = (g0 + i) * 16 + lane % 16;
    store_block(p, tb, rw, acc);
}

// ---------------------------------------------------------------------------

template <int TF, int XT>
static void dispatch(const GemmParams &p, int64_t max_rows, int64_t n_for_shape, unsigned nseg, hipStream_t s) {
    int64_t groups = (max_rows + 15) / 16;
    if (n_for_shape <= 64 || XT > 2) {
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
                   const int32_t *row_index, DevBuf *ws) {
    if (n <= 0 || w.rows <= 0) return;
    if (ws && !ep.exact && mx_gemm_takes(w, n)) {
        const int64_t ldst = w.units_k;
        void *xm = ws->get<uint8_t>(mx_frag_bytes(n, ldst));
        launch_split_mx(xm, x, row_index, n, w.cols, w.cols, ldst, s);
        launch_mx_gemm(w, out, w.rows, xm, ldst, n, ep, s);
        return;
    }
    if (ws && tile_gemm_takes(w, n)) {
        const int xt = ep.exact ? 3 : 2;
        const int64_t ldk = split_k_tiles(w);
        const size_t xb = (split_bytes_ldk(n, ldk, xt) + 255) & ~(size_t)255;
        size_t pb = tile_part_bytes(w, n, xt);
        // a borrowed scratch too small for the split-K partial sums: the
        // product runs unsplit (the same sums, added in one pass)
        if (ws->borrowed && xb + pb > ws->bytes) pb = 0;
        uint8_t *xs = ws->get<uint8_t>(xb + pb);
        launch_split(xs, x, row_index, n, w.cols, w.cols, ldk, xt, s);
        launch_tile_gemm(w, out, w.rows, xs, ldk, n, xt, ep, s, pb ? (float *)(xs + xb) : nullptr);
        return;
    }
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
    if (n <= 16) {
        launch_gemv(p, w.tf, w.rows, w.cols, ep.exact != 0, 1, ws, s);
        return;
    }
    if (f32_gemm_takes(w, n)) {  // exact products whatever ep.exact asks
        launch_f32_gemm(p, s);
        return;
    }
    dispatch_tf(w.tf, p, w.rows, n, 1, ep.exact != 0, s);
}

void launch_matmul_act(const TileView &w, float *out, const Act &x, int64_t n, const MatmulEpilogue &ep,
                       hipStream_t s, DevBuf *ws) {
    if (n <= 0 || w.rows <= 0) return;
    if (!ep.exact && mx_gemm_takes(w, n)) {
        if (x.xm && x.ldst >= w.units_k) {
            launch_mx_gemm(w, out, w.rows, x.xm, x.ldst, n, ep, s);
            return;
        }
        if (x.f32) {
            launch_matmul(w, out, x.f32, n, ep, s, nullptr, ws);
            return;
        }
    }
    if (x.xs && !ep.exact && tile_gemm_takes(w, n) && x.ldk >= split_k_tiles(w)) {
        const size_t pb = ws ? tile_part_bytes(w, n, 2) : 0;
        launch_tile_gemm(w, out, w.rows, x.xs, x.ldk, n, 2, ep, s, pb ? ws->get<float>(pb / sizeof(float)) : nullptr);
        return;
    }
    DITCH_CHECK(x.f32 != nullptr, DITCH_INVALID_ARGUMENT, "product: no activation form the weight's product takes");
    launch_matmul(w, out, x.f32, n, ep, s, nullptr, ws);
}

void launch_matmul_grouped(const GroupSeg *d_segs, const GroupSeg *h_segs, unsigned nseg, int tf, int64_t rows,
                           int64_t cols, int64_t max_cnt, float *out, const float *x, const int32_t *row_index,
                           const float *delta_xa, int delta_stride, hipStream_t s, DevBuf *ws, DevBuf *meta) {
    if (nseg == 0 || max_cnt <= 0) return;
    if (h_segs && ws && meta && tile_grouped_takes(h_segs, nseg, max_cnt)) {
        launch_tile_gemm_grouped(d_segs, h_segs, nseg, out, rows, x, cols, row_index, delta_xa, delta_stride, ws, meta,
                                 s);
        return;
    }
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
    if (max_cnt <= 16) {
        launch_gemv(p, tf, rows, cols, false, nseg, ws, s);
        return;
    }
    dispatch_tf(tf, p, rows, max_cnt, nseg, false, s);
}

}  // namespace ditch
