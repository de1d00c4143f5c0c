// gemm_tile.hip — the large-batch product (prompt forward, n >= 32 tokens).
//
// out[n][rows] = x[n][cols] @ W^T (tensor.matmulT, tensor.zig:1023-1045) for
// weights whose decode the gfx950 conversion instructions do exactly
// (TileView::fast): bf16, MXFP4, FP8, INT4.
//
// Two kernels:
//
// split_kernel writes the activations once as bf16 MFMA A fragments, XT
// terms per value (x = t0 + t1 (+ t2), each the round-to-nearest-even bf16
// of the remainder), in the order the product reads them:
//     xs[m16][kt][term][lane] (16 B each), lane l = token 16*m16 + l%16,
//     k = 32*kt + 8*(l/16) .. +8
// so every A fragment is one contiguous KiB. k tiles past the matrix are
// zero up to a whole number of pipeline stages.
//
// tile_gemm_kernel: a workgroup of waves side by side computes 64 tokens x
// 64 rows per wave (64 accumulator registers, two waves per SIMD). A stage
// covers 64 or 128 k: its A fragments, each wave's weight codes (1 KiB units
// of 16 rows) and per-row side words (scales) are copied global -> LDS with
// global_load_lds (no registers, double buffered; with two waves per SIMD
// only the younger wave of each SIMD issues them), then every wave decodes
// its weight tiles with v_cvt_scalef32_pk_bf16_fp4 (MXFP4), v_cvt_pk_f32_fp8
// + f32 scale + v_cvt_pk_bf16_f32 (FP8) or integer unpacking (INT4) and
// issues the MFMAs, reading k tile t + 1's A fragments and decoding its
// weights between k tile t's MFMAs (the order is fixed with
// sched_group_barrier). The block index is remapped so that the workgroups
// an XCD runs at the same time cover an 8 x (few) patch of output tiles:
// they share A and W tiles in that XCD's L2.
#include <type_traits>

#include "gemm_common.h"
#include "gemm_wide.h"
#include "tile_decode.h"

namespace ditch {

// ---------------------------------------------------------------------------
// activation fragments

struct SplitParams {
    u32x4 *xs;
    const float *x;
    const int32_t *row_index;  // optional gather of x rows
    const int32_t *prow;       // optional: fragment row -> row of the gathered space, -1 for a zero row
    int64_t n, ldx, K;
    int64_t kt_total;  // k tiles per 16-token block (the fragments' ldk)
    int64_t m16;       // 16-token blocks
    // optional: a delta's A [rank][K]; each 32-column k tile's x . A^T
    // partial sums go to xa_part [n][kt_total][rank]
    const float *da = nullptr;
    float *xa_part = nullptr;
    int rank = 0;
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
    int64_t gi = tok;
    bool valid = tok < p.n;
    if (valid && p.prow) {
        gi = p.prow[tok];
        valid = gi >= 0;
    }
    if (valid) {
        int64_t src = p.row_index ? (int64_t)p.row_index[gi] : gi;
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
    if (p.xa_part) {
        // the k tile's x . A^T: each lane's 8 products in column order, then
        // its k quarters added pairwise ((q0 + q1) + (q2 + q3))
        for (int j = 0; j < p.rank; j++) {
            const float *aj = p.da + (int64_t)j * p.K + k0;
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < 8; q++) s = __builtin_fmaf(v[q], k0 + q < p.K ? aj[q] : 0.f, s);
            s = __fadd_rn(s, __shfl_xor(s, 16, 64));
            s = __fadd_rn(s, __shfl_xor(s, 32, 64));
            if ((lane >> 4) == 0 && tok < p.n) p.xa_part[(tok * p.kt_total + kt) * p.rank + j] = s;
        }
    }
    u32x4 w[XT];
    a_words<false, XT>(v, w);
#pragma unroll
    for (int e = 0; e < XT; e++) p.xs[(f * XT + e) * 64 + lane] = w[e];
}

// xa[t][j] = the k tiles' partial sums of split_kernel, one wave a token:
// lane l adds tiles l, l + 64, ... in order, then the lanes' sums are added
// pairwise (xor 32, 16, .., 1)
__global__ __launch_bounds__(256) void xa_tiles_reduce_kernel(float *xa, const float *part, int64_t n,
                                                              int64_t kt_total, int rank) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const float *pp = part + t * kt_total * rank;
    for (int j = 0; j < rank; j++) {
        float s = 0.f;
        for (int64_t kt = lane; kt < kt_total; kt += 64) s = __fadd_rn(s, pp[kt * rank + j]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s = __fadd_rn(s, __shfl_xor(s, o, 64));
        if (lane == 0) xa[t * rank + j] = s;
    }
}

// Token-major activation terms for the routed products: out[token][k tile]
// [term][k quarter] (16 bytes each, the same words split_kernel writes for
// the token's fragment lanes), so that a routed tile gathers each pair's
// pieces from its token's row (64 contiguous bytes per k tile and term)
// instead of a copy of the row per pair.
template <int XT>
__global__ __launch_bounds__(256) void split_tok_kernel(u32x4 *out, const float *x, int64_t n, int64_t ldx, int64_t K,
                                                        int64_t kt_total) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n * kt_total * 4) return;
    const int kq = (int)(t & 3);
    const int64_t kt = (t >> 2) % kt_total, tok = (t >> 2) / kt_total;
    const int64_t k0 = kt * 32 + 8 * kq;
    const float *xr = x + tok * ldx;
    float v[8];
    if (k0 + 8 <= K && ((((uintptr_t)(xr + k0)) & 15) == 0)) {
        const float4 a = *(const float4 *)(xr + k0), b = *(const float4 *)(xr + k0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = k0 + j < K ? xr[k0 + j] : 0.f;
    }
    u32x4 w[XT];
    a_words<false, XT>(v, w);
#pragma unroll
    for (int e = 0; e < XT; e++) out[((tok * kt_total + kt) * XT + e) * 4 + kq] = w[e];
}

// ---------------------------------------------------------------------------

struct TileGemmParams {
    TileView w;
    TileView w2;            // GLU: the up projection (w is the gate)
    const u32x4 *xs;
    int64_t kt_total;       // k tiles the product runs over
    int64_t ldk;            // k tiles per 16-token block in xs (>= kt_total)
    uint32_t act;           // GLU: activation code (tensor.Activation order)
    u32x4 *xs_out;          // GLU: act(gate) * up as A fragments of the next product
    int64_t ldk_out;
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
    // grouped (routed experts): tile row mt is descriptor gdesc[4 mt ..]:
    // segment, first 16-token block, the segment's end block, the block's
    // first token within the segment; the segment's weight, output rows and
    // delta come from gsegs
    const GroupSeg *gsegs;
    const GroupSeg *gsegs2;  // GLU and grouped: the up projection of each segment
    const int32_t *gdesc;
    const int32_t *gcount;   // grouped, planned on the device: tile rows in use (the grid covers a bound)
    // split-K (plain products): blockIdx.y takes stages [y S / ksplit, (y + 1) S / ksplit)
    // and stores its raw sums in part[y][n][rows]; ksplit_reduce_kernel adds them
    int ksplit;
    float *part;
    // GLU, grouped: the routed down projections' delta products x . A^T
    // formed from act(gate) * up in the epilogue: segment z's delta A
    // [rank][rows of w] is xa_a[z] with rank xa_segs[z].delta_rank; each
    // wave writes the sums over its 32 output columns to xa_part[((tile
    // column * WGN + wave) * xa_pairs + pair) * xa_stride + j], for
    // xa_reduce_kernel to add
    const float *const *xa_a;
    const GroupSeg *xa_segs;
    float *xa_part;
    int64_t xa_pairs;
    int xa_parts, xa_stride;
    // GLU, grouped: the A fragments gathered from token-major terms
    // (split_tok_kernel) instead of xs: fragment row r of the plan is pair
    // a_prow[r] (-1: padding), token a_map[pair]; a_tok_stride bytes a token
    const u32x4 *a_tok;
    const int32_t *a_prow, *a_map;
    int64_t a_tok_stride;
};

// Where a tile's outputs go: a plain product's, or a routed segment's
struct TileOut {
    float *out;
    int64_t ldo, n, rows;
    const float *bias;
    int accumulate;
    const float *delta_b, *delta_xa;
    int delta_rank, delta_stride;
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

__device__ __forceinline__ void tile_store(const TileOut &p, int64_t tok, int64_t row, float v) {
    if (tok >= p.n || row >= p.rows) return;
    if (p.delta_rank > 0) {
        float d = 0.f;
        for (int j = 0; j < p.delta_rank; j++)
            d = __builtin_fmaf(p.delta_b[row * p.delta_rank + j], p.delta_xa[tok * p.delta_stride + j], d);
        v = __fadd_rn(v, d);
    }
    if (p.bias) v = __fadd_rn(v, p.bias[row]);
    float *o = p.out + tok * p.ldo + row;
    if (p.accumulate) v = __fadd_rn(*o, v);
    *o = v;
}

// tile_store over a lane's tile (tokens tb[m] + r, rows rw[i]) with the
// same arithmetic in the same order, one 16-token block at a time: the
// block's operands (delta factors, bias, old outputs) are all read before
// its first store, so their loads are in flight together. Element by
// element, each read of an output waits for the store before it (the
// addresses may alias), and the residual add then pays one memory latency
// per element.
// The lane's rows' delta factors of the first four directions (loaded when
// the kernel starts: the epilogue of each round of workgroups then waits on
// no load for them).
template <int NI>
__device__ __forceinline__ void delta_b_first(const TileOut &p, const int64_t (&rw)[NI], float (&b0)[4][NI]) {
    const int nj0 = p.delta_rank < 4 ? p.delta_rank : 4;
#pragma unroll
    for (int jj = 0; jj < 4; jj++)
#pragma unroll
        for (int i = 0; i < NI; i++)
            b0[jj][i] = jj < nj0 && rw[i] < p.rows ? p.delta_b[rw[i] * p.delta_rank + jj] : 0.f;
}

template <int NM, int NI, bool PRE = false>
__device__ __forceinline__ void tile_store_block(const TileOut &p, const int64_t (&tb)[NM], const int64_t (&rw)[NI],
                                                 floatx4 (&acc)[NM][NI], const float (*b0)[NI] = nullptr) {
    bool rin[NI];
    float bias[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        rin[i] = rw[i] < p.rows;
        bias[i] = p.bias && rin[i] ? p.bias[rw[i]] : 0.f;
    }
    // PRE: every block's tokens' first four x . A^T values, loaded before
    // the first store (a store may alias them, so loads after it wait)
    float x0[PRE ? NM : 1][4][4];
    if constexpr (PRE) {
        if (p.delta_rank > 0) {
            const int nj0 = p.delta_rank < 4 ? p.delta_rank : 4;
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        x0[m][jj][r] = jj < nj0 && tb[m] + r < p.n ? p.delta_xa[(tb[m] + r) * p.delta_stride + jj] : 0.f;
        }
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
            if constexpr (PRE) {
                // four directions' factors a load round (the first four:
                // b0, loaded when the kernel started, and x0)
                for (int j0 = 0; j0 < p.delta_rank; j0 += 4) {
                    const int nj = p.delta_rank - j0 < 4 ? p.delta_rank - j0 : 4;
                    float bj[4][NI], xj[4][4];
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
#pragma unroll
                        for (int i = 0; i < NI; i++)
                            bj[jj][i] = j0 == 0 ? b0[jj][i]
                                                : (jj < nj && rin[i] ? p.delta_b[rw[i] * p.delta_rank + j0 + jj] : 0.f);
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            xj[jj][r] = j0 == 0 ? x0[m][jj][r]
                                                : (jj < nj && tin[r] ? p.delta_xa[(tb[m] + r) * p.delta_stride + j0 + jj]
                                                                     : 0.f);
                    }
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        if (jj >= nj) break;
#pragma unroll
                        for (int i = 0; i < NI; i++)
#pragma unroll
                            for (int r = 0; r < 4; r++) d[i][r] = __builtin_fmaf(bj[jj][i], xj[jj][r], d[i][r]);
                    }
                }
            } else {
                for (int j = 0; j < p.delta_rank; j++) {
                    float bj[NI], xj[4];
#pragma unroll
                    for (int i = 0; i < NI; i++) bj[i] = rin[i] ? p.delta_b[rw[i] * p.delta_rank + j] : 0.f;
#pragma unroll
                    for (int r = 0; r < 4; r++) xj[r] = tin[r] ? p.delta_xa[(tb[m] + r) * p.delta_stride + j] : 0.f;
#pragma unroll
                    for (int i = 0; i < NI; i++)
#pragma unroll
                        for (int r = 0; r < 4; r++) d[i][r] = __builtin_fmaf(bj[i], xj[r], d[i][r]);
                }
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
                for (int r = 0; r < 4; r++) old[i][r] = rin[i] && tin[r] ? p.out[(tb[m] + r) * p.ldo + rw[i]] : 0.f;
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) v[i][r] = __fadd_rn(old[i][r], v[i][r]);
        }
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (rin[i] && tin[r]) p.out[(tb[m] + r) * p.ldo + rw[i]] = v[i][r];
    }
}

// s_waitcnt operand: wait until at most n vector memory loads are in flight
// (expcnt and lgkmcnt left at their no-wait maxima).
__host__ __device__ constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

typedef __attribute__((address_space(3))) void lds_void;

// The grouped and plain GLU epilogue of a wave's tile: act(gate) * up
// (tensor.gatedActivation), as f32 rows and/or as the A fragments of the
// next product; each 16-token block of the wave's 32-column k tile goes
// through the wave's LDS patch [16][32] (the stage buffers are idle: the
// last stage ended with a barrier). Grouped: tokens and output rows within
// the segment, fragment blocks in the padded order of the row map, and the
// routed down delta's x . A^T partial sums over the wave's columns (part
// `part`; xa0: the first four directions' A of its columns). tokb: the
// token of the wave's first row (within the output rows), mblk0 its block.
template <int WM, int OG, bool GR>
__device__ __forceinline__ void glu_epilogue(const TileGemmParams &p, const TileOut &to, int64_t rows,
                                             floatx4 (&acc)[WM][2 * OG], int64_t tokb, int64_t mblk0, int64_t m16_n,
                                             int64_t g0, float *patch, int lane, int seg, int part, int xa_rank,
                                             const float (&xa0)[4][OG]) {
    const int kq = lane >> 4;
    // the gates' activation first, the activation's switch outside the loops
    with_act(p.act, [&](auto ac) {
        constexpr int A = decltype(ac)::value;
#pragma unroll
        for (int m = 0; m < WM; m++)
#pragma unroll
            for (int i = 0; i < OG; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[m][i][r] = act_fused<A>(acc[m][i][r]);
    });
#pragma unroll
    for (int m = 0; m < WM; m++) {
        const int64_t mblk = mblk0 + m;
#pragma unroll
        for (int i = 0; i < OG; i++) {
            const int64_t col = (g0 + i) * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t tok = tokb + m * 16 + 4 * kq + r;
                float y = __fmul_rn(acc[m][i][r], acc[m][i + OG][r]);
                if (tok >= to.n || col >= rows) y = 0.f;
                else if (p.out) to.out[tok * to.ldo + col] = y;
                patch[(4 * kq + r) * 32 + (i & 1) * 16 + (lane & 15)] = y;
            }
            if ((i & 1) && p.xs_out && mblk < m16_n && ((g0 + i - 1) * 16) / 32 < p.ldk_out) {
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = patch[(lane & 15) * 32 + 8 * kq + j];
                u32x4 words[2];
                a_words<false, 2>(v, words);
                const int64_t kt = ((g0 + i - 1) * 16) / 32;
#pragma unroll
                for (int e = 0; e < 2; e++) p.xs_out[((mblk * p.ldk_out + kt) * 2 + e) * 64 + lane] = words[e];
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            }
        }
    }
    if constexpr (GR) {
        // the routed delta's x . A^T over this wave's columns: per token,
        // the 16 lanes of a DPP row hold 16 columns of each of the wave's
        // groups (y as stored above)
        const int rank = xa_rank;
        if (rank > 0) {
            const float *A = p.xa_a[seg];
            const int64_t base = p.gsegs[seg].off;
            float *xp = p.xa_part + (int64_t)part * p.xa_pairs * p.xa_stride;
            float y[WM][OG][4];
#pragma unroll
            for (int m = 0; m < WM; m++)
#pragma unroll
                for (int i = 0; i < OG; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int64_t tok = tokb + m * 16 + 4 * kq + r;
                        const int64_t col = (g0 + i) * 16 + (lane & 15);
                        y[m][i][r] = tok >= to.n || col >= rows ? 0.f : __fmul_rn(acc[m][i][r], acc[m][i + OG][r]);
                    }
            for (int j0 = 0; j0 < rank; j0 += 4) {
                float aj[4][OG];
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int i = 0; i < OG; i++) {
                        const int64_t col = (g0 + i) * 16 + (lane & 15);
                        aj[jj][i] = j0 == 0 ? xa0[jj][i]
                                            : (j0 + jj < rank && col < rows ? A[(int64_t)(j0 + jj) * rows + col] : 0.f);
                    }
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if (j0 + jj >= rank) break;
#pragma unroll
                    for (int m = 0; m < WM; m++)
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int64_t tok = tokb + m * 16 + 4 * kq + r;
                            float sum = 0.f;
#pragma unroll
                            for (int i = 0; i < OG; i++) sum = __builtin_fmaf(y[m][i][r], aj[jj][i], sum);
                            sum = row16_sum(sum);
                            if ((lane & 15) == 0 && tok < to.n) xp[(base + tok) * p.xa_stride + j0 + jj] = sum;
                        }
                }
            }
        }
    }
}

// the A of the routed down delta over a wave's columns, first four directions
template <int OG>
__device__ __forceinline__ int xa_first(const TileGemmParams &p, int seg, int64_t g0, int64_t rows, int lane,
                                        float (&xa0)[4][OG]) {
    const int rank = p.xa_part ? p.xa_segs[seg].delta_rank : 0;
    if (rank > 0) {
        const float *A = p.xa_a[seg];
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
            for (int i = 0; i < OG; i++) {
                const int64_t col = (g0 + i) * 16 + (lane & 15);
                xa0[jj][i] = jj < rank && col < rows ? A[(int64_t)jj * rows + col] : 0.f;
            }
    }
    return rank;
}

// Every operand of a stage travels global -> LDS by DMA (global_load_lds:
// lane l's bytes land at the destination + l * size), two stage buffers:
// stage s + 1 is copied while stage s is computed, and a stage ends with
// this wave's copies drained plus a barrier. No global load writes a
// register inside the loop.
template <int TF, int XT, int WGM, int WGN, int WM, int WN, bool GLU, bool GR = false>
__global__ __launch_bounds__(WGM * WGN * 64) void tile_gemm_kernel(TileGemmParams p) {
    constexpr int WAVES = WGM * WGN;
    constexpr int TPS = TileCfg<TF>::TPS, NU = TileCfg<TF>::NU, NS = TileCfg<TF>::NS;
    constexpr int NS1 = NS ? NS : 1;
    constexpr int FR = WGM * WM * TPS * XT;  // A fragments per stage: [m][t][term]
    // two stage buffers as distinct LDS objects, so that the compiler can
    // tell the DMA into one from the reads of the other (with one array it
    // waits for every copy in flight before any LDS read)
    __shared__ u32x4 As0[FR * 64], As1[FR * 64];                            // [fragment][lane]
    __shared__ u32x4 Bs0[WAVES * WN * NU * 64], Bs1[WAVES * WN * NU * 64];  // [wave][group][unit][lane]
    __shared__ uint32_t Ss0[WAVES * NS1 * 64], Ss1[WAVES * NS1 * 64];        // [wave][entry][group][row]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave_m = wave / WGN, wave_n = wave % WGN;
    int mt, nt;
    {
        // grouped and planned on the device: the grid covers a bound, the
        // tiles in use (the first *gcount tile rows) are spread over the
        // first blocks as a grid of their own size would be, and the rest
        // of the workgroups exit at once
        int tm = p.tiles_m, G = (int)gridDim.x;
        if (GR && p.gcount) {
            tm = *p.gcount;
            G = tm * p.tiles_n;
            if ((int)blockIdx.x >= G) return;
        }
        map_tile(blockIdx.x, G, tm, p.tiles_n, mt, nt);
    }
    const int32_t *gd = GR ? p.gdesc + 4 * mt : nullptr;
    // the weights' descriptions by value: read through a reference into the
    // segment table they would be loaded again at every stage (the copies
    // and stores in the loop might, as far as the compiler knows, change
    // them), and each stage's copies would wait for those loads
    const TileView w = GR ? p.gsegs[gd[0]].w : p.w;
    const TileView w2 = GR && GLU ? p.gsegs2[gd[0]].w : p.w2;
    TileOut to{p.out, p.ldo, p.n, w.rows, p.bias, p.accumulate, p.delta_b, p.delta_xa, p.delta_rank, p.delta_stride};
    int64_t tok0;  // token (within the output rows) of the tile's first block
    // row groups of this wave: WN of w, or (GLU) the same WN/2 output groups
    // of the gate (w) and of the up projection (w2)
    constexpr int OG = GLU ? WN / 2 : WN;  // output row groups per wave
    static_assert(!GLU || WN % 4 == 0, "a GLU wave covers whole 32-column k tiles of its output");
    const int64_t groups = (w.rows + 15) / 16;
    const int64_t g0 = (int64_t)nt * (OG * WGN) + wave_n * OG;
    int64_t m16_0, m16_n;
    if constexpr (GR) {
        const GroupSeg &sg = p.gsegs[gd[0]];
        m16_0 = gd[1];
        m16_n = gd[2];
        tok0 = gd[3];
        to.out = p.out + sg.off * p.ldo;
        to.n = sg.cnt;
        to.bias = nullptr;
        to.delta_b = sg.delta_b;
        to.delta_rank = sg.delta_rank;
        to.delta_xa = sg.delta_rank ? p.delta_xa + sg.off * p.delta_stride : nullptr;
    } else {
        m16_0 = (int64_t)mt * (WGM * WM);
        m16_n = (p.n + 15) / 16;
        tok0 = m16_0 * 16;
    }
    const int64_t S_all = p.kt_total / TPS;
    const int ks = GLU || GR ? 0 : (int)blockIdx.y, nks = GLU || GR ? 1 : p.ksplit;
    const int64_t s_begin = S_all * ks / nks, S = S_all * (ks + 1) / nks;  // this block's stages
    if (nks > 1) {
        to = TileOut{p.part + (int64_t)ks * p.n * w.rows, w.rows, p.n, w.rows, nullptr, 0, nullptr, nullptr, 0, 0};
    }
    const int64_t units = w.units_k;
    // the grouped epilogues' delta factors that depend on the rows only,
    // loaded now (routed products: the first four directions' B of the
    // wave's rows; grouped GLU: the first four directions' A of the routed
    // down delta over the wave's columns)
    float b0[4][WN];
    float xa0[4][OG];
    int xa_rank = 0;
    if constexpr (!GLU && GR) {
        if (to.delta_rank > 0) {
            int64_t rw0[WN];
#pragma unroll
            for (int i = 0; i < WN; i++) rw0[i] = (g0 + i) * 16 + (lane & 15);
            delta_b_first(to, rw0, b0);
        }
    } else if constexpr (GR) {
        xa_rank = xa_first<OG>(p, gd[0], g0, w.rows, lane, xa0);
    }

    // Copies: a global_load_lds stalls the issuing wave while the texture
    // unit's queue is full, so with two waves per SIMD only the younger one
    // (waves WAVES/2.., which the issue arbiter serves after the older one)
    // issues the copies of a stage, and the older waves run their products
    // undisturbed. With one wave per SIMD every wave copies its share.
    constexpr int CW = WAVES >= 8 ? WAVES / 2 : WAVES;  // copying waves
    constexpr int CA = FR / CW, CB = WAVES * WN * NU / CW, CS = NS ? WAVES * NS / CW : 0;
    static_assert(FR % CW == 0 && (WAVES * WN * NU) % CW == 0 && (WAVES * NS) % CW == 0, "copies split evenly");
    static_assert(WN == 4, "one side-word copy covers a wave's four row groups");
    // Copier ck takes a contiguous run of each stage array (A fragments
    // ck CA .., code pieces ck CB .., side words ck CS ..) and writes it in
    // 4 KiB windows: an LDS copy writes at M0 plus its instruction offset
    // (which moves the global address too, so the source pointer is lowered
    // by it): one M0 write per window instead of one per copy, so the
    // copies issue back to back (measured faster than an M0 write before
    // every copy).
    const bool copier = wave >= WAVES - CW;
    const int ck = copier ? wave - (WAVES - CW) : 0;
    // sources: a uniform base per copy (scalar registers) plus the lane's 16
    // bytes of the 1 KiB piece (one shared 32-bit register); per-lane 64-bit
    // pointers would not fit beside the products' registers, and a spilled
    // pointer's reload waits for every copy in flight
    // (computed per copy from a few uniform values in scalar registers:
    // arrays of precomputed bases exhaust them and end up spilled)
    const uint32_t lofs = (uint32_t)lane * 16;
    auto asrc = [&](int j) {  // copy j's A fragment, stage 0
        const int f = ck * CA + j;
        const int m = f / (TPS * XT), t = (f / XT) % TPS, e = f % XT;
        int64_t mb = m16_0 + m;
        mb = mb < m16_n ? mb : m16_n - 1;
        return (const char *)(p.xs + ((mb * p.ldk + t) * XT + e) * 64);
    };
    auto group_of = [&](int wq, int i) {
        const int64_t gi = (int64_t)nt * (OG * WGN) + (wq % WGN) * OG + (i % OG);
        return gi < groups ? gi : groups - 1;
    };
    auto bsrc = [&](int j) {  // copy j's code pieces, unit 0
        const int q = ck * CB + j, wq = q / (WN * NU), i = (q / NU) % WN;
        const TileView &wi = (GLU && i >= OG) ? w2 : w;
        return wi.codes + group_of(wq, i) * units * 1024;
    };
    const SideStep sst = side_step<TF>(w);
    const uint32_t *ssrc[CS > 0 ? CS : 1];
#pragma unroll
    for (int j = 0; j < CS; j++) {
        const int q = ck * CS + j, wq = q / NS1, i = lane >> 4;  // lane l: row l % 16 of row group l / 16
        const TileView &wi = (GLU && i >= OG) ? w2 : w;
        ssrc[j] = wi.side + side_row(wi, group_of(wq, i), lane);
    }

    // gathered A (grouped GLU with token-major terms): copier ck copies
    // every fragment of block m16_0 + ck (CA == TPS * XT), so each lane
    // keeps one pointer: its row's token, its k quarter
    constexpr bool GATHER = GR && GLU && TF != TF_Q8;  // (Q8: no registers to spare)
    const char *gsrc = nullptr;
    if constexpr (GATHER) {
        static_assert(CA == TPS * XT, "one copier per token block of the tile");
        if (p.a_tok && copier) {
            int64_t mb = m16_0 + ck;
            mb = mb < m16_n ? mb : m16_n - 1;
            const int32_t pr = p.a_prow[mb * 16 + (lane & 15)];
            const int64_t tok = pr >= 0 ? (int64_t)p.a_map[pr] : 0;
            gsrc = (const char *)p.a_tok + tok * p.a_tok_stride + (lane >> 4) * 16;
        }
    }
    auto copy_stage = [&](int64_t s, u32x4 *As, u32x4 *Bs, uint32_t *Ss) {
        if (!copier) return;
        // copy j of a run of 1 KiB pieces: window j / 4, offset (j % 4) KiB
        if (GATHER && gsrc) {
            // fragment (k tile s TPS + j / XT, term j % XT): 64 bytes of the
            // token's row per k tile and term
            static_for<CA>([&](auto jc) {
                constexpr int j = decltype(jc)::value, off = (j % 4) * 1024;
                __builtin_amdgcn_global_load_lds((const void *)(gsrc + (TPS * s * XT * 64 + j * 64 - off)),
                                                 (lds_void *)&As[(ck * CA + j / 4 * 4) * 64], 16, off, 0);
            });
        } else {
            static_for<CA>([&](auto jc) {
                constexpr int j = decltype(jc)::value, off = (j % 4) * 1024;
                __builtin_amdgcn_global_load_lds((const void *)(asrc(j) + (TPS * s * XT * 64 * 16 - off) + lofs),
                                                 (lds_void *)&As[(ck * CA + j / 4 * 4) * 64], 16, off, 0);
            });
        }
        static_for<CB>([&](auto jc) {
            constexpr int j = decltype(jc)::value, off = (j % 4) * 1024;
            const int q = ck * CB + j, u = q % NU;
            int64_t un = s * NU + u;
            un = un < units ? un : units - 1;  // a bf16 stage's missing second unit: decoded as zero
            __builtin_amdgcn_global_load_lds((const void *)(bsrc(j) + (un * 1024 - off) + lofs),
                                             (lds_void *)&Bs[(ck * CB + j / 4 * 4) * 64], 16, off, 0);
        });
        if constexpr (NS > 0) {
            // 256 B each: sixteen to a window
            static_for<CS>([&](auto jc) {
                constexpr int j = decltype(jc)::value, off = (j % 16) * 256;
                const int q = ck * CS + j;
                __builtin_amdgcn_global_load_lds(
                    (const void *)((const char *)side_word<TF>(sst, ssrc[j], s, q % NS1) - off),
                    (lds_void *)&Ss[(ck * CS + j / 16 * 16) * 64], 4, off, 0);
            });
        }
    };

    floatx4 acc[WM][WN];
#pragma unroll
    for (int m = 0; m < WM; m++)
#pragma unroll
        for (int i = 0; i < WN; i++) acc[m][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    copy_stage(s_begin, As0, Bs0, Ss0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // one stage: the copying waves copy stage s + 1 into the other buffers
    // (every wave finished reading them in stage s - 1; the last stage
    // repeats itself into the idle buffers), every wave computes stage s,
    // drains its copies and meets the others at the barrier
    auto step = [&](int64_t s, const u32x4 *As, const u32x4 *Bs, const uint32_t *Ss, u32x4 *An, u32x4 *Bn,
                    uint32_t *Sn) {
        copy_stage(s + 1 < S ? s + 1 : s, An, Bn, Sn);
        __builtin_amdgcn_sched_barrier(0);
        u32x4 c[WN][NU];
        uint32_t sd[WN][NS1];
#pragma unroll
        for (int i = 0; i < WN; i++) {
#pragma unroll
            for (int u = 0; u < NU; u++) c[i][u] = Bs[((wave * WN + i) * NU + u) * 64 + lane];
#pragma unroll
            for (int j = 0; j < NS1; j++) sd[i][j] = NS ? Ss[(wave * NS1 + j) * 64 + i * 16 + (lane & 15)] : 0u;
        }
        const bool second = TF != TF_BF16 || 2 * s + 1 < units;
        const u32x4 *A = As + wave_m * WM * TPS * XT * 64 + lane;
        // k tile t + 1's A fragments are read and its weight tiles decoded
        // while k tile t's products issue (two register sets). Q8_0 keeps one
        // A set, read again once k tile t's products have issued: its block-
        // scaled partial sums need the registers, and a kernel that spills
        // reloads its copy addresses behind a wait for every copy in flight.
        constexpr int AS = TF == TF_Q8 || WM > 4 ? 1 : 2;
        u32x4 a[AS][WM][XT], bf[2][WN];
#pragma unroll
        for (int m = 0; m < WM; m++)
#pragma unroll
            for (int e = 0; e < XT; e++) a[0][m][e] = A[(m * TPS * XT + e) * 64];
#pragma unroll
        for (int i = 0; i < WN; i++) bf[0][i] = decode_tile_lds<TF>(w, c[i], sd[i], 0, second);
        __builtin_amdgcn_sched_barrier(0);
        // issue order: each k tile's products interleaved with the next k
        // tile's A reads (one per product), then with its weight decode
        // VALU per product: roughly the decode's instruction count per k tile
        // over the products left after the A reads
        constexpr int NA = WM * XT, NM = WM * XT * WN, NV = NM - NA;
        constexpr int VPM = TF == TF_BF16 ? 1 : TF == TF_MX4 ? 2 : TF == TF_FP8 ? 3 : TF == TF_Q8 ? 5 : 4;
        auto order = [&](int t) {
            if (t + 1 < TPS && AS == 2) {
#pragma unroll
                for (int j = 0; j < NA; j++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
#pragma unroll
                for (int j = 0; j < NV; j++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
                }
            } else if (t + 1 < TPS) {  // one A set: the next tile's reads after the products
#pragma unroll
                for (int j = 0; j < NM; j++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, NA, 0);
            } else {
                __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
            }
        };
        // FP8: the wave's priority falls by a step a k tile, so of the two
        // waves that share a SIMD the one behind in the stage wins the
        // arbitration (each priority change ends a scheduling region: the k
        // tile's order is set inside it); measured 2 % faster on the C3 FP8
        // GLU, and 1 % slower on the INT4 products, which keep one region
        constexpr bool PRIO = TF == TF_FP8;
#pragma unroll
        for (int t = 0; t < TPS; t++) {
            if constexpr (PRIO) {
                const int pr = 3 - (3 * t) / (TPS > 1 ? TPS - 1 : 1);
                if (pr >= 3) __builtin_amdgcn_s_setprio(3);
                else if (pr == 2) __builtin_amdgcn_s_setprio(2);
                else if (pr == 1) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
            const int cu = t & 1, nx = cu ^ 1;
            const int ca = AS == 2 ? cu : 0;
            if (AS == 2 && t + 1 < TPS) {
#pragma unroll
                for (int m = 0; m < WM; m++)
#pragma unroll
                    for (int e = 0; e < XT; e++) a[AS == 2 ? nx : 0][m][e] = A[((m * TPS + t + 1) * XT + e) * 64];
            }
            if constexpr (TF == TF_Q8) {
                // Q8_0: each 32-column k tile is one block; its f16 scale
                // (side word half t) multiplies the tile's partial sum
                float sq[WN];
#pragma unroll
                for (int i = 0; i < WN; i++) sq[i] = f16_to_f32_hw((uint16_t)(sd[i][0] >> (16 * t)));
#pragma unroll
                for (int m = 0; m < WM; m++)
#pragma unroll
                    for (int i = 0; i < WN; i++) {
                        floatx4 pt = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int e = 0; e < XT; e++) pt = mfma_bf16(a[ca][m][e], bf[cu][i], pt);
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[m][i][r] = __builtin_fmaf(sq[i], pt[r], acc[m][i][r]);
                    }
            } else {
#pragma unroll
                for (int m = 0; m < WM; m++)
#pragma unroll
                    for (int e = 0; e < XT; e++)
#pragma unroll
                        for (int i = 0; i < WN; i++) acc[m][i] = mfma_bf16(a[ca][m][e], bf[cu][i], acc[m][i]);
            }
            if (AS == 1 && t + 1 < TPS) {
#pragma unroll
                for (int m = 0; m < WM; m++)
#pragma unroll
                    for (int e = 0; e < XT; e++) a[0][m][e] = A[((m * TPS + t + 1) * XT + e) * 64];
            }
            if (t + 1 < TPS) {
#pragma unroll
                for (int i = 0; i < WN; i++) bf[nx][i] = decode_tile_lds<TF>(w, c[i], sd[i], t + 1, second);
            }
            if constexpr (PRIO) order(t);
        }
        if constexpr (!PRIO) {
#pragma unroll
            for (int t = 0; t < TPS; t++) order(t);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of stage s + 1 landed
        __builtin_amdgcn_s_barrier();              // ... and every other wave's
        __builtin_amdgcn_sched_barrier(0);
    };
    int64_t s = s_begin;
    for (; s + 1 < S; s += 2) {
        step(s, As0, Bs0, Ss0, As1, Bs1, Ss1);
        step(s + 1, As1, Bs1, Ss1, As0, Bs0, Ss0);
    }
    if (s < S) step(s, As0, Bs0, Ss0, As1, Bs1, Ss1);

    const int kq = lane >> 4;
    if constexpr (!GLU) {
        int64_t tb[WM], rw[WN];
#pragma unroll
        for (int m = 0; m < WM; m++) tb[m] = tok0 + (wave_m * WM + m) * 16 + 4 * kq;
#pragma unroll
        for (int i = 0; i < WN; i++) rw[i] = (g0 + i) * 16 + (lane & 15);
        if constexpr (GR) tile_store_block<WM, WN, true>(to, tb, rw, acc, b0);
        else tile_store_block(to, tb, rw, acc);
    } else {
        glu_epilogue<WM, OG, GR>(p, to, w.rows, acc, tok0 + wave_m * WM * 16, m16_0 + wave_m * WM, m16_n, g0,
                                 (float *)As0 + wave * 16 * 32, lane, GR ? gd[0] : 0, nt * WGN + wave_n, xa_rank, xa0);
    }
}

// xa[p][j] = the sum of the parts' entries for pair p in part order (part
// k's [P][stride] slab at k P stride; j below a segment's rank only is used)
__global__ void xa_reduce_kernel(float *xa, const float *part, int64_t P, int parts, int stride) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < P * stride;
         t += (int64_t)gridDim.x * blockDim.x) {
        float sum = 0.f;
        for (int k0 = 0; k0 < parts; k0 += 8) {  // eight parts' loads in flight, then their sums in order
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = k0 + k < parts ? part[(int64_t)(k0 + k) * P * stride + t] : 0.f;
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (k0 + k < parts) sum = __fadd_rn(sum, v[k]);
        }
        xa[t] = sum;
    }
}

// ---------------------------------------------------------------------------
// MXFP4 weights on the scaled MFMA
//
// v_mfma_scale_f32_16x16x128_f8f6f4 multiplies a 16 x 128 A block by a 128 x 16
// B block where each lane supplies 32 consecutive k of one row / column with
// one E8M0 scale: lane l holds row l % 16, k = 32 (l / 16) .. +32. With B =
// the MXFP4 codes (e2m1) and their own E8M0 block scales, the weights enter
// exactly (the e2m1 value times 2^k is what the reference's bf16 decode
// yields). The activations enter as MX_TERMS fp6 (e2m3) terms with their own
// E8M0 scale per 32-k block: x = sum_e code_e * 2^s_e + r, each term the
// round-to-nearest-even e2m3 value of the remainder over the scale that puts
// the remainder's block maximum in (3.75, 7.5]; every subtraction is exact,
// so |r| <= 2^-3.9 of the previous remainder's block maximum, i.e. after four
// terms |r| <= 15^-4 * max|x over the block| ~ 2^-15.6 max|x|. The fp6 x fp4
// MFMA runs at four times the bf16 rate: four terms cost what one bf16 term
// does, against two bf16 terms on the bf16 path.
//
struct MxSplitParams {
    u32x4 *xm;
    const float *x;
    const int32_t *row_index;
    int64_t n, ldx, K, ldst, m16;
};

__global__ __launch_bounds__(256) void split_mx_kernel(MxSplitParams p) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= p.m16 * p.ldst * 64) return;
    const int lane = (int)(t & 63);
    const int64_t f = t >> 6;  // m16 * ldst + stage
    const int64_t st = f % p.ldst, mb = f / p.ldst;
    const int64_t tok = mb * 16 + (lane & 15);
    const int64_t k0 = st * 128 + 32 * (lane >> 4);
    float r[32];
    if (tok < p.n) {
        const int64_t src = p.row_index ? (int64_t)p.row_index[tok] : tok;
        const float *xr = p.x + src * p.ldx;
        if (k0 + 32 <= p.K && ((((uintptr_t)(xr + k0)) & 15) == 0)) {
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
                const float4 v = *(const float4 *)(xr + k0 + j);
                r[j] = v.x; r[j + 1] = v.y; r[j + 2] = v.z; r[j + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; j++) r[j] = (k0 + j < p.K) ? xr[k0 + j] : 0.f;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; j++) r[j] = 0.f;
    }
    mx_write_slot(r, (uint8_t *)p.xm + f * MX_BLOCK, lane);
}

typedef int v8i_t __attribute__((ext_vector_type(8)));

// Fourth word of a raw buffer resource (32-bit data format; with stride 0
// the record count is a byte count and reads past it return zero)
constexpr int BUF_RSRC_WORD3 = 0x00020000;

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));

// One A operand: the six code dwords of a fragment lane (128- and 64-bit LDS
// loads); its scale is byte E of the lane's scale word.
struct MxA {
    v4i_t lo;
    v2i_t hi;
};

template <int E>
__device__ __forceinline__ floatx4 mfma_mx(const MxA &a, int sa, const u32x4 &b, int sb, floatx4 c) {
    // A: fp6 e2m3 (format 2, six dwords read); B: fp4 e2m1 (format 4, four
    // dwords read)
    const v4i_t b0 = __builtin_bit_cast(v4i_t, b);
    const v4i_t h4 = __builtin_shufflevector(a.hi, a.hi, 0, 1, -1, -1);
    const v8i_t av = __builtin_shufflevector(a.lo, h4, 0, 1, 2, 3, 4, 5, -1, -1);
    const v8i_t bv = __builtin_shufflevector(b0, b0, 0, 1, 2, 3, -1, -1, -1, -1);
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 2, 4, E, sa, 0, sb);
}

// The scaled-MFMA product. A workgroup of 8 waves covers 64 tokens (4
// fragment blocks) x 512 rows (GLU: 256 output columns). Wave (wm, wn) =
// (wave / 4, wave % 4) takes token blocks 2 wm, 2 wm + 1 and 8 row groups
// (GLU: 4 gate groups and the same 4 groups of the up projection), so each A
// operand read from LDS feeds 8 products. A stage is 128 k: the A fragments
// of the 4 token blocks (4 x 6400 B: four fp6 terms and their E8M0 scales),
// the 32 row groups' fp4 codes (1 KiB a group) and their E8M0 bytes go to one
// of two LDS stage buffers by buffer_load_lds, every wave copying 1/8 of
// them, so each operand crosses the texture path once per workgroup (the two
// waves that share a row group read it from LDS). Every wave runs the same
// instruction stream, and the next stage's copies are spread between the
// MFMAs: a wave that issues a load while the texture unit's queue is full
// stalls, and a burst of loads at the top of the stage would hold back the
// MFMAs of every wave behind it. One barrier a stage. GLU: the epilogue
// writes act(gate) * up as f32 rows and/or as the MX fragments of the next
// product.
// (The body is a device function: the buffer-resource type exists on the
// device side only, and the host pass instantiates the kernel for its stub.)
template <int WM, bool GLU>
__device__ __forceinline__ void mx_gemm_body(const TileGemmParams &p) {
    constexpr int WAVES = 8, MB = 2 * WM, WN = 8, NT = MX_TERMS;
    constexpr int OG = GLU ? WN / 2 : WN;  // output row groups per wave
    constexpr int AQ = MX_BLOCK / 16;     // u32x4 per A block
    constexpr int PS = OG * 16 + 4;       // GLU patch row stride (floats)
    // one pipeline stage: A blocks [block][fragment], the workgroup's 32 row
    // groups' codes [wn][group][lane] and E8M0 bytes [wn][group][64 B]; two
    // stages as distinct LDS objects
    struct Stage {
        u32x4 A[MB * AQ];
        u32x4 B[4 * WN * 64];
        uint32_t S[4 * WN * 16];
    };
    __shared__ Stage st0, st1;
    const TileView &w = p.w;
    const TileOut to{p.out, p.ldo, p.n, w.rows, p.bias, p.accumulate, p.delta_b, p.delta_xa, p.delta_rank,
                     p.delta_stride};
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    int mt, nt;
    map_tile(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, mt, nt);
    const int64_t groups = (w.rows + 15) / 16;
    const int64_t G0 = (int64_t)nt * (OG * 4);  // the workgroup's first row group
    const int64_t g0 = G0 + wn * OG;
    const int64_t m16_0 = (int64_t)mt * MB, m16_n = (p.n + 15) / 16;
    const int64_t S = w.units_k;  // stages: one 128-column unit each

    // Copies through buffer resources (base and bounds in SGPRs, one per-lane
    // offset register, the rest a uniform offset), the same for every wave:
    // three of the 24 KiB A pieces (block q / 6, piece q % 6 for q = wave +
    // 8 j) and the 256 B of scale words of block wave / 2 (two waves write
    // the same words: an LDS copy writes a dword per lane); the codes of row
    // group `wave` of every wn (4 KiB) and the E8M0 bytes of groups 4 wave ..
    // 4 wave + 3 (of gate rows for even waves, up rows for odd ones, GLU).
    const int64_t a0 = m16_0 < m16_n ? m16_0 : m16_n - 1;
    const int64_t a_blocks = (m16_0 + MB < m16_n ? m16_0 + MB : m16_n) - a0;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void *)(p.xs + a0 * p.ldk * AQ), (short)0,
                                          (int)(a_blocks * p.ldk * MX_BLOCK), BUF_RSRC_WORD3);
    const int64_t gb = G0 < groups ? G0 : groups - 1;
    const int b_groups = (int)((gb + 4 * OG < groups ? gb + 4 * OG : groups) - gb);
    auto grp = [&](int q) {  // piece q = wn * 8 + i -> groups from the resource base
        const int64_t gi = G0 + (q / WN) * OG + (q % WN) % OG;
        return (int)((gi < groups ? gi : groups - 1) - gb);
    };
    const TileView &wb = (GLU && wave >= OG) ? p.w2 : w;      // the codes this wave copies
    const TileView &ws = (GLU && (wave & 1)) ? p.w2 : w;      // the scale bytes this wave copies
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(wb.mx + gb * S * 1024), (short)0, (int)(b_groups * S * 1024), BUF_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(ws.mx_scales + gb * S * 64), (short)0, (int)(b_groups * S * 64), BUF_RSRC_WORD3);
    static_assert(WN == WAVES, "each wave copies one row group of every wn");
    auto a_off = [&](int m) {  // bytes from the resource base to block m16_0 + m, stage 0
        const int64_t mb = m16_0 + m < m16_n ? m16_0 + m : m16_n - 1;
        return (int)((mb - a0) * p.ldk * MX_BLOCK);
    };
    // A pieces q = wave + 8 j (the last piece again where 8 does not divide
    // them: the same bytes to the same place), scale words of block
    // wave * MB / 8
    constexpr int NA = MB * 6, CA = (NA + WAVES - 1) / WAVES;
    int aoff[CA], boff[4];
#pragma unroll
    for (int j = 0; j < CA; j++) {
        const int q = wave + WAVES * j < NA ? wave + WAVES * j : NA - 1;
        aoff[j] = a_off(q / 6) + (q % 6) * 1024;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) boff[j] = grp(j * WN + wave) * (int)S * 1024;
    const int sblk = wave * MB / WAVES;
    const int soff = a_off(sblk) + 6144;
    const int sv = grp(4 * wave + (lane >> 4)) * (int)S * 64 + (lane & 15) * 4;  // per-lane scale source
    // copy j of a stage: 0..CA-1 A pieces, CA the A scale words, CA+1..CA+4
    // codes, CA+5 scale bytes
    auto copy = [&](int j, int64_t s, Stage &t) {
        if (j < CA) {
            const int q = wave + WAVES * j < NA ? wave + WAVES * j : NA - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)&t.A[(q / 6) * AQ + (q % 6) * 64], 16, lane * 16,
                                                     aoff[j] + (int)s * MX_BLOCK, 0, 0);
        } else if (j == CA) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)&t.A[sblk * AQ + 384], 4, lane * 4,
                                                     soff + (int)s * MX_BLOCK, 0, 0);
        } else if (j < CA + 5) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)&t.B[((j - CA - 1) * WN + wave) * 64], 16,
                                                     lane * 16, boff[j - CA - 1] + (int)s * 1024, 0, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)&t.S[wave * 64], 4, sv, (int)s * 64, 0, 0);
        }
    };
    constexpr int NCOPY = CA + 6;

    floatx4 acc[WM][WN];
#pragma unroll
    for (int m = 0; m < WM; m++)
#pragma unroll
        for (int i = 0; i < WN; i++) acc[m][i] = floatx4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int j = 0; j < NCOPY; j++) copy(j, 0, st0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    auto step = [&](int64_t s, const Stage &t, Stage &tn) {
        const int64_t sn = s + 1 < S ? s + 1 : s;
        const u32x4 *Aw = t.A + WM * wm * AQ;  // the wave's blocks
        auto read_a = [&](int m, int e) {
            MxA r;
            r.lo = __builtin_bit_cast(v4i_t, Aw[m * AQ + e * 64 + lane]);
            r.hi = ((const v2i_t *)(Aw + m * AQ + 256))[e * 64 + lane];
            return r;
        };
        MxA a[2];
        a[0] = read_a(0, 0);
        int sa[WM], sb[WN];
        u32x4 b[WN];
#pragma unroll
        for (int m = 0; m < WM; m++) sa[m] = (int)((const uint32_t *)(Aw + m * AQ + 384))[lane];
#pragma unroll
        for (int i = 0; i < WN; i++) {
            b[i] = t.B[(wn * WN + i) * 64 + lane];
            sb[i] = ((const uint8_t *)t.S)[(wn * WN + i) * 64 + lane];
        }
        __builtin_amdgcn_sched_barrier(0);
        // operand (block m, term e) feeds WN products; the next operand is
        // read while they issue, and one of the next stage's copies goes out
        // after every second product
        static_assert(NT == 4, "the operand sequence below is written out for four terms");
        auto block = [&](auto ec, int m, const MxA &at, int k) {
            constexpr int E = decltype(ec)::value;
#pragma unroll
            for (int i = 0; i < WN; i++) {
                acc[m][i] = mfma_mx<E>(at, sa[m], b[i], sb[i], acc[m][i]);
                const int l = k * (WN / 2) + i / 2;  // 0..31 over the stage
                if (i % 2 == 1 && l < NCOPY) copy(l, sn, tn);
            }
        };
        auto term = [&](auto ec) {
            constexpr int E = decltype(ec)::value;
#pragma unroll
            for (int m = 0; m < WM; m++) {
                const int k = E * WM + m;
                if (k > 0 && m == 0) __builtin_amdgcn_s_setprio(3 - E);
                if (k + 1 < NT * WM) a[(k + 1) & 1] = read_a((m + 1) % WM, m + 1 < WM ? E : E + 1);
                block(ec, m, a[k & 1], k);
            }
            // the order of the term's instructions (each priority change
            // ends a scheduling region)
#pragma unroll
            for (int m = 0; m < WM; m++) {
                const int k = E * WM + m;
                if (k + 1 < NT * WM) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
                for (int i = 0; i < WN; i += 2) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    if (k * (WN / 2) + i / 2 < NCOPY) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            }
        };
        // s_setprio (issue arbitration only): a wave issuing its products
        // outranks one still at the top of the stage, and the priority falls
        // by one a term, so of the two waves that share a SIMD the one behind
        // in the stage wins the MFMA pipe (with equal priorities the older
        // wave always does, and the other one issues the stage's tail alone,
        // at about half the rate)
        __builtin_amdgcn_s_setprio(3);
        term(std::integral_constant<int, 0>{});
        term(std::integral_constant<int, 1>{});
        term(std::integral_constant<int, 2>{});
        term(std::integral_constant<int, 3>{});
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    int64_t s = 0;
    for (; s + 1 < S; s += 2) {
        step(s, st0, st1);
        step(s + 1, st1, st0);
    }
    if (s < S) step(s, st0, st1);

    const int kq = lane >> 4;
    const int64_t mw = m16_0 + WM * wm;  // the wave's first token block
    if constexpr (!GLU) {
        int64_t tb[WM], rw[WN];
#pragma unroll
        for (int m = 0; m < WM; m++) tb[m] = (mw + m) * 16 + 4 * kq;
#pragma unroll
        for (int i = 0; i < WN; i++) rw[i] = (g0 + i) * 16 + (lane & 15);
        tile_store_block(to, tb, rw, acc);
    } else {
        // y = act(gate) * up (tensor.gatedActivation) for the wave's 64
        // columns (two E8M0 blocks of the next product's k) and 16 WM
        // tokens, through a per-wave LDS patch [16 WM tokens][64 columns] in
        // the idle stage buffers (the last stage ended with a barrier and no
        // copy is in flight); then slot l (token l % 16, columns 32 ((l / 16)
        // % 2).., block l / 32) is split by lane l % 64 into the next
        // product's fragments
        static_assert(OG * 16 == 64, "two 32-column blocks per wave");
        static_assert(WAVES / 2 * WM * 16 * PS * 4 <= (int)sizeof(Stage), "patches fit the stage buffers");
        float *pt = (float *)(wave < WAVES / 2 ? (void *)&st0 : (void *)&st1) + (wave % (WAVES / 2)) * (WM * 16 * PS);
        // the gates' activation first, the activation's switch outside the loops
        with_act(p.act, [&](auto ac) {
            constexpr int A = decltype(ac)::value;
#pragma unroll
            for (int m = 0; m < WM; m++)
#pragma unroll
                for (int i = 0; i < OG; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[m][i][r] = act_fused<A>(acc[m][i][r]);
        });
#pragma unroll
        for (int m = 0; m < WM; m++) {
#pragma unroll
            for (int i = 0; i < OG; i++) {
                const int64_t col = (g0 + i) * 16 + (lane & 15);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int64_t tok = (mw + m) * 16 + 4 * kq + r;
                    float y = __fmul_rn(acc[m][i][r], acc[m][i + OG][r]);
                    if (tok >= p.n || col >= w.rows) y = 0.f;
                    else if (p.out) p.out[tok * p.ldo + col] = y;
                    pt[(m * 16 + 4 * kq + r) * PS + i * 16 + (lane & 15)] = y;
                }
            }
        }
        if (p.xs_out) {
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
            for (int sl0 = 0; sl0 < WM * 32; sl0 += 64) {
                const int sl = sl0 + lane, mb = sl / 32, half = (sl / 16) % 2;
                const int64_t kb = (g0 * 16) / 32 + half;  // the next product's E8M0 block of these columns
                const int64_t mblk = mw + mb;
                float r[32];
#pragma unroll
                for (int j = 0; j < 32; j++) r[j] = pt[((mb < WM ? mb : 0) * 16 + (lane & 15)) * PS + half * 32 + j];
                if (sl < WM * 32 && mblk < m16_n && kb / 4 < p.ldk_out)
                    mx_write_slot(r, (uint8_t *)p.xs_out + (mblk * p.ldk_out + kb / 4) * MX_BLOCK,
                                  (lane & 15) + 16 * (int)(kb % 4));
            }
        }
    }
}

template <int WM, bool GLU>
__global__ __launch_bounds__(512) void mx_gemm_kernel(TileGemmParams p) {
    mx_gemm_body<WM, GLU>(p);
}

// ---------------------------------------------------------------------------

int64_t split_k_tiles(const TileView &w) {
    // a whole number of pipeline stages (4 k tiles; 2 for bf16 and FP8 weights)
    const int64_t tps = (w.tf == TF_BF16 || w.tf == TF_FP8 || w.tf == TF_Q8) ? 2 : 4;
    int64_t kt = w.units_k * (unit_k_of(w.tf) / 32);
    return (kt + tps - 1) / tps * tps;
}

bool tile_gemm_takes(const TileView &w, int64_t n) {
    if (!w.fast || n < 32) return false;
    return w.tf == TF_BF16 || w.tf == TF_MX4 || w.tf == TF_FP8 || w.tf == TF_INT4 || w.tf == TF_Q8;
}

bool launch_matmul_delta_split(const TileView &w, float *out, const float *x, int64_t n, const MatmulEpilogue &ep,
                               const float *da, int rank, float *xa, hipStream_t s, DevBuf *ws) {
    if (!ws || ep.exact || rank <= 0 || mx_gemm_takes(w, n) || !tile_gemm_takes(w, n)) return false;
    const int64_t ldk = split_k_tiles(w);
    const size_t xb = (split_bytes_ldk(n, ldk, 2) + 255) & ~(size_t)255;
    const size_t pb = tile_part_bytes(w, n, 2);
    const size_t qb = ((size_t)n * ldk * rank * 4 + 255) & ~(size_t)255;
    if (ws->borrowed && xb + pb + qb > ws->bytes) return false;
    uint8_t *xs = ws->get<uint8_t>(xb + pb + qb);
    float *xpart = (float *)(xs + xb + pb);
    SplitParams sp{(u32x4 *)xs, x, nullptr, nullptr, n, w.cols, w.cols, ldk, (n + 15) / 16};
    sp.da = da;
    sp.xa_part = xpart;
    sp.rank = rank;
    const int64_t total = sp.m16 * ldk * 64;
    hipLaunchKernelGGL(split_kernel<2>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, sp);
    DITCH_TRY_HIP(hipGetLastError());
    hipLaunchKernelGGL(xa_tiles_reduce_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, xa, xpart, n, ldk, rank);
    DITCH_TRY_HIP(hipGetLastError());
    MatmulEpilogue e2 = ep;
    e2.delta_xa = xa;
    launch_tile_gemm(w, out, w.rows, xs, ldk, n, 2, e2, s, pb ? (float *)(xs + xb) : nullptr);
    return true;
}

void launch_split(void *xs, const float *x, const int32_t *row_index, int64_t n, int64_t ldx, int64_t K,
                  int64_t kt_total, int xt, hipStream_t s) {
    SplitParams sp{(u32x4 *)xs, x, row_index, nullptr, n, ldx, K, kt_total, (n + 15) / 16};
    int64_t total = sp.m16 * kt_total * 64;
    dim3 grid((unsigned)((total + 255) / 256));
    if (xt == 3) hipLaunchKernelGGL(split_kernel<3>, grid, dim3(256), 0, s, sp);
    else hipLaunchKernelGGL(split_kernel<2>, grid, dim3(256), 0, s, sp);
    DITCH_TRY_HIP(hipGetLastError());
}

// out[t][r] = sum over the split-K parts (in part order) + delta + bias (+ out)
__global__ void ksplit_reduce_kernel(TileGemmParams p) {
    const int64_t rows = p.w.rows, total = p.n * rows;
    const TileOut to{p.out, p.ldo, p.n, rows, p.bias, p.accumulate, p.delta_b, p.delta_xa, p.delta_rank,
                     p.delta_stride};
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    if (rows % 4 == 0) {
        // four consecutive outputs of one token a thread: 16-byte loads of
        // every part, one division for the four
        for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 4 * j < total; j += step) {
            const int64_t i = 4 * j, t = i / rows, r = i % rows;
            float4 v = *(const float4 *)(p.part + i);
            for (int k = 1; k < p.ksplit; k++) {
                const float4 w = *(const float4 *)(p.part + (int64_t)k * total + i);
                v.x = __fadd_rn(v.x, w.x);
                v.y = __fadd_rn(v.y, w.y);
                v.z = __fadd_rn(v.z, w.z);
                v.w = __fadd_rn(v.w, w.w);
            }
            tile_store(to, t, r, v.x);
            tile_store(to, t, r + 1, v.y);
            tile_store(to, t, r + 2, v.z);
            tile_store(to, t, r + 3, v.w);
        }
        return;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        const int64_t t = i / rows, r = i % rows;
        float v = p.part[i];
        for (int k = 1; k < p.ksplit; k++) v = __fadd_rn(v, p.part[(int64_t)k * total + i]);
        tile_store(to, t, r, v);
    }
}

// Split-K parts for a plain product whose tiles would not give each of the
// GPU's 256 CUs a workgroup (and with at least 4 stages per part); a grid
// of one round takes no split (splitting it into two rounds measured 1-3 %
// slower on C3 FP8 and C4: the same stages, plus the partial sums' pass).
static int tile_ksplit(int64_t tiles, int64_t stages) {
    int ks = 1;
    while (ks < 8 && tiles * ks < 256 && stages / (2 * ks) >= 4) ks *= 2;
    // a last round of workgroups at most half full on a long K (C5's o and
    // dense down products, 896 tiles of 256-288 stages): two parts fill
    // whole rounds, and the partial sums' reduce costs less than the idle
    // half round
    if (ks == 1 && tiles > 256 && tiles % 256 != 0 && tiles % 256 <= 128 && stages >= 128) ks = 2;
    return ks;
}

// the tile a plain product launches: 64 tokens x (WGN x 64) rows
static constexpr int tile_wgn(int tf, int xt) { return tf == TF_BF16 || xt == 3 ? 4 : 8; }

static int tile_tps(int tf) {
    switch (tf) {
    case TF_BF16: return TileCfg<TF_BF16>::TPS;
    case TF_FP8: return TileCfg<TF_FP8>::TPS;
    case TF_MX4: return TileCfg<TF_MX4>::TPS;
    case TF_INT4: return TileCfg<TF_INT4>::TPS;
    default: return TileCfg<TF_Q8>::TPS;
    }
}

static int tile_ksplit_of(const TileView &w, int64_t n, int xt) {
    const int64_t tiles = (n + 63) / 64 * ((w.rows + 64 * tile_wgn(w.tf, xt) - 1) / (64 * tile_wgn(w.tf, xt)));
    return tile_ksplit(tiles, split_k_tiles(w) / tile_tps(w.tf));
}

size_t tile_part_bytes(const TileView &w, int64_t n, int xt) {
    if (wide_gemm_takes(w, n, xt, split_k_tiles(w))) return 0;  // no partial sums
    const int ks = tile_ksplit_of(w, n, xt);
    return ks > 1 ? (size_t)ks * n * w.rows * sizeof(float) : 0;
}

template <int TF, int XT, int WGM, int WGN, int WM, int WN, bool GLU>
static void launch_tile(TileGemmParams &p, hipStream_t s) {
    constexpr int BM = 16 * WM * WGM, BN = 16 * (GLU ? WN / 2 : WN) * WGN;
    p.tiles_m = (int)((p.n + BM - 1) / BM);
    p.tiles_n = (int)((p.w.rows + BN - 1) / BN);
    static_assert((BM == 64 || BM == 96) && (GLU || BN == 64 * tile_wgn(TF, XT)), "tile_ksplit_of sizes the same tile");
    // 96-token tiles only where the 64-token ones take no k split (the
    // partial-sum scratch is sized for those)
    p.ksplit = GLU || !p.part || BM != 64 ? 1 : tile_ksplit((int64_t)p.tiles_m * p.tiles_n, p.kt_total / TileCfg<TF>::TPS);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)p.ksplit);
    hipLaunchKernelGGL((tile_gemm_kernel<TF, XT, WGM, WGN, WM, WN, GLU>), grid, dim3(WGM * WGN * 64), 0, s, p);
    if (p.ksplit > 1) {
        DITCH_TRY_HIP(hipGetLastError());
        const int64_t total = p.n * p.w.rows;
        hipLaunchKernelGGL(ksplit_reduce_kernel, dim3((unsigned)std::min<int64_t>((total + 255) / 256, 4096)),
                           dim3(256), 0, s, p);
    }
}

template <int TF, int XT, bool GLU>
static void launch_tile_tf(TileGemmParams &p, hipStream_t s) {
    // waves side by side, each 64 tokens x 64 rows with 64 accumulator
    // registers: 8 waves (two per SIMD, a 64 x 512 tile) where the stage
    // buffers fit in LDS, 4 otherwise
    if constexpr (TF == TF_BF16 || XT == 3) {
        launch_tile<TF, XT, 1, 4, 4, 4, GLU>(p, s);
    } else if constexpr (TF == TF_FP8) {
        // FP8 (64-column stages): 96-token waves where the grid stays full.
        // The decode of a weight tile then feeds 12 MFMAs instead of 8, and
        // the decode's vector instructions do not overlap the MFMAs; the
        // tile is 1.5x the work, so it pays when the 96-token grid needs
        // fewer rounds of one workgroup a CU (counted 10 % cheaper per unit
        // of work) and the 64-token grid takes no k split.
        const int64_t bn = 16 * (GLU ? 2 : 4) * 8;
        const int64_t tn = (p.w.rows + bn - 1) / bn;
        const int64_t t64 = (p.n + 63) / 64 * tn, t96 = (p.n + 95) / 96 * tn;
        const bool split64 = !GLU && p.part && tile_ksplit(t64, p.kt_total / TileCfg<TF>::TPS) > 1;
        const double r64 = (double)((t64 + 255) / 256), r96 = 1.35 * (double)((t96 + 255) / 256);
        if (!split64 && r96 < r64) launch_tile<TF, XT, 1, 8, 6, 4, GLU>(p, s);
        else launch_tile<TF, XT, 1, 8, 4, 4, GLU>(p, s);
    } else {
        launch_tile<TF, XT, 1, 8, 4, 4, GLU>(p, s);
    }
}

template <bool GLU>
static void launch_tile_any(TileGemmParams &p, int xt, hipStream_t s) {
    if constexpr (GLU) {  // the forward's two activation terms only
        switch (p.w.tf) {
        case TF_BF16: launch_tile_tf<TF_BF16, 2, true>(p, s); break;
        case TF_MX4: launch_tile_tf<TF_MX4, 2, true>(p, s); break;
        case TF_FP8: launch_tile_tf<TF_FP8, 2, true>(p, s); break;
        case TF_INT4: launch_tile_tf<TF_INT4, 2, true>(p, s); break;
        case TF_Q8: launch_tile_tf<TF_Q8, 2, true>(p, s); break;
        default: throw Error{DITCH_UNSUPPORTED, "tiled GLU: tile format"};
        }
        DITCH_TRY_HIP(hipGetLastError());
    } else {
        const bool x3 = xt == 3;
        switch (p.w.tf) {
        case TF_BF16: x3 ? launch_tile_tf<TF_BF16, 3, false>(p, s) : launch_tile_tf<TF_BF16, 2, false>(p, s); break;
        case TF_MX4: x3 ? launch_tile_tf<TF_MX4, 3, false>(p, s) : launch_tile_tf<TF_MX4, 2, false>(p, s); break;
        case TF_FP8: x3 ? launch_tile_tf<TF_FP8, 3, false>(p, s) : launch_tile_tf<TF_FP8, 2, false>(p, s); break;
        case TF_INT4: x3 ? launch_tile_tf<TF_INT4, 3, false>(p, s) : launch_tile_tf<TF_INT4, 2, false>(p, s); break;
        case TF_Q8: x3 ? launch_tile_tf<TF_Q8, 3, false>(p, s) : launch_tile_tf<TF_Q8, 2, false>(p, s); break;
        default: throw Error{DITCH_UNSUPPORTED, "tiled GEMM: tile format"};
        }
        DITCH_TRY_HIP(hipGetLastError());
    }
}

void launch_tile_gemm(const TileView &w, float *out, int64_t ldo, const void *xs, int64_t ldk, int64_t n, int xt,
                      const MatmulEpilogue &ep, hipStream_t s, float *part) {
    if (wide_gemm_takes(w, n, xt, ldk)) {
        launch_wide_gemm(w, out, ldo, xs, ldk, n, ep, s);
        return;
    }
    TileGemmParams p{};
    p.part = ldo == w.rows ? part : nullptr;
    p.w = w;
    p.xs = (const u32x4 *)xs;
    p.kt_total = split_k_tiles(w);
    p.ldk = ldk;
    DITCH_CHECK(ldk >= p.kt_total, DITCH_INVALID_ARGUMENT, "tiled GEMM: activation fragments shorter than K");
    p.out = out;
    p.ldo = ldo;
    p.n = n;
    p.bias = ep.bias;
    p.accumulate = ep.accumulate;
    p.delta_b = ep.delta_b;
    p.delta_xa = ep.delta_xa;
    p.delta_rank = ep.delta_rank;
    p.delta_stride = ep.delta_rank;
    launch_tile_any<false>(p, xt, s);
}

// Routed experts on the tiled product: each segment's rows (gathered by
// row_index, or consecutive) are split into 16-token blocks of their own, a
// tile row covers up to 4 blocks of one segment, and the kernel reads the
// segment's weight, output rows and delta from the device segment table.
template <int TF, bool GLU>
static void launch_tile_grouped(TileGemmParams &p, hipStream_t s) {
    constexpr bool W4 = TF == TF_BF16;  // the stage buffers of the bf16 format need the 4-wave tile
    constexpr int WGN = W4 ? 4 : 8, BN = 16 * (GLU ? 2 : 4) * WGN;
    p.tiles_n = (int)((p.w.rows + BN - 1) / BN);
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n));
    hipLaunchKernelGGL((tile_gemm_kernel<TF, 2, 1, WGN, 4, 4, GLU, true>), grid, dim3(WGN * 64), 0, s, p);
}

template <bool GLU>
static void launch_tile_grouped_any(TileGemmParams &p, hipStream_t s) {
    switch (p.w.tf) {
    case TF_BF16: launch_tile_grouped<TF_BF16, GLU>(p, s); break;
    case TF_MX4: launch_tile_grouped<TF_MX4, GLU>(p, s); break;
    case TF_FP8: launch_tile_grouped<TF_FP8, GLU>(p, s); break;
    case TF_INT4: launch_tile_grouped<TF_INT4, GLU>(p, s); break;
    case TF_Q8: launch_tile_grouped<TF_Q8, GLU>(p, s); break;
    default: throw Error{DITCH_UNSUPPORTED, "grouped tiled GEMM: tile format"};
    }
    DITCH_TRY_HIP(hipGetLastError());
}

bool tile_grouped_takes(const GroupSeg *h_segs, unsigned nseg, int64_t max_cnt) {
    if (nseg == 0 || max_cnt <= 16) return false;
    for (unsigned i = 0; i < nseg; i++)
        if (!tile_gemm_takes(h_segs[i].w, 128) || h_segs[i].w.tf != h_segs[0].w.tf ||
            h_segs[i].w.units_k != h_segs[0].w.units_k)
            return false;
    return true;
}

// The row map and tile table of a grouped call (to `meta`), and unless the
// caller brings them (xs_pre), the split activation fragments (to `ws`).
struct GroupedPlan {
    const u32x4 *xs;
    const int32_t *dm;
    int64_t blocks, ndesc, kt;
};

static GroupedPlan grouped_plan(const GroupSeg *h_segs, unsigned nseg, const float *x, int64_t ldx,
                                const int32_t *row_index, const void *xs_pre, DevBuf *ws, DevBuf *meta, hipStream_t s) {
    const TileView &w0 = h_segs[0].w;
    const int64_t kt = split_k_tiles(w0);
    // blocks of each segment, the padded row map and the tile descriptors
    std::vector<int32_t> base(nseg);
    int64_t blocks = 0, ndesc = 0;
    for (unsigned z = 0; z < nseg; z++) {
        base[z] = (int32_t)blocks;
        const int64_t nb = (h_segs[z].cnt + 15) / 16;
        blocks += nb;
        ndesc += (nb + 3) / 4;
    }
    if (blocks == 0) return GroupedPlan{nullptr, nullptr, 0, 0, kt};
    std::vector<int32_t> hm((size_t)(blocks * 16 + ndesc * 4));
    int32_t *prow = hm.data(), *desc = hm.data() + blocks * 16;
    int64_t d = 0;
    for (unsigned z = 0; z < nseg; z++) {
        const int64_t nb = (h_segs[z].cnt + 15) / 16;
        for (int64_t i = 0; i < nb * 16; i++)
            prow[base[z] * 16 + i] = i < h_segs[z].cnt ? (int32_t)(h_segs[z].off + i) : -1;
        for (int64_t j = 0; j < nb; j += 4) {
            desc[4 * d] = (int32_t)z;
            desc[4 * d + 1] = (int32_t)(base[z] + j);
            desc[4 * d + 2] = (int32_t)(base[z] + nb);
            desc[4 * d + 3] = (int32_t)(j * 16);
            d++;
        }
    }
    int32_t *dm = meta->get<int32_t>(hm.size());
    DITCH_TRY_HIP(hipMemcpyAsync(dm, hm.data(), hm.size() * 4, hipMemcpyHostToDevice, s));
    if (xs_pre) return GroupedPlan{(const u32x4 *)xs_pre, dm, blocks, ndesc, kt};
    void *xs = ws->get<uint8_t>(split_bytes_ldk(blocks * 16, kt, 2));
    SplitParams sp{(u32x4 *)xs, x, row_index, dm, blocks * 16, ldx, w0.cols, kt, blocks};
    const int64_t total = blocks * kt * 64;
    hipLaunchKernelGGL(split_kernel<2>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, sp);
    DITCH_TRY_HIP(hipGetLastError());
    return GroupedPlan{(const u32x4 *)xs, dm, blocks, ndesc, kt};
}

int64_t grouped_blocks(const GroupSeg *h_segs, unsigned nseg) {
    int64_t blocks = 0;
    for (unsigned z = 0; z < nseg; z++) blocks += (h_segs[z].cnt + 15) / 16;
    return blocks;
}

void launch_tile_gemm_grouped(const GroupSeg *d_segs, const GroupSeg *h_segs, unsigned nseg, float *out, int64_t ldo,
                              const float *x, int64_t ldx, const int32_t *row_index, const float *delta_xa,
                              int delta_stride, DevBuf *ws, DevBuf *meta, hipStream_t s, const void *xs_pre) {
    const GroupedPlan g = grouped_plan(h_segs, nseg, x, ldx, row_index, xs_pre, ws, meta, s);
    if (g.blocks == 0) return;
    TileGemmParams p{};
    p.w = h_segs[0].w;
    p.xs = g.xs;
    p.kt_total = g.kt;
    p.ldk = g.kt;
    p.out = out;
    p.ldo = ldo;
    p.delta_xa = delta_xa;
    p.delta_stride = delta_stride;
    p.gsegs = d_segs;
    p.gdesc = g.dm + g.blocks * 16;
    p.tiles_m = (int)g.ndesc;
    launch_tile_grouped_any<false>(p, s);
}

void launch_tile_glu_grouped(const GroupSeg *d_gate, const GroupSeg *d_up, const GroupSeg *h_gate,
                             const GroupSeg *h_up, unsigned nseg, uint32_t act, float *out, void *xs_out,
                             int64_t ldk_out, const float *x, int64_t ldx, const int32_t *row_index, DevBuf *ws,
                             DevBuf *meta, hipStream_t s, int64_t n_tok) {
    DITCH_CHECK(tile_glu_takes(h_gate[0].w, h_up[0].w, 128), DITCH_INVALID_ARGUMENT,
                "grouped GLU: gate and up must share format and shape");
    DITCH_CHECK(!xs_out || ldk_out * 32 >= h_gate[0].w.rows, DITCH_INVALID_ARGUMENT,
                "grouped GLU: output fragments too short");
    // the tokens' terms once, token-major, for the tiles to gather
    const bool tok = n_tok > 0 && h_gate[0].w.tf != TF_Q8;
    const int64_t kt0 = split_k_tiles(h_gate[0].w);
    void *xt = nullptr;
    if (tok) {
        xt = ws->get<uint8_t>((size_t)(n_tok * kt0 * 2 * 64));
        const int64_t total = n_tok * kt0 * 4;
        hipLaunchKernelGGL(split_tok_kernel<2>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, (u32x4 *)xt, x,
                           n_tok, ldx, h_gate[0].w.cols, kt0);
        DITCH_TRY_HIP(hipGetLastError());
    }
    const GroupedPlan g = grouped_plan(h_gate, nseg, x, ldx, row_index, xt, ws, meta, s);
    if (g.blocks == 0) return;
    TileGemmParams p{};
    if (tok) {
        p.a_tok = (const u32x4 *)xt;
        p.a_prow = g.dm;
        p.a_map = row_index;
        p.a_tok_stride = kt0 * 2 * 64;
    }
    p.w = h_gate[0].w;
    p.w2 = h_up[0].w;
    p.act = act;
    p.xs = g.xs;
    p.kt_total = g.kt;
    p.ldk = g.kt;
    p.xs_out = (u32x4 *)xs_out;
    p.ldk_out = ldk_out;
    p.out = out;
    p.ldo = h_gate[0].w.rows;
    p.gsegs = d_gate;
    p.gsegs2 = d_up;
    p.gdesc = g.dm + g.blocks * 16;
    p.tiles_m = (int)g.ndesc;
    launch_tile_grouped_any<true>(p, s);
}

// Grouped products whose row map and tile table a device kernel wrote
// (GroupedDevPlan): the grid covers plan.max_desc tile rows and the rows past
// *plan.count exit at once; no host copy of the counts.
void launch_tile_glu_grouped_dev(const GroupSeg *d_gate, const GroupSeg *d_up, const TileView &gate0,
                                 const TileView &up0, uint32_t act, float *out, void *xs_out, int64_t ldk_out,
                                 const float *x, int64_t ldx, const int32_t *row_index, const GroupedDevPlan &plan,
                                 DevBuf *ws, hipStream_t s, const GroupedDeltaXa *dx, int64_t n_tok) {
    DITCH_CHECK(tile_glu_takes(gate0, up0, 128), DITCH_INVALID_ARGUMENT, "grouped GLU: gate and up must share format and shape");
    DITCH_CHECK(!xs_out || ldk_out * 32 >= gate0.rows, DITCH_INVALID_ARGUMENT, "grouped GLU: output fragments too short");
    const int64_t kt = split_k_tiles(gate0);
    TileGemmParams p{};
    void *xs = nullptr;
    if (n_tok > 0 && gate0.tf != TF_Q8) {
        // the tokens' terms once, token-major; the tiles gather each pair's
        // pieces (x: the n_tok token rows, row_index: pair -> token)
        xs = ws->get<uint8_t>((size_t)(n_tok * kt * 2 * 64));
        const int64_t total = n_tok * kt * 4;
        hipLaunchKernelGGL(split_tok_kernel<2>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, (u32x4 *)xs, x,
                           n_tok, ldx, gate0.cols, kt);
        DITCH_TRY_HIP(hipGetLastError());
        p.a_tok = (const u32x4 *)xs;
        p.a_prow = plan.prow;
        p.a_map = row_index;
        p.a_tok_stride = kt * 2 * 64;
    } else {
        xs = ws->get<uint8_t>(split_bytes_ldk(plan.max_blocks * 16, kt, 2));
        SplitParams sp{(u32x4 *)xs, x, row_index, plan.prow, plan.max_blocks * 16, ldx, gate0.cols, kt, plan.max_blocks};
        const int64_t total = plan.max_blocks * kt * 64;
        hipLaunchKernelGGL(split_kernel<2>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, sp);
        DITCH_TRY_HIP(hipGetLastError());
    }
    p.w = gate0;
    p.w2 = up0;
    p.act = act;
    p.xs = (const u32x4 *)xs;
    p.kt_total = kt;
    p.ldk = kt;
    p.xs_out = (u32x4 *)xs_out;
    p.ldk_out = ldk_out;
    p.out = out;
    p.ldo = gate0.rows;
    p.gsegs = d_gate;
    p.gsegs2 = d_up;
    p.gdesc = plan.desc;
    p.gcount = plan.count;
    p.tiles_m = (int)plan.max_desc;
    if (dx) {
        // the launch's tile columns times its waves: the parts of each pair
        const int wgn = gate0.tf == TF_BF16 ? 4 : 8, bn = 16 * 2 * wgn;  // the grouped GLU's tile columns
        p.xa_a = dx->a;
        p.xa_segs = dx->segs;
        p.xa_stride = dx->max_rank;
        p.xa_parts = (int)((gate0.rows + bn - 1) / bn) * wgn;
        p.xa_pairs = dx->pairs;
        p.xa_part = (float *)dx->ws->get<float>((size_t)dx->pairs * p.xa_parts * dx->max_rank);
    }
    launch_tile_grouped_any<true>(p, s);
    if (dx) {
        const int64_t total = dx->pairs * dx->max_rank;
        hipLaunchKernelGGL(xa_reduce_kernel, dim3((unsigned)std::min<int64_t>((total + 255) / 256, 4096)), dim3(256),
                           0, s, dx->xa, p.xa_part, dx->pairs, p.xa_parts, dx->max_rank);
        DITCH_TRY_HIP(hipGetLastError());
    }
}

void launch_tile_gemm_grouped_dev(const GroupSeg *d_segs, const TileView &w0, float *out, int64_t ldo,
                                  const void *xs, const GroupedDevPlan &plan, hipStream_t s, const float *delta_xa,
                                  int delta_stride) {
    TileGemmParams p{};
    p.w = w0;
    p.delta_xa = delta_xa;
    p.delta_stride = delta_stride;
    p.xs = (const u32x4 *)xs;
    p.kt_total = split_k_tiles(w0);
    p.ldk = p.kt_total;
    p.out = out;
    p.ldo = ldo;
    p.gsegs = d_segs;
    p.gdesc = plan.desc;
    p.gcount = plan.count;
    p.tiles_m = (int)plan.max_desc;
    launch_tile_grouped_any<false>(p, s);
}

bool tile_glu_takes(const TileView &g, const TileView &u, int64_t n) {
    // the fused pair has no split-K: it keeps to batches of 128 tokens and more
    if (n < 128 || !tile_gemm_takes(g, n) || !tile_gemm_takes(u, n)) return false;
    return g.tf == u.tf && g.rows == u.rows && g.cols == u.cols && g.units_k == u.units_k &&
           g.scale_type == u.scale_type && g.block_rows == u.block_rows && g.block_cols == u.block_cols &&
           g.row_shard == u.row_shard && g.group == u.group && g.side_cols == u.side_cols;
}

void launch_tile_glu(const TileView &gate, const TileView &up, uint32_t act, float *out, void *xs_out,
                     int64_t ldk_out, const void *xs, int64_t ldk, int64_t n, hipStream_t s) {
    TileGemmParams p{};
    p.w = gate;
    p.w2 = up;
    p.act = act;
    p.xs = (const u32x4 *)xs;
    p.kt_total = split_k_tiles(gate);
    p.ldk = ldk;
    DITCH_CHECK(ldk >= p.kt_total, DITCH_INVALID_ARGUMENT, "tiled GLU: activation fragments shorter than K");
    DITCH_CHECK(!xs_out || ldk_out * 32 >= gate.rows, DITCH_INVALID_ARGUMENT, "tiled GLU: output fragments too short");
    p.xs_out = (u32x4 *)xs_out;
    p.ldk_out = ldk_out;
    p.out = out;
    p.ldo = gate.rows;
    p.n = n;
    launch_tile_any<true>(p, 2, s);
}

// ---------------------------------------------------------------------------
// MXFP4 on the scaled MFMA: host side

bool mx_gemm_takes(const TileView &w, int64_t n) { return w.tf == TF_MX4 && w.fast && w.mx && n >= 128; }

size_t mx_frag_bytes(int64_t n, int64_t ldst) { return (size_t)((n + 15) / 16) * ldst * MX_BLOCK; }

void launch_split_mx(void *xm, const float *x, const int32_t *row_index, int64_t n, int64_t ldx, int64_t K,
                     int64_t ldst, hipStream_t s) {
    DITCH_CHECK(ldst * 128 >= K, DITCH_INVALID_ARGUMENT, "MX fragments shorter than K");
    MxSplitParams sp{(u32x4 *)xm, x, row_index, n, ldx, K, ldst, (n + 15) / 16};
    const int64_t total = sp.m16 * ldst * 64;
    hipLaunchKernelGGL(split_mx_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, sp);
    DITCH_TRY_HIP(hipGetLastError());
}

template <bool GLU>
static void launch_mx(TileGemmParams &p, hipStream_t s) {
    // 96 x BN tiles, or 64 x BN ones when the larger tiles would leave CUs
    // idle (the k and v projections: 172 tiles against 256 CUs)
    constexpr int BN = GLU ? 256 : 512;
    p.tiles_n = (int)((p.w.rows + BN - 1) / BN);
    if ((p.n + 95) / 96 * p.tiles_n >= 256) {
        p.tiles_m = (int)((p.n + 95) / 96);
        hipLaunchKernelGGL((mx_gemm_kernel<3, GLU>), dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(512), 0, s, p);
    } else {
        p.tiles_m = (int)((p.n + 63) / 64);
        hipLaunchKernelGGL((mx_gemm_kernel<2, GLU>), dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(512), 0, s, p);
    }
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_mx_gemm(const TileView &w, float *out, int64_t ldo, const void *xm, int64_t ldst, int64_t n,
                    const MatmulEpilogue &ep, hipStream_t s) {
    DITCH_CHECK(mx_gemm_takes(w, n), DITCH_INVALID_ARGUMENT, "scaled-MFMA product: not an MXFP4 tensor it takes");
    DITCH_CHECK(ldst >= w.units_k, DITCH_INVALID_ARGUMENT, "MX fragments shorter than K");
    TileGemmParams p{};
    p.w = w;
    p.xs = (const u32x4 *)xm;
    p.kt_total = w.units_k;
    p.ldk = ldst;
    p.out = out;
    p.ldo = ldo;
    p.n = n;
    p.bias = ep.bias;
    p.accumulate = ep.accumulate;
    p.delta_b = ep.delta_b;
    p.delta_xa = ep.delta_xa;
    p.delta_rank = ep.delta_rank;
    p.delta_stride = ep.delta_rank;
    launch_mx<false>(p, s);
}

bool mx_glu_takes(const TileView &g, const TileView &u, int64_t n) {
    return mx_gemm_takes(g, n) && mx_gemm_takes(u, n) && g.rows == u.rows && g.cols == u.cols && g.rows % 32 == 0;
}

void launch_mx_glu(const TileView &gate, const TileView &up, uint32_t act, float *out, void *xm_out, int64_t ldst_out,
                   const void *xm, int64_t ldst, int64_t n, hipStream_t s) {
    DITCH_CHECK(mx_glu_takes(gate, up, n), DITCH_INVALID_ARGUMENT, "scaled-MFMA gate/up: shapes or formats it does not take");
    DITCH_CHECK(ldst >= gate.units_k, DITCH_INVALID_ARGUMENT, "MX fragments shorter than K");
    DITCH_CHECK(!xm_out || ldst_out * 128 >= gate.rows, DITCH_INVALID_ARGUMENT, "MX output fragments shorter than the rows");
    TileGemmParams p{};
    p.w = gate;
    p.w2 = up;
    p.act = act;
    p.xs = (const u32x4 *)xm;
    p.kt_total = gate.units_k;
    p.ldk = ldst;
    p.xs_out = (u32x4 *)xm_out;
    p.ldk_out = ldst_out;
    p.out = out;
    p.ldo = gate.rows;
    p.n = n;
    launch_mx<true>(p, s);
}

}  // namespace ditch
