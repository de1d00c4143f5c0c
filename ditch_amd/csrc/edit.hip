// edit.hip — the rank-k weight edit in every row-normalisation mode, on the
// device (abliterate.computeDelta, abliterate.zig:223-350): `none`
// (A = V^T W, B = -lambda V), `pre` (row norms, A over the normalised rows,
// B scaled by the norms), `full` (the renormalised edit's delta approximated
// by a rank-r randomised SVD of the implicit operator D = diag(c) W +
// sum_l d_l a_l^T, abliterate.zig:282-349, 353-394, 473-538) and the optional
// input-side ablation (abliterate.zig:234-261).
//
// Every pass over W runs on the resident (re-tiled, still quantised) weight:
// row norms, W^T y for up to 16 vectors at a time, and the exact three-term
// product W x for the q vectors of the SVD. The rest is q or k vectors of
// the matrix's width: one workgroup orthonormalises them, one runs the
// Jacobi eigen-solver of the q x q Gram matrix.
#include <math.h>
#include <string.h>

#include <vector>

#include "internal.h"
#include "zig_random.h"

namespace ditch {

// ---------------------------------------------------------------------------
// helpers (blockDim.x a multiple of 64)

__device__ __forceinline__ double ed_wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ double ed_block_sum(double v, double *sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = ed_wave_sum(v);
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < nw; w++) r += sh[w];
    return r;
}

// an f32 dot product accumulated in f64 and rounded once
__device__ float ed_dot(const float *a, const float *b, int64_t n, double *sh) {
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) acc += (double)a[i] * (double)b[i];
    return (float)ed_block_sum(acc, sh);
}

// ---------------------------------------------------------------------------
// kernels

// vn[j][i] = v[j][i] / n_i (0 where n_i = 0)              (abliterate.zig:290-292)
__global__ void edit_vn_kernel(float *vn, const float *v, const float *norms, int64_t k, int64_t rows) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < k * rows; t += (int64_t)gridDim.x * blockDim.x) {
        const float n = norms[t % rows];
        vn[t] = n > 0.f ? __fdiv_rn(v[t], n) : 0.f;
    }
}

// b[i][j] = -lambda v[j][i] (x n_i for `pre`)        (abliterate.zig:275-278, 298-303)
__global__ void edit_b_kernel(float *b, const float *v, const float *norms, int64_t k, int64_t rows, float weight,
                              int64_t ldb) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < k * rows; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = t / k, j = t % k;
        float x = __fmul_rn(-weight, v[j * rows + i]);
        if (norms) x = __fmul_rn(x, norms[i]);
        b[i * ldb + j] = x;
    }
}

// out[j][l] = dot(p_l, x_j) for p [np][len], x [nx][len]: one block per pair
__global__ __launch_bounds__(256) void edit_dots_kernel(float *out, const float *p, const float *x, int64_t np,
                                                        int64_t len) {
    __shared__ double sh[8];
    const int64_t j = blockIdx.y, l = blockIdx.x;
    const float d = ed_dot(p + l * len, x + j * len, len, sh);
    if (threadIdx.x == 0) out[j * np + l] = d;
}

// The full edit's per-row factors (abliterate.zig:318-330): with
// b_ij = -lambda v_ji, s_i^2 = 1 + sum_j (2 b_ij (W_i.a_j)/n_i + sum_l b_ij b_il
// G_jl), c_i = 1/s_i - 1, d_ji = n_i b_ij / s_i.
__global__ void edit_cd_kernel(float *c, float *d, const float *v, const float *norms, const float *wa,
                               const float *gram, int64_t k, int64_t rows, float weight) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < rows; i += (int64_t)gridDim.x * blockDim.x) {
        const float n = norms[i];
        float s2 = 1.0f;
        for (int64_t j = 0; j < k; j++) {
            const float bij = __fmul_rn(-weight, v[j * rows + i]);
            const float wn_dot_a = n > 0.f ? __fdiv_rn(wa[j * rows + i], n) : 0.f;
            s2 = __fadd_rn(s2, __fmul_rn(__fmul_rn(2.0f, bij), wn_dot_a));
            for (int64_t l = 0; l < k; l++)
                s2 = __fadd_rn(s2, __fmul_rn(__fmul_rn(bij, __fmul_rn(-weight, v[l * rows + i])), gram[j * k + l]));
        }
        const float s = __fsqrt_rn(fmaxf(s2, 1e-12f));
        c[i] = __fsub_rn(__fdiv_rn(1.0f, s), 1.0f);
        for (int64_t j = 0; j < k; j++)
            d[j * rows + i] = __fdiv_rn(__fmul_rn(n, __fmul_rn(-weight, v[j * rows + i])), s);
    }
}

// D X: out[j][i] = (W x_j)_i c_i + sum_l dot(a_l, x_j) d_li (abliterate.zig:363-376)
__global__ void edit_apply_kernel(float *out, const float *c, const float *d, const float *ax, int64_t q, int64_t k,
                                  int64_t rows) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < q * rows; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t j = t / rows, i = t % rows;
        float o = __fmul_rn(out[t], c[i]);
        for (int64_t l = 0; l < k; l++) o = __fadd_rn(o, __fmul_rn(ax[j * k + l], d[l * rows + i]));
        out[t] = o;
    }
}

// cy[j][i] = c_i y_j[i]                                   (abliterate.zig:383-386)
__global__ void edit_scale_rows_kernel(float *cy, const float *y, const float *c, int64_t q, int64_t rows) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < q * rows; t += (int64_t)gridDim.x * blockDim.x)
        cy[t] = __fmul_rn(c[t % rows], y[t]);
}

// D^T Y: out[j][col] += sum_l dot(d_l, y_j) a_l[col]      (abliterate.zig:387-392)
__global__ void edit_applyT_kernel(float *out, const float *a, const float *dy, int64_t q, int64_t k, int64_t cols) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < q * cols; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t j = t / cols, col = t % cols;
        float o = out[t];
        for (int64_t l = 0; l < k; l++) o = __fadd_rn(o, __fmul_rn(dy[j * k + l], a[l * cols + col]));
        out[t] = o;
    }
}

// abliterate.orthonormalize (abliterate.zig:409-423): modified Gram-Schmidt,
// two passes, every row normalised (zeroed at norm <= 1e-20). One block.
__global__ __launch_bounds__(1024) void edit_orthonormalize_kernel(float *vecs, int64_t q, int64_t n) {
    __shared__ double sh[16];
    for (int64_t i = 0; i < q; i++) {
        float *vi = vecs + i * n;
        for (int pass = 0; pass < 2; pass++)
            for (int64_t j = 0; j < i; j++) {
                const float *vj = vecs + j * n;
                const float p = ed_dot(vi, vj, n, sh);
                for (int64_t t = threadIdx.x; t < n; t += blockDim.x) vi[t] = __fadd_rn(vi[t], __fmul_rn(-p, vj[t]));
                __syncthreads();
            }
        const float nrm = __fsqrt_rn(ed_dot(vi, vi, n, sh));
        const float s = nrm > 1e-20f ? __fdiv_rn(1.0f, nrm) : 0.f;
        for (int64_t t = threadIdx.x; t < n; t += blockDim.x) vi[t] = nrm > 1e-20f ? __fmul_rn(vi[t], s) : 0.f;
        __syncthreads();
    }
}

// The same Gram-Schmidt with the vector being orthonormalised held in
// registers (EPT elements a thread, element m * 1024 + tid): each step reads
// only v_j, whose successor is loaded before the step's reduction, and each
// reduction takes one barrier that waits on LDS alone (the wave sums
// alternate between two LDS slots, so a fast wave cannot overwrite sums a
// slow wave is still reading). Per element the arithmetic is the kernel
// above's: f64 dot rounded to f32, then v_i + (-p) v_j rounded twice.
template <int CTRL>
__device__ __forceinline__ double ed_dpp(double v) {
    const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xf, 0xf, false);
    return __hiloint2double(hi, lo);
}

// the sum of a wave's 64 values, the same in every lane: DPP butterflies
// within each row of 16 lanes (quad swaps, half-row and row mirrors), then
// the four row sums read as scalars
__device__ __forceinline__ double ed_wave_total(double v) {
    v += ed_dpp<0xB1>(v);
    v += ed_dpp<0x4E>(v);
    v += ed_dpp<0x141>(v);
    v += ed_dpp<0x140>(v);
    double r = 0.0;
#pragma unroll
    for (int row = 0; row < 4; row++)
        r += __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 16 * row),
                              __builtin_amdgcn_readlane(__double2loint(v), 16 * row));
    return r;
}

__device__ __forceinline__ void ed_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int EPT>
__global__ __launch_bounds__(1024) void edit_orth_reg_kernel(float *vecs, int64_t q, int64_t n) {
    __shared__ double sh[2][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int slot = 0;
    auto block_dot = [&](const float *a, const float *b) -> float {
        double acc = 0.0;
#pragma unroll
        for (int m = 0; m < EPT; m++) acc += (double)a[m] * (double)b[m];
        acc = ed_wave_total(acc);
        if (lane == 0) sh[slot][wave] = acc;
        ed_lds_barrier();
        double r = 0.0;
#pragma unroll
        for (int w = 0; w < 16; w++) r += sh[slot][w];
        slot ^= 1;
        return (float)r;
    };
    auto load = [&](float *dst, const float *src) {
#pragma unroll
        for (int m = 0; m < EPT; m++) {
            const int64_t t = (int64_t)m * 1024 + tid;
            dst[m] = t < n ? src[t] : 0.f;
        }
    };
    for (int64_t i = 0; i < q; i++) {
        float *vi_g = vecs + i * n;
        float vi[EPT], vj[EPT], vn[EPT];
        load(vi, vi_g);
        if (i > 0) load(vj, vecs);
        for (int pass = 0; pass < 2; pass++)
            for (int64_t j = 0; j < i; j++) {
                const int64_t nj = j + 1 < i ? j + 1 : (pass == 0 ? 0 : -1);
                if (nj >= 0) load(vn, vecs + nj * n);
                const float p = block_dot(vi, vj);
#pragma unroll
                for (int m = 0; m < EPT; m++) vi[m] = __fadd_rn(vi[m], __fmul_rn(-p, vj[m]));
                if (nj >= 0) {
#pragma unroll
                    for (int m = 0; m < EPT; m++) vj[m] = vn[m];
                }
            }
        const float nrm = __fsqrt_rn(block_dot(vi, vi));
        const float s = nrm > 1e-20f ? __fdiv_rn(1.0f, nrm) : 0.f;
#pragma unroll
        for (int m = 0; m < EPT; m++) {
            const int64_t t = (int64_t)m * 1024 + tid;
            if (t < n) vi_g[t] = nrm > 1e-20f ? __fmul_rn(vi[m], s) : 0.f;
        }
        __syncthreads();  // v_i (global) is read by the later vectors
    }
}

// SVD widths up to ED_LDS_Q keep the Jacobi's two q x q matrices in LDS;
// wider ones work on them in place in global memory.
constexpr int ED_LDS_Q = 128;

// abliterate.jacobiEigen (abliterate.zig:427-469): cyclic Jacobi in f32 on the
// q x q matrix m (in place: its diagonal ends as the eigenvalues),
// eigenvectors in the columns of vecs. One block; the rotation's updates
// are spread over the block's threads in the reference's order.
template <bool LDS>
__global__ __launch_bounds__(1024) void edit_jacobi_kernel(float *m_g, float *vecs_g, int n) {
    extern __shared__ float ed_dyn[];
    __shared__ int stop;
    float *m = LDS ? ed_dyn : m_g, *vecs = LDS ? ed_dyn + n * n : vecs_g;
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int t = tid; t < n * n; t += nt) {
        if (LDS) m[t] = m_g[t];
        vecs[t] = (t / n == t % n) ? 1.f : 0.f;
    }
    __syncthreads();
    for (int sweep = 0; sweep < 50; sweep++) {
        if (tid == 0) {
            double off = 0;
            for (int i = 0; i < n; i++)
                for (int j = 0; j < n; j++)
                    if (i != j) off += (double)m[i * n + j] * (double)m[i * n + j];
            stop = off < 1e-18;
        }
        __syncthreads();
        if (stop) break;
        for (int p = 0; p < n; p++)
            for (int q = p + 1; q < n; q++) {
                const float apq = m[p * n + q];
                if (fabsf(apq) < 1e-20f) continue;
                const float app = m[p * n + p], aqq = m[q * n + q];
                const float theta = __fdiv_rn(__fsub_rn(aqq, app), __fmul_rn(2.0f, apq));
                const float sg = theta > 0.f ? 1.f : theta < 0.f ? -1.f : 0.f;
                const float t = __fdiv_rn(sg, __fadd_rn(fabsf(theta), __fsqrt_rn(__fadd_rn(__fmul_rn(theta, theta), 1.0f))));
                const float tf = theta == 0.f ? 1.0f : t;
                const float cs = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fmul_rn(tf, tf), 1.0f)));
                const float sn = __fmul_rn(tf, cs);
                __syncthreads();  // every thread has read the pivot before it changes
                for (int k = tid; k < n; k += nt) {
                    const float akp = m[k * n + p], akq = m[k * n + q];
                    m[k * n + p] = __fsub_rn(__fmul_rn(cs, akp), __fmul_rn(sn, akq));
                    m[k * n + q] = __fadd_rn(__fmul_rn(sn, akp), __fmul_rn(cs, akq));
                    const float vkp = vecs[k * n + p], vkq = vecs[k * n + q];
                    vecs[k * n + p] = __fsub_rn(__fmul_rn(cs, vkp), __fmul_rn(sn, vkq));
                    vecs[k * n + q] = __fadd_rn(__fmul_rn(sn, vkp), __fmul_rn(cs, vkq));
                }
                __syncthreads();
                for (int k = tid; k < n; k += nt) {
                    const float apk = m[p * n + k], aqk = m[q * n + k];
                    m[p * n + k] = __fsub_rn(__fmul_rn(cs, apk), __fmul_rn(sn, aqk));
                    m[q * n + k] = __fadd_rn(__fmul_rn(sn, apk), __fmul_rn(cs, aqk));
                }
                __syncthreads();
            }
    }
    __syncthreads();
    if (LDS)
        for (int t = tid; t < n * n; t += nt) {
            m_g[t] = m[t];
            vecs_g[t] = vecs[t];
        }
}

// The SVD's factors and the LoRA pair (abliterate.zig:514-547): eigenvalues
// sorted descending (a stable sort), s_t = sqrt(max(lambda, 0)), u_t = Q e,
// v_t = B^T e / s_t; a[t] = sqrt(s_t) v_t, b[i][t] = u_t[i] sqrt(s_t). One
// block per output component t (rank of them).
__global__ __launch_bounds__(256) void edit_svd_out_kernel(float *a, float *b, const float *evals_m,
                                                           const float *evecs, const float *qy, const float *bt,
                                                           int q, int64_t rows, int64_t cols, int64_t rank,
                                                           int64_t ldb, int64_t b_off) {
    extern __shared__ int order[];  // q entries
    const int t = blockIdx.x;
    if (threadIdx.x == 0) {
        for (int i = 0; i < q; i++) order[i] = i;
        for (int i = 1; i < q; i++) {
            const int o = order[i];
            int j = i;
            while (j > 0 && evals_m[order[j - 1] * q + order[j - 1]] < evals_m[o * q + o]) {
                order[j] = order[j - 1];
                j--;
            }
            order[j] = o;
        }
    }
    __syncthreads();
    const int src = order[t];
    const float lambda = fmaxf(evals_m[src * q + src], 0.f);
    const float s = __fsqrt_rn(lambda);
    const float sq = __fsqrt_rn(fmaxf(s, 0.f));
    const float inv = s > 1e-12f ? __fdiv_rn(1.0f, s) : 0.f;
    for (int64_t i = threadIdx.x; i < rows; i += blockDim.x) {
        float u = 0.f;
        for (int c = 0; c < q; c++) u = __fadd_rn(u, __fmul_rn(evecs[c * q + src], qy[c * rows + i]));
        b[i * ldb + b_off + t] = __fmul_rn(u, sq);
    }
    for (int64_t j = threadIdx.x; j < cols; j += blockDim.x) {
        float v = 0.f;
        for (int c = 0; c < q; c++) v = __fadd_rn(v, __fmul_rn(evecs[c * q + src], bt[c * cols + j]));
        v = s > 1e-12f ? __fmul_rn(v, inv) : 0.f;
        a[t * cols + j] = __fmul_rn(sq, v);
    }
}

// B += B B^T-style Gram of q rows: g[i][j] = dot(x_i, x_j)
// (abliterate.zig:505-508) via edit_dots_kernel.

// ---------------------------------------------------------------------------
// host side

static int ed_grid(int64_t total) {
    int64_t g = (total + 255) / 256;
    return (int)(g < 1 ? 1 : g > 16384 ? 16384 : g);
}

// The full mode's random test matrix: the first n draws of
// Random.floatNorm(f32) from std.Random.DefaultPrng.init(seed), in the
// order the reference fills omega (abliterate.zig:474-479).
void edit_gaussian(float *out, size_t n, uint64_t seed) {
    ZigRandom rng(seed);
    for (size_t t = 0; t < n; t++) out[t] = rng.norm_f32();
}

int64_t edit_rank(int64_t rows, int64_t cols, int64_t k, int mode, int64_t lora_rank, int ablate) {
    int64_t r = k;
    if (mode == 2) {
        const int64_t rr = lora_rank > k ? lora_rank : k;
        int64_t q = 2 * rr + 4;
        q = q < rows ? q : rows;
        q = q < cols ? q : cols;
        r = rr < q ? rr : q;
    }
    return r + (ablate ? k : 0);
}

struct EditWork {
    DevBuf v, norms, vn, a, bp, wa, gram, c, d, omega, qy, qx, cy, dots, bbt, evecs, xs, xa, wu;
};

// b[i][0..r) = bp[i][0..r), b[i][r + j] = -lambda wu[j][i]  (abliterate.zig:252-257)
__global__ void edit_b_ablate_kernel(float *b, const float *bp, const float *wu, int64_t rows, int64_t r, int64_t k,
                                     float weight) {
    const int64_t rank = r + k;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < rows * rank;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = t / rank, j = t % rank;
        b[t] = j < r ? bp[i * r + j] : __fmul_rn(-weight, wu[(j - r) * rows + i]);
    }
}

static void edit_matmul(const TileView &w, float *out, const float *x, int64_t n, hipStream_t s, DevBuf *ws,
                        const float *delta_a = nullptr, const float *delta_b = nullptr, int delta_rank = 0,
                        float *xa = nullptr) {
    MatmulEpilogue ep;
    ep.exact = 1;  // three bf16 terms: the f32 products of tensor.matmulT
    if (delta_rank > 0) {
        launch_delta_xa(xa, x, delta_a, n, w.cols, delta_rank, s);
        ep.delta_b = delta_b;
        ep.delta_xa = xa;
        ep.delta_rank = delta_rank;
    }
    launch_matmul(w, out, x, n, ep, s, nullptr, ws);
}

// W^T y for q vectors
static void edit_matvecT(const TileView &w, float *out, const float *y, int64_t q, hipStream_t s) {
    launch_matvecT(out, w, y, q, s);
}

static void edit_orth(float *vecs, int64_t q, int64_t n, hipStream_t s) {
    const int64_t ept = (n + 1023) / 1024;
    if (ept <= 2)
        hipLaunchKernelGGL(edit_orth_reg_kernel<2>, dim3(1), dim3(1024), 0, s, vecs, q, n);
    else if (ept <= 4)
        hipLaunchKernelGGL(edit_orth_reg_kernel<4>, dim3(1), dim3(1024), 0, s, vecs, q, n);
    else if (ept <= 8)
        hipLaunchKernelGGL(edit_orth_reg_kernel<8>, dim3(1), dim3(1024), 0, s, vecs, q, n);
    else if (ept <= 16)
        hipLaunchKernelGGL(edit_orth_reg_kernel<16>, dim3(1), dim3(1024), 0, s, vecs, q, n);
    else if (ept <= 24)
        hipLaunchKernelGGL(edit_orth_reg_kernel<24>, dim3(1), dim3(1024), 0, s, vecs, q, n);
    else  // vectors above 24 576 elements: the global-memory form
        hipLaunchKernelGGL(edit_orthonormalize_kernel, dim3(1), dim3(1024), 0, s, vecs, q, n);
    DITCH_TRY_HIP(hipGetLastError());
}

static void edit_jacobi(float *m, float *vecs, int64_t q, hipStream_t s) {
    DITCH_CHECK(q <= 46340, DITCH_UNSUPPORTED, "edit: SVD width above 46340");
    const dim3 block(q <= 256 ? 256 : 1024);
    if (q <= ED_LDS_Q) {
        static const bool attr = [] {
            return hipFuncSetAttribute((const void *)edit_jacobi_kernel<true>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       2 * ED_LDS_Q * ED_LDS_Q * 4) == hipSuccess;
        }();
        DITCH_CHECK(attr, DITCH_DEVICE_FAILED, "edit: the Jacobi kernel's LDS size was refused");
        hipLaunchKernelGGL(edit_jacobi_kernel<true>, dim3(1), block, (size_t)(2 * q * q * 4), s, m, vecs, (int)q);
    } else {
        hipLaunchKernelGGL(edit_jacobi_kernel<false>, dim3(1), block, 0, s, m, vecs, (int)q);
    }
    DITCH_TRY_HIP(hipGetLastError());
}

static void edit_dots(float *out, const float *p, int64_t np, const float *x, int64_t nx, int64_t len, hipStream_t s) {
    hipLaunchKernelGGL(edit_dots_kernel, dim3((unsigned)np, (unsigned)nx), dim3(256), 0, s, out, p, x, np, len);
    DITCH_TRY_HIP(hipGetLastError());
}

// The delta of abliterate.computeDelta for the resident weight w and host
// directions v [k][rows]: device buffers da [rank][cols], db [rows][rank]
// (allocated here, owned by the caller), *rank set.
void edit_delta_device(ditch_hip *h, const TileView &w, const float *hv, int64_t k, float weight, int mode,
                       int64_t lora_rank, uint64_t seed, int ablate, hipStream_t s, float **da_out, float **db_out,
                       int64_t *rank_out) {
    const int64_t rows = w.rows, cols = w.cols;
    DITCH_CHECK(k >= 1 && mode >= 0 && mode <= 2, DITCH_INVALID_ARGUMENT, "edit: at least one direction, mode 0..2");
    if (!h->edit_work) h->edit_work = std::make_shared<EditWork>();
    EditWork &W = *static_cast<EditWork *>(h->edit_work.get());
    float *v = W.v.get<float>(k * rows);
    DITCH_TRY_HIP(hipMemcpyAsync(v, hv, k * rows * 4, hipMemcpyHostToDevice, s));
    const int64_t rank = edit_rank(rows, cols, k, mode, lora_rank, ablate);
    const int64_t r_out = rank - (ablate ? k : 0);  // the output-side edit's rank
    float *A = (float *)dev_alloc(rank * cols * 4), *B = (float *)dev_alloc(rows * rank * 4);
    try {
        // the output-side B, [rows][r_out] (a separate buffer when the input
        // side widens the final B)
        float *Bp = ablate ? W.bp.get<float>(rows * r_out) : B;
        float *norms = nullptr;
        float *a = A;  // none / pre: the output-side A is the first k rows of A
        if (mode == 0) {
            edit_matvecT(w, a, v, k, s);
        } else {
            norms = W.norms.get<float>(rows);
            launch_row_norms(norms, w, s);
            float *vn = W.vn.get<float>(k * rows);
            hipLaunchKernelGGL(edit_vn_kernel, dim3(ed_grid(k * rows)), dim3(256), 0, s, vn, v, norms, k, rows);
            DITCH_TRY_HIP(hipGetLastError());
            if (mode == 2) a = W.a.get<float>(k * cols);
            edit_matvecT(w, a, vn, k, s);
        }
        if (mode != 2) {
            hipLaunchKernelGGL(edit_b_kernel, dim3(ed_grid(k * rows)), dim3(256), 0, s, Bp, v, mode == 1 ? norms : nullptr,
                               k, rows, weight, r_out);
            DITCH_TRY_HIP(hipGetLastError());
        } else {
            // D = diag(c) W + sum_l d_l a_l^T and its randomised SVD
            float *wa = W.wa.get<float>(k * rows);
            edit_matmul(w, wa, a, k, s, &W.xs);
            float *gram = W.gram.get<float>(k * k);
            edit_dots(gram, a, k, a, k, cols, s);
            float *c = W.c.get<float>(rows), *d = W.d.get<float>(k * rows);
            hipLaunchKernelGGL(edit_cd_kernel, dim3(ed_grid(rows)), dim3(256), 0, s, c, d, v, norms, wa, gram, k, rows,
                               weight);
            DITCH_TRY_HIP(hipGetLastError());
            const int64_t rr = lora_rank > k ? lora_rank : k;
            int64_t q = 2 * rr + 4;
            q = q < rows ? q : rows;
            q = q < cols ? q : cols;
            std::vector<float> om((size_t)(q * cols));
            edit_gaussian(om.data(), om.size(), seed);
            float *omega = W.omega.get<float>(q * cols);
            DITCH_TRY_HIP(hipMemcpyAsync(omega, om.data(), om.size() * 4, hipMemcpyHostToDevice, s));
            float *qy = W.qy.get<float>(q * rows), *qx = W.qx.get<float>(q * cols), *cy = W.cy.get<float>(q * rows);
            float *dots = W.dots.get<float>(q * k);
            auto apply = [&](float *out, const float *x) {  // out [q][rows] = (D X)^T
                edit_matmul(w, out, x, q, s, &W.xs);
                edit_dots(dots, a, k, x, q, cols, s);
                hipLaunchKernelGGL(edit_apply_kernel, dim3(ed_grid(q * rows)), dim3(256), 0, s, out, c, d, dots, q, k,
                                   rows);
                DITCH_TRY_HIP(hipGetLastError());
            };
            auto applyT = [&](float *out, const float *y) {  // out [q][cols] = (D^T Y)^T
                hipLaunchKernelGGL(edit_scale_rows_kernel, dim3(ed_grid(q * rows)), dim3(256), 0, s, cy, y, c, q, rows);
                DITCH_TRY_HIP(hipGetLastError());
                edit_matvecT(w, out, cy, q, s);
                edit_dots(dots, d, k, y, q, rows, s);
                hipLaunchKernelGGL(edit_applyT_kernel, dim3(ed_grid(q * cols)), dim3(256), 0, s, out, a, dots, q, k,
                                   cols);
                DITCH_TRY_HIP(hipGetLastError());
            };
            apply(qy, omega);
            edit_orth(qy, q, rows, s);
            for (int it = 0; it < 6; it++) {
                applyT(qx, qy);
                edit_orth(qx, q, cols, s);
                apply(qy, qx);
                edit_orth(qy, q, rows, s);
            }
            applyT(qx, qy);  // B^T = (Q^T D)^T
            float *bbt = W.bbt.get<float>(q * q), *evecs = W.evecs.get<float>(q * q);
            edit_dots(bbt, qx, q, qx, q, cols, s);
            edit_jacobi(bbt, evecs, q, s);
            hipLaunchKernelGGL(edit_svd_out_kernel, dim3((unsigned)r_out), dim3(256), (size_t)q * 4, s, A, Bp, bbt,
                               evecs, qy, qx, (int)q, rows, cols, r_out, r_out, (int64_t)0);
            DITCH_TRY_HIP(hipGetLastError());
        }
        if (ablate) {
            // U = orth(W^T V) [k][cols]; W' U through the primary delta; the
            // rank grows by k (abliterate.zig:234-261)
            float *u = A + r_out * cols;
            edit_matvecT(w, u, v, k, s);
            edit_orth(u, k, cols, s);
            float *wu = W.wu.get<float>(k * rows);
            float *xa = W.xa.get<float>(k * r_out);
            edit_matmul(w, wu, u, k, s, &W.xs, A, Bp, (int)r_out, xa);
            hipLaunchKernelGGL(edit_b_ablate_kernel, dim3(ed_grid(rows * rank)), dim3(256), 0, s, B, Bp, wu, rows, r_out,
                               k, weight);
            DITCH_TRY_HIP(hipGetLastError());
        }
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    } catch (...) {
        dev_free(A);
        dev_free(B);
        throw;
    }
    *da_out = A;
    *db_out = B;
    *rank_out = rank;
}

}  // namespace ditch
