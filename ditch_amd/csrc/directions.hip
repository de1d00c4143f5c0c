// directions.hip — the step after residual capture, kept on the device: the
// per-prompt window mean and winsorising of the captured residuals with
// their f64 sums (Engine.forEachResidual / getResidualMeanObserved,
// engine.zig:314-337, 414-431), the per-coordinate moments
// (directions.Moments, directions.zig:184-213), the difference-of-means
// directions (abliterate.computeDirections, abliterate.zig:88-109), the
// Nystrom sketch of the bad residuals (directions.Sketch.add, directions.zig:
// 80-104) and the multi-direction basis built from it (Sketch.factor and
// computeBasisFrom, directions.zig:108-134, 371-455).
//
// Per-prompt and per-entry vectors are a few thousand floats: each is one
// workgroup's work (reductions in LDS), and every sum that the reference
// takes over prompts runs over the prompts in their order, one thread per
// coordinate, so those f64 sums are the reference's bit for bit.
#include <math.h>

#include "internal.h"

namespace ditch {

constexpr int DIR_MAX_HIDDEN = 16384;  // |v| keys of one vector in LDS
constexpr int DIR_LDS_M = 96;          // sketch widths whose basis works in LDS

// ---------------------------------------------------------------------------
// block reductions (blockDim.x a multiple of 64, at most 1024)

__device__ __forceinline__ double dir_wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// the block's sum; every thread gets it (sh: 16 doubles of LDS)
__device__ double dir_block_sum(double v, double *sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = dir_wave_sum(v);
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double r = 0.0;
    for (int w = 0; w < nw; w++) r += sh[w];
    return r;
}

// dot of two f32 vectors, accumulated in f64 and rounded once
__device__ float dir_dot_f32(const float *a, const float *b, int64_t n, double *sh) {
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) acc += (double)a[i] * (double)b[i];
    return (float)dir_block_sum(acc, sh);
}

// tensor.normalize (tensor.zig:580-584): x *= 1 / ||x|| unless ||x|| <= 1e-12
__device__ void dir_normalize(float *x, int64_t n, double *sh) {
    const float nrm = __fsqrt_rn(dir_dot_f32(x, x, n, sh));
    if (nrm > 1e-12f) {
        const float s = __fdiv_rn(1.0f, nrm);
        for (int64_t i = threadIdx.x; i < n; i += blockDim.x) x[i] = __fmul_rn(x[i], s);
    }
    __syncthreads();
}

// y += alpha * x without fusion (tensor.zig:560-570)
__device__ void dir_axpy(float *y, float alpha, const float *x, int64_t n) {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) y[i] = __fadd_rn(y[i], __fmul_rn(alpha, x[i]));
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Window mean and winsorising (engine.zig:414-431)

struct WindowArgs {
    const float *res;      // [entries][n_capture][hidden]
    const uint32_t *first; // [prompts] first capture index of each prompt
    const uint32_t *take;  // [prompts] captured rows of each prompt
    float *vout;           // [prompts][entries][hidden]
    int64_t entries, n_capture, hidden, prompts;
    float q;               // quantile of |v|; outside [0, 1): none
    int winsor;
};

// One workgroup per (prompt, entry): v = sum_t (1/take) r_t by the
// reference's axpy (a product, then a sum, each rounded), then the values
// clamped to +-quantile(|v|, q) with torch.quantile's interpolation
// (engine.zig:492-499). The order statistics come from a bitonic sort of
// the |v| bit patterns in LDS (non-negative floats order as their bits).
__global__ __launch_bounds__(1024) void residual_window_kernel(WindowArgs a) {
    __shared__ uint32_t keys[DIR_MAX_HIDDEN];
    const int64_t b = blockIdx.x, e = blockIdx.y, H = a.hidden;
    uint32_t first = a.first[b], take = a.take[b];
    // a capture range outside the residual buffer is not read (clamped empty)
    if ((int64_t)first >= a.n_capture) take = 0;
    else if ((int64_t)first + take > a.n_capture) take = (uint32_t)(a.n_capture - first);
    const float inv = __fdiv_rn(1.0f, (float)(take > 1 ? take : 1));
    float *v = a.vout + (b * a.entries + e) * H;
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) {
        float acc = 0.f;
        for (uint32_t t = 0; t < take; t++)
            acc = __fadd_rn(acc, __fmul_rn(inv, a.res[(e * a.n_capture + first + t) * H + i]));
        v[i] = acc;
        if (a.winsor) keys[i] = __float_as_uint(fabsf(acc));
    }
    if (!a.winsor) return;
    int N = 1;
    while (N < H) N <<= 1;
    for (int64_t i = H + threadIdx.x; i < N; i += blockDim.x) keys[i] = 0xFFFFFFFFu;  // after every value
    __syncthreads();
    for (int k = 2; k <= N; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < N; i += blockDim.x) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint32_t x = keys[i], y = keys[ixj];
                    const bool up = (i & k) == 0;
                    if ((x > y) == up) {
                        keys[i] = y;
                        keys[ixj] = x;
                    }
                }
            }
            __syncthreads();
        }
    const float pos = __fmul_rn(a.q, (float)(H - 1));
    const float fl = floorf(pos);
    const int64_t lo = (int64_t)fl, hi = lo + 1 < H - 1 ? lo + 1 : H - 1;
    const float frac = __fsub_rn(pos, fl);
    const float s_lo = __uint_as_float(keys[lo]), s_hi = __uint_as_float(keys[hi]);
    const float thr = __fadd_rn(s_lo, __fmul_rn(frac, __fsub_rn(s_hi, s_lo)));
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) v[i] = fmaxf(-thr, fminf(v[i], thr));
}

// sum[e][i] += v[b][e][i] and (with sq) sq[e][i] += v^2 over the prompts in
// order (Acc.add engine.zig:320-326; Moments.add directions.zig:196-205)
__global__ void residual_accum_kernel(double *sum, double *sq, const float *vout, int64_t prompts, int64_t entries,
                                      int64_t hidden) {
    const int64_t total = entries * hidden;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        double s = sum ? sum[t] : 0.0, q = sq ? sq[t] : 0.0;
        for (int64_t b = 0; b < prompts; b++) {
            const double x = (double)vout[b * total + t];
            s += x;
            q += x * x;
        }
        if (sum) sum[t] = s;
        if (sq) sq[t] = q;
    }
}

// mean = f32(sum / max(count, 1)) (engine.zig:333-335)
__global__ void residual_mean_kernel(float *mean, const double *sum, double count, int64_t n) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (int64_t)gridDim.x * blockDim.x)
        mean[t] = (float)(sum[t] / count);
}

// ---------------------------------------------------------------------------
// Difference-of-means directions (abliterate.zig:88-109), one block per entry

__global__ __launch_bounds__(1024) void directions_kernel(float *dirs, float *gd_scratch, const float *good,
                                                          const float *bad, int64_t hidden, int orthogonalize) {
    __shared__ double sh[16];
    const int64_t e = blockIdx.x;
    float *d = dirs + e * hidden;
    const float *g = good + e * hidden, *b = bad + e * hidden;
    for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) d[i] = __fsub_rn(b[i], g[i]);
    __syncthreads();
    dir_normalize(d, hidden, sh);
    if (!orthogonalize) return;
    float *gd = gd_scratch + e * hidden;
    for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) gd[i] = g[i];
    __syncthreads();
    dir_normalize(gd, hidden, sh);
    const float p = dir_dot_f32(d, gd, hidden, sh);
    dir_axpy(d, -p, gd, hidden);
    dir_normalize(d, hidden, sh);
}

// ---------------------------------------------------------------------------
// Nystrom sketch (directions.zig:80-104): z = r - center, p = Omega^T z

__global__ __launch_bounds__(256) void sketch_proj_kernel(double *proj, const float *omega, int64_t m,
                                                          const float *center, const float *v, int64_t entries,
                                                          int64_t hidden) {
    __shared__ double sh[16];
    const int64_t b = blockIdx.x, e = blockIdx.y;
    const float *r = v + (b * entries + e) * hidden, *c = center + e * hidden;
    for (int64_t j = 0; j < m; j++) {
        double acc = 0.0;
        for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x)
            acc += ((double)r[i] - (double)c[i]) * (double)omega[j * hidden + i];
        acc = dir_block_sum(acc, sh);
        if (threadIdx.x == 0) proj[(b * entries + e) * m + j] = acc;
    }
}

// Y[e][j][i] += z_b[i] p_b[j] and W[e][j][l] += p_b[j] p_b[l], the prompts
// in order
__global__ void sketch_accum_kernel(double *y, double *w, const double *proj, int64_t m, const float *center,
                                    const float *v, int64_t prompts, int64_t entries, int64_t hidden) {
    const int64_t per = m * hidden + m * m, total = entries * per;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = t / per, u = t % per;
        if (u < m * hidden) {
            const int64_t j = u / hidden, i = u % hidden;
            double acc = y[(e * m + j) * hidden + i];
            const double c = (double)center[e * hidden + i];
            for (int64_t b = 0; b < prompts; b++) {
                const double z = (double)v[(b * entries + e) * hidden + i] - c;
                acc += z * proj[(b * entries + e) * m + j];
            }
            y[(e * m + j) * hidden + i] = acc;
        } else {
            const int64_t jl = u - m * hidden, j = jl / m, l = jl % m;
            double acc = w[(e * m + j) * m + l];
            for (int64_t b = 0; b < prompts; b++)
                acc += proj[(b * entries + e) * m + j] * proj[(b * entries + e) * m + l];
            w[(e * m + j) * m + l] = acc;
        }
    }
}

// ---------------------------------------------------------------------------
// Basis (Sketch.factor + computeBasisFrom), one block per entry

// directions.symmetricEigen (directions.zig:463-500): cyclic Jacobi in f64 on
// an n x n matrix in LDS or global memory (overwritten by its
// diagonalisation), eigenvectors
// in the columns of vecs; the rotation's rows and columns are updated by the
// block's threads in the reference's operation order.
__device__ void dir_symmetric_eigen(double *mat, double *vecs, int n, double *flag) {
    const int tid = threadIdx.x;
    for (int k = tid; k < n * n; k += blockDim.x) vecs[k] = (k / n == k % n) ? 1.0 : 0.0;
    __syncthreads();
    for (int sweep = 0; sweep < 60; sweep++) {
        if (tid == 0) {
            double off = 0, diag = 0;
            for (int i = 0; i < n; i++)
                for (int j = 0; j < n; j++) {
                    const double x = mat[i * n + j];
                    if (i != j) off += x * x;
                    else diag += x * x;
                }
            flag[0] = off <= 1e-24 * (diag > 1e-300 ? diag : 1e-300) ? 1.0 : 0.0;
        }
        __syncthreads();
        if (flag[0] != 0.0) break;
        __syncthreads();
        for (int p = 0; p < n; p++)
            for (int q = p + 1; q < n; q++) {
                const double apq = mat[p * n + q];
                if (fabs(apq) < 1e-300) continue;
                const double theta = (mat[q * n + q] - mat[p * n + p]) / (2.0 * apq);
                const double sg = theta > 0 ? 1.0 : theta < 0 ? -1.0 : 0.0;
                const double t = theta == 0 ? 1.0 : sg / (fabs(theta) + sqrt(theta * theta + 1.0));
                const double cs = 1.0 / sqrt(t * t + 1.0), sn = t * cs;
                __syncthreads();  // every thread has read the pivot before it changes
                for (int k = tid; k < n; k += blockDim.x) {
                    const double akp = mat[k * n + p], akq = mat[k * n + q];
                    mat[k * n + p] = cs * akp - sn * akq;
                    mat[k * n + q] = sn * akp + cs * akq;
                    const double vkp = vecs[k * n + p], vkq = vecs[k * n + q];
                    vecs[k * n + p] = cs * vkp - sn * vkq;
                    vecs[k * n + q] = sn * vkp + cs * vkq;
                }
                __syncthreads();
                for (int k = tid; k < n; k += blockDim.x) {
                    const double apk = mat[p * n + k], aqk = mat[q * n + k];
                    mat[p * n + k] = cs * apk - sn * aqk;
                    mat[q * n + k] = sn * apk + cs * aqk;
                }
                __syncthreads();
            }
    }
    __syncthreads();
}

struct BasisArgs {
    float *dirs;           // [entries][k][hidden]
    const float *first;    // [entries][hidden]
    const float *good;     // [entries][hidden] good means
    const double *y;       // [entries][m][hidden]
    const double *w;       // [entries][m][m]
    double *bf;            // scratch [entries][m][hidden]
    float *gd;             // scratch [entries][hidden]
    int64_t hidden, k, m;
    int orthogonalize;
    // the sketch's m x m matrices and index lists: in dynamic LDS (lds = 1)
    // or, for wide sketches, per entry in `work` (2 m^2 doubles + 2 m ints)
    int lds;
    double *work;
};

__global__ __launch_bounds__(256) void basis_kernel(BasisArgs a) {
    extern __shared__ double dir_dyn[];
    __shared__ double sh[16], flag[1];
    __shared__ int r_sh;
    const int64_t e = blockIdx.x, H = a.hidden, K = a.k;
    const int m = (int)a.m, tid = threadIdx.x;
    double *wm = a.lds ? dir_dyn : a.work + e * (2 * a.m * a.m + a.m);
    double *vecs = wm + m * m;
    int *valid = (int *)(vecs + m * m), *order = valid + m;
    float *basis = a.dirs + e * K * H;
    float *gd = a.gd + e * H;
    double *bf = a.bf + e * a.m * H;
    const double *ye = a.y + e * a.m * H;
    for (int64_t i = tid; i < K * H; i += blockDim.x) basis[i] = i < H ? a.first[e * H + i] : 0.f;
    for (int64_t i = tid; i < H; i += blockDim.x) gd[i] = a.good[e * H + i];
    for (int i = tid; i < m * m; i += blockDim.x) wm[i] = a.w[e * m * m + i];
    __syncthreads();
    dir_normalize(gd, H, sh);
    // Sketch.factor: B = Y W^{-1/2} over W's significant eigenvalues
    dir_symmetric_eigen(wm, vecs, m, flag);
    if (tid == 0) {
        double max_ev = 0;
        for (int j = 0; j < m; j++) max_ev = wm[j * m + j] > max_ev ? wm[j * m + j] : max_ev;
        int r = 0;
        for (int j = 0; j < m; j++) {
            const double ev = wm[j * m + j];
            if (ev <= max_ev * 1e-9 || ev <= 0) continue;
            valid[r++] = j;
        }
        r_sh = r;
    }
    __syncthreads();
    const int r = r_sh;
    for (int64_t i = tid; i < H; i += blockDim.x)
        for (int c = 0; c < r; c++) {
            const int j = valid[c];
            const double s = 1.0 / sqrt(wm[j * m + j]);
            double col = 0.0;
            for (int l = 0; l < m; l++) {
                const double coef = vecs[l * m + j] * s;
                if (coef == 0) continue;
                col += coef * ye[l * H + i];
            }
            bf[c * H + i] = col;
        }
    __syncthreads();
    // the first direction (and the good direction) projected out of B's columns
    for (int c = 0; c < r; c++)
        for (int pass = 0; pass < 1 + a.orthogonalize; pass++) {
            const float *unit = pass == 0 ? basis : gd;
            double acc = 0.0;
            for (int64_t i = tid; i < H; i += blockDim.x) acc += bf[c * H + i] * (double)unit[i];
            const double p = dir_block_sum(acc, sh);
            for (int64_t i = tid; i < H; i += blockDim.x) bf[c * H + i] -= p * (double)unit[i];
            __syncthreads();
        }
    // Gram matrix of B and its eigen-decomposition (reusing wm / vecs)
    for (int i = 0; i < r; i++)
        for (int j = i; j < r; j++) {
            double acc = 0.0;
            for (int64_t t = tid; t < H; t += blockDim.x) acc += bf[i * H + t] * bf[j * H + t];
            const double g = dir_block_sum(acc, sh);
            if (tid == 0) {
                wm[i * r + j] = g;
                wm[j * r + i] = g;
            }
        }
    __syncthreads();
    dir_symmetric_eigen(wm, vecs, r, flag);
    if (tid == 0) {  // descending eigenvalues, ties in index order (a stable sort)
        for (int i = 0; i < r; i++) order[i] = i;
        for (int i = 1; i < r; i++) {
            const int o = order[i];
            int j = i;
            while (j > 0 && wm[order[j - 1] * r + order[j - 1]] < wm[o * r + o]) {
                order[j] = order[j - 1];
                j--;
            }
            order[j] = o;
        }
    }
    __syncthreads();
    for (int64_t d = 1; d < K; d++) {
        if (d - 1 >= r) continue;
        const int src = order[d - 1];
        const double lambda = wm[src * r + src];
        if (lambda <= 0) continue;
        float *dir = basis + d * H;
        for (int64_t i = tid; i < H; i += blockDim.x) {
            float acc = 0.f;
            for (int c = 0; c < r; c++) {
                const float coef = (float)(vecs[c * r + src] / sqrt(lambda));
                acc = __fadd_rn(acc, __fmul_rn(coef, (float)bf[c * H + i]));
            }
            dir[i] = acc;
        }
    }
    __syncthreads();
    // abliterate.orthonormalize (abliterate.zig:409-423)
    for (int64_t i = 0; i < K; i++) {
        float *vi = basis + i * H;
        for (int pass = 0; pass < 2; pass++)
            for (int64_t j = 0; j < i; j++) {
                const float p = dir_dot_f32(vi, basis + j * H, H, sh);
                dir_axpy(vi, -p, basis + j * H, H);
            }
        const float nrm = __fsqrt_rn(dir_dot_f32(vi, vi, H, sh));
        const float s = nrm > 1e-20f ? __fdiv_rn(1.0f, nrm) : 0.f;
        for (int64_t t = tid; t < H; t += blockDim.x) vi[t] = nrm > 1e-20f ? __fmul_rn(vi[t], s) : 0.f;
        __syncthreads();
    }
}

// Every component oriented like the same component of the previous entry
// (directions.zig:446-452), entries in order (one block).
__global__ __launch_bounds__(1024) void orient_kernel(float *dirs, int64_t entries, int64_t k, int64_t hidden) {
    __shared__ double sh[16];
    for (int64_t e = 1; e < entries; e++)
        for (int64_t d = 1; d < k; d++) {
            float *dir = dirs + (e * k + d) * hidden;
            const float *prev = dirs + ((e - 1) * k + d) * hidden;
            const float p = dir_dot_f32(dir, prev, hidden, sh);
            if (p < 0)
                for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) dir[i] = -dir[i];
            __syncthreads();
        }
}

// ---------------------------------------------------------------------------
// host side

static int dir_grid(int64_t total) {
    int64_t g = (total + 255) / 256;
    return (int)(g < 1 ? 1 : g > 8192 ? 8192 : g);
}

void launch_residual_reduce(const float *res, int64_t entries, int64_t n_capture, int64_t hidden,
                            const uint32_t *first, const uint32_t *take, int64_t prompts, float q, float *vout,
                            double *sum, double *sq, hipStream_t s) {
    if (prompts <= 0 || entries <= 0 || hidden <= 0) return;
    const bool winsor = q >= 0.f && q < 1.f;
    DITCH_CHECK(!winsor || hidden <= DIR_MAX_HIDDEN, DITCH_UNSUPPORTED, "winsorising: hidden above 16384");
    DITCH_CHECK(prompts <= 65535 && entries <= 65535, DITCH_UNSUPPORTED, "residual reduce: grid");
    WindowArgs a{res, first, take, vout, entries, n_capture, hidden, prompts, q, winsor ? 1 : 0};
    hipLaunchKernelGGL(residual_window_kernel, dim3((unsigned)prompts, (unsigned)entries), dim3(1024), 0, s, a);
    DITCH_TRY_HIP(hipGetLastError());
    if (sum || sq) {
        hipLaunchKernelGGL(residual_accum_kernel, dim3(dir_grid(entries * hidden)), dim3(256), 0, s, sum, sq, vout,
                           prompts, entries, hidden);
        DITCH_TRY_HIP(hipGetLastError());
    }
}

void launch_residual_mean(float *mean, const double *sum, uint64_t count, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(residual_mean_kernel, dim3(dir_grid(n)), dim3(256), 0, s, mean, sum,
                       (double)(count > 1 ? count : 1), n);
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_directions(float *dirs, const float *good, const float *bad, int64_t entries, int64_t hidden,
                       int orthogonalize, hipStream_t s, DevBuf *tmp) {
    if (entries <= 0 || hidden <= 0) return;
    float *gd = orthogonalize ? tmp->get<float>((size_t)(entries * hidden)) : nullptr;
    hipLaunchKernelGGL(directions_kernel, dim3((unsigned)entries), dim3(1024), 0, s, dirs, gd, good, bad, hidden,
                       orthogonalize);
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_sketch_add(double *y, double *w, const float *omega, int64_t m, const float *center, const float *v,
                       int64_t prompts, int64_t entries, int64_t hidden, hipStream_t s, DevBuf *tmp) {
    if (prompts <= 0 || entries <= 0) return;
    DITCH_CHECK(m >= 1, DITCH_INVALID_ARGUMENT, "sketch: width 0");
    double *proj = tmp->get<double>((size_t)(prompts * entries * m));
    hipLaunchKernelGGL(sketch_proj_kernel, dim3((unsigned)prompts, (unsigned)entries), dim3(256), 0, s, proj, omega,
                       m, center, v, entries, hidden);
    DITCH_TRY_HIP(hipGetLastError());
    hipLaunchKernelGGL(sketch_accum_kernel, dim3(dir_grid(entries * (m * hidden + m * m))), dim3(256), 0, s, y, w,
                       proj, m, center, v, prompts, entries, hidden);
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_basis(float *dirs, const float *first, const float *good, int64_t entries, int64_t hidden, int64_t k,
                  int orthogonalize, const double *y, const double *w, int64_t m, hipStream_t s, DevBuf *tmp) {
    if (entries <= 0) return;
    DITCH_CHECK(k >= 1 && m >= 1, DITCH_INVALID_ARGUMENT, "basis: no directions or an empty sketch");
    DITCH_CHECK(m <= 46340, DITCH_UNSUPPORTED, "basis: sketch width above 46340");
    if (k == 1) {
        DITCH_TRY_HIP(hipMemcpyAsync(dirs, first, (size_t)(entries * hidden) * 4, hipMemcpyDeviceToDevice, s));
        return;
    }
    // per entry: 2 m^2 doubles and 2 m ints (m doubles' room) of eigen-solver state
    const int64_t per = 2 * m * m + m;
    const bool lds = m <= DIR_LDS_M;
    double *bf = tmp->get<double>((size_t)(entries * m * hidden + (entries * hidden + 1) / 2 + (lds ? 0 : entries * per)));
    BasisArgs a{dirs, first, good, y, w, bf, (float *)(bf + entries * m * hidden), hidden, k, m, orthogonalize,
                lds ? 1 : 0, lds ? nullptr : bf + entries * m * hidden + (entries * hidden + 1) / 2};
    const size_t shmem = lds ? (size_t)per * 8 : 0;
    if (lds) {
        static const bool attr = [] {
            return hipFuncSetAttribute((const void *)basis_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (2 * DIR_LDS_M * DIR_LDS_M + DIR_LDS_M) * 8) == hipSuccess;
        }();
        DITCH_CHECK(attr, DITCH_DEVICE_FAILED, "basis: the kernel's LDS size was refused");
    }
    hipLaunchKernelGGL(basis_kernel, dim3((unsigned)entries), dim3(256), shmem, s, a);
    DITCH_TRY_HIP(hipGetLastError());
    hipLaunchKernelGGL(orient_kernel, dim3(1), dim3(1024), 0, s, dirs, entries, k, hidden);
    DITCH_TRY_HIP(hipGetLastError());
}

}  // namespace ditch
