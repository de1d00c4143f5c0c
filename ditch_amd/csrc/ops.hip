// ops.hip — element-wise and reduction kernels of the forward pass and of
// the VTable's per-row operations (compute.zig:107-119), plus row norms and
// W^T y over resident weights (tensor.zig:1056-1122).
#include "decode.h"
#include "internal.h"
#include "gemm_common.h"
#include "tiled.h"

namespace ditch {

static int grid_1d(int64_t total, int block = 256) {
    int64_t g = (total + block - 1) / block;
    if (g > 65536) g = 65536;
    return g < 1 ? 1 : (int)g;
}

// ---------------------------------------------------------------------------
// Reductions inside one 256-thread block.

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, Op op, T *sh) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    T r = sh[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) r = op(r, sh[w]);
    return r;
}

__device__ __forceinline__ float block_sum(float v, float *sh) {
    v = wave_sum(v);
    return block_reduce(v, [](float a, float b) { return a + b; }, sh);
}
__device__ __forceinline__ double block_sum_d(double v, double *sh) {
    v = wave_sum_d(v);
    return block_reduce(v, [](double a, double b) { return a + b; }, sh);
}
__device__ __forceinline__ float block_max(float v, float *sh) {
    v = wave_max(v);
    return block_reduce(v, [](float a, float b) { return fmaxf(a, b); }, sh);
}


// ---------------------------------------------------------------------------
// RMSNorm / LayerNorm rows (tensor.zig:1167-1179, 1343-1358): one block per
// row. `row_index` gathers input rows (the logit rows of model.zig:4798-4852).

__global__ void rmsnorm_kernel(float *out, const float *x, const float *w, int64_t wlen, int64_t len, float eps,
                               int gemma, const int64_t *row_index, int64_t n_src, int64_t in_stride,
                               int64_t out_stride) {
    __shared__ float sh[8];
    int64_t r = blockIdx.x;
    int64_t src = row_index ? row_index[r] : r;
    src = (uint64_t)src < (uint64_t)n_src ? src : n_src - 1;  // the row lists are unsigned
    const float *xr = x + src * in_stride;
    float ss = 0.f;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) ss = __builtin_fmaf(xr[i], xr[i], ss);
    ss = block_sum(ss, sh);
    float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)len), eps)));
    float *o = out + r * out_stride;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) {
        float v = __fmul_rn(xr[i], inv);
        if (wlen > 0) v = __fmul_rn(v, gemma ? __fadd_rn(1.0f, w[i]) : w[i]);
        o[i] = v;
    }
}

// rmsnorm_kernel for rows of 256 NV columns: a wave per row holds it in
// registers (NV float4 a lane, one read of the row), sums its squares over
// the wave and writes the normalised row; four rows a workgroup.
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(float *out, const float *x, const float *w, int64_t wlen,
                                                           int64_t n, float eps, int gemma, const int64_t *row_index,
                                                           int64_t n_src) {
    constexpr int64_t LEN = 256 * NV;
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= n) return;
    int64_t src = row_index ? row_index[r] : r;
    src = (uint64_t)src < (uint64_t)n_src ? src : n_src - 1;  // the row lists are unsigned
    const float4 *xr = (const float4 *)(x + src * LEN);
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) v[j] = xr[64 * j + lane];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        ss = __builtin_fmaf(v[j].x, v[j].x, ss);
        ss = __builtin_fmaf(v[j].y, v[j].y, ss);
        ss = __builtin_fmaf(v[j].z, v[j].z, ss);
        ss = __builtin_fmaf(v[j].w, v[j].w, ss);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o, 64));
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)LEN), eps)));
    float4 *o = (float4 *)(out + r * LEN);
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int64_t i = 4 * (64 * j + lane);
        float e[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            e[q] = __fmul_rn(e[q], inv);
            if (wlen > 0) e[q] = __fmul_rn(e[q], gemma ? __fadd_rn(1.0f, w[i + q]) : w[i + q]);
        }
        o[64 * j + lane] = make_float4(e[0], e[1], e[2], e[3]);
    }
}

// RMS norm of rows (tensor.zig:1167-1179) written straight into the tiled
// GEMM's two-term bf16 A fragments ([n/16][ldk][2][64 lanes] x 16 bytes,
// columns past len are zero) and, when `out` is given, as f32 rows too. One
// block per 16 rows: the inverse RMS of each row first (a wave per 4 rows),
// then one (k tile, lane) fragment word pair per thread step.
__global__ __launch_bounds__(256) void rmsnorm_split_kernel(u32x4 *xs, int64_t ldk, float *out, const float *x,
                                                            const float *w, int64_t wlen, int64_t len, float eps,
                                                            int gemma, int64_t n) {
    __shared__ float inv_s[16];
    const int64_t m16 = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool vec = (len % 4) == 0;  // rows of whole float4s (the bases are 16-byte aligned)
    for (int rr = 0; rr < 4; rr++) {
        const int row = wave * 4 + rr;
        const int64_t r = m16 * 16 + row;
        float ss = 0.f;
        if (r < n) {
            const float *xr = x + r * len;
            if (vec) {
                for (int64_t i = 4 * lane; i < len; i += 256) {
                    float4 v = *(const float4 *)(xr + i);
                    ss = __builtin_fmaf(v.x, v.x, ss);
                    ss = __builtin_fmaf(v.y, v.y, ss);
                    ss = __builtin_fmaf(v.z, v.z, ss);
                    ss = __builtin_fmaf(v.w, v.w, ss);
                }
            } else {
                for (int64_t i = lane; i < len; i += 64) ss = __builtin_fmaf(xr[i], xr[i], ss);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o, 64));
        if (lane == 0)
            inv_s[row] = r < n ? __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)len), eps))) : 0.f;
    }
    __syncthreads();
    for (int64_t q = threadIdx.x; q < ldk * 64; q += 256) {
        const int64_t kt = q >> 6;
        const int l = (int)(q & 63), row = l & 15;
        const int64_t r = m16 * 16 + row;
        const int64_t k0 = kt * 32 + 8 * (l >> 4);
        const float inv = inv_s[row];
        float xv[8], wv[8];
        if (r < n && vec && k0 + 8 <= len) {
            float4 a = *(const float4 *)(x + r * len + k0), b = *(const float4 *)(x + r * len + k0 + 4);
            xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w; xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) xv[j] = (r < n && k0 + j < len) ? x[r * len + k0 + j] : 0.f;
        }
        if (wlen > 0 && (wlen % 4) == 0 && k0 + 8 <= wlen) {
            float4 a = *(const float4 *)(w + k0), b = *(const float4 *)(w + k0 + 4);
            wv[0] = a.x; wv[1] = a.y; wv[2] = a.z; wv[3] = a.w; wv[4] = b.x; wv[5] = b.y; wv[6] = b.z; wv[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) wv[j] = (wlen > 0 && k0 + j < wlen) ? w[k0 + j] : 1.f;
        }
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float y = 0.f;
            if (r < n && k0 + j < len) {
                y = __fmul_rn(xv[j], inv);
                if (wlen > 0) y = __fmul_rn(y, gemma ? __fadd_rn(1.0f, wv[j]) : wv[j]);
            }
            v[j] = y;
        }
        if (out && r < n) {
            if (vec && k0 + 8 <= len) {
                *(float4 *)(out + r * len + k0) = make_float4(v[0], v[1], v[2], v[3]);
                *(float4 *)(out + r * len + k0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (k0 + j < len) out[r * len + k0 + j] = v[j];
            }
        }
        u32x4 words[2];
        a_words<false, 2>(v, words);
        xs[((m16 * ldk + kt) * 2 + 0) * 64 + l] = words[0];
        xs[((m16 * ldk + kt) * 2 + 1) * 64 + l] = words[1];
    }
}

// RMSNorm of 16 rows per block written as the MX fragments of a scaled-MFMA
// product (and, when `out`, as f32 rows). Pass 1: each wave sums the squares
// of 4 rows with 16 loads in flight. Pass 2: 512 columns at a time, the 16
// rows are staged in LDS by coalesced loads, then each thread normalises one
// lane slot (a token's 32-column E8M0 block) of one of the chunk's 4 stages.
constexpr int RS_CHUNK = 512;  // columns per LDS chunk: 4 stages of 128
__global__ __launch_bounds__(256) void rmsnorm_split_mx_kernel(uint8_t *xm, int64_t ldst, float *out, const float *x,
                                                               const float *w, int64_t wlen, int64_t len, float eps,
                                                               int gemma, int64_t n) {
    __shared__ float inv_s[16];
    __shared__ float chunk[16][RS_CHUNK + 4];
    const int64_t m16 = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool vec = (len % 4) == 0 && ((uintptr_t)x & 15) == 0;
    {
        float ss[4] = {0.f, 0.f, 0.f, 0.f};
        const int64_t r0 = m16 * 16 + wave * 4;
        if (vec) {
            for (int64_t i0 = 4 * lane; i0 < len; i0 += 1024) {
                float4 v[4][4];
#pragma unroll
                for (int rr = 0; rr < 4; rr++)
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int64_t i = i0 + 256 * u;
                        v[rr][u] = (r0 + rr < n && i < len) ? *(const float4 *)(x + (r0 + rr) * len + i)
                                                            : make_float4(0.f, 0.f, 0.f, 0.f);
                    }
#pragma unroll
                for (int rr = 0; rr < 4; rr++)
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        ss[rr] = __builtin_fmaf(v[rr][u].x, v[rr][u].x, ss[rr]);
                        ss[rr] = __builtin_fmaf(v[rr][u].y, v[rr][u].y, ss[rr]);
                        ss[rr] = __builtin_fmaf(v[rr][u].z, v[rr][u].z, ss[rr]);
                        ss[rr] = __builtin_fmaf(v[rr][u].w, v[rr][u].w, ss[rr]);
                    }
            }
        } else {
#pragma unroll
            for (int rr = 0; rr < 4; rr++)
                if (r0 + rr < n)
                    for (int64_t i = lane; i < len; i += 64)
                        ss[rr] = __builtin_fmaf(x[(r0 + rr) * len + i], x[(r0 + rr) * len + i], ss[rr]);
        }
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            float t = ss[rr];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) t = __fadd_rn(t, __shfl_xor(t, o, 64));
            if (lane == 0)
                inv_s[wave * 4 + rr] =
                    r0 + rr < n ? __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(t, (float)len), eps))) : 0.f;
        }
    }
    __syncthreads();
    const int st_l = threadIdx.x >> 6, l = lane, row = l & 15, kb = l >> 4;
    const int64_t r = m16 * 16 + row;
    const float inv = inv_s[row];
    // the 16 rows' columns c0 .. c0 + 512 (zero past the matrix), 8 float4
    // a thread; chunk c + 1 is loaded into registers while chunk c is split
    constexpr int QT = 16 * RS_CHUNK / 4 / 256;
    auto fetch = [&](int64_t c0, float4 (&buf)[QT]) {
#pragma unroll
        for (int j = 0; j < QT; j++) {
            const int q = threadIdx.x + 256 * j;
            const int qr = q / (RS_CHUNK / 4), qc = (q % (RS_CHUNK / 4)) * 4;
            const int64_t rq = m16 * 16 + qr, k = c0 + qc;
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
            if (rq < n) {
                if (vec && k + 4 <= len) a = *(const float4 *)(x + rq * len + k);
                else {
                    a.x = k < len ? x[rq * len + k] : 0.f;
                    a.y = k + 1 < len ? x[rq * len + k + 1] : 0.f;
                    a.z = k + 2 < len ? x[rq * len + k + 2] : 0.f;
                    a.w = k + 3 < len ? x[rq * len + k + 3] : 0.f;
                }
            }
            buf[j] = a;
        }
    };
    float4 pre[QT];
    fetch(0, pre);
    for (int64_t c0 = 0; c0 < ldst * 128; c0 += RS_CHUNK) {
#pragma unroll
        for (int j = 0; j < QT; j++) {
            const int q = threadIdx.x + 256 * j;
            *(float4 *)&chunk[q / (RS_CHUNK / 4)][(q % (RS_CHUNK / 4)) * 4] = pre[j];
        }
        __syncthreads();
        if (c0 + RS_CHUNK < ldst * 128) fetch(c0 + RS_CHUNK, pre);
        const int64_t st = c0 / 128 + st_l;
        if (st < ldst) {
            const int kl = st_l * 128 + kb * 32;
            const int64_t k0 = c0 + kl;
            float v[32];
#pragma unroll
            for (int j = 0; j < 32; j += 4) {
                const float4 a = *(const float4 *)&chunk[row][kl + j];
                float4 b = make_float4(1.f, 1.f, 1.f, 1.f);
                if (wlen > 0 && (wlen % 4) == 0 && k0 + j + 4 <= wlen) b = *(const float4 *)(w + k0 + j);
                else if (wlen > 0) {
                    b.x = k0 + j < wlen ? w[k0 + j] : 1.f;
                    b.y = k0 + j + 1 < wlen ? w[k0 + j + 1] : 1.f;
                    b.z = k0 + j + 2 < wlen ? w[k0 + j + 2] : 1.f;
                    b.w = k0 + j + 3 < wlen ? w[k0 + j + 3] : 1.f;
                }
                const float xa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    float y = 0.f;
                    if (r < n && k0 + j + u < len) {
                        y = __fmul_rn(xa[u], inv);
                        if (wlen > 0) y = __fmul_rn(y, gemma ? __fadd_rn(1.0f, wb[u]) : wb[u]);
                    }
                    v[j + u] = y;
                }
            }
            if (out && r < n) {
                if (vec && k0 + 32 <= len) {
#pragma unroll
                    for (int j = 0; j < 32; j += 4)
                        *(float4 *)(out + r * len + k0 + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 32; j++)
                        if (k0 + j < len) out[r * len + k0 + j] = v[j];
                }
            }
            mx_write_slot(v, xm + (m16 * ldst + st) * MX_BLOCK, l);
        }
        __syncthreads();
    }
}

// The same as rmsnorm_split_kernel with each row read once: wave w of 16
// holds row 16 m16 + w in registers (lane l: columns 1024 j + 16 l .. +16,
// j < NPH), sums its squares with a butterfly over the wave, normalises, and
// writes each phase's two-term words (32 k tiles) into LDS in fragment
// order; the workgroup then copies the phase's 64 KiB to the fragments in
// whole 16-byte words.
template <int NPH>
__global__ __launch_bounds__(1024) void rmsnorm_split_rows_kernel(u32x4 *xs, int64_t ldk, float *out, const float *x,
                                                                  const float *w, int64_t wlen, int64_t len,
                                                                  float eps, int gemma, int64_t n) {
    __shared__ u32x4 phase_buf[32 * 2 * 64];  // [k tile][term][lane], 64 KiB
    const int64_t m16 = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r = m16 * 16 + wave;
    const bool row_in = r < n;
    const bool vec = (len % 4) == 0 && ((uintptr_t)x & 15) == 0;
    float xv[NPH][16];
#pragma unroll
    for (int j = 0; j < NPH; j++) {
        const int64_t k0 = 1024 * j + 16 * lane;
        if (row_in && vec && k0 + 16 <= len) {
#pragma unroll
            for (int q = 0; q < 16; q += 4) {
                const float4 a = *(const float4 *)(x + r * len + k0 + q);
                xv[j][q] = a.x; xv[j][q + 1] = a.y; xv[j][q + 2] = a.z; xv[j][q + 3] = a.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 16; q++) xv[j][q] = row_in && k0 + q < len ? x[r * len + k0 + q] : 0.f;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NPH; j++)
#pragma unroll
        for (int q = 0; q < 16; q++) ss = __builtin_fmaf(xv[j][q], xv[j][q], ss);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o, 64));
    const float inv = row_in ? __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)len), eps))) : 0.f;
#pragma unroll
    for (int j = 0; j < NPH; j++) {
        const int64_t kt0 = 32 * j;
        if (kt0 >= ldk) break;
        const int64_t k0 = 1024 * j + 16 * lane;
        float v[16];
#pragma unroll
        for (int q = 0; q < 16; q += 4) {
            float4 b = make_float4(1.f, 1.f, 1.f, 1.f);
            if (wlen > 0 && (wlen % 4) == 0 && k0 + q + 4 <= wlen) b = *(const float4 *)(w + k0 + q);
            else if (wlen > 0) {
                b.x = k0 + q < wlen ? w[k0 + q] : 1.f;
                b.y = k0 + q + 1 < wlen ? w[k0 + q + 1] : 1.f;
                b.z = k0 + q + 2 < wlen ? w[k0 + q + 2] : 1.f;
                b.w = k0 + q + 3 < wlen ? w[k0 + q + 3] : 1.f;
            }
            const float wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float y = 0.f;
                if (row_in && k0 + q + u < len) {
                    y = __fmul_rn(xv[j][q + u], inv);
                    if (wlen > 0) y = __fmul_rn(y, gemma ? __fadd_rn(1.0f, wb[u]) : wb[u]);
                }
                v[q + u] = y;
            }
        }
        if (out && row_in) {
            if (vec && k0 + 16 <= len) {
#pragma unroll
                for (int q = 0; q < 16; q += 4) *(float4 *)(out + r * len + k0 + q) = make_float4(v[q], v[q + 1], v[q + 2], v[q + 3]);
            } else {
#pragma unroll
                for (int q = 0; q < 16; q++)
                    if (k0 + q < len) out[r * len + k0 + q] = v[q];
            }
        }
        // k tile kt0 + lane / 2, its 8-column chunks 2 (lane % 2) and 2 (lane % 2) + 1
        const int ktl = lane >> 1;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            float v8[8];
#pragma unroll
            for (int q = 0; q < 8; q++) v8[q] = v[8 * c + q];
            u32x4 words[2];
            a_words<false, 2>(v8, words);
            const int slot = wave + 16 * (2 * (lane & 1) + c);
            phase_buf[(ktl * 2 + 0) * 64 + slot] = words[0];
            phase_buf[(ktl * 2 + 1) * 64 + slot] = words[1];
        }
        __syncthreads();
        const int64_t nkt = ldk - kt0 < 32 ? ldk - kt0 : 32;
        u32x4 *dst = xs + (m16 * ldk + kt0) * 2 * 64;
        for (int64_t i = threadIdx.x; i < nkt * 128; i += 1024) dst[i] = phase_buf[i];
        __syncthreads();
    }
}

// RMSNorm of 8 rows written as MX fragments, each row read once: wave w of
// 8 holds row 16 m16 + 8 h + w (h = blockIdx.x % 2: the two halves of a
// 16-token block) in registers (lane l: 32-column blocks l + 64 j, j < NB),
// sums its squares with a butterfly over the wave, normalises, and splits its
// blocks into fp6 terms into LDS, 16 stages (64 blocks) a phase, in a copy
// of the fragment layout that holds only the half's 32 slots; the workgroup
// then writes them to their slots (128-byte runs). Two workgroups fit a CU,
// so one's loads overlap the other's splits. (The two-pass kernel above
// reads every row twice: once for the sum of squares, once for the split.)
template <int NB>
__global__ __launch_bounds__(512) void rmsnorm_split_mx_rows_kernel(uint8_t *xm, int64_t ldst, const float *x,
                                                                    const float *w, int64_t wlen, int64_t len,
                                                                    float eps, int gemma, int64_t n) {
    constexpr int HS = 32;                         // slots of a half block
    constexpr int HB = 25 * MX_TERMS * HS;         // bytes of a half block: 16 + 8 per term and slot, + scale words
    __shared__ u32x4 stage_buf[16 * HB / 16];      // 16 stages, 50 KiB
    const int64_t m16 = blockIdx.x >> 1;
    const int half = blockIdx.x & 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r = m16 * 16 + half * 8 + wave;
    const bool row_in = r < n;
    const bool vec = (len % 4) == 0 && ((uintptr_t)x & 15) == 0;
    float xv[NB][32];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int64_t k0 = (int64_t)(lane + 64 * j) * 32;
        if (row_in && vec && k0 + 32 <= len) {
#pragma unroll
            for (int q = 0; q < 32; q += 4) {
                const float4 a = *(const float4 *)(x + r * len + k0 + q);
                xv[j][q] = a.x; xv[j][q + 1] = a.y; xv[j][q + 2] = a.z; xv[j][q + 3] = a.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 32; q++) xv[j][q] = row_in && k0 + q < len ? x[r * len + k0 + q] : 0.f;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int q = 0; q < 32; q++) ss = __builtin_fmaf(xv[j][q], xv[j][q], ss);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, o, 64));
    const float inv = row_in ? __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)len), eps))) : 0.f;
    const int64_t nst = ldst;  // stages in the fragments
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int64_t st0 = 16 * j;
        if (st0 >= nst) break;
        // this lane's block: stage st0 + lane / 4, block lane % 4 of it
        const int64_t k0 = (int64_t)(lane + 64 * j) * 32;
        float v[32];
#pragma unroll
        for (int q = 0; q < 32; q += 4) {
            float4 b = make_float4(1.f, 1.f, 1.f, 1.f);
            if (wlen > 0 && (wlen % 4) == 0 && k0 + q + 4 <= wlen) b = *(const float4 *)(w + k0 + q);
            else if (wlen > 0) {
                b.x = k0 + q < wlen ? w[k0 + q] : 1.f;
                b.y = k0 + q + 1 < wlen ? w[k0 + q + 1] : 1.f;
                b.z = k0 + q + 2 < wlen ? w[k0 + q + 2] : 1.f;
                b.w = k0 + q + 3 < wlen ? w[k0 + q + 3] : 1.f;
            }
            const float wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float y = 0.f;
                if (row_in && k0 + q + u < len) {
                    y = __fmul_rn(xv[j][q + u], inv);
                    if (wlen > 0) y = __fmul_rn(y, gemma ? __fadd_rn(1.0f, wb[u]) : wb[u]);
                }
                v[q + u] = y;
            }
        }
        // half slot: token wave, block lane % 4 (fragment slot 8 half + wave + 16 (lane % 4))
        if (st0 + lane / 4 < nst)
            mx_write_slot<HS>(v, (uint8_t *)stage_buf + (lane / 4) * HB, wave + 8 * (lane % 4));
        __syncthreads();
        const int nphase = (int)(nst - st0 < 16 ? nst - st0 : 16);
        uint8_t *dst = xm + (m16 * ldst + st0) * MX_BLOCK;
        const uint8_t *src = (const uint8_t *)stage_buf;
        // per stage: 16 (term, block) runs of 8 slots in each of the two code
        // parts, 4 runs of 8 scale words
        for (int i = threadIdx.x; i < nphase * 16 * 8; i += 512) {
            const int st = i >> 7, run = (i >> 3) & 15, t = i & 7;
            const int e = run >> 2, kb = run & 3;
            const int hs = 8 * kb + t, fs = 8 * half + 16 * kb + t;  // half-block and fragment slot
            *(u32x4 *)(dst + st * MX_BLOCK + (64 * e + fs) * 16) = *(const u32x4 *)(src + st * HB + (HS * e + hs) * 16);
            *(uint2 *)(dst + st * MX_BLOCK + 4096 + (64 * e + fs) * 8) =
                *(const uint2 *)(src + st * HB + 16 * MX_TERMS * HS + (HS * e + hs) * 8);
            if (e == 0)
                *(uint32_t *)(dst + st * MX_BLOCK + 6144 + fs * 4) =
                    *(const uint32_t *)(src + st * HB + 24 * MX_TERMS * HS + hs * 4);
        }
        __syncthreads();
    }
}

__global__ void layernorm_kernel(float *out, const float *x, const float *w, int64_t wlen, const float *bias,
                                 int64_t len, float eps, int one_plus) {
    __shared__ float sh[8];
    int64_t r = blockIdx.x;
    const float *xr = x + r * len;
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) s += xr[i];
    float mean = __fdiv_rn(block_sum(s, sh), (float)len);
    float v2 = 0.f;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) {
        float d = __fsub_rn(xr[i], mean);
        v2 = __builtin_fmaf(d, d, v2);
    }
    float var = __fdiv_rn(block_sum(v2, sh), (float)len);
    float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
    float *o = out + r * len;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) {
        float y = __fmul_rn(__fsub_rn(xr[i], mean), inv);
        if (wlen > 0) y = __fmul_rn(y, one_plus ? __fadd_rn(1.0f, w[i]) : w[i]);
        if (bias) y = __fadd_rn(y, bias[i]);
        o[i] = y;
    }
}

// In-place softmax (tensor.zig:1181-1200).
__global__ void softmax_kernel(float *x, int64_t len) {
    __shared__ float sh[8];
    float *xr = x + (int64_t)blockIdx.x * len;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) m = fmaxf(m, xr[i]);
    m = block_max(m, sh);
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) {
        float e = exp_cephes(__fsub_rn(xr[i], m));
        xr[i] = e;
        s += e;
    }
    s = block_sum(s, sh);
    float inv = __fdiv_rn(1.0f, s);
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) xr[i] = __fmul_rn(xr[i], inv);
}

// log-softmax (tensor.zig:1203-1210): f32 max, f64 sum of exp, f32 x - lse.
// log-softmax and KL over long rows (tensor.zig:1203-1210, scorers.zig:
// 387-394), each row split into `S` chunks so that a few rows of a 128 k
// vocabulary still spread over every CU. The arithmetic is the reference's:
// the f32 row maximum m (exact in any order), then s = sum exp(f64(x - m))
// in f64 with x - m taken in f32, lse = m + f32(log s), out = x - lse.
//   pass 1  per chunk: its maximum                         -> part_m[row][S]
//   pass 2  per chunk: m = max of the row's part_m, the chunk's f64 sum
//                                                          -> part_s[row][S]
//   pass 3  per chunk: s = the row's part_s added in chunk order, lse, and
//           the chunk's outputs (log-probs, or the KL terms -> part_k)
//   pass 4  (KL only) per row: part_k added in chunk order.
struct RowSplit {
    int64_t len, chunk;
    int S;
};

__global__ __launch_bounds__(256) void rowsplit_max_kernel(float *part_m, const float *x, RowSplit rs) {
    __shared__ float sh[8];
    const int64_t row = blockIdx.y, c = blockIdx.x;
    const float *xr = x + row * rs.len;
    const int64_t i0 = c * rs.chunk, i1 = i0 + rs.chunk < rs.len ? i0 + rs.chunk : rs.len;
    float m = -INFINITY;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) m = fmaxf(m, xr[i]);
    m = block_max(m, sh);
    if (threadIdx.x == 0) part_m[row * rs.S + c] = m;
}

__device__ __forceinline__ float rowsplit_row_max(const float *part_m, int64_t row, int S) {
    float m = -INFINITY;
    for (int c = 0; c < S; c++) m = fmaxf(m, part_m[row * S + c]);
    return m;
}

__global__ __launch_bounds__(256) void rowsplit_sum_kernel(double *part_s, const float *part_m, const float *x,
                                                           RowSplit rs) {
    __shared__ double sh[8];
    const int64_t row = blockIdx.y, c = blockIdx.x;
    const float m = rowsplit_row_max(part_m, row, rs.S);
    const float *xr = x + row * rs.len;
    const int64_t i0 = c * rs.chunk, i1 = i0 + rs.chunk < rs.len ? i0 + rs.chunk : rs.len;
    double acc = 0.0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) acc += exp((double)__fsub_rn(xr[i], m));
    acc = block_sum_d(acc, sh);
    if (threadIdx.x == 0) part_s[row * rs.S + c] = acc;
}

__device__ __forceinline__ float rowsplit_lse(const double *part_s, const float *part_m, int64_t row, int S) {
    const float m = rowsplit_row_max(part_m, row, S);
    double s = 0.0;
    for (int c = 0; c < S; c++) s += part_s[row * S + c];
    return __fadd_rn(m, (float)log(s));
}

__global__ __launch_bounds__(256) void rowsplit_logsoftmax_kernel(float *out, const double *part_s,
                                                                  const float *part_m, const float *x, RowSplit rs) {
    const int64_t row = blockIdx.y, c = blockIdx.x;
    const float lse = rowsplit_lse(part_s, part_m, row, rs.S);
    const float *xr = x + row * rs.len;
    float *o = out + row * rs.len;
    const int64_t i0 = c * rs.chunk, i1 = i0 + rs.chunk < rs.len ? i0 + rs.chunk : rs.len;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) o[i] = __fsub_rn(xr[i], lse);
}

// KL terms of one chunk: sum exp(lb) (lb - lt) in f64 with lt = t - lse
// (scorers.zig:390-394)
__global__ __launch_bounds__(256) void rowsplit_kl_kernel(double *part_k, const double *part_s, const float *part_m,
                                                          const float *base, const float *trial, RowSplit rs) {
    __shared__ double sh[8];
    const int64_t row = blockIdx.y, c = blockIdx.x;
    const float lse = rowsplit_lse(part_s, part_m, row, rs.S);
    const float *tr = trial + row * rs.len, *br = base + row * rs.len;
    const int64_t i0 = c * rs.chunk, i1 = i0 + rs.chunk < rs.len ? i0 + rs.chunk : rs.len;
    double acc = 0.0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
        const double lb = (double)br[i];
        const double lt = (double)__fsub_rn(tr[i], lse);
        acc += exp(lb) * (lb - lt);
    }
    acc = block_sum_d(acc, sh);
    if (threadIdx.x == 0) part_k[row * rs.S + c] = acc;
}

__global__ void rowsplit_kl_total_kernel(double *kl, const double *part_k, int64_t n, int S) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n) return;
    double s = 0.0;
    for (int c = 0; c < S; c++) s += part_k[row * S + c];
    kl[row] = s;
}

// out[i][j] = act(gate[i][j]) * up[i][j] (tensor.zig:1296-1337)
__global__ void gated_act_kernel(uint32_t act, float *out, const float *gate, const float *up, int64_t n, int64_t len,
                                 int64_t in_stride, int64_t out_stride) {
    int64_t total = n * len;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i / len, j = i % len;
        float v = act_apply(act, gate[r * in_stride + j]);
        if (up) v = __fmul_rn(v, up[r * in_stride + j]);
        out[r * out_stride + j] = v;
    }
}

// RoPE (tensor.zig:1360-1381) of n head vectors at pos[i].
__global__ void rope_kernel(float *x, int64_t n, int64_t dim, const float *cos_t, const float *sin_t, int64_t half,
                            const uint32_t *pos, uint32_t style) {
    int64_t hd = dim / 2;
    int64_t total = n * hd;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = t / hd, i = t % hd;
        float c = cos_t[(int64_t)pos[r] * half + i], s = sin_t[(int64_t)pos[r] * half + i];
        float *row = x + r * dim;
        int64_t a = style == DITCH_ROPE_GPTJ ? 2 * i : i, b = style == DITCH_ROPE_GPTJ ? 2 * i + 1 : i + hd;
        float x1 = row[a], x2 = row[b];
        row[a] = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
        row[b] = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
    }
}

// scores[p] = scale * dot(q, k[p]) (tensor.zig:1126-1144): one wave per key.
__global__ void attn_scores_kernel(float *scores, int64_t n_keys, const float *q, int64_t hd, const float *k,
                                   int64_t stride, float scale) {
    int lane = threadIdx.x & 63;
    int64_t p = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (p >= n_keys) return;
    float a = 0.f;
    for (int64_t d = lane; d < hd; d += 64) a = __builtin_fmaf(k[p * stride + d], q[d], a);
    a = wave_sum(a);
    if (lane == 0) scores[p] = __fmul_rn(a, scale);
}

// out[j] = sum_p scores[p] v[p][j] (tensor.zig:1148-1160)
__global__ void attn_values_kernel(float *out, int64_t vd, const float *scores, int64_t n_keys, const float *v,
                                   int64_t stride) {
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= vd) return;
    float a = 0.f;
    for (int64_t p = 0; p < n_keys; p++) a = __builtin_fmaf(v[p * stride + j], scores[p], a);
    out[j] = a;
}

// Row norms of a resident weight: one block per row.
__global__ void row_norms_kernel(float *out, TileView w) {
    __shared__ float sh[8];
    int64_t r = blockIdx.x;
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < w.cols; c += blockDim.x) {
        uint16_t b;
        float v = tiled_element_f32(w, r, c, &b);
        s = __builtin_fmaf(v, v, s);
    }
    s = block_sum(s, sh);
    if (threadIdx.x == 0) out[r] = __fsqrt_rn(s);
}

// xa[i][j] = dot(a_j, x_i) for the low-rank delta (tensor.zig:1036-1042)
// (a wave per row and 4 directions: delta_dot4)
__global__ void delta_xa_kernel(float *xa, const float *x, const float *a, int64_t n, int64_t cols, int64_t rank) {
    int lane = threadIdx.x & 63;
    const int64_t nb = (rank + 3) / 4;
    int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (t >= n * nb) return;
    const int64_t i = t / nb, j0 = (t % nb) * 4;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    delta_dot4(x + i * cols, a, cols, j0, rank, lane, s);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const float v = wave_sum(s[jj]);
        if (lane == 0 && j0 + jj < rank) xa[i * rank + j0 + jj] = v;
    }
}

// The same with A staged in LDS once per workgroup of 8 rows (one wave a
// row and its 4-direction blocks): the waves then read A from LDS instead
// of all of them fetching the same lines from L2.
__global__ __launch_bounds__(512) void delta_xa_lds_kernel(float *xa, const float *x, const float *a, int64_t n,
                                                           int64_t cols, int64_t rank) {
    extern __shared__ float4 a_lds4[];
    const float4 *a4 = (const float4 *)a;
    const int64_t n4 = rank * cols / 4;
    for (int64_t t = threadIdx.x; t < n4; t += blockDim.x) a_lds4[t] = a4[t];
    __syncthreads();
    const float *al = (const float *)a_lds4;
    const int lane = threadIdx.x & 63;
    const int64_t i = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (i >= n) return;
    for (int64_t j0 = 0; j0 < rank; j0 += 4) {
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        delta_dot4(x + i * cols, al, cols, j0, rank, lane, s);
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const float v = wave_sum(s[jj]);
            if (lane == 0 && j0 + jj < rank) xa[i * rank + j0 + jj] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Launchers

void launch_rmsnorm(float *out, const float *x, const float *w, int64_t wlen, int64_t n, int64_t len, float eps,
                    int gemma, hipStream_t s, const int64_t *row_index, int64_t n_src) {
    if (n <= 0) return;
    const int64_t ns = row_index ? n_src : n;
    const dim3 g4((unsigned)((n + 3) / 4));
    // rows of whole 256-column steps up to 4096, 16-byte aligned: a wave per row
    const bool rows = len % 256 == 0 && len <= 4096 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)out & 15) == 0;
    if (rows && len == 512) hipLaunchKernelGGL(rmsnorm_rows_kernel<2>, g4, dim3(256), 0, s, out, x, w, wlen, n, eps, gemma, row_index, ns);
    else if (rows && len == 1024) hipLaunchKernelGGL(rmsnorm_rows_kernel<4>, g4, dim3(256), 0, s, out, x, w, wlen, n, eps, gemma, row_index, ns);
    else if (rows && len == 2048) hipLaunchKernelGGL(rmsnorm_rows_kernel<8>, g4, dim3(256), 0, s, out, x, w, wlen, n, eps, gemma, row_index, ns);
    else if (rows && len == 4096) hipLaunchKernelGGL(rmsnorm_rows_kernel<16>, g4, dim3(256), 0, s, out, x, w, wlen, n, eps, gemma, row_index, ns);
    else
        hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)n), dim3(256), 0, s, out, x, w, wlen, len, eps, gemma,
                           row_index, ns, len, len);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_rmsnorm_split(void *xs, int64_t ldk, float *out, const float *x, const float *w, int64_t wlen, int64_t n,
                          int64_t len, float eps, int gemma, hipStream_t s) {
    if (n <= 0) return;
    DITCH_CHECK(ldk * 32 >= len, DITCH_INVALID_ARGUMENT, "rmsnorm_split: fragments shorter than the row");
    const dim3 grid((unsigned)((n + 15) / 16));
    // rows up to 4096 columns (fragments up to 128 k tiles): one read of each row
    if (ldk <= 32) hipLaunchKernelGGL(rmsnorm_split_rows_kernel<1>, grid, dim3(1024), 0, s, (u32x4 *)xs, ldk, out, x, w, wlen, len, eps, gemma, n);
    else if (ldk <= 64) hipLaunchKernelGGL(rmsnorm_split_rows_kernel<2>, grid, dim3(1024), 0, s, (u32x4 *)xs, ldk, out, x, w, wlen, len, eps, gemma, n);
    else if (ldk <= 128) hipLaunchKernelGGL(rmsnorm_split_rows_kernel<4>, grid, dim3(1024), 0, s, (u32x4 *)xs, ldk, out, x, w, wlen, len, eps, gemma, n);
    else hipLaunchKernelGGL(rmsnorm_split_kernel, grid, dim3(256), 0, s, (u32x4 *)xs, ldk, out, x, w, wlen, len, eps, gemma, n);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_rmsnorm_split_mx(void *xm, int64_t ldst, float *out, const float *x, const float *w, int64_t wlen,
                             int64_t n, int64_t len, float eps, int gemma, hipStream_t s) {
    if (n <= 0) return;
    DITCH_CHECK(ldst * 128 >= len, DITCH_INVALID_ARGUMENT, "rmsnorm_split_mx: fragments shorter than the row");
    if (!out && ldst <= 32) {  // rows up to 4096 columns, no f32 copy asked: one read of each row
        hipLaunchKernelGGL(rmsnorm_split_mx_rows_kernel<2>, dim3((unsigned)((n + 15) / 16 * 2)), dim3(512), 0, s,
                           (uint8_t *)xm, ldst, x, w, wlen, len, eps, gemma, n);
    } else {
        hipLaunchKernelGGL(rmsnorm_split_mx_kernel, dim3((unsigned)((n + 15) / 16)), dim3(256), 0, s, (uint8_t *)xm,
                           ldst, out, x, w, wlen, len, eps, gemma, n);
    }
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_rmsnorm_strided(float *out, const float *x, const float *w, int64_t wlen, int64_t n, int64_t len,
                            int64_t in_stride, int64_t out_stride, float eps, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)n), dim3(256), 0, s, out, x, w, wlen, len, eps, 0, nullptr, n,
                       in_stride, out_stride);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_layernorm(float *out, const float *x, const float *w, int64_t wlen, const float *bias, int64_t n,
                      int64_t len, float eps, int one_plus, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(layernorm_kernel, dim3((unsigned)n), dim3(256), 0, s, out, x, w, wlen, bias, len, eps, one_plus);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_softmax_rows(float *x, int64_t n, int64_t len, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)n), dim3(256), 0, s, x, len);
    DITCH_TRY_HIP(hipGetLastError());
}
// Chunks per row: enough workgroups to cover the CUs about twice, chunks
// of at least 2048 elements.
static RowSplit row_split(int64_t n, int64_t len) {
    int64_t S = (512 + n - 1) / n;
    const int64_t most = (len + 2047) / 2048;
    S = S < most ? S : most;
    S = S < 1 ? 1 : S;
    RowSplit rs;
    rs.len = len;
    rs.chunk = (len + S - 1) / S;
    rs.S = (int)((len + rs.chunk - 1) / rs.chunk);
    return rs;
}

// part_m [n][S] f32, part_s [n][S] f64 (and part_k [n][S] f64 for KL) in `tmp`
static void row_split_passes(const RowSplit &rs, const float *x, int64_t n, float *&pm, double *&ps, double **pk,
                             hipStream_t s, DevBuf *tmp) {
    const size_t cells = (size_t)n * rs.S;
    double *d = tmp->get<double>(3 * cells);
    ps = d;
    if (pk) *pk = d + cells;
    pm = (float *)(d + 2 * cells);
    dim3 grid((unsigned)rs.S, (unsigned)n);
    hipLaunchKernelGGL(rowsplit_max_kernel, grid, dim3(256), 0, s, pm, x, rs);
    DITCH_TRY_HIP(hipGetLastError());
    hipLaunchKernelGGL(rowsplit_sum_kernel, grid, dim3(256), 0, s, ps, pm, x, rs);
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_log_softmax_rows(float *out, const float *x, int64_t n, int64_t len, hipStream_t s, DevBuf *tmp) {
    if (n <= 0 || len <= 0) return;
    DITCH_CHECK(n <= 65535, DITCH_UNSUPPORTED, "log-softmax: more than 65535 rows in one call");
    const RowSplit rs = row_split(n, len);
    float *pm;
    double *ps;
    row_split_passes(rs, x, n, pm, ps, nullptr, s, tmp);
    hipLaunchKernelGGL(rowsplit_logsoftmax_kernel, dim3((unsigned)rs.S, (unsigned)n), dim3(256), 0, s, out, ps, pm, x,
                       rs);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_kl_rows(double *kl, const float *base, const float *trial, int64_t n, int64_t vocab, hipStream_t s,
                    DevBuf *tmp) {
    if (n <= 0) return;
    DITCH_CHECK(n <= 65535, DITCH_UNSUPPORTED, "KL: more than 65535 rows in one call");
    DITCH_CHECK(vocab > 0, DITCH_INVALID_ARGUMENT, "KL: empty rows");
    const RowSplit rs = row_split(n, vocab);
    float *pm;
    double *ps, *pk;
    row_split_passes(rs, trial, n, pm, ps, &pk, s, tmp);
    hipLaunchKernelGGL(rowsplit_kl_kernel, dim3((unsigned)rs.S, (unsigned)n), dim3(256), 0, s, pk, ps, pm, base, trial,
                       rs);
    DITCH_TRY_HIP(hipGetLastError());
    hipLaunchKernelGGL(rowsplit_kl_total_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kl, pk, n, rs.S);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_gated_act(uint32_t act, float *out, const float *gate, const float *up, int64_t n, int64_t len,
                      int64_t in_stride, int64_t out_stride, hipStream_t s) {
    if (n * len <= 0) return;
    hipLaunchKernelGGL(gated_act_kernel, dim3(grid_1d(n * len)), dim3(256), 0, s, act, out, gate, up, n, len,
                       in_stride, out_stride);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_rope_rows(float *x, int64_t n, int64_t dim, const float *cos_t, const float *sin_t, int64_t half,
                      const uint32_t *pos, uint32_t style, hipStream_t s) {
    if (n * dim <= 0) return;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_1d(n * dim / 2)), dim3(256), 0, s, x, n, dim, cos_t, sin_t, half, pos,
                       style);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_attention_scores(float *scores, int64_t n_keys, const float *q, int64_t hd, const float *k,
                             int64_t stride, float scale, hipStream_t s) {
    if (n_keys <= 0) return;
    hipLaunchKernelGGL(attn_scores_kernel, dim3((unsigned)((n_keys + 3) / 4)), dim3(256), 0, s, scores, n_keys, q, hd,
                       k, stride, scale);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_attention_values(float *out, int64_t vd, const float *scores, int64_t n_keys, const float *v,
                             int64_t stride, hipStream_t s) {
    if (vd <= 0) return;
    hipLaunchKernelGGL(attn_values_kernel, dim3(grid_1d(vd)), dim3(256), 0, s, out, vd, scores, n_keys, v, stride);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_row_norms(float *out, const TileView &w, hipStream_t s) {
    if (w.rows <= 0) return;
    hipLaunchKernelGGL(row_norms_kernel, dim3((unsigned)w.rows), dim3(256), 0, s, out, w);
    DITCH_TRY_HIP(hipGetLastError());
}
void launch_delta_xa(float *xa, const float *x, const float *a, int64_t n, int64_t cols, int64_t rank, hipStream_t s) {
    if (n * rank <= 0) return;
    const size_t abytes = (size_t)(rank * cols) * 4;
    if (n >= 64 && (cols & 3) == 0 && (((uintptr_t)x | (uintptr_t)a) & 15) == 0 && abytes <= 65536) {
        static const bool attr = [] {
            return hipFuncSetAttribute((const void *)delta_xa_lds_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       65536) == hipSuccess;
        }();
        if (attr) {
            hipLaunchKernelGGL(delta_xa_lds_kernel, dim3((unsigned)((n + 7) / 8)), dim3(512), abytes, s, xa, x, a, n,
                               cols, rank);
            DITCH_TRY_HIP(hipGetLastError());
            return;
        }
    }
    const int64_t waves = n * ((rank + 3) / 4);
    hipLaunchKernelGGL(delta_xa_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, xa, x, a, n, cols, rank);
    DITCH_TRY_HIP(hipGetLastError());
}

}  // namespace ditch
