// model.hip — the resident forward pass (model.zig:4619-4959), routed MoE
// (moe.zig:998-1228) and DeepSeek MLA (model.zig:3292-3342) over weights
// registered in HBM. Activations stay on the device for the whole call.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <memory>

#include "decode.h"
#include "internal.h"
#include "attention_rope.h"
#include "tiled.h"
#include "model.h"

namespace ditch {


static int grid_for(int64_t total, int block = 256) {
    int64_t g = (total + block - 1) / block;
    if (g > 65536) g = 65536;
    return g < 1 ? 1 : (int)g;
}

// ---------------------------------------------------------------------------
// Kernels

// x[i] = embedding row tokens[i] widened to f32 (model.zig:4673-4675).
__global__ void embed_kernel(float *x, TileView w, const uint32_t *tokens, int64_t n) {
    int64_t total = n * w.cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i / w.cols, c = i % w.cols;
        int64_t t = (int64_t)tokens[r];
        t = t < w.rows ? t : w.rows - 1;  // ids are checked on the host; clamp device-side inputs
        uint16_t b;
        x[i] = tiled_element_f32(w, t, c, &b);
    }
}

// residuals[entry][ci] = x[capture_rows[ci]] (model.zig:4856-4862)
__global__ void capture_kernel(float *res, const float *x, const uint64_t *rows, int64_t n_capture, int64_t hidden,
                               int64_t n) {
    int64_t total = n_capture * hidden;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t ci = i / hidden, c = i % hidden;
        const uint64_t ru = rows[ci];
        const int64_t r = ru < (uint64_t)n ? (int64_t)ru : n - 1;
        res[i] = x[r * hidden + c];
    }
}

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Per row: q/k head RMSNorm (qwen3 "head"), RoPE of [off, off + rot) of every
// head, and the k/v rows written into the cache slot (b, pos)
// (model.zig:4253-4295). One block per row, one wave per head.
struct RopeArgs {
    float *q, *k;
    const float *v;
    float *kc, *vc;
    const ditch_row *rows;
    const float *cos_t, *sin_t;
    const float *q_norm, *k_norm;
    int64_t n, heads, kv_heads, hd, rope_off, rot, half, rope_len, T, kvd, nb;
    float eps;
    int style;
    // the whole-prompt attention rotates the queries itself when *dense is
    // set (q_in_attn: head_dim 128, whole-head neox, no query norm): the
    // query heads are then left as they are
    const int *dense;
    int q_in_attn;
};

// One head vector: optional RMSNorm (x * inv * w, tensor.zig:1167-1179), then
// RoPE of [rope_off, rope_off + rot) on the normalised values. Every element
// is read and then written by exactly one lane, after the wave has reduced
// the sum of squares, so the update is in place without a hazard. `dst2`
// (the cache slot of a key head) receives the same values.
__device__ void head_norm_rope(float *x, float *dst2, const float *nw, const RopeArgs &a, int64_t pos) {
    int lane = threadIdx.x & 63;
    float inv = 1.0f;
    if (nw) {
        float ss = 0.f;
        for (int64_t d = lane; d < a.hd; d += 64) ss = __builtin_fmaf(x[d], x[d], ss);
        ss = wave_sum64(ss);
        inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)a.hd), a.eps)));
    }
    auto val = [&](int64_t d) { return nw ? __fmul_rn(__fmul_rn(x[d], inv), nw[d]) : x[d]; };
    int64_t r0 = a.rot > 0 ? a.rope_off : a.hd, r1 = a.rot > 0 ? a.rope_off + 2 * a.half : a.hd;
    // coordinates outside the rotated range
    for (int64_t d = lane; d < a.hd; d += 64) {
        if (d >= r0 && d < r1) continue;
        float v = val(d);
        x[d] = v;
        if (dst2) dst2[d] = v;
    }
    if (a.rot > 0) {
        int64_t p = pos < a.rope_len - 1 ? pos : a.rope_len - 1;
        const float *cr = a.cos_t + p * a.half, *sr = a.sin_t + p * a.half;
        for (int64_t i = lane; i < a.half; i += 64) {
            int64_t ia = a.rope_off + (a.style == DITCH_ROPE_GPTJ ? 2 * i : i);
            int64_t ib = a.rope_off + (a.style == DITCH_ROPE_GPTJ ? 2 * i + 1 : i + a.half);
            float x1 = val(ia), x2 = val(ib), c = cr[i], s = sr[i];
            float ya = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
            float yb = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
            x[ia] = ya;
            x[ib] = yb;
            if (dst2) {
                dst2[ia] = ya;
                dst2[ib] = yb;
            }
        }
    }
}

// head_norm_rope for head_dim 128 rotated whole in neox order (element d and
// d + 64 form a pair, both held by lane d): HB heads of the wave at a time,
// every load of the group issued before the first use; the same operations
// in the same order as head_norm_rope.
template <int HB>
__device__ void heads_rope_128(const RopeArgs &a, int64_t i, int64_t pos, float *kd, int64_t h_first) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int64_t H = a.heads + a.kv_heads;
    const int64_t p = pos < a.rope_len - 1 ? pos : a.rope_len - 1;
    const float c = a.cos_t[p * 64 + lane], sn = a.sin_t[p * 64 + lane];
    for (int64_t h0 = h_first + (int64_t)wave * HB; h0 < H; h0 += (int64_t)nw * HB) {
        float x0[HB], x1[HB];
#pragma unroll
        for (int j = 0; j < HB; j++) {
            const int64_t h = h0 + j;
            x0[j] = x1[j] = 0.f;
            if (h < H) {
                const float *x = h < a.heads ? a.q + (i * a.heads + h) * 128 : a.k + (i * a.kv_heads + (h - a.heads)) * 128;
                x0[j] = x[lane];
                x1[j] = x[lane + 64];
            }
        }
#pragma unroll
        for (int j = 0; j < HB; j++) {
            const int64_t h = h0 + j;
            if (h >= H) continue;
            const bool qh = h < a.heads;
            const float *nwt = qh ? a.q_norm : a.k_norm;
            float v0 = x0[j], v1 = x1[j];
            if (nwt) {
                float ss = __builtin_fmaf(v1, v1, __builtin_fmaf(v0, v0, 0.f));
                ss = wave_sum64(ss);
                const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, 128.f), a.eps)));
                v0 = __fmul_rn(__fmul_rn(v0, inv), nwt[lane]);
                v1 = __fmul_rn(__fmul_rn(v1, inv), nwt[lane + 64]);
            }
            const float ya = __fsub_rn(__fmul_rn(v0, c), __fmul_rn(v1, sn));
            const float yb = __fadd_rn(__fmul_rn(v1, c), __fmul_rn(v0, sn));
            float *x = qh ? a.q + (i * a.heads + h) * 128 : a.k + (i * a.kv_heads + (h - a.heads)) * 128;
            x[lane] = ya;
            x[lane + 64] = yb;
            if (!qh) {
                float *d2 = kd + (h - a.heads) * 128;
                d2[lane] = ya;
                d2[lane + 64] = yb;
            }
        }
    }
}

__global__ void qk_rope_cache_kernel(RopeArgs a) {
    int64_t i = blockIdx.x;
    int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int64_t pos = a.rows[i].pos, b = a.rows[i].b;
    if (b >= a.nb || pos >= a.T) return;  // outside the KV cache: the row is skipped
    float *kd = a.kc + (b * a.T + pos) * a.kvd, *vd = a.vc + (b * a.T + pos) * a.kvd;
    if (a.hd == 128 && a.rope_off == 0 && a.rot == 128 && a.half == 64 && a.style == DITCH_ROPE_NEOX) {
        const bool keys_only = a.q_in_attn && *a.dense;
        heads_rope_128<4>(a, i, pos, kd, keys_only ? a.heads : 0);
        for (int64_t d = threadIdx.x; d < a.kvd; d += blockDim.x) vd[d] = a.v[i * a.kvd + d];
        return;
    }
    for (int64_t h = wave; h < a.heads + a.kv_heads; h += nw) {
        if (h < a.heads) {
            head_norm_rope(a.q + (i * a.heads + h) * a.hd, nullptr, a.q_norm, a, pos);
        } else {
            int64_t kh = h - a.heads;
            head_norm_rope(a.k + (i * a.kv_heads + kh) * a.hd, kd + kh * a.hd, a.k_norm, a, pos);
        }
    }
    for (int64_t d = threadIdx.x; d < a.kvd; d += blockDim.x) vd[d] = a.v[i * a.kvd + d];
}

// Causal attention of one (row, head) per wave (model.zig:2935-2986): scores
// for keys 0..pos of the row's prompt, softmax (Cephes exp, tensor.zig:
// 1181-1200), then the weighted sum of values. Output compacted to
// [n][heads][vd] (model.zig:4338-4345).
constexpr int ATT_MAXK = 1024;  // keys per row held in LDS

__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
    __shared__ float sc[4][ATT_MAXK];
    __shared__ float qs[4][512];
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int64_t task = (int64_t)blockIdx.x * 4 + wave;
    if (task >= a.n * a.heads) return;
    int64_t r = task / a.heads, h = task % a.heads;
    int64_t pos = a.rows[r].pos, b = a.rows[r].b;
    if (b >= a.nb || pos >= a.T) return;  // outside the KV cache: the row is skipped
    int64_t kvh = h / a.groups;
    const float *q = a.q + (r * a.heads + h) * a.hd;
    for (int64_t d = lane; d < a.hd; d += 64) qs[wave][d] = q[d];
    __builtin_amdgcn_wave_barrier();
    int64_t n_keys = pos + 1;
    const float *kb = a.kc + (b * a.T) * a.kvd + kvh * a.hd;
    const float *vb = a.vc + (b * a.T) * a.kvd + kvh * a.hd;
    float m = -INFINITY;
    for (int64_t p = lane; p < n_keys; p += 64) {
        const float *kr = kb + p * a.kvd;
        float s = 0.f;
        for (int64_t d = 0; d < a.hd; d++) s = __builtin_fmaf(kr[d], qs[wave][d], s);
        s = __fmul_rn(s, a.scale);
        sc[wave][p] = s;
        m = fmaxf(m, s);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float sum = 0.f;
    for (int64_t p = lane; p < n_keys; p += 64) {
        float e = exp_cephes(__fsub_rn(sc[wave][p], m));
        sc[wave][p] = e;
        sum += e;
    }
    sum = wave_sum64(sum);
    float inv = __fdiv_rn(1.0f, sum);
    __builtin_amdgcn_wave_barrier();
    float *o = a.out + (r * a.heads + h) * a.vd;
    for (int64_t d = lane; d < a.vd; d += 64) {
        float acc = 0.f;
        for (int64_t p = 0; p < n_keys; p++) acc = __builtin_fmaf(vb[p * a.kvd + d], __fmul_rn(sc[wave][p], inv), acc);
        o[d] = acc;
    }
}

// MLA: k = [kv_b nope | k_pe], v = [kv_b v | 0] per head (model.zig:3330-3341)
__global__ void mla_assemble_kernel(float *k, float *v, const float *kvb, const float *kva, int64_t n, int64_t heads,
                                    int64_t hd, int64_t nope, int64_t rd, int64_t vd, int64_t kv_lora) {
    int64_t total = n * heads * hd;
    int64_t kvr = kv_lora + rd, kvb_rows = heads * (nope + vd);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t t = i / (heads * hd), h = (i / hd) % heads, d = i % hd;
        const float *src = kvb + t * kvb_rows + h * (nope + vd);
        k[i] = d < nope ? src[d] : kva[t * kvr + kv_lora + (d - nope)];
        v[i] = d < vd ? src[nope + d] : 0.f;
    }
}

// MLA keys and values written straight into the KV cache, one block per row
// (the assembly of model.zig:3330-3341 and the RoPE of model.zig:4253-4295
// in one pass): head h's key is [kv_b nope part | k_pe], k_pe (the row's
// kv_a tail, shared by every head) rotated once per row; its value is [kv_b
// v part | 0]; the queries' rope coordinates are rotated in place. The same
// values as assembling k and v per head and rotating each head's copy of
// k_pe, without the two row-sized intermediates. Needs hd == nope + rd and
// every width a multiple of 4 (float4 rows).
struct MlaCacheArgs {
    float *q;
    const float *kvb, *kva;
    float *kc, *vc;
    const ditch_row *rows;
    const float *cos_t, *sin_t;
    int64_t heads, hd, nope, rd, vd, kv_lora, half, rope_len, T, nb, kvd;
    int style;
};

__global__ __launch_bounds__(256) void mla_rope_cache_kernel(MlaCacheArgs a) {
    __shared__ __align__(16) float kpe[512];
    const int64_t i = blockIdx.x;
    const int64_t pos = a.rows[i].pos, b = a.rows[i].b;
    if (b >= a.nb || pos >= a.T) return;  // outside the KV cache: the row is skipped
    const int64_t p = pos < a.rope_len - 1 ? pos : a.rope_len - 1;
    const float *cr = a.cos_t + p * a.half, *sr = a.sin_t + p * a.half;
    const bool gptj = a.style == DITCH_ROPE_GPTJ;
    const float *pe = a.kva + i * (a.kv_lora + a.rd) + a.kv_lora;
    for (int64_t d = threadIdx.x; d < a.rd; d += blockDim.x) {
        float y = pe[d];
        if (d < 2 * a.half) {
            const int64_t j = gptj ? d / 2 : d % a.half;
            const int64_t ia = gptj ? 2 * j : j, ib = gptj ? 2 * j + 1 : j + a.half;
            const float x1 = pe[ia], x2 = pe[ib], c = cr[j], sn = sr[j];
            y = d == ia ? __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, sn)) : __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, sn));
        }
        kpe[d] = y;
    }
    // the queries' rope pairs, one pair a thread (in place)
    float *qr = a.q + i * a.heads * a.hd + a.nope;
    for (int64_t t = threadIdx.x; t < a.heads * a.half; t += blockDim.x) {
        const int64_t h = t / a.half, j = t % a.half;
        float *x = qr + h * a.hd;
        const int64_t ia = gptj ? 2 * j : j, ib = gptj ? 2 * j + 1 : j + a.half;
        const float x1 = x[ia], x2 = x[ib], c = cr[j], sn = sr[j];
        x[ia] = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, sn));
        x[ib] = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, sn));
    }
    __syncthreads();
    const int64_t hd4 = a.hd / 4, kvb_row = a.heads * (a.nope + a.vd);
    const float *src = a.kvb + i * kvb_row;
    float4 *kd = (float4 *)(a.kc + (b * a.T + pos) * a.kvd), *vdst = (float4 *)(a.vc + (b * a.T + pos) * a.kvd);
    for (int64_t t = threadIdx.x; t < a.heads * hd4; t += blockDim.x) {
        const int64_t h = t / hd4, d = (t % hd4) * 4;
        const float *hs = src + h * (a.nope + a.vd);
        kd[t] = d < a.nope ? *(const float4 *)(hs + d) : *(const float4 *)(kpe + (d - a.nope));
        vdst[t] = d < a.vd ? *(const float4 *)(hs + a.nope + d) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// Router (moe.zig:1011-1101) for one token per thread: softmax or sigmoid
// scores, correction bias, group-limited masking, top-k with strict '>',
// renormalisation and scaling.
struct RouteArgs {
    float *logits;          // [n][E], scores in place
    const float *corr;      // [E] or null
    int32_t *sel;           // [n][k]
    float *selw;            // [n][k]
    int32_t *ord;           // [n][k]: the selections in ascending expert index
    int64_t n, E, k, n_group, topk_group;
    int scoring, group_limited, norm_topk;
    float scaling;
};

constexpr int ROUTE_MAXE = 512;
constexpr int ROUTE_MAXG = 64;
constexpr int ROUTE_EJ = ROUTE_MAXE / 64;  // experts per lane

// (value, index) of the better of two candidates of a top-k pass: the
// larger value, the lower index on ties (moe.zig:971-985: strict > in index
// order); a candidate that is not above -inf (or NaN) never wins.
__device__ __forceinline__ void better(float &v, int &i, float v2, int i2) {
    const bool ok2 = v2 > -INFINITY, ok = v > -INFINITY;
    if (ok2 && (!ok || v2 > v || (v2 == v && i2 < i))) {
        v = v2;
        i = i2;
    }
}
__device__ __forceinline__ int wave_argmax(float v, int i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(v, o, 64);
        const int i2 = __shfl_xor(i, o, 64);
        better(v, i, v2, i2);
    }
    return v > -INFINITY ? i : 0;  // nothing above -inf: the reference's initial best, index 0
}

// Router of one token per wave (moe.zig:998-1110): softmax (max, Cephes exp,
// sum, 1/sum) or sigmoid scores, correction bias for the choice,
// group-limited selection (a group's score is its best, or with the bias its
// best two, in index order; kept groups chosen by repeated argmax), top-k by
// repeated argmax with ties to the lower index, renormalisation and scaling.
// Lane l holds experts l + 64 j.
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
    __shared__ float chs[4][ROUTE_MAXE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + wave;
    if (t >= a.n) return;
    float *row = a.logits + t * a.E;
    float p[ROUTE_EJ], ch[ROUTE_EJ];
#pragma unroll
    for (int j = 0; j < ROUTE_EJ; j++) {
        const int64_t e = lane + 64 * j;
        p[j] = e < a.E ? row[e] : -INFINITY;
    }
    if (a.scoring == DITCH_SCORING_SOFTMAX) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++) m = fmaxf(m, p[j]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float sm = 0.f;
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++) {
            p[j] = lane + 64 * j < a.E ? exp_cephes(__fsub_rn(p[j], m)) : 0.f;
            sm = __fadd_rn(sm, p[j]);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sm = __fadd_rn(sm, __shfl_xor(sm, o, 64));
        const float inv = __fdiv_rn(1.0f, sm);
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++) p[j] = __fmul_rn(p[j], inv);
    } else {
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++) p[j] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-p[j])));
    }
#pragma unroll
    for (int j = 0; j < ROUTE_EJ; j++) {
        const int64_t e = lane + 64 * j;
        ch[j] = e < a.E ? __fadd_rn(p[j], a.corr ? a.corr[e] : 0.0f) : -INFINITY;
        if (e < a.E) chs[wave][e] = ch[j];
    }
    if (a.group_limited && a.n_group > 1) {
        // lane g scores group g over its experts in index order
        const int64_t per = a.E / a.n_group;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        float gs = -INFINITY;
        if (lane < a.n_group) {
            const float *sg = chs[wave] + lane * per;
            if (a.corr) {
                float b1 = -INFINITY, b2 = -INFINITY;
                for (int64_t i = 0; i < per; i++) {
                    if (sg[i] > b1) { b2 = b1; b1 = sg[i]; }
                    else if (sg[i] > b2) b2 = sg[i];
                }
                gs = __fadd_rn(b1, per > 1 ? b2 : 0.0f);
            } else {
                float best = -INFINITY;
                for (int64_t i = 0; i < per; i++) best = fmaxf(best, sg[i]);
                gs = best;
            }
        }
        // kept groups: repeated argmax; a kept group never wins again
        bool kept = false;
        const int64_t keep = a.topk_group < a.n_group ? a.topk_group : a.n_group;
        for (int64_t kk = 0; kk < keep; kk++) {
            const int best = wave_argmax(lane < a.n_group && !kept ? gs : -INFINITY, lane);
            if (lane == best) kept = true;
        }
        const uint64_t kept_mask = __ballot(kept);
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++) {
            const int64_t e = lane + 64 * j;
            if (e < a.E && !((kept_mask >> (e / per)) & 1ull)) ch[j] = -INFINITY;
        }
    }
    // top k, in selection order (k <= 16; the selections stay in registers:
    // arrays indexed at run time would live in scratch memory)
    float sum = 0.f;
    int32_t selj[16];
    float pbs[16];
#pragma unroll
    for (int jk = 0; jk < 16; jk++) {
        if (jk >= a.k) break;
        float v = -INFINITY;
        int idx = 0;
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++) better(v, idx, ch[j], lane + 64 * j);
        const int best = wave_argmax(v, idx);
        // the winner's probability, from the lane that holds it
        float pb = 0.f;
#pragma unroll
        for (int j = 0; j < ROUTE_EJ; j++)
            if (lane + 64 * j == best) {
                pb = p[j];
                ch[j] = -INFINITY;
            }
        pb = __shfl(pb, best % 64, 64);
        selj[jk] = best;
        pbs[jk] = pb;
        sum = __fadd_rn(sum, pb);
    }
    // lane j < k finishes selection j: its weight (renormalised by the sum,
    // then scaled), and its place in ascending expert index (the combine's
    // order): the count of smaller experts plus the earlier selections of
    // the same expert. Experts repeat when fewer than k choices are above
    // -inf (NaN router scores, or group-limited routing that keeps fewer
    // than k experts): the argmax then returns expert 0 again, as topk
    // does (moe.zig:971-985), and the repeats keep their selection order.
    int32_t my_sel = 0;
    float my_w = 0.f;
#pragma unroll
    for (int jk = 0; jk < 16; jk++)
        if (lane == jk) {
            my_sel = selj[jk];
            my_w = pbs[jk];
        }
    if (lane < a.k) {
        float w = my_w;
        if (a.norm_topk && sum > 0) w = __fdiv_rn(w, sum);
        if (a.scaling != 1.0f) w = __fmul_rn(w, a.scaling);
        a.sel[t * a.k + lane] = my_sel;
        a.selw[t * a.k + lane] = w;
        int rank = 0;
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (i < a.k && (selj[i] < my_sel || (selj[i] == my_sel && i < lane))) rank++;
        a.ord[t * a.k + rank] = lane;
    }
}

// Per-expert token counts.
// Selections per expert: a histogram in LDS per block, then one global
// atomic per expert and block (the selections of a layer hit ~E addresses).
__global__ __launch_bounds__(256) void expert_count_kernel(const int32_t *sel, int64_t nk, int32_t *counts, int64_t E) {
    __shared__ int32_t hist[ROUTE_MAXE];
    for (int64_t e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nk; i += (int64_t)gridDim.x * blockDim.x)
        atomicAdd(&hist[sel[i]], 1);
    __syncthreads();
    for (int64_t e = threadIdx.x; e < E; e += blockDim.x)
        if (hist[e]) atomicAdd(&counts[e], hist[e]);
}

// Expert e's pair list in (token, slot) order (moe.zig:1174-1188): one block
// per expert; each wave takes a contiguous run of the selections, counts its
// matches, and after one block-wide prefix writes them in order.
constexpr int LIST_WAVES = 16;
__global__ __launch_bounds__(LIST_WAVES * 64) void expert_list_kernel(const int32_t *sel, int64_t n, int64_t k,
                                                                     const int32_t *offsets, int32_t *pair_token,
                                                                     int32_t *pair_of) {
    __shared__ int32_t wave_cnt[LIST_WAVES];
    const int e = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t nk = n * k;
    const int64_t seg = (nk + LIST_WAVES * 64 - 1) / (LIST_WAVES * 64) * 64;
    const int64_t lo = wave * seg, hi = lo + seg < nk ? lo + seg : nk;
    // both passes take 8 steps of 64 selections at a time, their loads
    // issued together (one step at a time waits for each load in turn)
    constexpr int LU = 8;
    int32_t cnt = 0;
    for (int64_t c = lo; c < hi; c += 64 * LU) {
        int32_t v[LU];
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int64_t i = c + 64 * u + lane;
            v[u] = i < hi ? sel[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < LU; u++) cnt += __popcll(__ballot(v[u] == e));
    }
    if (lane == 0) wave_cnt[wave] = cnt;
    __syncthreads();
    int32_t base = offsets[e];
    for (int w = 0; w < wave; w++) base += wave_cnt[w];
    for (int64_t c = lo; c < hi; c += 64 * LU) {
        int32_t v[LU];
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int64_t i = c + 64 * u + lane;
            v[u] = i < hi ? sel[i] : -1;
        }
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int64_t i = c + 64 * u + lane;
            const bool hit = v[u] == e;
            const unsigned long long ballot = __ballot(hit);
            if (hit) {
                const int32_t p = base + __popcll(ballot & ((1ull << lane) - 1ull));
                pair_token[p] = (int32_t)(i / k);
                pair_of[i] = p;
            }
            base += __popcll(ballot);
        }
    }
}

// Device planning of a routed layer's grouped products, every expert a
// segment in index order (no count read-back): the offsets of each expert's
// pairs, off/cnt of the nt segment tables, the padded row map (16-row blocks
// per expert, -1 for padding and for the rows past the last block up to
// max_blocks) and the tile table (one entry per 4 blocks of an expert).
__global__ __launch_bounds__(1024) void moe_plan_kernel(const int32_t *counts, int64_t E, GroupSeg *segs, int nt,
                                                        int32_t *offsets, int32_t *prow, int32_t *desc, int32_t *count,
                                                        int64_t max_blocks) {
    __shared__ int32_t cnt_s[ROUTE_MAXE], off_s[ROUTE_MAXE], base_s[ROUTE_MAXE], dbase_s[ROUTE_MAXE];
    __shared__ int32_t tot_blocks;
    __shared__ int32_t wsum[3][16];
    // exclusive prefix sums over the experts of their pairs, 16-row blocks
    // and 4-block tile rows (thread e holds expert e, E <= 512 < 1024):
    // inclusive scans within each wave, then the earlier waves' totals
    {
        const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const int64_t e = threadIdx.x;
        const int32_t c = e < E ? counts[e] : 0, nb = (c + 15) / 16, nd = (nb + 3) / 4;
        int32_t ic = c, ib = nb, id = nd;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t tc = __shfl_up(ic, o, 64), tb = __shfl_up(ib, o, 64), td = __shfl_up(id, o, 64);
            if (lane >= o) {
                ic += tc;
                ib += tb;
                id += td;
            }
        }
        if (lane == 63) {
            wsum[0][wv] = ic;
            wsum[1][wv] = ib;
            wsum[2][wv] = id;
        }
        __syncthreads();
        int32_t pc = 0, pb = 0, pd = 0;
        for (int w = 0; w < wv; w++) {
            pc += wsum[0][w];
            pb += wsum[1][w];
            pd += wsum[2][w];
        }
        if (e < E) {
            cnt_s[e] = c;
            off_s[e] = pc + ic - c;
            base_s[e] = pb + ib - nb;
            dbase_s[e] = pd + id - nd;
        }
        if (threadIdx.x == 0) {
            int32_t b = 0, d = 0;
            for (int w = 0; w < (int)(blockDim.x >> 6); w++) {
                b += wsum[1][w];
                d += wsum[2][w];
            }
            tot_blocks = b;
            *count = d;
        }
    }
    __syncthreads();
    for (int64_t e = threadIdx.x; e < E; e += blockDim.x) {
        offsets[e] = off_s[e];
        for (int t = 0; t < nt; t++) {
            segs[t * E + e].off = off_s[e];
            segs[t * E + e].cnt = cnt_s[e];
        }
        const int32_t nb = (cnt_s[e] + 15) / 16;
        for (int32_t j = 0; j < nb; j += 4) {
            int32_t *dd = desc + 4 * (int64_t)(dbase_s[e] + j / 4);
            dd[0] = (int32_t)e;
            dd[1] = base_s[e] + j;
            dd[2] = base_s[e] + nb;
            dd[3] = j * 16;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int64_t e = wave; e < E; e += nw) {
        const int32_t c = cnt_s[e], nb = (c + 15) / 16;
        for (int32_t i = lane; i < nb * 16; i += 64) prow[(int64_t)base_s[e] * 16 + i] = i < c ? off_s[e] + i : -1;
    }
    for (int64_t r = (int64_t)tot_blocks * 16 + threadIdx.x; r < max_blocks * 16; r += blockDim.x) prow[r] = -1;
}

// out[t] = x[t] + (sum over the token's experts in ascending index of
// w * eo + shared) (moe.zig:1197-1227 then the residual add); ord holds each
// token's selections in that order. Four columns per thread. UNI: a row is a
// whole number of waves (hidden a multiple of 256), so a wave's token is
// one value and its selections, weights and pair rows are scalar loads.
template <bool UNI>
__global__ void moe_combine_kernel(float *x, const float *eo, const float *eo_shared,
                                   const int32_t *__restrict__ ord, const float *__restrict__ selw,
                                   const int32_t *__restrict__ pair_of, int64_t n, int64_t k, int64_t hidden) {
    const int64_t h4 = (hidden + 3) / 4, total = n * h4;
    const bool vec = (hidden % 4) == 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t t = i / h4;
        if constexpr (UNI) t = (int64_t)__builtin_amdgcn_readfirstlane((int)t);
        const int64_t c0 = (i % h4) * 4;
        // the token's k (<= 16) rows and weights first, then every row load
        // in flight together, added in the order ord gives (fixed-size
        // register arrays, entries j >= k unused)
        const float *er[16];
        float wt[16];
        float4 ev[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            wt[j] = 0.f;
            er[j] = eo;
            if (j < k) {
                const int64_t sidx = t * k + ord[t * k + j];
                wt[j] = selw[sidx];
                er[j] = eo + (int64_t)pair_of[sidx] * hidden + c0;
            }
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            ev[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (j < k) {
                if (vec) ev[j] = *(const float4 *)er[j];
                else {
                    ev[j].x = er[j][0];
                    ev[j].y = c0 + 1 < hidden ? er[j][1] : 0.f;
                    ev[j].z = c0 + 2 < hidden ? er[j][2] : 0.f;
                    ev[j].w = c0 + 3 < hidden ? er[j][3] : 0.f;
                }
            }
        }
        float m[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (j >= k) continue;
            m[0] = __fadd_rn(m[0], __fmul_rn(wt[j], ev[j].x));
            m[1] = __fadd_rn(m[1], __fmul_rn(wt[j], ev[j].y));
            m[2] = __fadd_rn(m[2], __fmul_rn(wt[j], ev[j].z));
            m[3] = __fadd_rn(m[3], __fmul_rn(wt[j], ev[j].w));
        }
        if (vec) {
            float4 *xo = (float4 *)(x + t * hidden + c0);
            float4 o = *xo;
            if (eo_shared) {
                const float4 sh = *(const float4 *)(eo_shared + t * hidden + c0);
                m[0] = __fadd_rn(m[0], sh.x);
                m[1] = __fadd_rn(m[1], sh.y);
                m[2] = __fadd_rn(m[2], sh.z);
                m[3] = __fadd_rn(m[3], sh.w);
            }
            *xo = make_float4(__fadd_rn(o.x, m[0]), __fadd_rn(o.y, m[1]), __fadd_rn(o.z, m[2]), __fadd_rn(o.w, m[3]));
            continue;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (c0 + u >= hidden) continue;
            float v = m[u];
            if (eo_shared) v = __fadd_rn(v, eo_shared[t * hidden + c0 + u]);
            x[t * hidden + c0 + u] = __fadd_rn(x[t * hidden + c0 + u], v);
        }
    }
}

__global__ void add_rows_kernel(float *x, const float *y, int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
        x[i] = __fadd_rn(x[i], y[i]);
}

// xa[p][j] = dot(a_e_j, x_row(p)) for the pairs of every expert segment
struct SegDelta {
    const float *a;  // [rank][cols] or null
    int64_t off, cnt;
    int rank;
};
__global__ void grouped_delta_xa_kernel(float *xa, const float *x, const int32_t *row_index, const SegDelta *segs,
                                        int64_t cols, int max_rank) {
    int lane = threadIdx.x & 63;
    const SegDelta &s = segs[blockIdx.y];
    int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (s.rank == 0 || t >= s.cnt * s.rank) return;
    int64_t pl = t / s.rank, j = t % s.rank;
    int64_t p = s.off + pl;
    int64_t src = row_index ? row_index[p] : p;
    float acc = 0.f;
    for (int64_t c = lane; c < cols; c += 64) acc = __builtin_fmaf(s.a[j * cols + c], x[src * cols + c], acc);
    acc = wave_sum64(acc);
    if (lane == 0) xa[p * max_rank + j] = acc;
}

// ---------------------------------------------------------------------------
// Host side

}  // namespace ditch

namespace ditch {

static void host_fill_rope(const ditch_model_config &c, std::vector<float> &cos_t, std::vector<float> &sin_t);

static Vec upload_vec(const ditch_weight *w, hipStream_t s) {
    // norms / biases: widen to f32 on the host side of the upload
    int64_t len = (int64_t)(w->rows * w->cols);
    std::vector<float> host(len);
    for (int64_t i = 0; i < len; i++) {
        switch (w->dtype) {
        case DITCH_F32: host[i] = ((const float *)w->data)[i]; break;
        case DITCH_BF16: {
            uint32_t b = (uint32_t)((const uint16_t *)w->data)[i] << 16;
            memcpy(&host[i], &b, 4);
            break;
        }
        case DITCH_F16: {
            uint16_t hb = ((const uint16_t *)w->data)[i];
            uint32_t sign = (uint32_t)(hb & 0x8000u) << 16, e = (hb >> 10) & 0x1fu, m = hb & 0x3ffu, bits;
            if (e == 0) {
                float f = (float)m * 5.9604644775390625e-08f;
                host[i] = sign ? -f : f;
                continue;
            }
            bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
            memcpy(&host[i], &bits, 4);
            break;
        }
        default: throw Error{DITCH_UNSUPPORTED, "norm/bias vectors must be f32, f16 or bf16"};
        }
    }
    Vec v;
    v.len = len;
    v.p = (float *)dev_alloc(len * 4);
    DITCH_TRY_HIP(hipMemcpyAsync(v.p, host.data(), len * 4, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipStreamSynchronize(s));
    return v;
}

static bool vector_slot(int slot) {
    switch (slot) {
    case DITCH_SLOT_FINAL_NORM: case DITCH_SLOT_ATTN_NORM: case DITCH_SLOT_Q_BIAS: case DITCH_SLOT_K_BIAS:
    case DITCH_SLOT_V_BIAS: case DITCH_SLOT_Q_NORM: case DITCH_SLOT_K_NORM: case DITCH_SLOT_FFN_NORM:
    case DITCH_SLOT_ROUTER_CORRECTION: case DITCH_SLOT_MLA_Q_A_NORM: case DITCH_SLOT_MLA_KV_A_NORM: return true;
    default: return false;
    }
}

static Vec *vec_slot(ditch_hip_model *m, int layer, int slot) {
    if (slot == DITCH_SLOT_FINAL_NORM) return &m->final_norm;
    DITCH_CHECK(layer >= 0 && (uint64_t)layer < m->c.layers, DITCH_INVALID_ARGUMENT, "layer index");
    Layer &L = m->layers[layer];
    switch (slot) {
    case DITCH_SLOT_ATTN_NORM: return &L.attn_norm;
    case DITCH_SLOT_Q_BIAS: return &L.q_bias;
    case DITCH_SLOT_K_BIAS: return &L.k_bias;
    case DITCH_SLOT_V_BIAS: return &L.v_bias;
    case DITCH_SLOT_Q_NORM: return &L.q_norm;
    case DITCH_SLOT_K_NORM: return &L.k_norm;
    case DITCH_SLOT_FFN_NORM: return &L.ffn_norm;
    case DITCH_SLOT_ROUTER_CORRECTION: return &L.corr;
    case DITCH_SLOT_MLA_Q_A_NORM: return &L.q_a_norm;
    case DITCH_SLOT_MLA_KV_A_NORM: return &L.kv_a_norm;
    default: throw Error{DITCH_INVALID_ARGUMENT, "not a vector slot"};
    }
}

static Mat *mat_slot(ditch_hip_model *m, int layer, int slot, int expert) {
    if (slot == DITCH_SLOT_EMBED) return &m->embed;
    if (slot == DITCH_SLOT_LM_HEAD) return &m->lm_head;
    DITCH_CHECK(layer >= 0 && (uint64_t)layer < m->c.layers, DITCH_INVALID_ARGUMENT, "layer index");
    Layer &L = m->layers[layer];
    switch (slot) {
    case DITCH_SLOT_Q: return &L.q;
    case DITCH_SLOT_K: return &L.k;
    case DITCH_SLOT_V: return &L.v;
    case DITCH_SLOT_O: return &L.o;
    case DITCH_SLOT_GATE: return &L.gate;
    case DITCH_SLOT_UP: return &L.up;
    case DITCH_SLOT_DOWN: return &L.down;
    case DITCH_SLOT_ROUTER: return &L.router;
    case DITCH_SLOT_SHARED_GATE: return &L.sh_gate;
    case DITCH_SLOT_SHARED_UP: return &L.sh_up;
    case DITCH_SLOT_SHARED_DOWN: return &L.sh_down;
    case DITCH_SLOT_MLA_Q_A: return &L.q_a;
    case DITCH_SLOT_MLA_Q_B: return &L.q_b;
    case DITCH_SLOT_MLA_KV_A: return &L.kv_a;
    case DITCH_SLOT_MLA_KV_B: return &L.kv_b;
    case DITCH_SLOT_EXPERT_GATE: case DITCH_SLOT_EXPERT_UP: case DITCH_SLOT_EXPERT_DOWN: {
        DITCH_CHECK(expert >= 0 && (uint64_t)expert < m->c.n_experts && !L.eg.empty(), DITCH_INVALID_ARGUMENT,
                    "expert index (or the layer is not a routed MoE layer)");
        return slot == DITCH_SLOT_EXPERT_GATE ? &L.eg[expert] : slot == DITCH_SLOT_EXPERT_UP ? &L.eu[expert] : &L.ed[expert];
    }
    default: throw Error{DITCH_INVALID_ARGUMENT, "unknown slot " + std::to_string(slot)};
    }
}

ditch_hip_model *model_create(ditch_hip *h, const ditch_model_config *cfg) {
    DITCH_CHECK(cfg->hidden > 0 && cfg->layers > 0 && cfg->heads > 0 && cfg->head_dim > 0, DITCH_INVALID_ARGUMENT,
                "model config");
    DITCH_CHECK(cfg->n_experts <= (uint64_t)ROUTE_MAXE && cfg->n_group <= (uint64_t)ROUTE_MAXG && cfg->top_k <= 16,
                DITCH_UNSUPPORTED, "router limits: <= 512 experts, <= 64 groups, top_k <= 16");
    auto *m = new ditch_hip_model();
    m->h = h;
    m->c = *cfg;
    m->moe_layers.assign(cfg->layers, 0);
    if (cfg->moe_layers) memcpy(m->moe_layers.data(), cfg->moe_layers, cfg->layers);
    m->c.moe_layers = m->moe_layers.data();
    m->layers.resize(cfg->layers);
    for (uint64_t l = 0; l < cfg->layers; l++)
        if (cfg->n_experts && m->moe_layers[l]) {
            m->layers[l].eg.resize(cfg->n_experts);
            m->layers[l].eu.resize(cfg->n_experts);
            m->layers[l].ed.resize(cfg->n_experts);
        }
    std::vector<float> cs, sn;
    host_fill_rope(m->c, cs, sn);
    m->c.rope_factors = nullptr;  // not kept past creation
    size_t bytes = (cs.size() + 1) * 4;
    try {
        m->rope_cos = (float *)dev_alloc(bytes);
        m->rope_sin = (float *)dev_alloc(bytes);
        if (!cs.empty()) {
            DITCH_TRY_HIP(hipMemcpyAsync(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, h->stream));
            DITCH_TRY_HIP(hipMemcpyAsync(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, h->stream));
        }
        DITCH_TRY_HIP(hipStreamSynchronize(h->stream));
    } catch (...) {
        delete m;
        throw;
    }
    return m;
}

// The shape every matrix slot must have under the model's configuration
// (the reference's Layer fields, model.zig:312-390, and MoE experts,
// moe.zig:95-123); a mismatch is refused before anything reaches the device,
// so no kernel is ever launched on a matrix its grid was not sized for.
// Dense gate/up widths may differ per layer (DeepSeek's first dense layers):
// only their hidden side is fixed here, the forward checks the three agree.
static void check_mat_shape(const ditch_hip_model *m, int slot, const ditch_weight *w) {
    const ditch_model_config &c = m->c;
    const uint64_t H = c.hidden, r = w->rows, k = w->cols;
    const uint64_t qd = c.heads * c.head_dim, kvd = c.kv_heads * c.head_dim, od = c.heads * c.v_head_dim;
    auto want = [&](bool ok, const char *what) {
        DITCH_CHECK(ok, DITCH_INVALID_ARGUMENT,
                    std::string("model_set: ") + what + " has the wrong shape (" + std::to_string(r) + " x " +
                        std::to_string(k) + ")");
    };
    switch (slot) {
    case DITCH_SLOT_EMBED: want(k == H && r > 0, "embedding"); break;
    case DITCH_SLOT_LM_HEAD: want(k == H && r == c.vocab, "lm_head"); break;
    case DITCH_SLOT_Q: want(r == qd && k == H, "q_proj"); break;
    case DITCH_SLOT_K:
    case DITCH_SLOT_V: want(r == kvd && k == H, "k/v_proj"); break;
    case DITCH_SLOT_O: want(r == H && k == (c.mla ? od : qd), "o_proj"); break;
    case DITCH_SLOT_GATE:
    case DITCH_SLOT_UP: want(k == H && r > 0, "gate/up_proj"); break;
    case DITCH_SLOT_DOWN: want(r == H && k > 0, "down_proj"); break;
    case DITCH_SLOT_ROUTER: want(r == c.n_experts && k == H, "router"); break;
    case DITCH_SLOT_EXPERT_GATE:
    case DITCH_SLOT_EXPERT_UP: want(r == c.moe_inter && k == H, "expert gate/up"); break;
    case DITCH_SLOT_EXPERT_DOWN: want(r == H && k == c.moe_inter, "expert down"); break;
    case DITCH_SLOT_SHARED_GATE:
    case DITCH_SLOT_SHARED_UP: want(k == H && (c.shared_inter == 0 || r == c.shared_inter), "shared gate/up"); break;
    case DITCH_SLOT_SHARED_DOWN: want(r == H && (c.shared_inter == 0 || k == c.shared_inter), "shared down"); break;
    case DITCH_SLOT_MLA_Q_A: want(r == c.q_lora_rank && k == H, "q_a_proj"); break;
    case DITCH_SLOT_MLA_Q_B: want(r == qd && k == (c.q_lora_rank ? c.q_lora_rank : H), "q_b_proj"); break;
    case DITCH_SLOT_MLA_KV_A: want(r == c.kv_lora_rank + c.qk_rope_dim && k == H, "kv_a_proj"); break;
    case DITCH_SLOT_MLA_KV_B:
        want(r == c.heads * (c.qk_nope_dim + c.v_head_dim) && k == c.kv_lora_rank, "kv_b_proj");
        break;
    default: break;
    }
}

void model_set(ditch_hip_model *m, int layer, int slot, int expert, const ditch_weight *w) {
    hipStream_t s = m->h->stream;
    if (vector_slot(slot)) {
        Vec *v = vec_slot(m, layer, slot);
        Vec nv = upload_vec(w, s);
        v->release();
        *v = nv;
        return;
    }
    Mat *mt = mat_slot(m, layer, slot, expert);
    check_mat_shape(m, slot, w);
    ditch_hip_tensor *t = upload_weight(m->h, w, s);
    mt->release();
    mt->t = t;
    m->weights_version++;
    if (m->expert_budget > 0 &&
        (slot == DITCH_SLOT_EXPERT_GATE || slot == DITCH_SLOT_EXPERT_UP || slot == DITCH_SLOT_EXPERT_DOWN)) {
        DITCH_CHECK(!m->cache, DITCH_INVALID_ARGUMENT, "expert registered after the expert cache was built");
        uint64_t limit = EXPERT_PINNED_LIMIT;
        if (const char *ev = getenv("DITCH_HIP_EXPERT_PINNED_LIMIT")) limit = strtoull(ev, nullptr, 10);
        const uint64_t routed = std::max<uint64_t>(
            1, (uint64_t)std::count_if(m->moe_layers.begin(), m->moe_layers.end(), [](uint8_t f) { return f != 0; }));
        if (m->expert_pinned_layer.size() != m->layers.size()) m->expert_pinned_layer.assign(m->layers.size(), 0);
        stream_out(*mt, m->expert_pinned_layer[layer], limit / routed, m->expert_pinned, m->expert_pinned_exhausted);
    }
}

// Slots whose product the forward runs without a delta epilogue: the
// embedding is a row lookup, and a routed expert carries a delta on its down
// projection only (moe.zig:99-100). A delta there would have no effect, so it
// is refused rather than dropped.
static void check_delta_slot(int slot) {
    DITCH_CHECK(slot != DITCH_SLOT_EMBED && slot != DITCH_SLOT_EXPERT_GATE && slot != DITCH_SLOT_EXPERT_UP,
                DITCH_UNSUPPORTED, "a delta on the embedding or a routed expert's gate/up projection is not applied "
                                   "by the forward");
}
void check_edit_slot(int slot) { check_delta_slot(slot); }
Mat *mat_slot_of(ditch_hip_model *m, int layer, int slot, int expert) { return mat_slot(m, layer, slot, expert); }

void model_set_delta(ditch_hip_model *m, int layer, int slot, int expert, uint64_t rank, const float *a,
                     const float *b) {
    if (rank > 0) check_delta_slot(slot);
    Mat *mt = mat_slot(m, layer, slot, expert);
    DITCH_CHECK(mt->ok(), DITCH_INVALID_ARGUMENT, "delta on an empty slot");
    DITCH_CHECK(rank <= (uint64_t)INT32_MAX, DITCH_UNSUPPORTED, "delta rank above 2^31");
    mt->clear_delta();
    if (rank == 0) return;
    hipStream_t s = m->h->stream;
    size_t ab = rank * mt->t->v.cols * 4, bb = mt->t->v.rows * rank * 4;
    mt->da = (float *)dev_alloc(ab);
    mt->db = (float *)dev_alloc(bb);
    DITCH_TRY_HIP(hipMemcpyAsync(mt->da, a, ab, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipMemcpyAsync(mt->db, b, bb, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipStreamSynchronize(s));
    mt->rank = (int)rank;
}

// The same edit as abliterate.computeOutputDelta (none mode): a = V^T W on
// the device over the resident codes, b = -weight V.
void model_edit(ditch_hip_model *m, int layer, int slot, int expert, const float *v, uint64_t k, float weight) {
    check_delta_slot(slot);
    Mat *mt = mat_slot(m, layer, slot, expert);
    DITCH_CHECK(mt->ok(), DITCH_INVALID_ARGUMENT, "edit of an empty slot");
    hipStream_t s = m->h->stream;
    DevBuf staged;
    TileView w = mt->t->v;
    if (mt->streamed()) {  // a streamed expert: the edit reads a device copy of its blob
        uint8_t *d = staged.get<uint8_t>(mt->hm.bytes);
        DITCH_TRY_HIP(hipMemcpyAsync(d, mt->hm.host, mt->hm.bytes, hipMemcpyHostToDevice, s));
        w = view_at(*mt, d);
    }
    // the directions and the partial sums in the model's edit scratch (an
    // edit of thousands of matrices allocates and frees nothing per matrix
    // there); a and b in one allocation, a written by the product itself
    float *d_v = m->edit_v.get<float>(k * w.rows);
    DITCH_TRY_HIP(hipMemcpyAsync(d_v, v, k * w.rows * 4, hipMemcpyHostToDevice, s));
    mt->clear_delta();
    float *dab = (float *)dev_alloc((k * w.cols + w.rows * k) * 4);
    mt->da = dab;
    mt->db = dab + k * w.cols;
    mt->joint = true;
    launch_matvecT(mt->da, w, d_v, (int64_t)k, s);
    std::vector<float> b(w.rows * k);
    for (int64_t i = 0; i < w.rows; i++)
        for (uint64_t j = 0; j < k; j++) b[i * k + j] = -weight * v[j * w.rows + i];
    DITCH_TRY_HIP(hipMemcpyAsync(mt->db, b.data(), w.rows * k * 4, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipStreamSynchronize(s));
    mt->rank = (int)k;
}

// abliterate.computeDelta in any mode on a registered matrix, installed as
// its delta (a streamed expert's blob is staged on the device for the passes)
void model_edit_ex(ditch_hip_model *m, int layer, int slot, int expert, const float *v, uint64_t k, float weight,
                   int mode, int64_t lora_rank, uint64_t seed, int ablate) {
    check_delta_slot(slot);
    Mat *mt = mat_slot(m, layer, slot, expert);
    DITCH_CHECK(mt->ok(), DITCH_INVALID_ARGUMENT, "edit of an empty slot");
    hipStream_t s = m->h->stream;
    DevBuf staged;
    TileView w = mt->t->v;
    if (mt->streamed()) {
        uint8_t *d = staged.get<uint8_t>(mt->hm.bytes);
        DITCH_TRY_HIP(hipMemcpyAsync(d, mt->hm.host, mt->hm.bytes, hipMemcpyHostToDevice, s));
        w = view_at(*mt, d);
    }
    float *da = nullptr, *db = nullptr;
    int64_t rank = 0;
    edit_delta_device(m->h, w, v, (int64_t)k, weight, mode, lora_rank, seed, ablate, s, &da, &db, &rank);
    mt->clear_delta();
    mt->da = da;
    mt->db = db;
    mt->rank = (int)rank;
}

void model_reset_deltas(ditch_hip_model *m) {
    for (auto &L : m->layers) {
        for (Mat *mt : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down, &L.router, &L.sh_gate, &L.sh_up, &L.sh_down,
                        &L.q_a, &L.q_b, &L.kv_a, &L.kv_b})
            mt->clear_delta();
        for (auto *vec : {&L.eg, &L.eu, &L.ed})
            for (auto &mt : *vec) mt.clear_delta();
    }
    m->embed.clear_delta();
    m->lm_head.clear_delta();
}

uint64_t model_bytes(const ditch_hip_model *m) {
    uint64_t b = 0;
    auto add = [&](const Mat &mt) {
        if (mt.t) b += mt.t->bytes;
    };
    add(m->embed);
    add(m->lm_head);
    for (auto &L : m->layers) {
        for (const Mat *mt : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down, &L.router, &L.sh_gate, &L.sh_up,
                              &L.sh_down, &L.q_a, &L.q_b, &L.kv_a, &L.kv_b})
            add(*mt);
        for (auto *vec : {&L.eg, &L.eu, &L.ed})
            for (auto &mt : *vec) add(mt);
    }
    return b;
}

// matmul with the slot's delta (tensor.zig:1036-1042) and an epilogue.
static void mm(ditch_hip_model *m, const Mat &mt, float *out, const float *x, int64_t n, const float *bias,
               int accumulate, hipStream_t s) {
    DITCH_CHECK(mt.ok(), DITCH_INVALID_ARGUMENT, "forward: a weight slot is empty");
    MatmulEpilogue ep;
    ep.bias = bias;
    ep.accumulate = accumulate;
    if (mt.rank > 0) {
        float *xa = m->xa.get<float>((size_t)n * mt.rank);
        launch_delta_xa(xa, x, mt.da, n, mt.t->v.cols, mt.rank, s);
        ep.delta_b = mt.db;
        ep.delta_xa = xa;
        ep.delta_rank = mt.rank;
    }
    launch_matmul(mt.t->v, out, x, n, ep, s, nullptr, &m->xsplit);
}

// The same on an activation that may come as pre-split A fragments (the
// delta's x A^T needs the f32 rows).
static void mm_act(ditch_hip_model *m, const Mat &mt, float *out, const Act &x, int64_t n, const float *bias,
                   int accumulate, hipStream_t s) {
    DITCH_CHECK(mt.ok(), DITCH_INVALID_ARGUMENT, "forward: a weight slot is empty");
    MatmulEpilogue ep;
    ep.bias = bias;
    ep.accumulate = accumulate;
    if (mt.rank > 0) {
        DITCH_CHECK(x.f32, DITCH_INVALID_ARGUMENT, "forward: a delta needs the f32 activation");
        float *xa = m->xa.get<float>((size_t)n * mt.rank);
        if (!x.xs && !x.xm) {
            // the split of the f32 rows forms x . A^T on the way
            MatmulEpilogue e2 = ep;
            e2.delta_b = mt.db;
            e2.delta_rank = mt.rank;
            if (launch_matmul_delta_split(mt.t->v, out, x.f32, n, e2, mt.da, mt.rank, xa, s, &m->xsplit)) return;
        }
        launch_delta_xa(xa, x.f32, mt.da, n, mt.t->v.cols, mt.rank, s);
        ep.delta_b = mt.db;
        ep.delta_xa = xa;
        ep.delta_rank = mt.rank;
    }
    launch_matmul_act(mt.t->v, out, x, n, ep, s, &m->xsplit);
}

// Whether the tiled product takes `mt` with fragments alone (no f32 rows).
// A product whose input may come as bf16-term fragments alone (no f32 rows):
// the bf16 tiled kernel takes it (MXFP4 included: its producers write bf16
// terms; given f32 rows an MXFP4 product takes the scaled-MFMA path).
constexpr bool attn_split_fragments = false;

static bool frag_only(const Mat &mt, int64_t n) { return mt.ok() && mt.rank == 0 && tile_gemm_takes(mt.t->v, n); }
// A product that reads MX fragments alone (MXFP4 on the scaled MFMA).
static bool mx_only(const Mat &mt, int64_t n) { return mt.ok() && mt.rank == 0 && mx_gemm_takes(mt.t->v, n); }

// Whether a routed layer's grouped products can be planned on the device:
// every expert resident (no cache), gate/up/down of one tiled format and
// shape (the fused GLU then the down product, whose epilogue adds each
// expert's down delta), and enough pairs per expert on average for the
// 16-token blocks.
static bool moe_device_plan(ditch_hip_model *m, const Layer &L, int64_t n) {
    const ditch_model_config &c = m->c;
    const int64_t E = (int64_t)c.n_experts, k = (int64_t)c.top_k;
    if (E <= 0 || E > ROUTE_MAXE || n * k < 16 * E) return false;
    for (int64_t e = 0; e < E; e++) {
        if (!L.eg[e].ok() || !L.eu[e].ok() || !L.ed[e].ok() || L.eg[e].streamed()) return false;
        const TileView &g = L.eg[e].t->v, &u = L.eu[e].t->v, &d = L.ed[e].t->v, &g0 = L.eg[0].t->v,
                       &d0 = L.ed[0].t->v;
        if (!tile_gemm_takes(g, 128) || !tile_gemm_takes(d, 128) || !tile_glu_takes(g, u, 128) || g.tf != g0.tf ||
            g.units_k != g0.units_k || d.tf != d0.tf || d.units_k != d0.units_k || g.rows != g0.rows ||
            d.rows != d0.rows)
            return false;
    }
    return true;
}

// Routed experts (moe.zig:998-1228) with the residual add: x += moe(h).
static void moe_forward(ditch_hip_model *m, Layer &L, float *x, const float *h, int64_t n, hipStream_t s) {
    const ditch_model_config &c = m->c;
    int64_t E = (int64_t)c.n_experts, k = (int64_t)c.top_k, hidden = (int64_t)c.hidden, inter = (int64_t)c.moe_inter;
    float *logits = m->r_logits.get<float>(n * E);
    mm(m, L.router, logits, h, n, nullptr, 0, s);
    int32_t *sel = m->r_sel.get<int32_t>(n * k);
    float *selw = m->r_selw.get<float>(n * k);
    int32_t *ord = m->r_ord.get<int32_t>(n * k);
    DITCH_CHECK(E <= ROUTE_MAXE && k <= 16 && (!c.group_limited || c.n_group <= ROUTE_MAXG), DITCH_UNSUPPORTED,
                "router: more than 512 experts, 16 per token or 64 groups");
    RouteArgs ra{logits, L.corr.p, sel, selw, ord, n, E, k, (int64_t)c.n_group, (int64_t)c.topk_group, c.scoring,
                 c.group_limited, c.norm_topk_prob, c.routed_scaling};
    hipLaunchKernelGGL(route_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, ra);
    DITCH_TRY_HIP(hipGetLastError());
    int32_t *counts = m->r_counts.get<int32_t>(E);
    DITCH_TRY_HIP(hipMemsetAsync(counts, 0, E * 4, s));
    hipLaunchKernelGGL(expert_count_kernel, dim3((unsigned)std::min<int64_t>((n * k + 2047) / 2048, 64)), dim3(256), 0,
                       s, sel, n * k, counts, E);
    DITCH_TRY_HIP(hipGetLastError());
    int32_t *pair_of = m->r_pair_of.get<int32_t>(n * k);
    float *eo = nullptr;
    if (moe_device_plan(m, L, n)) {
        // every expert resident and on the tiled product: the grouped
        // products are planned on the device
        m->moe_device_planned++;
        const int64_t P = n * k, max_blocks = (P + 15) / 16 + E, max_desc = (max_blocks + 3) / 4 + E;
        int32_t *offsets = m->r_offsets.get<int32_t>(E);
        int32_t *pair_token = m->r_pair_token.get<int32_t>(P);
        eo = m->e_out.get<float>(P * hidden);
        int max_rank = 0;
        std::vector<uintptr_t> key;
        key.reserve((size_t)(6 * E + 1));
        key.push_back((uintptr_t)m->weights_version);
        for (int64_t e = 0; e < E; e++) {
            key.insert(key.end(), {(uintptr_t)L.eg[e].t, (uintptr_t)L.eu[e].t, (uintptr_t)L.ed[e].t,
                                   (uintptr_t)L.ed[e].db, (uintptr_t)L.ed[e].da, (uintptr_t)L.ed[e].rank});
            max_rank = std::max(max_rank, L.ed[e].rank);
        }
        GroupSeg *dsegs = L.plan_tab.get<GroupSeg>(3 * E);
        const float **dda = L.plan_da.get<const float *>(E);
        if (key != L.plan_key) {
            std::vector<GroupSeg> tab((size_t)(3 * E));
            std::vector<const float *> das((size_t)E);
            for (int64_t e = 0; e < E; e++) {
                tab[e] = GroupSeg{L.eg[e].t->v, 0, 0, nullptr, 0};
                tab[E + e] = GroupSeg{L.eu[e].t->v, 0, 0, nullptr, 0};
                tab[2 * E + e] = GroupSeg{L.ed[e].t->v, 0, 0, L.ed[e].db, L.ed[e].rank};
                das[e] = L.ed[e].rank ? L.ed[e].da : nullptr;
            }
            DITCH_TRY_HIP(hipMemcpyAsync(dsegs, tab.data(), tab.size() * sizeof(GroupSeg), hipMemcpyHostToDevice, s));
            DITCH_TRY_HIP(hipMemcpyAsync(dda, das.data(), E * sizeof(float *), hipMemcpyHostToDevice, s));
            L.plan_key = std::move(key);
        }
        int32_t *meta = m->gmeta.get<int32_t>(max_blocks * 16 + max_desc * 4 + 1);
        const GroupedDevPlan plan{meta, meta + max_blocks * 16, meta + max_blocks * 16 + max_desc * 4, max_blocks,
                                  max_desc};
        hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(1024), 0, s, counts, E, dsegs, 3, offsets, plan.prow,
                           plan.desc, plan.count, max_blocks);
        DITCH_TRY_HIP(hipGetLastError());
        hipLaunchKernelGGL(expert_list_kernel, dim3((unsigned)E), dim3(LIST_WAVES * 64), 0, s, sel, n, k, offsets,
                           pair_token, pair_of);
        DITCH_TRY_HIP(hipGetLastError());
        const TileView &vd = L.ed[0].t->v;
        const int64_t ldk_d = split_k_tiles(vd);
        void *fr = m->acts.get<uint8_t>(split_bytes_ldk(max_blocks * 16, ldk_d, 2));
        // routed down deltas: their x . A^T formed by the GLU's epilogue
        float *dxa = nullptr;
        GroupedDeltaXa dx{};
        if (max_rank > 0) {
            dxa = m->e_xa.get<float>(P * max_rank);
            dx = GroupedDeltaXa{dda, dsegs + 2 * E, dxa, P, max_rank, &m->e_xa_part};
        }
        launch_tile_glu_grouped_dev(dsegs, dsegs + E, L.eg[0].t->v, L.eu[0].t->v, 0, nullptr, fr, ldk_d, h, hidden,
                                    pair_token, plan, &m->xsplit, s, max_rank > 0 ? &dx : nullptr, n);
        launch_tile_gemm_grouped_dev(dsegs + 2 * E, vd, eo, hidden, fr, plan, s, dxa, max_rank);
    } else {
    m->moe_host_planned++;
    std::vector<int32_t> hc(E), ho(E);
    DITCH_TRY_HIP(hipMemcpyAsync(hc.data(), counts, E * 4, hipMemcpyDeviceToHost, s));
    DITCH_TRY_HIP(hipStreamSynchronize(s));
    cache_synced(m);
    int32_t acc = 0, max_cnt = 0;
    for (int64_t e = 0; e < E; e++) {
        ho[e] = acc;
        acc += hc[e];
        max_cnt = std::max(max_cnt, hc[e]);
    }
    int64_t P = acc;  // == n * k
    int32_t *offsets = m->r_offsets.get<int32_t>(E);
    DITCH_TRY_HIP(hipMemcpyAsync(offsets, ho.data(), E * 4, hipMemcpyHostToDevice, s));
    int32_t *pair_token = m->r_pair_token.get<int32_t>(P);
    hipLaunchKernelGGL(expert_list_kernel, dim3((unsigned)E), dim3(LIST_WAVES * 64), 0, s, sel, n, k, offsets, pair_token,
                       pair_of);
    DITCH_TRY_HIP(hipGetLastError());
    // segments (experts with tokens), in index order; with expert streaming
    // in chunks of experts resident together in the cache
    std::vector<int32_t> used;
    for (int64_t e = 0; e < E; e++) {
        if (hc[e] == 0) continue;
        DITCH_CHECK(L.eg[e].ok() && L.eu[e].ok() && L.ed[e].ok(), DITCH_INVALID_ARGUMENT, "forward: expert weights missing");
        used.push_back((int32_t)e);
    }
    const bool streamed = !used.empty() && L.eg[used[0]].streamed();
    const int64_t li = &L - m->layers.data();
    float *gate = m->e_gate.get<float>(P * inter), *up = m->e_up.get<float>(P * inter);
    eo = m->e_out.get<float>(P * hidden);
    size_t from = 0;
    while (from < used.size()) {
        std::vector<int> slots;
        size_t cnt = used.size() - from;
        if (streamed) {
            slots = cache_acquire(m, li, used, from, s);
            cnt = slots.size();
        }
        std::vector<GroupSeg> sg, su, sd;
        std::vector<SegDelta> dd;
        int max_rank = 0;
        int32_t max_cnt = 0;
        for (size_t q = 0; q < cnt; q++) {
            const int64_t e = used[from + q];
            TileView vg = L.eg[e].t->v, vu = L.eu[e].t->v, vdn = L.ed[e].t->v;
            if (streamed) expert_views(*m->cache, slots[q], L, e, vg, vu, vdn);
            sg.push_back(GroupSeg{vg, ho[e], hc[e], nullptr, 0});
            su.push_back(GroupSeg{vu, ho[e], hc[e], nullptr, 0});
            sd.push_back(GroupSeg{vdn, ho[e], hc[e], L.ed[e].db, L.ed[e].rank});
            dd.push_back(SegDelta{L.ed[e].da, ho[e], hc[e], L.ed[e].rank});
            max_rank = std::max(max_rank, L.ed[e].rank);
            max_cnt = std::max(max_cnt, hc[e]);
        }
        unsigned nseg = (unsigned)sg.size();
        for (unsigned i = 0; i < nseg; i++)
            DITCH_CHECK(sg[i].w.tf == sg[0].w.tf && su[i].w.tf == su[0].w.tf && sd[i].w.tf == sd[0].w.tf &&
                            sg[i].w.rows == inter && sg[i].w.cols == hidden && sd[i].w.rows == hidden &&
                            sd[i].w.cols == inter,
                        DITCH_INVALID_ARGUMENT, "experts of one layer must share shape and format");
        GroupSeg *dsegs = m->segs.get<GroupSeg>(3 * nseg);
        DITCH_TRY_HIP(hipMemcpyAsync(dsegs, sg.data(), nseg * sizeof(GroupSeg), hipMemcpyHostToDevice, s));
        DITCH_TRY_HIP(hipMemcpyAsync(dsegs + nseg, su.data(), nseg * sizeof(GroupSeg), hipMemcpyHostToDevice, s));
        DITCH_TRY_HIP(hipMemcpyAsync(dsegs + 2 * nseg, sd.data(), nseg * sizeof(GroupSeg), hipMemcpyHostToDevice, s));
        const TileView &vg = sg[0].w, &vd = sd[0].w;
        // gate, up and SwiGLU in one tiled product whose epilogue writes the
        // down product's fragments (f32 rows too when a down delta needs them)
        const bool fused = tile_grouped_takes(sg.data(), nseg, max_cnt) && tile_grouped_takes(sd.data(), nseg, max_cnt) &&
                           tile_glu_takes(vg, su[0].w, 128);
        const void *dfr = nullptr;
        if (fused) {
            const int64_t ldk_d = split_k_tiles(vd);
            void *fr = m->acts.get<uint8_t>(split_bytes_ldk(grouped_blocks(sg.data(), nseg) * 16, ldk_d, 2));
            // a chunk of at least n pairs: the n token rows split once and gathered
            const int64_t chunk_pairs = (int64_t)sg[nseg - 1].off + sg[nseg - 1].cnt - sg[0].off;
            launch_tile_glu_grouped(dsegs, dsegs + nseg, sg.data(), su.data(), nseg, 0, max_rank > 0 ? gate : nullptr,
                                    fr, ldk_d, h, hidden, pair_token, &m->xsplit, &m->gmeta, s,
                                    chunk_pairs >= n ? n : 0);
            dfr = fr;
        } else {
            launch_matmul_grouped(dsegs, sg.data(), nseg, vg.tf, inter, hidden, max_cnt, gate, h, pair_token, nullptr, 0,
                                  s, &m->xsplit, &m->gmeta);
            launch_matmul_grouped(dsegs + nseg, su.data(), nseg, su[0].w.tf, inter, hidden, max_cnt, up, h, pair_token,
                                  nullptr, 0, s, &m->xsplit, &m->gmeta);
            // act(gate) * up on this chunk's pairs (consecutive experts: one run of pairs)
            const int64_t p0 = sg[0].off, p1 = (int64_t)sg[nseg - 1].off + sg[nseg - 1].cnt;
            launch_gated_act(0, gate + p0 * inter, gate + p0 * inter, up + p0 * inter, p1 - p0, inter, inter, inter, s);
        }
        float *dxa = nullptr;
        if (max_rank > 0) {
            SegDelta *dsd = m->segd.get<SegDelta>(nseg);
            DITCH_TRY_HIP(hipMemcpyAsync(dsd, dd.data(), nseg * sizeof(SegDelta), hipMemcpyHostToDevice, s));
            dxa = m->e_xa.get<float>(P * max_rank);
            dim3 grid((unsigned)((max_cnt * max_rank + 3) / 4), nseg);
            hipLaunchKernelGGL(grouped_delta_xa_kernel, grid, dim3(256), 0, s, dxa, gate, nullptr, dsd, inter, max_rank);
            DITCH_TRY_HIP(hipGetLastError());
        }
        if (dfr)
            launch_tile_gemm_grouped(dsegs + 2 * nseg, sd.data(), nseg, eo, hidden, nullptr, inter, nullptr, dxa, max_rank,
                                     &m->xsplit, &m->gmeta, s, dfr);
        else
            launch_matmul_grouped(dsegs + 2 * nseg, sd.data(), nseg, vd.tf, hidden, inter, max_cnt, eo, gate, nullptr,
                                  dxa, max_rank, s, &m->xsplit, &m->gmeta);
        if (streamed) {
            cache_release(m, slots, s);
            // a layer in several chunks: the host tables of this chunk go out
            // of scope before the next is built (the degraded case, when the
            // cache holds fewer experts than the layer routes to)
            if (from + cnt < used.size()) {
                DITCH_TRY_HIP(hipStreamSynchronize(s));
                cache_synced(m);
            }
        }
        from += cnt;
    }
    if (streamed) {
        cache_note_layer(m, li, used);
        cache_prefetch_next(m, li);
    }
    }
    float *esh = nullptr;
    if (L.sh_gate.ok()) {
        int64_t si = L.sh_gate.t->v.rows;
        DITCH_CHECK(L.sh_up.ok() && L.sh_down.ok() && L.sh_up.t->v.rows == si && L.sh_down.t->v.cols == si,
                    DITCH_INVALID_ARGUMENT, "forward: shared expert gate/up/down widths disagree");
        esh = m->e_shared.get<float>(n * hidden);
        if (n >= 128 && L.sh_gate.rank == 0 && L.sh_up.rank == 0 && tile_glu_takes(L.sh_gate.t->v, L.sh_up.t->v, n) &&
            frag_only(L.sh_down, n)) {
            // gate, up and the activation in one tiled product whose epilogue
            // writes the down product's fragments (as the dense layers' MLP)
            const int64_t ldk_h = split_ldk(hidden), ldk_i = split_ldk(si);
            void *hs = m->hs.get<uint8_t>(split_bytes_ldk(n, ldk_h, 2));
            launch_split(hs, h, nullptr, n, hidden, hidden, ldk_h, 2, s);
            void *as = m->acts.get<uint8_t>(split_bytes_ldk(n, ldk_i, 2));
            launch_tile_glu(L.sh_gate.t->v, L.sh_up.t->v, 0, nullptr, as, ldk_i, hs, ldk_h, n, s);
            mm_act(m, L.sh_down, esh, Act{nullptr, as, ldk_i}, n, nullptr, 0, s);
        } else {
            float *sgb = m->g.get<float>(n * si), *sub = m->u.get<float>(n * si);
            mm(m, L.sh_gate, sgb, h, n, nullptr, 0, s);
            mm(m, L.sh_up, sub, h, n, nullptr, 0, s);
            launch_gated_act(0, sgb, sgb, sub, n, si, si, si, s);
            mm(m, L.sh_down, esh, sgb, n, nullptr, 0, s);
        }
    }
    // a wave of 64 threads covers 256 columns; grid_for's block count keeps
    // every grid-stride step a whole number of waves
    if (hidden % 256 == 0 && n * (hidden / 4) < INT32_MAX)
        hipLaunchKernelGGL(moe_combine_kernel<true>, dim3(grid_for(n * ((hidden + 3) / 4))), dim3(256), 0, s, x, eo,
                           esh, ord, selw, pair_of, n, k, hidden);
    else
        hipLaunchKernelGGL(moe_combine_kernel<false>, dim3(grid_for(n * ((hidden + 3) / 4))), dim3(256), 0, s, x, eo,
                           esh, ord, selw, pair_of, n, k, hidden);
    DITCH_TRY_HIP(hipGetLastError());
}

// `B` prompt slots of `T` positions size the KV cache (KvCache.initFor,
// engine.zig:388-390); rows outside it are skipped by the kernels that read
// the row descriptors.
// With `pc`, the keys and values of every layer live in that persistent
// cache (its B x T), so later calls attend to the positions earlier calls
// wrote (decode steps after a prefill).
void model_forward(ditch_hip_model *m, const uint32_t *d_tokens, const ditch_row *d_rows, int64_t n, int64_t B,
                   int64_t T, const uint64_t *d_capture, int64_t n_capture, float *d_res, const uint64_t *d_logit_rows,
                   int64_t n_logit, float *d_logits, ditch_hip_kv_cache *pc) {
    const ditch_model_config &c = m->c;
    hipStream_t s = m->h->stream;
    if (n <= 0) return;
    DITCH_CHECK(m->embed.ok(), DITCH_INVALID_ARGUMENT, "forward: no embedding");
    int64_t hidden = (int64_t)c.hidden;
    DITCH_CHECK(B > 0 && T > 0 && B <= (int64_t)INT32_MAX, DITCH_INVALID_ARGUMENT, "forward: KV cache shape");
    DITCH_CHECK(T <= ATT_MAXK, DITCH_UNSUPPORTED, "forward: positions beyond 1024 per prompt");
    int64_t nh = (int64_t)c.heads, nkv = c.mla ? nh : (int64_t)c.kv_heads, hd = (int64_t)c.head_dim;
    int64_t vd = c.mla ? (int64_t)c.v_head_dim : hd;
    DITCH_CHECK(hd <= 512, DITCH_UNSUPPORTED, "forward: head_dim above 512");
    int64_t qd = nh * hd, kvd = nkv * hd;
    float *x = m->x.get<float>(n * hidden);
    float *h = m->hbuf.get<float>(n * hidden);
    float *q = m->q.get<float>(n * qd), *kk = m->k.get<float>(n * kvd), *vv = m->v.get<float>(n * kvd);
    float *att = m->att.get<float>(n * nh * vd);
    if (pc) {
        DITCH_CHECK(pc->m == m && pc->B == B && pc->T == T && pc->kvd == kvd, DITCH_INVALID_ARGUMENT,
                    "forward: the KV cache belongs to another model or shape");
    }
    float *kc = pc ? pc->k : m->kc.get<float>(B * T * kvd), *vc = pc ? pc->v : m->vc.get<float>(B * T * kvd);
    int *dense_flag = m->attn_dense.get<int>(1);  // checked at the first layer that can use it
    bool dense_checked = false;

    hipLaunchKernelGGL(embed_kernel, dim3(grid_for(n * hidden)), dim3(256), 0, s, x, m->embed.t->v, d_tokens, n);
    DITCH_TRY_HIP(hipGetLastError());
    auto capture = [&](int64_t entry) {
        if (!d_res || n_capture == 0) return;
        hipLaunchKernelGGL(capture_kernel, dim3(grid_for(n_capture * hidden)), dim3(256), 0, s,
                           d_res + entry * n_capture * hidden, x, d_capture, n_capture, hidden, n);
        DITCH_TRY_HIP(hipGetLastError());
    };
    capture(0);
    // Large batches hand the products pre-split A fragments written by the
    // producing kernel (RMS norm, attention, the gate/up product); f32 rows
    // are kept only for consumers that need them.
    const bool frags = n >= 128;
    const int64_t ldk_h = split_ldk(hidden);
    for (int64_t li = 0; li < (int64_t)c.layers; li++) {
        Layer &L = m->layers[li];
        Act hact{h, nullptr, 0};
        const bool mx_qkv = frags && !c.mla && mx_only(L.q, n) && mx_only(L.k, n) && mx_only(L.v, n) &&
                            L.q.t->v.units_k == L.k.t->v.units_k && L.q.t->v.units_k == L.v.t->v.units_k;
        if (mx_qkv) {
            const int64_t ldst = L.q.t->v.units_k;
            void *hm = m->hs.get<uint8_t>(mx_frag_bytes(n, ldst));
            launch_rmsnorm_split_mx(hm, ldst, nullptr, x, L.attn_norm.p, L.attn_norm.len, n, hidden, c.rms_eps, 0, s);
            hact = Act{nullptr, nullptr, 0, hm, ldst};
        } else if (frags) {
            // the f32 rows only for a product that cannot take the fragments
            // alone (MLA: q_a and kv_a, or q_b without a q_a; an MXFP4 one
            // keeps its scaled-MFMA path, which splits the f32 rows itself)
            const Mat &mq = L.q_a.ok() ? L.q_a : L.q_b;
            const bool f32_needed =
                c.mla ? !frag_only(L.kv_a, n) || !frag_only(mq, n) || mx_only(L.kv_a, n) || mx_only(mq, n)
                      : !frag_only(L.q, n) || !frag_only(L.k, n) || !frag_only(L.v, n);
            void *hs = m->hs.get<uint8_t>(split_bytes_ldk(n, ldk_h, 2));
            launch_rmsnorm_split(hs, ldk_h, f32_needed ? h : nullptr, x, L.attn_norm.p, L.attn_norm.len, n, hidden,
                                 c.rms_eps, 0, s);
            hact = Act{f32_needed ? h : nullptr, hs, ldk_h};
        } else {
            launch_rmsnorm(h, x, L.attn_norm.p, L.attn_norm.len, n, hidden, c.rms_eps, 0, s);
        }
        // MLA: keys and values go to the cache in one kernel with the RoPE
        bool mla_fused = false;
        const float *mla_kvb = nullptr, *mla_kva = nullptr;
        if (c.mla) {
            int64_t nope = (int64_t)c.qk_nope_dim, rd = (int64_t)c.qk_rope_dim, kvl = (int64_t)c.kv_lora_rank;
            if (L.q_a.ok()) {
                int64_t qlr = (int64_t)c.q_lora_rank;
                float *qa = m->mla_a.get<float>(n * qlr);
                mm_act(m, L.q_a, qa, hact, n, nullptr, 0, s);
                launch_rmsnorm(qa, qa, L.q_a_norm.p, L.q_a_norm.len, n, qlr, c.mla_norm_eps, 0, s);
                mm(m, L.q_b, q, qa, n, nullptr, 0, s);
            } else {
                mm_act(m, L.q_b, q, hact, n, nullptr, 0, s);
            }
            float *kva = m->mla_b.get<float>(n * (kvl + rd));
            mm_act(m, L.kv_a, kva, hact, n, nullptr, 0, s);
            float *ckv = m->mla_c.get<float>(n * kvl);
            launch_rmsnorm_strided(ckv, kva, L.kv_a_norm.p, L.kv_a_norm.len, n, kvl, kvl + rd, kvl, c.mla_norm_eps, s);
            float *kvb = m->o.get<float>(n * nh * (nope + vd));
            mm(m, L.kv_b, kvb, ckv, n, nullptr, 0, s);
            mla_fused = !c.qk_norm && hd == nope + rd && rd <= 512 && vd <= hd && hd % 4 == 0 && nope % 4 == 0 &&
                        vd % 4 == 0 && kvl % 4 == 0 && rd % 4 == 0 && 2 * (int64_t)(c.rotary_dim / 2) <= rd;
            if (mla_fused) {
                mla_kvb = kvb;
                mla_kva = kva;
            } else {
                hipLaunchKernelGGL(mla_assemble_kernel, dim3(grid_for(n * nh * hd)), dim3(256), 0, s, kk, vv, kvb, kva,
                                   n, nh, hd, nope, rd, vd, kvl);
                DITCH_TRY_HIP(hipGetLastError());
            }
        } else {
            mm_act(m, L.q, q, hact, n, L.q_bias.p, 0, s);
            mm_act(m, L.k, kk, hact, n, L.k_bias.p, 0, s);
            mm_act(m, L.v, vv, hact, n, L.v_bias.p, 0, s);
        }
        if (pc) {  // this layer's slice of the persistent cache
            kc = pc->k + li * B * T * kvd;
            vc = pc->v + li * B * T * kvd;
        }
        // the attention kernels this layer takes; with the whole-prompt kernel
        // (decided on the device by the dense check) and a whole-head neox
        // RoPE of head_dim 128 without a query norm, that kernel rotates the
        // queries as it loads them and the RoPE kernel leaves them alone
        const bool mfma_attn = attention_mfma_takes(hd, vd, nh / nkv);
        const bool frag_epi = attn_split_fragments && frags && mfma_attn && (nh * vd) % 128 == 0 &&
                              frag_only(L.o, n) && !mx_only(L.o, n);
        const bool prompt_attn = mfma_attn && !frag_epi && attention_prompt_takes(hd, vd, T);
        const bool q_rope_in_attn = prompt_attn && !c.mla && hd == 128 && c.rotary_dim == 128 &&
                                    c.rope_style == DITCH_ROPE_NEOX && !c.qk_norm;
        if (prompt_attn && !dense_checked) {
            launch_attention_dense_check(d_rows, n, T, B, dense_flag, s);
            dense_checked = true;
        }
        RopeArgs ra{};
        ra.q = q;
        ra.k = kk;
        ra.v = vv;
        ra.kc = kc;
        ra.vc = vc;
        ra.rows = d_rows;
        ra.cos_t = m->rope_cos;
        ra.sin_t = m->rope_sin;
        ra.q_norm = c.qk_norm ? L.q_norm.p : nullptr;
        ra.k_norm = c.qk_norm ? L.k_norm.p : nullptr;
        ra.n = n;
        ra.heads = nh;
        ra.kv_heads = nkv;
        ra.hd = hd;
        ra.rope_off = c.mla ? (int64_t)c.qk_nope_dim : 0;
        ra.rot = (int64_t)(c.rotary_dim / 2 * 2);
        ra.half = (int64_t)(c.rotary_dim / 2);
        ra.rope_len = (int64_t)c.rope_len;
        ra.T = T;
        ra.nb = B;
        ra.kvd = kvd;
        ra.eps = c.rms_eps;
        ra.style = c.rope_style;
        ra.dense = q_rope_in_attn ? dense_flag : nullptr;
        ra.q_in_attn = q_rope_in_attn ? 1 : 0;
        if (mla_fused) {
            MlaCacheArgs ma{q, mla_kvb, mla_kva, kc, vc, d_rows, m->rope_cos, m->rope_sin, nh, hd,
                            (int64_t)c.qk_nope_dim, (int64_t)c.qk_rope_dim, vd, (int64_t)c.kv_lora_rank, ra.half,
                            ra.rope_len, T, B, kvd, c.rope_style};
            hipLaunchKernelGGL(mla_rope_cache_kernel, dim3((unsigned)n), dim3(256), 0, s, ma);
        } else {
            hipLaunchKernelGGL(qk_rope_cache_kernel, dim3((unsigned)n), dim3(256), 0, s, ra);
        }
        DITCH_TRY_HIP(hipGetLastError());
        AttnArgs aa{q, kc, vc, att, d_rows, n, nh, nh / nkv, hd, vd, T, kvd, c.attn_scale, nullptr, 0, B, nullptr};
        Act aact{att, nullptr, 0};
        // (the kernel's own bf16-fragment epilogue needs 34 KB more LDS a
        // workgroup, which halves its occupancy: the o product splitting the
        // f32 rows costs less)
        if (frag_epi) {
            aa.ldk = split_ldk(nh * vd);
            aa.xs = m->atts.get<uint8_t>(split_bytes_ldk(n, aa.ldk, 2));
            aact = Act{att, aa.xs, aa.ldk};
        }
        if (prompt_attn) aa.dense = dense_flag;
        if (q_rope_in_attn) launch_attention_mfma_rope(aa, AttnRope{m->rope_cos, m->rope_sin, (int64_t)c.rope_len}, nkv, s);
        else if (mfma_attn) launch_attention_mfma(aa, nkv, s);
        else hipLaunchKernelGGL(attention_kernel, dim3((unsigned)((n * nh + 3) / 4)), dim3(256), 0, s, aa);
        DITCH_TRY_HIP(hipGetLastError());
        mm_act(m, L.o, x, aact, n, nullptr, 1, s);  // x += o(att)
        const bool moe_layer = c.n_experts && m->moe_layers[li];
        if (!moe_layer)
            DITCH_CHECK(L.gate.ok() && L.up.ok() && L.down.ok() && L.up.t->v.rows == L.gate.t->v.rows &&
                            L.down.t->v.cols == L.gate.t->v.rows,
                        DITCH_INVALID_ARGUMENT, "forward: gate/up/down missing or their widths disagree");
        // MXFP4 gate/up in one scaled-MFMA product whose epilogue applies the
        // activation and writes the down projection's MX fragments
        const bool mx_glu = frags && !moe_layer && L.gate.ok() && L.up.ok() && L.gate.rank == 0 && L.up.rank == 0 &&
                            mx_glu_takes(L.gate.t->v, L.up.t->v, n) && L.gate.t->v.rows % 128 == 0 &&
                            mx_only(L.down, n) && L.down.t->v.units_k * 128 == L.gate.t->v.rows;
        if (mx_glu) {
            const int64_t ldst = L.gate.t->v.units_k, ldst_i = L.down.t->v.units_k;
            void *hm = m->hs.get<uint8_t>(mx_frag_bytes(n, ldst));
            launch_rmsnorm_split_mx(hm, ldst, nullptr, x, L.ffn_norm.p, L.ffn_norm.len, n, hidden, c.rms_eps, 0, s);
            void *am = m->acts.get<uint8_t>(mx_frag_bytes(n, ldst_i));
            launch_mx_glu(L.gate.t->v, L.up.t->v, 0, nullptr, am, ldst_i, hm, ldst, n, s);
            mm_act(m, L.down, x, Act{nullptr, nullptr, 0, am, ldst_i}, n, nullptr, 1, s);  // x += down(act)
            capture(li + 1);
            continue;
        }
        // gate and up in one tiled product whose epilogue applies the
        // activation and writes the down projection's fragments
        const bool glu = frags && !moe_layer && L.gate.ok() && L.up.ok() && L.gate.rank == 0 && L.up.rank == 0 &&
                         tile_glu_takes(L.gate.t->v, L.up.t->v, n) && frag_only(L.down, n);
        if (glu) {
            void *hs = m->hs.get<uint8_t>(split_bytes_ldk(n, ldk_h, 2));
            launch_rmsnorm_split(hs, ldk_h, nullptr, x, L.ffn_norm.p, L.ffn_norm.len, n, hidden, c.rms_eps, 0, s);
            const int64_t inter = L.gate.t->v.rows, ldk_i = split_ldk(inter);
            void *as = m->acts.get<uint8_t>(split_bytes_ldk(n, ldk_i, 2));
            launch_tile_glu(L.gate.t->v, L.up.t->v, 0, nullptr, as, ldk_i, hs, ldk_h, n, s);
            mm_act(m, L.down, x, Act{nullptr, as, ldk_i}, n, nullptr, 1, s);  // x += down(act)
            capture(li + 1);
            continue;
        }
        launch_rmsnorm(h, x, L.ffn_norm.p, L.ffn_norm.len, n, hidden, c.rms_eps, 0, s);
        if (moe_layer) {
            moe_forward(m, L, x, h, n, s);
        } else {
            int64_t inter = L.gate.t->v.rows;
            float *g = m->g.get<float>(n * inter), *u = m->u.get<float>(n * inter);
            mm(m, L.gate, g, h, n, nullptr, 0, s);
            mm(m, L.up, u, h, n, nullptr, 0, s);
            launch_gated_act(0, g, g, u, n, inter, inter, inter, s);
            mm(m, L.down, x, g, n, nullptr, 1, s);  // x += down(act)
        }
        capture(li + 1);
    }
    if (n_logit > 0 && d_logits) {
        float *hl = m->logit_h.get<float>(n_logit * hidden);
        launch_rmsnorm(hl, x, m->final_norm.p, m->final_norm.len, n_logit, hidden, c.rms_eps, 0, s,
                       (const int64_t *)d_logit_rows, n);
        const Mat &lm = m->lm_head.ok() ? m->lm_head : m->embed;
        mm(m, lm, d_logits, hl, n_logit, nullptr, 0, s);
    }
}

// RoPE tables (model.zig:2200-2282), computed in f64 on the host as the
// reference does.
static void host_fill_rope(const ditch_model_config &c, std::vector<float> &cos_t, std::vector<float> &sin_t) {
    size_t len = c.rope_len, dim = c.rotary_dim, half = dim / 2;
    cos_t.assign(len * half, 0.f);
    sin_t.assign(len * half, 0.f);
    if (half == 0) return;
    std::vector<double> inv(half);
    double theta = (double)c.rope_theta;
    for (size_t i = 0; i < half; i++) inv[i] = 1.0 / pow(theta, (double)(2 * i) / (double)dim);
    double attention_factor = 1.0;
    const double pi = 3.14159265358979323846;
    if (c.rope_scaling == DITCH_ROPE_SCALING_LINEAR) {
        for (auto &f : inv) f /= (double)c.rope_factor;
    } else if (c.rope_scaling == DITCH_ROPE_SCALING_LLAMA3) {
        double low_wavelen = (double)(c.rope_original_max_position / c.rope_low_freq_factor);
        double high_wavelen = (double)(c.rope_original_max_position / c.rope_high_freq_factor);
        double band = (double)(c.rope_high_freq_factor - c.rope_low_freq_factor);
        for (auto &f : inv) {
            double wavelen = 2.0 * pi / f;
            if (wavelen < high_wavelen) {
            } else if (wavelen > low_wavelen) {
                f /= (double)c.rope_factor;
            } else {
                double smooth = ((double)c.rope_original_max_position / wavelen - (double)c.rope_low_freq_factor) / band;
                f = (1.0 - smooth) * f / (double)c.rope_factor + smooth * f;
            }
        }
    } else if (c.rope_scaling == DITCH_ROPE_SCALING_YARN) {
        double dimf = (double)dim, maxp = (double)c.rope_original_max_position;
        double low = (dimf * log(maxp / ((double)c.yarn_beta_fast * 2.0 * pi))) / (2.0 * log(theta));
        double high = (dimf * log(maxp / ((double)c.yarn_beta_slow * 2.0 * pi))) / (2.0 * log(theta));
        if (c.yarn_truncate) {
            low = floor(low);
            high = ceil(high);
        }
        if (low < 0) low = 0;
        if (high > dimf - 1) high = dimf - 1;
        if (low == high) high += 0.001;
        for (size_t i = 0; i < half; i++) {
            double ramp = ((double)i - low) / (high - low);
            ramp = ramp < 0 ? 0 : ramp > 1 ? 1 : ramp;
            double extrapolation = 1.0 - ramp;
            double interp = inv[i] / (double)c.rope_factor;
            inv[i] = interp * (1.0 - extrapolation) + inv[i] * extrapolation;
        }
        attention_factor = (double)c.yarn_attention_factor;
    } else if (c.rope_scaling == DITCH_ROPE_SCALING_FACTORS && c.rope_factors) {
        for (size_t i = 0; i < half; i++) inv[i] /= (double)c.rope_factors[i];
    }
    for (size_t pos = 0; pos < len; pos++)
        for (size_t i = 0; i < half; i++) {
            double angle = (double)pos * inv[i];
            cos_t[pos * half + i] = (float)(cos(angle) * attention_factor);
            sin_t[pos * half + i] = (float)(sin(angle) * attention_factor);
        }
}

}  // namespace ditch

ditch_hip_kv_cache::~ditch_hip_kv_cache() {
    ditch::dev_free(k);
    ditch::dev_free(v);
}

namespace ditch {

ditch_hip_kv_cache *kv_cache_create(ditch_hip_model *m, int64_t B, int64_t T) {
    const ditch_model_config &c = m->c;
    DITCH_CHECK(B > 0 && T > 0 && T <= ATT_MAXK && B <= (int64_t)INT32_MAX, DITCH_INVALID_ARGUMENT,
                "kv cache: 1..1024 positions and at least one prompt");
    const int64_t nkv = c.mla ? (int64_t)c.heads : (int64_t)c.kv_heads;
    auto *kc = new ditch_hip_kv_cache();
    kc->m = m;
    kc->B = B;
    kc->T = T;
    kc->kvd = nkv * (int64_t)c.head_dim;
    kc->layers = (int64_t)c.layers;
    const size_t bytes = (size_t)(kc->layers * B * T * kc->kvd) * 4;
    try {
        kc->k = (float *)dev_alloc(bytes);
        kc->v = (float *)dev_alloc(bytes);
    } catch (...) {
        delete kc;
        throw;
    }
    return kc;
}

}  // namespace ditch

ditch_hip_model::~ditch_hip_model() {
    delete cache;  // drains its copy stream before the host blobs go
    cache = nullptr;
    for (auto &L : layers) {
        for (ditch::Vec *v : {&L.attn_norm, &L.q_bias, &L.k_bias, &L.v_bias, &L.q_norm, &L.k_norm, &L.ffn_norm,
                              &L.corr, &L.q_a_norm, &L.kv_a_norm})
            v->release();
        for (ditch::Mat *mt : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down, &L.router, &L.sh_gate, &L.sh_up,
                               &L.sh_down, &L.q_a, &L.q_b, &L.kv_a, &L.kv_b})
            mt->release();
        for (auto *vec : {&L.eg, &L.eu, &L.ed})
            for (auto &mt : *vec) mt.release();
    }
    embed.release();
    lm_head.release();
    final_norm.release();
    ditch::dev_free(rope_cos);
    ditch::dev_free(rope_sin);
}
