// attention.hip — prompt attention on the fp32 matrix cores.
//
// For every row (query token) and head: scores[p] = scale * dot(q, k_p) over
// the keys p <= pos of the row's prompt, softmax (max, Cephes exp of the
// difference, sum), out = sum_p softmax_p * v_p: the per-(row, head) work of
// model.zig:2935-2986 (attentionWorker) with the GQA head mapping of
// model.zig:4314 and the KV slot layout [prompt][position][kv_dim].
//
// A workgroup takes 16 consecutive rows and one KV head; each wave is one
// query head of that KV head's group. Keys and values are staged in LDS in
// chunks of 32 positions (shared by the group's waves) and multiplied on
// v_mfma_f32_16x16x4f32, whose products are exact: only the order of the f32
// additions differs from the CPU's dot products. The softmax is two-pass in
// the reference's order: the row maximum over every key first, then
// exp(s - max), the sum, and the value accumulation; the output is scaled by
// 1/sum at the end. Rows of the block that belong to different prompts are
// processed one prompt at a time.
#include "decode.h"
#include "gemm_common.h"
#include "internal.h"

namespace ditch {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// max / sum over the 16 lanes that share lane / 16
__device__ __forceinline__ float max16(float v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v = __fadd_rn(v, __shfl_xor(v, o, 64));
    return v;
}

constexpr int AK = 32;  // keys per LDS chunk

// MFMA operand layouts (v_mfma_f32_16x16x4f32): A lane l = row l%16, k l/16;
// B lane l = k l/16, column l%16; D lane l = rows 4*(l/16) + r, column l%16.
// The k index of step j is assigned per lane group g = l/16: QK^T steps over
// head dims g*HD/4 + j, PV steps over keys (AK/4) g + j, so every lane reads
// contiguous runs (ds_read_b128) from padded, bank-conflict-free rows.
template <int HD, int VD, int NW, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void attn_mfma_kernel(AttnArgs a) {
    constexpr int KS = HD + 4;  // K row stride (floats)
    constexpr int VS = AK + 4;  // transposed V row stride
    constexpr int PS = AK + 4;  // P row stride
    constexpr int QJ = HD / 4;  // QK^T k steps
    constexpr int VB = VD / 16; // output column blocks
    static_assert(HD % 16 == 0 && VD % 16 == 0, "head dims");
    __shared__ float Ks[AK * KS];
    __shared__ float Vt[VD * VS];
    __shared__ float Ps[NW][16 * PS];
    __shared__ int32_t rb[16], rp[16];
    // SPLIT: the block's finished output rows per wave, for the fragments
    constexpr int OS = VD + 4;
    __shared__ float Ot[SPLIT ? NW : 1][SPLIT ? 16 * OS : 1];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t r0 = (int64_t)blockIdx.x * 16;
    const int64_t hkv = blockIdx.y;
    const int64_t hq = (int64_t)blockIdx.z * NW + wave;  // query head within the group
    const bool head_ok = hq < a.groups;
    const int64_t h = hkv * a.groups + (head_ok ? hq : 0);
    if (threadIdx.x < 16) {
        int64_t r = r0 + threadIdx.x;
        rb[threadIdx.x] = r < a.n ? (int32_t)a.rows[r].b : -1;
        rp[threadIdx.x] = r < a.n ? (int32_t)a.rows[r].pos : -1;
    }
    if constexpr (SPLIT) {
        for (int i = lane; i < 16 * OS; i += 64) Ot[wave][i] = 0.f;
    }
    __syncthreads();

    // this lane's query (A operand): row c16, head dims g*QJ .. +QJ
    float qv[QJ];
    {
        const int64_t r = r0 + c16;
        const bool ok = head_ok && r < a.n;
        const float *q = a.q + ((ok ? r : 0) * a.heads + h) * a.hd + g * QJ;
#pragma unroll
        for (int j = 0; j < QJ; j += 4) {
            float4 v = ok ? *(const float4 *)(q + j) : make_float4(0.f, 0.f, 0.f, 0.f);
            qv[j] = v.x; qv[j + 1] = v.y; qv[j + 2] = v.z; qv[j + 3] = v.w;
        }
    }

    const int nthreads = NW * 64;
    auto stage = [&](int64_t b, int64_t c0, int64_t kmax, bool with_v) {
        const float *kb = a.kc + (b * a.T) * a.kvd + hkv * a.hd;
        const float *vb = a.vc + (b * a.T) * a.kvd + hkv * a.hd;
        for (int i = threadIdx.x; i < AK * (HD / 4); i += nthreads) {
            const int key = i / (HD / 4), d = (i % (HD / 4)) * 4;
            const int64_t p = c0 + key;
            float4 v = p <= kmax ? *(const float4 *)(kb + p * a.kvd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
            *(float4 *)&Ks[key * KS + d] = v;
        }
        if (with_v) {
            for (int i = threadIdx.x; i < AK * (VD / 4); i += nthreads) {
                const int key = i / (VD / 4), d = (i % (VD / 4)) * 4;
                const int64_t p = c0 + key;
                float4 v = p <= kmax ? *(const float4 *)(vb + p * a.kvd + d) : make_float4(0.f, 0.f, 0.f, 0.f);
                Vt[(d + 0) * VS + key] = v.x;
                Vt[(d + 1) * VS + key] = v.y;
                Vt[(d + 2) * VS + key] = v.z;
                Vt[(d + 3) * VS + key] = v.w;
            }
        }
    };
    // scores of the staged chunk's key blocks (16 keys each), D layout,
    // masked; the blocks' MFMA chains are interleaved
    constexpr int KB = AK / 16;
    auto scores = [&](floatx4 (&s)[KB], int64_t c0, const int (&pos)[4]) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) s[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < QJ; j += 4) {
#pragma unroll
            for (int kb = 0; kb < KB; kb++) {
                float4 k4 = *(const float4 *)&Ks[(kb * 16 + c16) * KS + g * QJ + j];
                s[kb] = mfma4(qv[j], k4.x, s[kb]);
                s[kb] = mfma4(qv[j + 1], k4.y, s[kb]);
                s[kb] = mfma4(qv[j + 2], k4.z, s[kb]);
                s[kb] = mfma4(qv[j + 3], k4.w, s[kb]);
            }
        }
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int64_t key = c0 + kb * 16 + c16;
#pragma unroll
            for (int r = 0; r < 4; r++) s[kb][r] = key <= pos[r] ? __fmul_rn(s[kb][r], a.scale) : -INFINITY;
        }
    };

    int done = 0;
    for (;;) {
        // the next prompt among the block's rows
        int first = -1;
        for (int i = 0; i < 16; i++)
            if (!((done >> i) & 1) && rb[i] >= 0) {
                first = i;
                break;
            }
        if (first < 0) break;
        const int64_t b = rb[first];
        int in_mask = 0, kmax = -1;
        for (int i = 0; i < 16; i++)
            if (rb[i] == b) {
                in_mask |= 1 << i;
                kmax = rp[i] > kmax ? rp[i] : kmax;
            }
        done |= in_mask;
        // positions of this lane's four D-layout rows (-1: not in this prompt)
        int pos[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = 4 * g + r;
            pos[r] = ((in_mask >> row) & 1) ? rp[row] : -1;
        }

        // pass 1: the row maxima
        float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        for (int64_t c0 = 0; c0 <= kmax; c0 += AK) {
            __syncthreads();
            stage(b, c0, kmax, false);
            __syncthreads();
            floatx4 sc[KB];
            scores(sc, c0, pos);
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) m[r] = fmaxf(m[r], sc[kb][r]);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) m[r] = max16(m[r]);

        // pass 2: exp, sums and P V
        float sum[4] = {0.f, 0.f, 0.f, 0.f};
        floatx4 o[VB];
#pragma unroll
        for (int db = 0; db < VB; db++) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
        float *P = Ps[wave];
        for (int64_t c0 = 0; c0 <= kmax; c0 += AK) {
            __syncthreads();
            stage(b, c0, kmax, true);
            __syncthreads();
            floatx4 sc[KB];
            scores(sc, c0, pos);
#pragma unroll
            for (int kb = 0; kb < KB; kb++) {
                const floatx4 &s = sc[kb];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float e = pos[r] >= 0 && s[r] != -INFINITY ? exp_cephes(__fsub_rn(s[r], m[r])) : 0.f;
                    sum[r] = __fadd_rn(sum[r], e);
                    P[(4 * g + r) * PS + kb * 16 + c16] = e;
                }
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            // out[row][dim] += sum_key P[row][key] V[key][dim]; keys (AK/4) g + j
            constexpr int KG = AK / 4;
            const float *pa = &P[c16 * PS + KG * g];
#pragma unroll
            for (int j = 0; j < KG; j += 4) {
                float4 p4 = *(const float4 *)(pa + j);
#pragma unroll
                for (int db = 0; db < VB; db++) {
                    float4 v4 = *(const float4 *)&Vt[(db * 16 + c16) * VS + KG * g + j];
                    o[db] = mfma4(p4.x, v4.x, o[db]);
                    o[db] = mfma4(p4.y, v4.y, o[db]);
                    o[db] = mfma4(p4.z, v4.z, o[db]);
                    o[db] = mfma4(p4.w, v4.w, o[db]);
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float t = sum16(sum[r]);
            inv[r] = t > 0.f ? __fdiv_rn(1.0f, t) : 0.f;
        }
        if (head_ok) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (pos[r] < 0) continue;
                float *orow = a.out + ((r0 + 4 * g + r) * a.heads + h) * a.vd;
#pragma unroll
                for (int db = 0; db < VB; db++) {
                    const float y = __fmul_rn(o[db][r], inv[r]);
                    orow[db * 16 + c16] = y;
                    if constexpr (SPLIT) Ot[wave][(4 * g + r) * OS + db * 16 + c16] = y;
                }
            }
        }
    }
    if constexpr (SPLIT) {
        // this head's k tiles (k = h * vd + dim) of the block's 16 rows
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        if (head_ok) {
            u32x4 *xs = (u32x4 *)a.xs;
#pragma unroll
            for (int kt = 0; kt < VD / 32; kt++) {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = Ot[wave][c16 * OS + kt * 32 + 8 * g + j];
                u32x4 words[2];
                a_words<false, 2>(v, words);
                const int64_t ktg = (h * VD) / 32 + kt;
#pragma unroll
                for (int e = 0; e < 2; e++) xs[(((int64_t)blockIdx.x * a.ldk + ktg) * 2 + e) * 64 + lane] = words[e];
            }
        }
    }
}

bool attention_mfma_takes(int64_t hd, int64_t vd, int64_t groups) {
    return groups >= 1 && ((hd == 64 && vd == 64) || (hd == 128 && vd == 128) || (hd == 192 && vd == 128));
}

template <int HD, int VD, int NW>
static void launch_attn_nw(const AttnArgs &a, int64_t kv_heads, hipStream_t s) {
    dim3 grid((unsigned)((a.n + 15) / 16), (unsigned)kv_heads, (unsigned)((a.groups + NW - 1) / NW));
    if (a.xs) {
        DITCH_CHECK((a.heads * VD) % 128 == 0 && a.ldk * 32 >= a.heads * VD, DITCH_INVALID_ARGUMENT,
                    "attention: fragment output needs heads * v_head_dim a multiple of 128");
        hipLaunchKernelGGL((attn_mfma_kernel<HD, VD, NW, true>), grid, dim3(NW * 64), 0, s, a);
    } else {
        hipLaunchKernelGGL((attn_mfma_kernel<HD, VD, NW, false>), grid, dim3(NW * 64), 0, s, a);
    }
}

// one wave per query head of the group, up to four per workgroup
template <int HD, int VD>
static void launch_attn(const AttnArgs &a, int64_t kv_heads, hipStream_t s) {
    if (a.groups >= 4) launch_attn_nw<HD, VD, 4>(a, kv_heads, s);
    else if (a.groups == 2 || a.groups == 3) launch_attn_nw<HD, VD, 2>(a, kv_heads, s);
    else launch_attn_nw<HD, VD, 1>(a, kv_heads, s);
}

void launch_attention_mfma(const AttnArgs &a, int64_t kv_heads, hipStream_t s) {
    if (a.hd == 64) launch_attn<64, 64>(a, kv_heads, s);
    else if (a.hd == 128) launch_attn<128, 128>(a, kv_heads, s);
    else launch_attn<192, 128>(a, kv_heads, s);
    DITCH_TRY_HIP(hipGetLastError());
}

}  // namespace ditch
