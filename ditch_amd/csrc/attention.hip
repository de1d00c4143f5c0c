// attention.hip — prompt attention on the bf16 matrix cores.
//
// For every row (query token) and head: scores[p] = scale * dot(q, k_p) over
// the keys p <= pos of the row's prompt, softmax (max, Cephes exp of the
// difference, sum), out = sum_p softmax_p * v_p: the per-(row, head) work of
// model.zig:2935-2986 (attentionWorker) with the GQA head mapping of
// model.zig:4314 and the KV slot layout [prompt][position][kv_dim].
//
// A workgroup takes 16 consecutive rows and one KV head; each wave is one
// query head of that KV head's group. Keys and values are staged in LDS in
// chunks of 32 positions (shared by the group's waves), each f32 value as
// two bf16 terms (hi = rne(v), lo = rne(v - hi)), and multiplied on
// v_mfma_f32_16x16x32_bf16 with three products per pair of operands
// (hi.hi + hi.lo + lo.hi): each product of two f32 values is taken to within
// 2^-16 of its magnitude, and the f32 accumulation order differs from the
// CPU's dot products. The scores are computed transposed (keys x rows), so
// the lanes that hold a row's scores also hold the A operand of P.V with the
// k index running over their own keys, and the value operand is read for
// the same keys: no transposition of P. The softmax is two-pass in the
// reference's order: the row maximum over every key first (the scores of up
// to CACHED chunks kept in LDS, each lane its own, longer prompts'
// recomputed), then
// exp(s - max), the sum and the value accumulation; the output is scaled by
// 1/sum at the end. Rows of the block that belong to different prompts are
// processed one prompt at a time.
#include "decode.h"
#include "gemm_common.h"
#include "internal.h"
#include "attention_rope.h"

namespace ditch {

constexpr int AK = 32;      // keys per LDS chunk
constexpr int CACHED = 4;   // chunks whose scores stay in LDS between the passes

// bf16 terms of two f32 values: hi = rne pair, lo = rne pair of the remainders
__device__ __forceinline__ uint2 split_pair(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f2_t __attribute__((ext_vector_type(2)));
    const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{a, b}, bf16x2_t));
    const float ra = __fsub_rn(a, u2f(hi << 16)), rb = __fsub_rn(b, u2f(hi & 0xffff0000u));
    return make_uint2(hi, __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{ra, rb}, bf16x2_t)));
}
// the four pairs of 8 values as the hi and lo words of an MFMA operand
__device__ __forceinline__ void split8_words(const float (&v)[8], u32x4 &hi, u32x4 &lo) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint2 t = split_pair(v[2 * j], v[2 * j + 1]);
        hi[j] = t.x;
        lo[j] = t.y;
    }
}

// acc += (ah + al) . (bh + bl) without the al . bl term
__device__ __forceinline__ floatx4 mfma3(u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl, floatx4 acc) {
    acc = mfma_bf16(ah, bh, acc);
    acc = mfma_bf16(ah, bl, acc);
    return mfma_bf16(al, bh, acc);
}

// v_mfma_f32_16x16x32_bf16 layouts: A lane l = row l%16, k 8(l/16)..+8;
// B lane l = k 8(l/16)..+8, column l%16; D lane l = rows 4(l/16)+r, column
// l%16. Scores S^T = K Q^T: A = keys (lane: key c16 of a 16-key block, head
// dims 32 s + 8 g ..), B = the query (dims 32 s + 8 g .., row c16), so lane
// (g, c16) holds row c16's scores of keys 4 g + r and 16 + 4 g + r of the
// chunk. P.V: A = P (row c16, k = those 8 keys), B = V (the same 8 keys,
// dim c16 of a 16-dim block), D = out rows 4 g + r, dim c16.
// RB (one query head a KV head, groups == 1): the NW waves take NW
// consecutive 16-row blocks of the one head instead of NW query heads of one
// block, so every staged chunk serves 16 NW rows. A row's arithmetic is the
// same either way: chunks past its own last key give it scores of -inf,
// exp 0 and no change to its sums.
template <int HD, int VD, int NW, bool SPLIT, bool RB = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void attn_mfma_kernel(AttnArgs a) {
    constexpr int KRS = HD + 8;  // K row stride (bf16): 16 keys of one read hit distinct banks
    constexpr int VRS = AK + 8;  // transposed V row stride (bf16)
    constexpr int QS = HD / 32;  // k steps of the scores
    constexpr int VB = VD / 16;  // output column blocks
    constexpr int KB = AK / 16;  // 16-key blocks per chunk
    static_assert(HD % 32 == 0 && VD % 16 == 0, "head dims");
    __shared__ __attribute__((aligned(16))) uint16_t Kh[AK * KRS], Kl[AK * KRS];
    __shared__ __attribute__((aligned(16))) uint16_t Vh[VD * VRS], Vl[VD * VRS];
    constexpr int NR = RB ? 16 * NW : 16;  // rows of the workgroup
    static_assert(NR <= 64, "row masks are 64-bit");
    __shared__ int32_t rb[NR], rp[NR];
    __shared__ floatx4 Sc[NW][CACHED * KB][64];  // pass 1's scores, [wave][chunk, key block][lane]
    // SPLIT: the block's finished output rows per wave, for the fragments
    constexpr int OS = VD + 4;
    __shared__ float Ot[SPLIT ? NW : 1][SPLIT ? 16 * OS : 1];

    if (a.dense && *a.dense) return;  // the whole-prompt kernel took these rows
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int wr = RB ? 16 * wave : 0;                   // the wave's first row within the workgroup's
    // (row block, KV head) of this workgroup: the hardware deals workgroups
    // to the 8 XCDs in turn, so consecutive ids are remapped to give each
    // XCD a contiguous run of row blocks of one head (the row blocks of a
    // prompt read the same keys and values, then from that XCD's L2)
    uint32_t bx, by;
    {
        const uint32_t X = gridDim.x, N = X * gridDim.y, L = blockIdx.x + X * blockIdx.y;
        const uint32_t per = N / 8, G = L < per * 8 ? (L % 8) * per + L / 8 : L;
        bx = G % X;
        by = G / X;
    }
    const int64_t r0 = (int64_t)bx * NR + wr;    // the wave's first row
    const int64_t hkv = by;
    const int64_t hq = RB ? 0 : (int64_t)blockIdx.z * NW + wave;  // query head within the group
    const bool head_ok = hq < a.groups;
    const int64_t h = hkv * a.groups + (head_ok ? hq : 0);
    if (threadIdx.x < NR) {
        int64_t r = (int64_t)bx * NR + threadIdx.x;
        // rows outside the KV cache are skipped like the padding rows
        const bool in = r < a.n && (int64_t)a.rows[r].b < a.nb && (int64_t)a.rows[r].pos < a.T;
        rb[threadIdx.x] = in ? (int32_t)a.rows[r].b : -1;
        rp[threadIdx.x] = in ? (int32_t)a.rows[r].pos : -1;
    }
    if constexpr (SPLIT) {
        for (int i = lane; i < 16 * OS; i += 64) Ot[wave][i] = 0.f;
    }
    __syncthreads();

    // this lane's query words (B operand): row c16, head dims 32 s + 8 g .. +8
    u32x4 qh[QS], ql[QS];
    {
        const int64_t r = r0 + c16;
        const bool ok = head_ok && r < a.n;
        const float *q = a.q + ((ok ? r : 0) * a.heads + h) * a.hd + 8 * g;
#pragma unroll
        for (int st = 0; st < QS; st++) {
            float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
            if (ok) {
                v0 = *(const float4 *)(q + 32 * st);
                v1 = *(const float4 *)(q + 32 * st + 4);
            }
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            split8_words(v, qh[st], ql[st]);
        }
    }

    const int nthreads = NW * 64;
    // Chunks are staged in two steps so that the next chunk's global loads
    // are in flight while the current one is multiplied: load_* fetches a
    // chunk into registers, put_* writes it (as bf16 terms) into LDS.
    constexpr bool PF = NW >= 4;
    constexpr int KI = PF ? (AK * (HD / 8) + NW * 64 - 1) / (NW * 64) : 1;        // K items per thread
    constexpr int VI = PF ? ((AK / 2) * (VD / 4) + NW * 64 - 1) / (NW * 64) : 1;  // V items per thread
    float4 kr[KI][2], vr[VI][2];
    // keys c0 .. c0 + AK of prompt b (zero past kmax): item = (key, 8 dims)
    auto load_k = [&](int64_t b, int64_t c0, int64_t kmax) {
        const float *kb = a.kc + (b * a.T) * a.kvd + hkv * a.hd;
#pragma unroll
        for (int t = 0; t < KI; t++) {
            const int i = threadIdx.x + t * nthreads;
            const int key = i / (HD / 8), d = (i % (HD / 8)) * 8;
            const int64_t p = c0 + key;
            kr[t][0] = kr[t][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < AK * (HD / 8) && p <= kmax) {
                kr[t][0] = *(const float4 *)(kb + p * a.kvd + d);
                kr[t][1] = *(const float4 *)(kb + p * a.kvd + d + 4);
            }
        }
    };
    auto put_k = [&]() {
#pragma unroll
        for (int t = 0; t < KI; t++) {
            const int i = threadIdx.x + t * nthreads;
            if (i >= AK * (HD / 8)) continue;
            const int key = i / (HD / 8), d = (i % (HD / 8)) * 8;
            const float v[8] = {kr[t][0].x, kr[t][0].y, kr[t][0].z, kr[t][0].w,
                                kr[t][1].x, kr[t][1].y, kr[t][1].z, kr[t][1].w};
            u32x4 hi, lo;
            split8_words(v, hi, lo);
            *(u32x4 *)&Kh[key * KRS + d] = hi;
            *(u32x4 *)&Kl[key * KRS + d] = lo;
        }
    };
    // without prefetch: a chunk loaded and written item by item
    auto stage_k = [&](int64_t b, int64_t c0, int64_t kmax) {
        const float *kb = a.kc + (b * a.T) * a.kvd + hkv * a.hd;
        for (int i = threadIdx.x; i < AK * (HD / 8); i += nthreads) {
            const int key = i / (HD / 8), d = (i % (HD / 8)) * 8;
            const int64_t p = c0 + key;
            float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
            if (p <= kmax) {
                v0 = *(const float4 *)(kb + p * a.kvd + d);
                v1 = *(const float4 *)(kb + p * a.kvd + d + 4);
            }
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            u32x4 hi, lo;
            split8_words(v, hi, lo);
            *(u32x4 *)&Kh[key * KRS + d] = hi;
            *(u32x4 *)&Kl[key * KRS + d] = lo;
        }
    };
    auto stage_v = [&](int64_t b, int64_t c0, int64_t kmax) {
        const float *vb = a.vc + (b * a.T) * a.kvd + hkv * a.hd;
        for (int i = threadIdx.x; i < (AK / 2) * (VD / 4); i += nthreads) {
            const int kp = i % (AK / 2), d = (i / (AK / 2)) * 4;
            const int64_t p = c0 + 2 * kp;
            float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
            if (p <= kmax) v0 = *(const float4 *)(vb + p * a.kvd + d);
            if (p + 1 <= kmax) v1 = *(const float4 *)(vb + (p + 1) * a.kvd + d);
            const float x0[4] = {v0.x, v0.y, v0.z, v0.w}, x1[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint2 w2 = split_pair(x0[j], x1[j]);
                *(uint32_t *)&Vh[(d + j) * VRS + 2 * kp] = w2.x;
                *(uint32_t *)&Vl[(d + j) * VRS + 2 * kp] = w2.y;
            }
        }
    };
    // values of the same keys: item = (key pair, 4 dims), written transposed
    // [dim][key]; the key pair runs fastest over the lanes, so the 64 lanes'
    // 32-bit writes of a wave fall in 64 distinct banks
    auto load_v = [&](int64_t b, int64_t c0, int64_t kmax) {
        const float *vb = a.vc + (b * a.T) * a.kvd + hkv * a.hd;
#pragma unroll
        for (int t = 0; t < VI; t++) {
            const int i = threadIdx.x + t * nthreads;
            const int kp = i % (AK / 2), d = (i / (AK / 2)) * 4;
            const int64_t p = c0 + 2 * kp;
            vr[t][0] = vr[t][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < (AK / 2) * (VD / 4)) {
                if (p <= kmax) vr[t][0] = *(const float4 *)(vb + p * a.kvd + d);
                if (p + 1 <= kmax) vr[t][1] = *(const float4 *)(vb + (p + 1) * a.kvd + d);
            }
        }
    };
    auto put_v = [&]() {
#pragma unroll
        for (int t = 0; t < VI; t++) {
            const int i = threadIdx.x + t * nthreads;
            if (i >= (AK / 2) * (VD / 4)) continue;
            const int kp = i % (AK / 2), d = (i / (AK / 2)) * 4;
            const float x0[4] = {vr[t][0].x, vr[t][0].y, vr[t][0].z, vr[t][0].w};
            const float x1[4] = {vr[t][1].x, vr[t][1].y, vr[t][1].z, vr[t][1].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint2 w2 = split_pair(x0[j], x1[j]);
                *(uint32_t *)&Vh[(d + j) * VRS + 2 * kp] = w2.x;
                *(uint32_t *)&Vl[(d + j) * VRS + 2 * kp] = w2.y;
            }
        }
    };
    // the staged chunk's scores (transposed D layout), scaled and masked for
    // this lane's row position
    auto scores = [&](floatx4 (&sc)[KB], int64_t c0, int row_pos) {
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < QS; st++) {
                const u32x4 kh = *(const u32x4 *)&Kh[(kb * 16 + c16) * KRS + 32 * st + 8 * g];
                const u32x4 kl = *(const u32x4 *)&Kl[(kb * 16 + c16) * KRS + 32 * st + 8 * g];
                acc = mfma3(kh, kl, qh[st], ql[st], acc);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t key = c0 + kb * 16 + 4 * g + r;
                sc[kb][r] = key <= row_pos ? __fmul_rn(acc[r], a.scale) : -INFINITY;
            }
        }
    };

    // lane i (< NR) holds row i's prompt and position: the row sets below
    // are wave ballots
    const int lb = lane < NR ? rb[lane] : -1, lp = lane < NR ? rp[lane] : -1;
    uint64_t done = 0;
    for (;;) {
        // the next prompt among the workgroup's rows (the first row not done)
        const uint64_t open = __ballot(lb >= 0) & ~done;
        if (open == 0) break;
        const int first = __builtin_ctzll(open);
        const int64_t b = __builtin_amdgcn_readlane(lb, first);
        const uint64_t in_mask = __ballot(lb == b);
        int kmax = lb == b ? lp : -1;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) kmax = max(kmax, __shfl_xor(kmax, o, 64));
        kmax = __builtin_amdgcn_readfirstlane(kmax);
        done |= in_mask;
        // this lane's row (c16) position, and those of its four output rows
        const int row_pos = ((in_mask >> (wr + c16)) & 1) ? rp[wr + c16] : -1;
        int pos[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = wr + 4 * g + r;
            pos[r] = ((in_mask >> row) & 1) ? rp[row] : -1;
        }
        const int nch = (kmax + AK) / AK;
        const bool cached = nch <= CACHED;

        // pass 1: the row maximum (scores of the first CACHED chunks kept).
        // With four waves the next chunk's loads are issued before the
        // current one is multiplied (PF); smaller groups load just in time
        // (their threads would need 2-4x the registers).
        float m = -INFINITY;
        if constexpr (PF) load_k(b, 0, kmax);
        for (int c = 0; c < nch; c++) {
            __syncthreads();
            if constexpr (!PF) stage_k(b, (int64_t)c * AK, kmax);
            else put_k();
            __syncthreads();
            if constexpr (PF) {
                if (c + 1 < nch) load_k(b, (int64_t)(c + 1) * AK, kmax);
                else {
                    load_v(b, 0, kmax);
                    if (!cached) load_k(b, 0, kmax);
                }
            }
            floatx4 sc[KB];
            scores(sc, (int64_t)c * AK, row_pos);
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) m = fmaxf(m, sc[kb][r]);
            if (cached) {
#pragma unroll
                for (int kb = 0; kb < KB; kb++) Sc[wave][c * KB + kb][lane] = sc[kb];
            }
        }
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));

        // pass 2: exp, sums and P V
        float sum = 0.f;
        floatx4 o[VB];
#pragma unroll
        for (int db = 0; db < VB; db++) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < nch; c++) {
            __syncthreads();
            if constexpr (!PF) {
                stage_v(b, (int64_t)c * AK, kmax);
                if (!cached) stage_k(b, (int64_t)c * AK, kmax);
            } else {
                if (!cached) put_k();
                put_v();
            }
            __syncthreads();
            if constexpr (PF) {
                if (c + 1 < nch) {
                    load_v(b, (int64_t)(c + 1) * AK, kmax);
                    if (!cached) load_k(b, (int64_t)(c + 1) * AK, kmax);
                }
            }
            floatx4 sc[KB];
            if (cached) {
#pragma unroll
                for (int kb = 0; kb < KB; kb++) sc[kb] = Sc[wave][c * KB + kb][lane];
            } else {
                scores(sc, (int64_t)c * AK, row_pos);
            }
            float e[8];
#pragma unroll
            for (int kb = 0; kb < KB; kb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float s = sc[kb][r];
                    const float v = row_pos >= 0 && s != -INFINITY ? exp_cephes(__fsub_rn(s, m)) : 0.f;
                    sum = __fadd_rn(sum, v);
                    e[kb * 4 + r] = v;
                }
            u32x4 ph, pl;
            split8_words(e, ph, pl);
            // out[row][dim] += sum over the lane's 8 keys of P[row][key] V[key][dim]
#pragma unroll
            for (int db = 0; db < VB; db++) {
                const uint16_t *vh = &Vh[(db * 16 + c16) * VRS + 4 * g], *vl = &Vl[(db * 16 + c16) * VRS + 4 * g];
                const uint2 h0 = *(const uint2 *)vh, h1 = *(const uint2 *)(vh + 16);
                const uint2 l0 = *(const uint2 *)vl, l1 = *(const uint2 *)(vl + 16);
                o[db] = mfma3(ph, pl, u32x4{h0.x, h0.y, h1.x, h1.y}, u32x4{l0.x, l0.y, l1.x, l1.y}, o[db]);
            }
        }
        // the row sums over all keys; output row 4 g + r's from lane 4 g + r
        sum = __fadd_rn(sum, __shfl_xor(sum, 16, 64));
        sum = __fadd_rn(sum, __shfl_xor(sum, 32, 64));
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float t = __shfl(sum, 4 * g + r, 64);
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
                for (int e = 0; e < 2; e++) xs[((r0 / 16 * a.ldk + ktg) * 2 + e) * 64 + lane] = words[e];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Whole-prompt attention for dense batches (row r = prompt r / T at position
// r % T) of at most PK positions: one workgroup per (prompt, KV head) stages
// the prompt's keys and values in LDS once, as bf16 terms (the per-block
// kernel stages a block's chunks again for every 16 rows), then each wave
// takes (query head, 16-row block) units with no further barrier, the
// scores of a unit's keys kept in registers between the max and the exp.
// The arithmetic is the per-block kernel's, operation for operation (the
// same three-product score and P.V MFMAs in the same chunk order, the row
// max, the Cephes exp and the sum in the lane's key order), and the values
// past a block's last row are read as zero as that kernel stages them, so
// both give the same bits.
constexpr int PK = 128;  // positions a prompt may have

// flag = 1 when every row r < n is (r / T, r % T) and inside the KV cache
__global__ __launch_bounds__(1024) void attn_dense_check_kernel(const ditch_row *rows, int64_t n, int64_t T,
                                                                int64_t nb, int *flag) {
    int bad = 0;
    for (int64_t r = threadIdx.x; r < n; r += 1024) {
        const ditch_row w = rows[r];
        bad |= (int64_t)w.b != r / T || (int64_t)w.pos != r % T;
    }
    bad = __syncthreads_or(bad);
    if (threadIdx.x == 0) *flag = !bad && (n + T - 1) / T <= nb;
}

template <int HD>
__global__ __launch_bounds__(512) void attn_prompt_kernel(AttnArgs a, AttnRope rope) {
    if (*a.dense == 0) return;  // the per-block kernel takes these rows
    constexpr int NW = 8, VD = HD, QS = HD / 32, VB = VD / 16, KB = AK / 16, NCH = PK / AK;
    constexpr int KRS = HD + 8, VRS = PK + 8;  // row strides (bf16), as in the per-block kernel
    __shared__ __attribute__((aligned(16))) uint16_t Kh[PK * KRS], Kl[PK * KRS];
    __shared__ __attribute__((aligned(16))) uint16_t Vh[VD * VRS], Vl[VD * VRS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t b = blockIdx.x, hkv = blockIdx.y;
    const int64_t L = a.n - b * a.T < a.T ? a.n - b * a.T : a.T;  // the prompt's positions 0 .. L - 1
    if (L <= 0) return;

    // keys (item = key, 8 dims) and values (item = key pair, 4 dims, stored
    // [dim][key]) of positions 0 .. PK, zero past L; every load first
    {
        constexpr int KI = PK * (HD / 8) / (NW * 64), VI = (PK / 2) * (VD / 4) / (NW * 64);
        static_assert(KI * NW * 64 == PK * (HD / 8) && VI * NW * 64 == (PK / 2) * (VD / 4), "items per thread");
        const float *kb = a.kc + (b * a.T) * a.kvd + hkv * a.hd, *vb = a.vc + (b * a.T) * a.kvd + hkv * a.hd;
        float4 kr[KI][2], vr[VI][2];
#pragma unroll
        for (int t = 0; t < KI; t++) {
            const int i = threadIdx.x + t * NW * 64, key = i / (HD / 8), d = (i % (HD / 8)) * 8;
            kr[t][0] = kr[t][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (key < L) {
                kr[t][0] = *(const float4 *)(kb + key * a.kvd + d);
                kr[t][1] = *(const float4 *)(kb + key * a.kvd + d + 4);
            }
        }
#pragma unroll
        for (int t = 0; t < VI; t++) {
            const int i = threadIdx.x + t * NW * 64, kp = i / (VD / 4), d = (i % (VD / 4)) * 4, p = 2 * kp;
            vr[t][0] = vr[t][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p < L) vr[t][0] = *(const float4 *)(vb + p * a.kvd + d);
            if (p + 1 < L) vr[t][1] = *(const float4 *)(vb + (p + 1) * a.kvd + d);
        }
#pragma unroll
        for (int t = 0; t < KI; t++) {
            const int i = threadIdx.x + t * NW * 64, key = i / (HD / 8), d = (i % (HD / 8)) * 8;
            const float v[8] = {kr[t][0].x, kr[t][0].y, kr[t][0].z, kr[t][0].w,
                                kr[t][1].x, kr[t][1].y, kr[t][1].z, kr[t][1].w};
            u32x4 hi, lo;
            split8_words(v, hi, lo);
            *(u32x4 *)&Kh[key * KRS + d] = hi;
            *(u32x4 *)&Kl[key * KRS + d] = lo;
        }
#pragma unroll
        for (int t = 0; t < VI; t++) {
            const int i = threadIdx.x + t * NW * 64, kp = i / (VD / 4), d = (i % (VD / 4)) * 4;
            const float x0[4] = {vr[t][0].x, vr[t][0].y, vr[t][0].z, vr[t][0].w};
            const float x1[4] = {vr[t][1].x, vr[t][1].y, vr[t][1].z, vr[t][1].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint2 w2 = split_pair(x0[j], x1[j]);
                *(uint32_t *)&Vh[(d + j) * VRS + 2 * kp] = w2.x;
                *(uint32_t *)&Vl[(d + j) * VRS + 2 * kp] = w2.y;
            }
        }
    }
    __syncthreads();

    // units (row block rb, query head j), rb-major: wave w takes w, w + NW, ..
    const int64_t nrb = (L + 15) / 16, units = nrb * a.groups;
    for (int64_t u = wave; u < units; u += NW) {
        const int64_t rb = u / a.groups, h = hkv * a.groups + u % a.groups;
        const int p0 = (int)(rb * 16);
        const int kmax = (int)(p0 + 15 < L - 1 ? p0 + 15 : L - 1);  // the block's last position
        const int nch = (kmax + AK) / AK;
        const int row_pos = p0 + c16 <= kmax ? p0 + c16 : -1;  // this lane's score row
        int pos[4];                                            // its four output rows
#pragma unroll
        for (int r = 0; r < 4; r++) pos[r] = p0 + 4 * g + r <= kmax ? p0 + 4 * g + r : -1;
        const int64_t r0 = b * a.T + p0;

        u32x4 qh[QS], ql[QS];
        {
            const bool ok = row_pos >= 0;
            const float *q = a.q + ((ok ? r0 + c16 : r0) * a.heads + h) * a.hd + 8 * g;
            float v[QS][8];
#pragma unroll
            for (int st = 0; st < QS; st++) {
                float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
                if (ok) {
                    v0 = *(const float4 *)(q + 32 * st);
                    v1 = *(const float4 *)(q + 32 * st + 4);
                }
                v[st][0] = v0.x; v[st][1] = v0.y; v[st][2] = v0.z; v[st][3] = v0.w;
                v[st][4] = v1.x; v[st][5] = v1.y; v[st][6] = v1.z; v[st][7] = v1.w;
            }
            if constexpr (HD == 128) {
                // the query's RoPE: dims 8 g + 32 st + j (st = 0, 1) pair with
                // the same lane's dims 64 further (st + 2), with the RoPE
                // kernel's operations in its order
                if (rope.cos_t && ok) {
                    const int64_t rp = row_pos < rope.rope_len - 1 ? row_pos : rope.rope_len - 1;
                    const float *cr = rope.cos_t + rp * 64 + 8 * g, *sr = rope.sin_t + rp * 64 + 8 * g;
#pragma unroll
                    for (int st = 0; st < 2; st++) {
                        const float4 c0 = *(const float4 *)(cr + 32 * st), c1 = *(const float4 *)(cr + 32 * st + 4);
                        const float4 s0 = *(const float4 *)(sr + 32 * st), s1 = *(const float4 *)(sr + 32 * st + 4);
                        const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
                        const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const float x0 = v[st][j], x1 = v[st + 2][j];
                            v[st][j] = __fsub_rn(__fmul_rn(x0, c[j]), __fmul_rn(x1, sn[j]));
                            v[st + 2][j] = __fadd_rn(__fmul_rn(x1, c[j]), __fmul_rn(x0, sn[j]));
                        }
                    }
                }
            }
#pragma unroll
            for (int st = 0; st < QS; st++) split8_words(v[st], qh[st], ql[st]);
        }

        // scores of chunks 0 .. nch (transposed D layout), scaled and masked
        floatx4 sc[NCH][KB];
        float m = -INFINITY;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            if (c < nch) {
#pragma unroll
                for (int kb = 0; kb < KB; kb++) {
                    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int st = 0; st < QS; st++) {
                        const int key = c * AK + kb * 16 + c16;
                        const u32x4 kh = *(const u32x4 *)&Kh[key * KRS + 32 * st + 8 * g];
                        const u32x4 kl = *(const u32x4 *)&Kl[key * KRS + 32 * st + 8 * g];
                        acc = mfma3(kh, kl, qh[st], ql[st], acc);
                    }
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int key = c * AK + kb * 16 + 4 * g + r;
                        sc[c][kb][r] = key <= row_pos ? __fmul_rn(acc[r], a.scale) : -INFINITY;
                        m = fmaxf(m, sc[c][kb][r]);
                    }
                }
            }
        }
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));

        float sum = 0.f;
        floatx4 o[VB];
#pragma unroll
        for (int db = 0; db < VB; db++) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            if (c < nch) {
                float e[8];
#pragma unroll
                for (int kb = 0; kb < KB; kb++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float s = sc[c][kb][r];
                        const float v = row_pos >= 0 && s != -INFINITY ? exp_cephes(__fsub_rn(s, m)) : 0.f;
                        sum = __fadd_rn(sum, v);
                        e[kb * 4 + r] = v;
                    }
                u32x4 ph, pl;
                split8_words(e, ph, pl);
                // keys 16 .. 31 of the chunk past the block's last row: zero
                // values, as the per-block kernel stages them
                const bool upper = c * AK + 16 <= kmax;
#pragma unroll
                for (int db = 0; db < VB; db++) {
                    const uint16_t *vh = &Vh[(db * 16 + c16) * VRS + c * AK + 4 * g];
                    const uint16_t *vl = &Vl[(db * 16 + c16) * VRS + c * AK + 4 * g];
                    const uint2 h0 = *(const uint2 *)vh, l0 = *(const uint2 *)vl;
                    uint2 h1 = *(const uint2 *)(vh + 16), l1 = *(const uint2 *)(vl + 16);
                    if (!upper) h1 = l1 = make_uint2(0u, 0u);
                    o[db] = mfma3(ph, pl, u32x4{h0.x, h0.y, h1.x, h1.y}, u32x4{l0.x, l0.y, l1.x, l1.y}, o[db]);
                }
            }
        }
        sum = __fadd_rn(sum, __shfl_xor(sum, 16, 64));
        sum = __fadd_rn(sum, __shfl_xor(sum, 32, 64));
        float inv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float t = __shfl(sum, 4 * g + r, 64);
            inv[r] = t > 0.f ? __fdiv_rn(1.0f, t) : 0.f;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (pos[r] < 0) continue;
            float *orow = a.out + ((r0 + 4 * g + r) * a.heads + h) * a.vd;
#pragma unroll
            for (int db = 0; db < VB; db++) orow[db * 16 + c16] = __fmul_rn(o[db][r], inv[r]);
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

// one query head a KV head (MHA, MLA): four waves on four 16-row blocks of
// the head, sharing each staged chunk
template <int HD, int VD>
static void launch_attn_rows(const AttnArgs &a, int64_t kv_heads, hipStream_t s) {
    constexpr int NW = 4;
    dim3 grid((unsigned)((a.n + 16 * NW - 1) / (16 * NW)), (unsigned)kv_heads, 1);
    if (a.xs) {
        DITCH_CHECK((a.heads * VD) % 128 == 0 && a.ldk * 32 >= a.heads * VD, DITCH_INVALID_ARGUMENT,
                    "attention: fragment output needs heads * v_head_dim a multiple of 128");
        hipLaunchKernelGGL((attn_mfma_kernel<HD, VD, NW, true, true>), grid, dim3(NW * 64), 0, s, a);
    } else {
        hipLaunchKernelGGL((attn_mfma_kernel<HD, VD, NW, false, true>), grid, dim3(NW * 64), 0, s, a);
    }
}

// one wave per query head of the group, up to four per workgroup
template <int HD, int VD>
static void launch_attn(const AttnArgs &a, int64_t kv_heads, hipStream_t s) {
    if (a.groups >= 4) launch_attn_nw<HD, VD, 4>(a, kv_heads, s);
    else if (a.groups == 2 || a.groups == 3) launch_attn_nw<HD, VD, 2>(a, kv_heads, s);
    else launch_attn_rows<HD, VD>(a, kv_heads, s);
}

// Whether the whole-prompt kernel can take a forward's attention (head dims
// 64 or 128, at most PK positions a prompt, f32 output), and the check of
// its rows into `flag` (once a forward: every layer has the same rows).
bool attention_prompt_takes(int64_t hd, int64_t vd, int64_t T) {
    return hd == vd && (hd == 64 || hd == 128) && T <= PK;
}
void launch_attention_dense_check(const ditch_row *rows, int64_t n, int64_t T, int64_t nb, int *flag, hipStream_t s) {
    hipLaunchKernelGGL(attn_dense_check_kernel, dim3(1), dim3(1024), 0, s, rows, n, T, nb, flag);
    DITCH_TRY_HIP(hipGetLastError());
}

// With a.dense (set by launch_attention_dense_check for these rows), both
// kernels are launched and the one the flag does not select exits at once.
static void launch_attention(const AttnArgs &a, const AttnRope &rope, int64_t kv_heads, hipStream_t s) {
    if (a.dense) {
        DITCH_CHECK(!a.xs && attention_prompt_takes(a.hd, a.vd, a.T), DITCH_INVALID_ARGUMENT,
                    "attention: the whole-prompt kernel does not take this shape");
        DITCH_CHECK(!rope.cos_t || a.hd == 128, DITCH_INVALID_ARGUMENT,
                    "attention: the whole-prompt kernel rotates queries of head_dim 128 only");
        const dim3 grid((unsigned)((a.n + a.T - 1) / a.T), (unsigned)kv_heads);
        if (a.hd == 64) hipLaunchKernelGGL(attn_prompt_kernel<64>, grid, dim3(512), 0, s, a, rope);
        else hipLaunchKernelGGL(attn_prompt_kernel<128>, grid, dim3(512), 0, s, a, rope);
        DITCH_TRY_HIP(hipGetLastError());
    }
    if (a.hd == 64) launch_attn<64, 64>(a, kv_heads, s);
    else if (a.hd == 128) launch_attn<128, 128>(a, kv_heads, s);
    else launch_attn<192, 128>(a, kv_heads, s);
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_attention_mfma(const AttnArgs &a, int64_t kv_heads, hipStream_t s) {
    launch_attention(a, AttnRope{}, kv_heads, s);
}

void launch_attention_mfma_rope(const AttnArgs &a, const AttnRope &rope, int64_t kv_heads, hipStream_t s) {
    DITCH_CHECK(a.dense && rope.cos_t && rope.sin_t && rope.rope_len > 0, DITCH_INVALID_ARGUMENT,
                "attention: query rotation needs the dense flag and the rope tables");
    launch_attention(a, rope, kv_heads, s);
}

}  // namespace ditch
