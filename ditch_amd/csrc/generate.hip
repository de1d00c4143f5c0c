// generate.hip — token generation after a batched prefill (model.generate /
// generateKeep, model.zig:5358-5444): the keys and values of every layer
// stay in a persistent HBM cache (ditch_hip_kv_cache), each decode step runs
// the active prompts' rows through the resident forward, and the next token
// of every row is picked on the device: the first maximum (model.zig:
// 5194-5204), or the Sampler's temperature / top-k / top-p draw (model.zig:
// 5208-5264), whose uniform draws come from the Sampler's own Zig
// DefaultPrng on the host, one per sampled row in row order.
#include <math.h>
#include <string.h>

#include <vector>

#include "internal.h"
#include "model.h"
#include "zig_random.h"

namespace ditch {

void model_forward(ditch_hip_model *m, const uint32_t *d_tokens, const ditch_row *d_rows, int64_t n, int64_t B,
                   int64_t T, const uint64_t *d_capture, int64_t n_capture, float *d_res, const uint64_t *d_logit_rows,
                   int64_t n_logit, float *d_logits, ditch_hip_kv_cache *pc);

constexpr int PICK_MAXK = 256;  // Sampler.max_top_k
constexpr int PICK_ROWS = 256;  // rows per launch: their draws travel in the arguments

struct PickArgs {
    uint32_t *out;
    const float *logits;
    int64_t vocab;
    float temperature, top_p;
    int top_k;
    double u[PICK_ROWS];  // each row's Random.float(f64) draw
};

// floats ordered as unsigned keys (larger key = larger value)
__device__ __forceinline__ uint32_t pick_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float pick_val(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// One block per logit row.
__global__ __launch_bounds__(1024) void pick_kernel(PickArgs a) {
    __shared__ uint32_t hist[256];
    __shared__ uint64_t cand[PICK_MAXK];
    __shared__ float bv_s[16];
    __shared__ uint32_t bi_s[16];
    __shared__ uint32_t prefix_s, remaining_s, n_gt, eq_base[1024];
    __shared__ double probs[PICK_MAXK];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = blockIdx.x, V = a.vocab;
    const float *x = a.logits + row * V;

    if (a.temperature <= 0.f) {
        // argmax: the first index of the largest value (strict >, NaN never wins)
        float bv = -INFINITY;
        uint32_t bi = 0;
        for (int64_t i = tid; i < V; i += nt) {
            const float v = x[i];
            if (v > bv) {
                bv = v;
                bi = (uint32_t)i;
            }
        }
        // reduce: larger value, then smaller index
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const uint32_t oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if ((tid & 63) == 0) {
            bv_s[tid >> 6] = bv;
            bi_s[tid >> 6] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            float v = bv_s[0];
            uint32_t id = bi_s[0];
            for (int w = 1; w < nt / 64; w++)
                if (bv_s[w] > v || (bv_s[w] == v && bi_s[w] < id)) {
                    v = bv_s[w];
                    id = bi_s[w];
                }
            a.out[row] = id;
        }
        return;
    }

    // the k largest logits, highest first, earlier index first among equals
    // (the Sampler's insertion order): the k-th key by radix select, then
    // every larger key and the first equal ones in index order
    const int k = (int)((int64_t)a.top_k < V ? a.top_k : V);
    if (tid == 0) {
        prefix_s = 0;
        remaining_s = (uint32_t)k;
        n_gt = 0;
    }
    uint32_t mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += nt) hist[i] = 0;
        __syncthreads();
        const uint32_t prefix = prefix_s;
        for (int64_t i = tid; i < V; i += nt) {
            const uint32_t key = pick_key(x[i]);
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t cum = 0, rem = remaining_s;
            for (int b = 255; b >= 0; b--) {
                if (cum + hist[b] >= rem) {
                    prefix_s = prefix | ((uint32_t)b << shift);
                    remaining_s = rem - cum;
                    break;
                }
                cum += hist[b];
            }
        }
        __syncthreads();
        mask |= 255u << shift;
    }
    const uint32_t kth = prefix_s, need_eq = remaining_s;
    // candidates: key << 32 | ~index (descending sort: larger key, then smaller index)
    for (int i = tid; i < PICK_MAXK; i += nt) cand[i] = 0;
    __syncthreads();
    for (int64_t i = tid; i < V; i += nt) {
        const uint32_t key = pick_key(x[i]);
        if (key > kth) {
            const uint32_t slot = atomicAdd(&n_gt, 1u);
            if (slot < (uint32_t)PICK_MAXK) cand[slot] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
        }
    }
    // the equal keys in index order: contiguous chunks, counts, a scan
    const int64_t chunk = (V + nt - 1) / nt, c0 = tid * chunk, c1 = c0 + chunk < V ? c0 + chunk : V;
    uint32_t cnt = 0;
    for (int64_t i = c0; i < c1; i++) cnt += pick_key(x[i]) == kth;
    eq_base[tid] = cnt;
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        for (int t = 0; t < nt; t++) {
            const uint32_t c = eq_base[t];
            eq_base[t] = acc;
            acc += c;
        }
    }
    __syncthreads();
    const uint32_t gt = n_gt;
    uint32_t r = eq_base[tid];
    for (int64_t i = c0; i < c1 && r < need_eq; i++)
        if (pick_key(x[i]) == kth) {
            const uint32_t slot = gt + r;
            if (slot < (uint32_t)PICK_MAXK) cand[slot] = ((uint64_t)kth << 32) | (uint32_t)~(uint32_t)i;
            r++;
        }
    __syncthreads();
    // bitonic sort of the 256 candidates, descending
    for (int size = 2; size <= PICK_MAXK; size <<= 1)
        for (int j = size >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < PICK_MAXK; i += nt) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t p = cand[i], q = cand[ixj];
                    const bool desc = (i & size) == 0;
                    if (desc ? p < q : p > q) {
                        cand[i] = q;
                        cand[ixj] = p;
                    }
                }
            }
            __syncthreads();
        }
    if (tid == 0) {
        // softmax at the temperature in f64, the smallest prefix holding
        // top_p of the mass, one draw (model.zig:5243-5262)
        const float v0 = pick_val((uint32_t)(cand[0] >> 32));
        double total = 0;
        for (int i = 0; i < k; i++) {
            const float vi = pick_val((uint32_t)(cand[i] >> 32));
            probs[i] = exp((double)__fsub_rn(vi, v0) / (double)a.temperature);
            total += probs[i];
        }
        int kept = 0;
        double kept_mass = 0;
        while (kept < k) {
            kept_mass += probs[kept];
            kept++;
            if (kept_mass >= (double)a.top_p * total) break;
        }
        double u = a.u[row] * kept_mass;
        uint32_t id = ~(uint32_t)(cand[kept - 1] & 0xFFFFFFFFu);
        for (int i = 0; i < kept; i++) {
            u -= probs[i];
            if (u <= 0) {
                id = ~(uint32_t)(cand[i] & 0xFFFFFFFFu);
                break;
            }
        }
        a.out[row] = id;
    }
}

void launch_pick(uint32_t *out, const float *logits, int64_t n, int64_t vocab, ditch_sampler *smp, hipStream_t s) {
    if (n <= 0) return;
    DITCH_CHECK(vocab > 0 && n <= INT32_MAX, DITCH_INVALID_ARGUMENT, "pick: empty rows");
    const bool sample = smp && smp->temperature > 0.f;
    ZigRandom rng;
    PickArgs a{};
    a.vocab = vocab;
    a.temperature = 0.f;
    a.top_p = 1.f;
    a.top_k = 1;
    if (sample) {
        rng = ZigRandom::from_state(smp->rng);
        a.temperature = smp->temperature;
        a.top_p = smp->top_p;
        a.top_k = (int)(smp->top_k < 1 ? 1 : smp->top_k > (uint32_t)PICK_MAXK ? PICK_MAXK : smp->top_k);
    }
    for (int64_t r0 = 0; r0 < n; r0 += PICK_ROWS) {
        const int64_t rows = n - r0 < PICK_ROWS ? n - r0 : PICK_ROWS;
        a.out = out + r0;
        a.logits = logits + r0 * vocab;
        for (int64_t i = 0; i < rows; i++) a.u[i] = sample ? rng.float64() : 0.0;
        hipLaunchKernelGGL(pick_kernel, dim3((unsigned)rows), dim3(1024), 0, s, a);
        DITCH_TRY_HIP(hipGetLastError());
    }
    if (sample)
        for (int i = 0; i < 4; i++) smp->rng[i] = rng.s[i];
}

void sampler_init(ditch_sampler *smp, uint64_t seed, float temperature, uint64_t top_k, float top_p) {
    const ZigRandom rng(seed);
    smp->temperature = temperature;
    smp->top_k = (uint32_t)(top_k < 1 ? 1 : top_k > (uint64_t)PICK_MAXK ? PICK_MAXK : top_k);
    smp->top_p = top_p;
    smp->reserved = 0;
    for (int i = 0; i < 4; i++) smp->rng[i] = rng.s[i];
}

// ---------------------------------------------------------------------------
// the generation loop (generateKeep, model.zig:5378-5444)

void generate(ditch_hip_model *m, ditch_hip_kv_cache *kc, const uint32_t *tokens, const uint64_t *lens, int64_t B,
              int64_t max_new, const uint32_t *eos, int64_t n_eos, ditch_sampler *smp, uint32_t *out_tokens,
              uint64_t *out_lens, float *first_logits) {
    const ditch_model_config &c = m->c;
    hipStream_t s = m->h->stream;
    DITCH_CHECK(kc && kc->m == m, DITCH_INVALID_ARGUMENT, "generate: the KV cache belongs to another model");
    DITCH_CHECK(B >= 1 && B <= kc->B, DITCH_INVALID_ARGUMENT, "generate: more prompts than the KV cache holds");
    DITCH_CHECK(max_new >= 1, DITCH_INVALID_ARGUMENT, "generate: max_new_tokens must be at least 1");
    const int64_t V = (int64_t)c.vocab;
    const uint64_t rows_embed = m->embed.ok() ? (uint64_t)m->embed.t->v.rows : 0;
    int64_t total = 0;
    for (int64_t b = 0; b < B; b++) {
        DITCH_CHECK(lens[b] >= 1 && (int64_t)lens[b] <= kc->T, DITCH_INVALID_ARGUMENT,
                    "generate: a prompt is empty or longer than the KV cache");
        total += (int64_t)lens[b];
    }
    for (int64_t i = 0; i < total; i++)
        DITCH_CHECK(tokens[i] < rows_embed, DITCH_INVALID_ARGUMENT, "generate: token id outside the embedding table");
    // prefill: every prompt row, the last row of each prompt gives its logits
    std::vector<ditch_row> rows(total);
    std::vector<uint64_t> last(B);
    int64_t idx = 0;
    for (int64_t b = 0; b < B; b++) {
        for (uint64_t p = 0; p < lens[b]; p++) rows[idx++] = ditch_row{(uint32_t)b, (uint32_t)p};
        last[b] = (uint64_t)idx - 1;
    }
    const int64_t cap = total > B ? total : B;
    DevBuf d_tok, d_rows, d_lr, d_log, d_pick;
    uint32_t *dt = d_tok.get<uint32_t>(cap);
    ditch_row *dr = d_rows.get<ditch_row>(cap);
    uint64_t *dl = d_lr.get<uint64_t>(B);
    float *dlog = d_log.get<float>((size_t)B * V);
    uint32_t *dp = d_pick.get<uint32_t>(B);
    DITCH_TRY_HIP(hipMemcpyAsync(dt, tokens, total * 4, hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipMemcpyAsync(dr, rows.data(), total * sizeof(ditch_row), hipMemcpyHostToDevice, s));
    DITCH_TRY_HIP(hipMemcpyAsync(dl, last.data(), B * 8, hipMemcpyHostToDevice, s));
    model_forward(m, dt, dr, total, kc->B, kc->T, nullptr, 0, nullptr, dl, B, dlog, kc);
    launch_pick(dp, dlog, B, V, smp, s);
    std::vector<uint32_t> picked(B), ids;
    DITCH_TRY_HIP(hipMemcpyAsync(picked.data(), dp, B * 4, hipMemcpyDeviceToHost, s));
    if (first_logits) DITCH_TRY_HIP(hipMemcpyAsync(first_logits, dlog, (size_t)B * V * 4, hipMemcpyDeviceToHost, s));
    DITCH_TRY_HIP(hipStreamSynchronize(s));
    auto is_eos = [&](uint32_t t) {
        for (int64_t e = 0; e < n_eos; e++)
            if (eos[e] == t) return true;
        return false;
    };
    std::vector<uint64_t> pos(B);
    std::vector<bool> active(B);
    int64_t n_active = 0;
    for (int64_t b = 0; b < B; b++) {
        pos[b] = lens[b];
        out_tokens[b * max_new] = picked[b];
        out_lens[b] = 1;
        active[b] = !(is_eos(picked[b]) || max_new <= 1 || (int64_t)pos[b] >= kc->T);
        n_active += active[b];
    }
    std::vector<uint32_t> step_tok;
    std::vector<ditch_row> step_rows;
    std::vector<uint64_t> step_lr;
    for (int64_t step = 1; step < max_new && n_active > 0; step++) {
        step_tok.clear();
        step_rows.clear();
        step_lr.clear();
        ids.clear();
        for (int64_t b = 0; b < B; b++) {
            if (!active[b]) continue;
            step_tok.push_back(out_tokens[b * max_new + out_lens[b] - 1]);
            step_rows.push_back(ditch_row{(uint32_t)b, (uint32_t)pos[b]});
            step_lr.push_back(step_lr.size());
            ids.push_back((uint32_t)b);
        }
        const int64_t n = (int64_t)step_tok.size();
        for (int64_t i = 0; i < n; i++)
            DITCH_CHECK(step_tok[i] < rows_embed, DITCH_INVALID_ARGUMENT, "generate: picked a token outside the embedding");
        DITCH_TRY_HIP(hipMemcpyAsync(dt, step_tok.data(), n * 4, hipMemcpyHostToDevice, s));
        DITCH_TRY_HIP(hipMemcpyAsync(dr, step_rows.data(), n * sizeof(ditch_row), hipMemcpyHostToDevice, s));
        DITCH_TRY_HIP(hipMemcpyAsync(dl, step_lr.data(), n * 8, hipMemcpyHostToDevice, s));
        model_forward(m, dt, dr, n, kc->B, kc->T, nullptr, 0, nullptr, dl, n, dlog, kc);
        launch_pick(dp, dlog, n, V, smp, s);
        DITCH_TRY_HIP(hipMemcpyAsync(picked.data(), dp, n * 4, hipMemcpyDeviceToHost, s));
        DITCH_TRY_HIP(hipStreamSynchronize(s));
        for (int64_t i = 0; i < n; i++) {
            const int64_t b = ids[i];
            const uint32_t t = picked[i];
            pos[b]++;
            out_tokens[b * max_new + out_lens[b]] = t;
            out_lens[b]++;
            if (is_eos(t) || (int64_t)pos[b] >= kc->T) {
                active[b] = false;
                n_active--;
            }
        }
    }
}

}  // namespace ditch
