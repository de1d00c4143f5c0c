/*
 * ditch_hip.h — C ABI of the MI355X (gfx950) device backend for ditch's
 * operator seam.
 *
 * The reference routes every matrix product of its forward pass through
 * `compute.zig` (compute.zig:90-117, `VTable`): a backend fills function
 * pointers that take host slices, compute synchronously and return
 * `error{Unsupported, DeviceFailed, OutOfMemory}` (compute.zig:54-60).
 * The entry points below are exactly those operations as `extern "C"`
 * functions (host pointers + sizes), plus the extensions the north star asks
 * for: packed quantised weights handed to the device as-is (the `Dequant`
 * descriptor of dequant.zig:346-375 folded into `ditch_weight`), weights
 * registered once in HBM, the resident forward (model.zig:4619
 * `forward(..., ForwardOptions)`), routed MoE (moe.zig:998), the rank-k edit
 * (abliterate.zig:264-280) and the KL scorer's log-softmax/KL
 * (tensor.zig:1203-1210, scorers.zig:378-402).
 *
 * Conventions follow the Metal shim (src/metal/shim.h:6-7): every function is
 * safe to call with a NULL context (it then fails cleanly), nothing throws
 * across the boundary, and the caller owns every buffer it passes. Calls on
 * one context are serialised by a mutex inside the library (the Vulkan
 * backend's one lock, vulkan/backend.zig:146-148, 229-230).
 */
#ifndef DITCH_HIP_H
#define DITCH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status codes. 0..3 map one to one onto compute.zig:54-60
 * (ok, error.Unsupported, error.DeviceFailed, error.OutOfMemory). A Zig
 * caller maps DITCH_INVALID_ARGUMENT to error.DeviceFailed.                 */
enum {
    DITCH_OK = 0,
    DITCH_UNSUPPORTED = 1,
    DITCH_DEVICE_FAILED = 2,
    DITCH_OUT_OF_MEMORY = 3,
    DITCH_INVALID_ARGUMENT = 4
};

/* ------------------------------------------------------------------------ */
/* Storage formats. 0..12 keep the numbering of tensor.zig:11-33 (`DType`:
 * f32, f16, bf16, i64, i32, q8_0, q4_0, q4_1, q5_0, q5_1, q4_k, q6_k, q8_k);
 * the quantised-safetensors formats of dequant.zig:70 (`Method`) follow.    */
enum {
    DITCH_F32 = 0,
    DITCH_F16 = 1,
    DITCH_BF16 = 2,
    DITCH_I64 = 3,
    DITCH_I32 = 4,
    DITCH_Q8_0 = 5,
    DITCH_Q4_0 = 6,
    DITCH_Q4_1 = 7,
    DITCH_Q5_0 = 8,
    DITCH_Q5_1 = 9,
    DITCH_Q4_K = 10,
    DITCH_Q6_K = 11,
    DITCH_Q8_K = 12,
    /* FP8 (dequant.zig:477-514): `data` = E4M3 (or E5M2) codes [rows][cols],
     * `scale` = grid [scale_rows][scale_cols] of f32/bf16/f16 or E8M0 bytes,
     * one value per block_rows x block_cols elements. Value = bf16_rne(code * s). */
    DITCH_FP8 = 32,
    /* MXFP4 natural layout (mxfp4-pack-quantized / store_dtype,
     * dequant.zig:643-673): `data` = [rows][cols/2] nibble pairs, low nibble
     * first; `scale` = E8M0 [rows][cols/32]. Value = bf16_rne(e2m1 * 2^(s-127)). */
    DITCH_MXFP4 = 33,
    /* MXFP4 gpt-oss layout (dequant.zig:603-637): `data` = [cols][rows/32][16]
     * blocks of the transpose, `scale` = E8M0 [cols][rows/32].               */
    DITCH_MXFP4_T = 34,
    /* compressed-tensors pack-quantized (dequant.zig:518-597): `data` = I32
     * words [rows][ceil(cols*bits/32)], `scale` [rows][groups] (f16/bf16/f32),
     * `zero` packed along rows [ceil(rows*bits/32)][groups] I32 or NULL,
     * `g_idx` I32 [cols] or NULL. Value = bf16_rne((q - zp) * scale).       */
    DITCH_INT_PACKED = 35,
    /* Scale dtype only: E8M0 exponent bytes (2^(b-127), dequant.zig:446). */
    DITCH_E8M0 = 40
};

/* A weight matrix as the kernels see it: `tensor.Weight{data, dtype, rows,
 * cols}` (tensor.zig:517-521) widened with the pieces of a quantised group
 * (dequant.zig:346-375). `rows` x `cols` is the logical matrix (the virtual
 * bf16 tensor for FP8/MXFP4/INT, the f32 view for float and GGUF types).
 * Unused fields are zero / NULL.                                           */
typedef struct ditch_weight {
    const void *data;
    int32_t dtype;
    int32_t scale_dtype;
    uint64_t rows;
    uint64_t cols;
    const void *scale;
    uint64_t scale_rows;   /* FP8 grid rows; INT: rows                      */
    uint64_t scale_cols;   /* FP8 grid cols; INT: groups per row            */
    uint64_t block_rows;   /* FP8 weight_block_size[0]                      */
    uint64_t block_cols;   /* FP8 weight_block_size[1]                      */
    uint64_t row_shard;    /* FP8 attn_row_shards (dequant.zig:471-475), 0 = none */
    int32_t fp8_e5m2;      /* FP8: codes are E5M2 instead of E4M3           */
    int32_t bits;          /* INT: field width (1..8)                       */
    uint64_t group;        /* INT: columns per scale group                  */
    const void *zero;      /* INT: packed zero points, NULL = symmetric     */
    const int32_t *g_idx;  /* INT: actorder group per column, NULL = none   */
} ditch_weight;

/* ------------------------------------------------------------------------ */
/* Context (one GPU).                                                        */
typedef struct ditch_hip ditch_hip;

/* Opens HIP device `device`. NULL on failure, with a message in `err`.     */
ditch_hip *ditch_hip_open(int32_t device, char *err, size_t err_len);
void ditch_hip_close(ditch_hip *h);
/* Device name, e.g. "AMD Instinct MI355X (gfx950)". Owned by the context. */
const char *ditch_hip_name(ditch_hip *h);
/* Message of the last failed call on this context ("" if none).           */
const char *ditch_hip_last_error(ditch_hip *h);
/* VTable.forgetWeights (compute.zig:96-97, 325-327): drops every weight the
 * per-call entry points keep resident. Registered tensors are unaffected. */
void ditch_hip_forget_weights(ditch_hip *h);
/* compute.Residency (compute.zig:567-693, the `--gpu-memory N` budget): the
 * per-call entry points that take a ditch_weight (matmulT, matvecTMulti,
 * rowNorms, edit_delta, edit_delta_ex) keep the registered (re-tiled) copy
 * of each weight in a least-recently-used set of at most `budget_bytes`
 * device bytes, keyed by the host address and length of its codes and the
 * rest of its descriptor, with a signature of sampled bytes of its buffers:
 * new contents at a cached address are a miss. Keying by address is sound
 * only while host weights stay valid and unique (memory-mapped files,
 * compute.weights_stable); with weights_stable = 0 or a zero budget every
 * call uploads, computes and drops (the default). A smaller budget evicts
 * at once; forget_weights clears.                                          */
int32_t ditch_hip_set_residency(ditch_hip *h, uint64_t budget_bytes, int32_t weights_stable);
typedef struct ditch_residency_stats {
    uint64_t budget;
    uint64_t used;
    uint64_t entries;
    uint64_t hits;
    uint64_t misses;
    uint64_t evictions;
    uint64_t enabled;
} ditch_residency_stats;
int32_t ditch_hip_residency_stats(ditch_hip *h, ditch_residency_stats *out);
/* The HIP stream every call of this context runs on (hipStream_t).         */
void *ditch_hip_stream(ditch_hip *h);
/* Waits for the context's stream.                                          */
int32_t ditch_hip_sync(ditch_hip *h);

/* ------------------------------------------------------------------------ */
/* VTable operations (compute.zig:98-116). Host memory in and out; each call
 * uploads, computes and copies back before it returns
 * (vulkan/backend.zig:21-23). Replaces the bodies of `matmulTOn`,
 * `matvecTMultiOn`, `rowNormsOn`, `attentionScoresOn`, ... (compute.zig:343-
 * 560) when a Zig backend fills `VTable` with these.                       */

/* out[n][w.rows] = x[n][w.cols] @ W^T          (compute.zig:100, tensor.zig:1023) */
int32_t ditch_hip_matmulT(ditch_hip *h, float *out, const float *x, uint64_t n,
                          const ditch_weight *w);
/* out[q][w.cols] = y[q][w.rows] @ W            (compute.zig:102, tensor.zig:1079) */
int32_t ditch_hip_matvecTMulti(ditch_hip *h, float *out, const ditch_weight *w,
                               const float *y, uint64_t q);
/* out[w.rows] = ||W_i||_2                      (compute.zig:104, tensor.zig:1114) */
int32_t ditch_hip_rowNorms(ditch_hip *h, float *out, const ditch_weight *w);
/* scores[p] = scale * dot(q[0..hd], k[p*stride ..])   (compute.zig:107, tensor.zig:1126) */
int32_t ditch_hip_attentionScores(ditch_hip *h, float *scores, uint64_t n_keys,
                                  const float *q, uint64_t hd, const float *k,
                                  uint64_t stride, float scale);
/* out[j] = sum_p scores[p] * v[p*stride + j], j < vd (compute.zig:109, tensor.zig:1148) */
int32_t ditch_hip_attentionValues(ditch_hip *h, float *out, uint64_t vd,
                                  const float *scores, uint64_t n_keys,
                                  const float *v, uint64_t stride);
/* out[i][j] = act(gate[i][j]) * up[i][j] (up may be NULL); `act` follows
 * tensor.Activation order: silu, gelu_tanh, gelu, relu, relu2, quick_gelu
 * (compute.zig:81-83, 111; tensor.zig:1227-1334)                           */
int32_t ditch_hip_gatedActivation(ditch_hip *h, uint32_t act, float *out,
                                  const float *gate, const float *up, uint64_t n,
                                  uint64_t len, uint64_t in_stride,
                                  uint64_t out_stride);
/* RMS norm of n rows of len (weight_len 0 = weightless)  (compute.zig:113, tensor.zig:1167) */
int32_t ditch_hip_rmsnormRows(ditch_hip *h, float *out, const float *x,
                              const float *weight, uint64_t weight_len,
                              uint64_t n, uint64_t len, float eps,
                              int32_t gemma_style);
/* LayerNorm of n rows (bias may be NULL)       (compute.zig:115, tensor.zig:1343) */
int32_t ditch_hip_layernormRows(ditch_hip *h, float *out, const float *x,
                                const float *weight, uint64_t weight_len,
                                const float *bias, uint64_t n, uint64_t len,
                                float eps, int32_t one_plus);
/* In-place softmax of n rows of len             (compute.zig:117, tensor.zig:1181) */
int32_t ditch_hip_softmaxRows(ditch_hip *h, float *x, uint64_t n, uint64_t len);
/* RoPE of n head vectors of dim at pos[i] against [table_len][half] tables;
 * style 0 = neox (rotate half), 1 = gptj (pairs)  (compute.zig:85, 119)     */
int32_t ditch_hip_ropeRows(ditch_hip *h, float *x, uint64_t n, uint64_t dim,
                           const float *cos_table, const float *sin_table,
                           uint64_t table_len, uint64_t half, const uint32_t *pos,
                           uint32_t style);

/* ------------------------------------------------------------------------ */
/* Decode (bit-exact with the CPU decoders). Rows [row0, row0+nrows) of `w`
 * into host `out`: bf16 for DITCH_FP8/MXFP4/MXFP4_T/INT_PACKED (the virtual
 * tensor of dequant.zig), f32 for float and GGUF types (tensor.Weight.row,
 * tensor.zig:523-526 -> quant.zig:57-79).                                   */
int32_t ditch_hip_dequant(ditch_hip *h, void *out, const ditch_weight *w,
                          uint64_t row0, uint64_t nrows);

/* ------------------------------------------------------------------------ */
/* Weights resident in HBM. `ditch_hip_upload` copies a weight from host
 * memory once and re-tiles it for the kernels (same bytes, no loss): the
 * explicit-registration form of compute.zig's `Residency` (compute.zig:580-
 * 693), for weights the caller keeps stable.                               */
typedef struct ditch_hip_tensor ditch_hip_tensor;
ditch_hip_tensor *ditch_hip_upload(ditch_hip *h, const ditch_weight *w);
void ditch_hip_tensor_free(ditch_hip *h, ditch_hip_tensor *t);
/* HBM bytes the tensor occupies (codes + scales).                          */
uint64_t ditch_hip_tensor_bytes(const ditch_hip_tensor *t);
/* Decode of a resident tensor into device memory (`d_out`, `out_bytes`
 * long), same output types as ditch_hip_dequant: 2 bytes per element for the
 * virtual-bf16 formats, 4 otherwise. A buffer shorter than nrows * cols
 * elements is refused. Runs on the context stream.                         */
int32_t ditch_hip_tensor_dequant(ditch_hip *h, void *d_out, uint64_t out_bytes,
                                 const ditch_hip_tensor *t, uint64_t row0,
                                 uint64_t nrows);
/* d_out[n][rows] (=|+=) d_x[n][cols] @ W^T (+ d_bias[rows]) on device
 * memory, enqueued on `stream` (NULL = the context stream), not waited for.
 * `accumulate` != 0 adds into d_out (the residual add of model.zig:4944).
 * `out_bytes` / `x_bytes` are the buffers' lengths (the `out` and `x`
 * slices of compute.zig:100); shorter than n * rows * 4 / n * cols * 4 is
 * refused before anything is launched.                                     */
int32_t ditch_hip_matmulT_device(ditch_hip *h, float *d_out, uint64_t out_bytes,
                                 const float *d_x, uint64_t x_bytes,
                                 uint64_t n, const ditch_hip_tensor *w,
                                 const float *d_bias, int32_t accumulate,
                                 void *stream);

/* ditch_hip_matmulT_device for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The same kernels, with their
 * scratch (activation fragments, GEMV staging, split-K partial sums) in a
 * static device array of ditch_hip_static_scratch_bytes() (64 MiB) that
 * each GPU holds for the life of the process: the call allocates nothing.
 * A call needing more scratch than that is refused (InvalidArgument) before
 * anything is launched; when only the split-K partial sums do not fit, the
 * product runs unsplit. Every call on one GPU shares that GPU's array: the
 * calls are ordered on the device in the order they are made (each call's
 * stream first waits for an event the previous call recorded after its last
 * kernel, whatever its stream or context), so calls on different streams
 * do not overlap (under graph capture the graph orders the captured calls:
 * make them depend on each other). The array keeps the last call's
 * contents.                                                               */
int32_t ditch_hip_matmulT_device_noalloc(ditch_hip *h, float *d_out,
                                         uint64_t out_bytes, const float *d_x,
                                         uint64_t x_bytes, uint64_t n,
                                         const ditch_hip_tensor *w,
                                         const float *d_bias,
                                         int32_t accumulate, void *stream);
uint64_t ditch_hip_static_scratch_bytes(void);

/* Activation fragments: the activations already in the layout the
 * large-batch product over a given tensor reads, for callers that multiply
 * the same activations by several tensors or keep them resident (the
 * resident forward's own producers write them). The layout depends on the
 * tensor's format and n: four fp6 (e2m3) terms with E8M0 block scales for
 * MXFP4 tensors on n >= 128 rows (the operands of the scaled MFMA), else
 * two bf16 terms per value in MFMA operand order (BF16, FP8, INT4, Q8_0 and
 * MXFP4 tensors on n >= 32). No reference counterpart: matmulT
 * (compute.zig:100) takes f32 rows.
 * ditch_hip_frag_bytes: bytes for n rows of activations against w, or 0
 * when the large-batch product does not take w (n < 32, or a format it does
 * not decode exactly); the f32 entry point then applies.                  */
uint64_t ditch_hip_frag_bytes(const ditch_hip_tensor *w, uint64_t n);
/* Writes the fragments of d_x [n][cols of w] (f32) for products over w into
 * d_frags (frag_bytes long), on `stream` (NULL = the context stream).     */
int32_t ditch_hip_split_device(ditch_hip *h, void *d_frags, uint64_t frag_bytes,
                               const float *d_x, uint64_t n,
                               const ditch_hip_tensor *w, void *stream);
/* ditch_hip_matmulT_device on fragments that ditch_hip_split_device wrote
 * for w (or for a tensor of the same format and cols). Unsupported where
 * ditch_hip_frag_bytes is 0; buffers shorter than n * rows * 4 (out) or
 * ditch_hip_frag_bytes(w, n) (frags) are refused.                          */
int32_t ditch_hip_matmulT_frags_device(ditch_hip *h, float *d_out,
                                       uint64_t out_bytes, const void *d_frags,
                                       uint64_t frag_bytes, uint64_t n,
                                       const ditch_hip_tensor *w,
                                       const float *d_bias, int32_t accumulate,
                                       void *stream);

/* The MLP block's fused first product (model.zig:4430-4486: gate and up
 * projections, then act(gate) * up, tensor.zig:1309-1337) on activation
 * fragments written by ditch_hip_split_device for `gate`; the result is
 * written as the fragments a product over a gate.rows-column tensor of the
 * same format reads (the down projection's input), never as f32 rows.
 * `act` follows tensor.Activation (0 = silu). No reference counterpart as
 * one call: the reference runs two matmulT and gatedActivation.
 * ditch_hip_glu_frag_bytes: the output's bytes, 0 when the fused product
 * does not take the pair (formats or shapes differ, n < 128).             */
uint64_t ditch_hip_glu_frag_bytes(const ditch_hip_tensor *gate,
                                  const ditch_hip_tensor *up, uint64_t n);
int32_t ditch_hip_glu_device(ditch_hip *h, void *d_out_frags, uint64_t out_bytes,
                             const void *d_frags, uint64_t frag_bytes,
                             uint64_t n, const ditch_hip_tensor *gate,
                             const ditch_hip_tensor *up, uint32_t act,
                             void *stream);

/* ------------------------------------------------------------------------ */
/* Resident forward pass (model.zig:4619-4853 with ForwardOptions,
 * model.zig:3136-3144), for the families of the benchmark configurations:
 * dense GQA decoders (llama, qwen2 with q/k/v bias, qwen3 q/k head norm),
 * routed MoE (qwen3_moe softmax top-k; deepseek_v3 sigmoid, correction bias,
 * group-limited top-k, routed scaling, shared experts) and DeepSeek MLA.   */

enum { DITCH_ROPE_NEOX = 0, DITCH_ROPE_GPTJ = 1 };
enum {
    DITCH_ROPE_SCALING_NONE = 0,
    DITCH_ROPE_SCALING_LINEAR = 1,
    DITCH_ROPE_SCALING_LLAMA3 = 2,
    DITCH_ROPE_SCALING_YARN = 3,
    /* per-frequency divisors (GGUF rope_freqs.weight, gguf_model.zig:171-180) */
    DITCH_ROPE_SCALING_FACTORS = 4
};
enum { DITCH_SCORING_SOFTMAX = 0, DITCH_SCORING_SIGMOID = 1 };

typedef struct ditch_model_config {
    uint64_t hidden;        /* hidden_size                                  */
    uint64_t inter;         /* intermediate_size (dense MLP)                */
    uint64_t layers;        /* num_hidden_layers                            */
    uint64_t heads;         /* num_attention_heads                          */
    uint64_t kv_heads;      /* num_key_value_heads                          */
    uint64_t head_dim;      /* q/k head dim (MLA: nope + rope)              */
    uint64_t v_head_dim;    /* value head dim (== head_dim unless MLA)      */
    uint64_t vocab;         /* vocab_size                                   */
    float rms_eps;          /* rms_norm_eps                                 */
    float attn_scale;       /* layer_attn_scale (arch.zig:1539, 1584-1591)  */
    int32_t qkv_bias;       /* q/k/v biases present (qwen2)                 */
    int32_t qk_norm;        /* per-head q/k RMSNorm before RoPE (qwen3 "head") */
    int32_t tie_embeddings; /* lm_head = embedding                          */
    /* RoPE (model.zig:2176-2282)                                           */
    int32_t rope_style;     /* DITCH_ROPE_*                                 */
    uint64_t rotary_dim;    /* rotated coordinates per head (MLA: rope dim) */
    uint64_t rope_len;      /* table rows: clamp(max_position, 512, 8192)   */
    float rope_theta;
    int32_t rope_scaling;   /* DITCH_ROPE_SCALING_*                         */
    float rope_factor;
    float rope_low_freq_factor;
    float rope_high_freq_factor;
    float rope_original_max_position;
    float yarn_beta_fast;
    float yarn_beta_slow;
    float yarn_attention_factor;
    int32_t yarn_truncate;
    const float *rope_factors; /* [rotary_dim / 2] for DITCH_ROPE_SCALING_FACTORS */
    /* MoE (moe.zig:177-389, 998-1228)                                      */
    uint64_t n_experts;     /* routed experts (0 = dense model)             */
    uint64_t top_k;
    uint64_t moe_inter;     /* expert FFN width                             */
    uint64_t shared_inter;  /* shared-expert FFN width (0 = none)           */
    int32_t scoring;        /* DITCH_SCORING_*                              */
    int32_t norm_topk_prob;
    int32_t group_limited;  /* topk_method group_limited (noaux_tc)         */
    uint64_t n_group;
    uint64_t topk_group;
    float routed_scaling;
    const uint8_t *moe_layers; /* [layers]: 1 = routed MoE MLP              */
    /* MLA (model.zig:3292-3342); q_lora_rank 0 = q_b reads h directly       */
    int32_t mla;
    uint64_t q_lora_rank;
    uint64_t kv_lora_rank;
    uint64_t qk_nope_dim;
    uint64_t qk_rope_dim;
    float mla_norm_eps;     /* latent_norm_eps                              */
} ditch_model_config;

/* Tensor slots of ditch_hip_model_set. Per layer unless marked global.    */
enum {
    DITCH_SLOT_EMBED = 0,        /* global [vocab][hidden]                  */
    DITCH_SLOT_FINAL_NORM = 1,   /* global [hidden]                         */
    DITCH_SLOT_LM_HEAD = 2,      /* global [vocab][hidden] (absent if tied) */
    DITCH_SLOT_ATTN_NORM = 10,
    DITCH_SLOT_Q = 11,
    DITCH_SLOT_K = 12,
    DITCH_SLOT_V = 13,
    DITCH_SLOT_O = 14,
    DITCH_SLOT_Q_BIAS = 15,
    DITCH_SLOT_K_BIAS = 16,
    DITCH_SLOT_V_BIAS = 17,
    DITCH_SLOT_Q_NORM = 18,
    DITCH_SLOT_K_NORM = 19,
    DITCH_SLOT_FFN_NORM = 20,
    DITCH_SLOT_GATE = 21,
    DITCH_SLOT_UP = 22,
    DITCH_SLOT_DOWN = 23,
    DITCH_SLOT_ROUTER = 30,
    DITCH_SLOT_ROUTER_CORRECTION = 31, /* e_score_correction_bias [n_experts] */
    DITCH_SLOT_EXPERT_GATE = 32,       /* `expert` selects the expert       */
    DITCH_SLOT_EXPERT_UP = 33,
    DITCH_SLOT_EXPERT_DOWN = 34,
    DITCH_SLOT_SHARED_GATE = 35,
    DITCH_SLOT_SHARED_UP = 36,
    DITCH_SLOT_SHARED_DOWN = 37,
    DITCH_SLOT_MLA_Q_A = 40,
    DITCH_SLOT_MLA_Q_A_NORM = 41,
    DITCH_SLOT_MLA_Q_B = 42,
    DITCH_SLOT_MLA_KV_A = 43,
    DITCH_SLOT_MLA_KV_A_NORM = 44,
    DITCH_SLOT_MLA_KV_B = 45
};

/* model.Row (model.zig): prompt slot `b` and position `pos` of a token.   */
typedef struct ditch_row {
    uint32_t b;
    uint32_t pos;
} ditch_row;

typedef struct ditch_hip_model ditch_hip_model;
ditch_hip_model *ditch_hip_model_create(ditch_hip *h, const ditch_model_config *cfg);
void ditch_hip_model_free(ditch_hip_model *m);
/* Registers (uploads) one tensor. Norm/bias slots take DITCH_F32/BF16/F16
 * vectors (rows = 1). `expert` is ignored except for expert slots.        */
int32_t ditch_hip_model_set(ditch_hip_model *m, int32_t layer, int32_t slot,
                            int32_t expert, const ditch_weight *w);
/* Low-rank delta W' = W + B A on a matrix slot (tensor.zig:588-592; applied
 * as the matmul epilogue of tensor.zig:871-880): a [rank][cols], b [rows][rank]. */
int32_t ditch_hip_model_set_delta(ditch_hip_model *m, int32_t layer,
                                  int32_t slot, int32_t expert, uint64_t rank,
                                  const float *a, const float *b);
/* model.resetDeltas (model.zig:2348).                                      */
/* Routed-expert streaming (the reference's ExpertCache, expert_cache.zig:
 * 108-607). Call before registering experts: each routed expert matrix set
 * afterwards is re-tiled on the device, kept in pinned host memory and freed
 * from HBM; the forward keeps a device cache of `bytes` (whole experts: gate
 * + up + down) and copies a layer's routed experts in on a copy stream of
 * its own once the router has picked them, evicting the experts whose layer
 * comes back last; a layer whose experts do not fit runs in chunks that do.
 * InvalidArgument when experts were registered before, or at the first
 * forward when `bytes` holds less than one expert.                         */
int32_t ditch_hip_model_set_expert_cache(ditch_hip_model *m, uint64_t bytes);

typedef struct ditch_expert_cache_stats {
    uint64_t capacity;    /* bytes given                                     */
    uint64_t slots;       /* experts the cache holds at once                  */
    uint64_t resident;    /* experts resident now                             */
    uint64_t hits;        /* routed experts found resident                    */
    uint64_t misses;      /* routed experts copied in on demand               */
    uint64_t prefetched;  /* experts copied ahead for the next routed layer   */
    uint64_t bytes_read;  /* host -> device bytes                             */
    uint64_t evictions;
    uint64_t slot_bytes;  /* bytes of one expert's slot                       */
    uint64_t warmed;      /* experts copied in by ditch_hip_model_warm_experts */
    uint64_t bytes_staged; /* of bytes_read, through the pinned staging ring  */
} ditch_expert_cache_stats;
/* The experts' host copies are pinned up to 48 GiB per model, shared
 * evenly by its routed layers (the environment variable
 * DITCH_HIP_EXPERT_PINNED_LIMIT, in bytes, read at registration, overrides
 * the total) and while pinning succeeds; the rest stay in pageable memory
 * and reach the cache through a small pinned staging ring, as stream.zig's
 * pinned buffers feed the reference's expert cache. Refills prefer pinned
 * experts, and copies ahead spread a cache's shortfall over the layers.
 * Zeros before the first forward of a streaming model. An expert copied in
 * ahead of its use (prefetched or warmed) counts as a miss at its first use
 * (expert_cache.zig:403-410).                                              */
int32_t ditch_hip_model_expert_cache_stats(const ditch_hip_model *m, ditch_expert_cache_stats *out);
/* ExpertCache.hotExperts / warm (expert_cache.zig:501-607): the routed
 * experts acquired so far with their use counts, most used first (ties by
 * layer, then expert), for the caller to keep (ditch writes it as a hotlist
 * file) and give back to the next run's model: warm copies the hottest
 * streamed experts that fit the free slots in before the first forward,
 * stopping at the first entry with no uses; entries naming no streamed
 * routed expert of the model are skipped. hot_experts writes min(capacity,
 * count) entries and sets *count to the number there are.                  */
typedef struct ditch_hot_expert {
    uint32_t layer;
    uint32_t expert;
    uint64_t uses;
} ditch_hot_expert;
int32_t ditch_hip_model_hot_experts(ditch_hip_model *m, ditch_hot_expert *out, uint64_t capacity,
                                    uint64_t *count);
int32_t ditch_hip_model_warm_experts(ditch_hip_model *m, const ditch_hot_expert *hot, uint64_t n,
                                     uint64_t *warmed);

int32_t ditch_hip_model_reset_deltas(ditch_hip_model *m);
/* HBM bytes held by the model's weights.                                   */
uint64_t ditch_hip_model_bytes(const ditch_hip_model *m);

/* Loads a checkpoint from disk into a resident model (Model.load,
 * model.zig, with safetensors.zig / gguf_model.zig underneath): `path` is a
 * Hugging Face directory (config.json and *.safetensors shards: plain
 * f32/f16/bf16, FP8 with block scales, compressed-tensors pack-quantized
 * INT and mxfp4-pack-quantized, all kept packed) or a GGUF v3 file (block
 * types kept packed; llama's q/k rows restored to the Hugging Face order).
 * Families: llama, qwen2, qwen3, qwen3_moe, deepseek_v3. The files are
 * memory-mapped and each weight goes through pinned host memory to HBM.
 * expert_cache_bytes > 0 streams the routed experts as
 * ditch_hip_model_set_expert_cache does. NULL on failure, with the message
 * in ditch_hip_last_error(h).                                              */
ditch_hip_model *ditch_hip_model_load(ditch_hip *h, const char *path,
                                      uint64_t expert_cache_bytes);
/* The model's configuration (moe_layers points into the model; valid while
 * it lives; rope_factors is NULL).                                         */
int32_t ditch_hip_model_get_config(const ditch_hip_model *m, ditch_model_config *out);

/* model.forward with ForwardOptions{capture_rows, residuals, logit_rows}:
 * host buffers. residuals: [(layers+1)][n_capture][hidden] (entry 0 = the
 * embedding, entry l+1 = after layer l, model.zig:4856-4862); logits:
 * [n_logit][vocab]. Either output may be NULL when its count is 0.        */
int32_t ditch_hip_forward(ditch_hip_model *m, const uint32_t *tokens,
                          const ditch_row *rows, uint64_t n,
                          const uint64_t *capture_rows, uint64_t n_capture,
                          float *residuals, const uint64_t *logit_rows,
                          uint64_t n_logit, float *logits);
/* The same with every buffer in device memory, enqueued on the context
 * stream (for callers that keep activations resident). The caller sizes the
 * KV cache as the engine does (KvCache.initFor(model, batch, max_len),
 * engine.zig:388-390): `n_prompts` prompt slots of `max_len` positions.
 * Nothing is read back: a dense model's call returns once its kernels are
 * enqueued. A routed layer whose grouped products are planned on the host
 * (streamed experts, a delta on a routed down projection, too few tokens
 * per expert) reads its expert counts back and waits for them.
 * The row descriptors stay on the device, so they are checked there: a row
 * with b >= n_prompts or pos >= max_len, a token id outside the embedding
 * or a capture/logit row >= n is clamped or skipped (no access leaves its
 * buffer) and its outputs are unspecified. `residuals_bytes` / `logits_bytes`
 * are the output buffers' lengths, checked against
 * (layers+1) * n_capture * hidden * 4 and n_logit * vocab * 4.            */
int32_t ditch_hip_forward_device(ditch_hip_model *m, const uint32_t *d_tokens,
                                 const ditch_row *d_rows, uint64_t n,
                                 uint32_t n_prompts, uint32_t max_len,
                                 const uint64_t *d_capture_rows,
                                 uint64_t n_capture, float *d_residuals,
                                 uint64_t residuals_bytes,
                                 const uint64_t *d_logit_rows, uint64_t n_logit,
                                 float *d_logits, uint64_t logits_bytes);

/* Which plan the routed layers took since the model was created: grouped
 * products planned on the device (no host round trip) or on the host after
 * reading the expert counts back. No reference counterpart (diagnostics).  */
typedef struct ditch_model_path_stats {
    uint64_t moe_device_planned;
    uint64_t moe_host_planned;
} ditch_model_path_stats;
int32_t ditch_hip_model_path_stats(const ditch_hip_model *m, ditch_model_path_stats *out);

/* ------------------------------------------------------------------------ */
/* Generation (model.generate / generateKeep, model.zig:5358-5444; the
 * keyword scorer's decode loop, engine.zig:254-268).                       */

/* KvCache.initFor(model, batch, max_len) (model.zig:2586-2724): every
 * layer's keys and values for n_prompts x max_len positions in HBM, kept
 * across calls (max_len <= 1024).                                          */
typedef struct ditch_hip_kv_cache ditch_hip_kv_cache;
ditch_hip_kv_cache *ditch_hip_kv_cache_create(ditch_hip_model *m, uint32_t n_prompts,
                                              uint32_t max_len);
void ditch_hip_kv_cache_free(ditch_hip_kv_cache *c);
/* model.forward through the persistent cache: rows {b, pos} write their
 * keys and values at (b, pos) of every layer and attend to positions
 * 0..pos of their prompt, including those earlier calls wrote (a prefill,
 * then one row per prompt a step). Device buffers, the context stream; rows
 * outside the cache are skipped as in ditch_hip_forward_device.            */
int32_t ditch_hip_forward_cached(ditch_hip_model *m, ditch_hip_kv_cache *c,
                                 const uint32_t *d_tokens, const ditch_row *d_rows,
                                 uint64_t n, const uint64_t *d_logit_rows,
                                 uint64_t n_logit, float *d_logits,
                                 uint64_t logits_bytes);
/* model.Sampler (model.zig:5208-5264): temperature <= 0 is greedy; top_k is
 * clamped to 1..256; rng is the state of the Sampler's
 * std.Random.DefaultPrng (Xoshiro256++), set by ditch_hip_sampler_init
 * (Sampler.init, model.zig:5216-5218). Every sampled pick takes one
 * Random.float(f64) draw from it, in row order, so a sampler used for the
 * same logits in the same order picks the reference's tokens.             */
typedef struct ditch_sampler {
    float temperature;
    uint32_t top_k;
    float top_p;
    uint32_t reserved;
    uint64_t rng[4];
} ditch_sampler;
/* Sampler.init(seed, temperature, top_k, top_p). Host only.               */
int32_t ditch_hip_sampler_init(ditch_sampler *s, uint64_t seed, float temperature,
                               uint64_t top_k, float top_p);
/* The next token of each of n logit rows on the device: the first maximum
 * (argmax, model.zig:5194-5204) when `sampler` is NULL or greedy, else
 * Sampler.pick of each row in order, advancing sampler->rng by the rows'
 * draws (taken on the host when the call is made).                        */
int32_t ditch_hip_pick_tokens_device(ditch_hip *h, uint32_t *d_out, const float *d_logits,
                                     uint64_t n, uint64_t vocab,
                                     ditch_sampler *sampler, void *stream);
/* generateKeep: prefill of n_prompts prompts (tokens flattened, prompt_lens
 * each), then up to max_new_tokens tokens per prompt, a prompt stopping at
 * an EOS id or a full cache. Host buffers: out_tokens [n_prompts]
 * [max_new_tokens], out_lens [n_prompts], first_logits (NULL or
 * [n_prompts][vocab], the prefill's next-token logits). A sampler's rng
 * advances by one draw per sampled token, as the reference's does.        */
int32_t ditch_hip_generate(ditch_hip_model *m, ditch_hip_kv_cache *c,
                           const uint32_t *tokens, const uint64_t *prompt_lens,
                           uint64_t n_prompts, uint64_t max_new_tokens,
                           const uint32_t *eos_ids, uint64_t n_eos,
                           ditch_sampler *sampler, uint32_t *out_tokens,
                           uint64_t *out_lens, float *first_logits);

/* ------------------------------------------------------------------------ */
/* Rank-k edit, `none` mode (abliterate.zig:264-280): a = V^T W ([k][cols]),
 * b = -weight * V ([rows][k]) for directions v [k][rows]. Host buffers.    */
int32_t ditch_hip_edit_delta(ditch_hip *h, float *a, float *b,
                             const ditch_weight *w, const float *v, uint64_t k,
                             float weight);
/* The same on a registered model matrix, installing the delta in place of
 * model.setDelta (abliterate.zig:193-197).                                 */
int32_t ditch_hip_model_edit(ditch_hip_model *m, int32_t layer, int32_t slot,
                             int32_t expert, const float *v, uint64_t k,
                             float weight);

/* One matrix of a batch edit: the slot (expert -1 for a dense slot), the
 * edit's weight and its k directions v [k][rows] (host memory, rows = the
 * matrix's rows; several targets may share one v).                        */
typedef struct ditch_edit_target {
    int32_t layer, slot, expert;
    float weight;
    const float *v;
} ditch_edit_target;
/* ditch_hip_model_edit for n matrices in one call (abliterate.apply's loop
 * over layers, components and experts, abliterate.zig:148-210, `none`
 * mode): every resident matrix's a = V^T W in one grouped launch over the
 * resident tiles, every b = -weight V in another, all deltas in one device
 * allocation (freed with the last of them); a streamed expert is staged on
 * the device on its own. Returns when the deltas are installed.           */
int32_t ditch_hip_model_edit_batch(ditch_hip_model *m,
                                   const ditch_edit_target *targets, uint64_t n,
                                   uint64_t k);

/* The edit in every row-normalisation mode (abliterate.computeDelta,
 * abliterate.zig:223-350; Options abliterate.zig:63-84): `none` as above,
 * `pre` (directions over the row-normalised matrix, B scaled by the row
 * norms), `full` (the default: the renormalised edit's delta approximated by
 * a rank-max(lora_rank, k) randomised SVD with 2r+4 columns and 6 power
 * iterations, abliterate.zig:282-349, 473-538), and the input-side
 * ablation that widens the delta by k (abliterate.zig:234-261). All passes
 * over W run on the device over the resident (quantised) weight.
 * The SVD's Gaussian test matrix is ditch_hip_edit_gaussian(q * cols, seed),
 * the reference's own draws (abliterate.zig:474-479).                      */
enum { DITCH_ROWNORM_NONE = 0, DITCH_ROWNORM_PRE = 1, DITCH_ROWNORM_FULL = 2 };
typedef struct ditch_edit_options {
    int32_t row_normalization; /* DITCH_ROWNORM_*                              */
    uint32_t lora_rank;        /* `full`: rank r (the reference's default: 3)   */
    uint64_t seed;             /* `full`: the test matrix's seed                */
    int32_t ablate_inputs;     /* nonzero: the input-side ablation as well      */
} ditch_edit_options;
/* Rank of the delta for a rows x cols matrix and k directions.            */
uint64_t ditch_hip_edit_rank(uint64_t rows, uint64_t cols, uint64_t k,
                             const ditch_edit_options *opts);
/* Host buffers: a [rank][cols], b [rows][rank] with rank = ditch_hip_edit_rank
 * (a_len / b_len: their lengths in floats, checked).                       */
int32_t ditch_hip_edit_delta_ex(ditch_hip *h, float *a, uint64_t a_len, float *b,
                                uint64_t b_len, const ditch_weight *w,
                                const float *v, uint64_t k, float weight,
                                const ditch_edit_options *opts);
/* The same on a registered model matrix, installing the delta
 * (model.setDelta, abliterate.zig:193-197).                                */
int32_t ditch_hip_model_edit_ex(ditch_hip_model *m, int32_t layer, int32_t slot,
                                int32_t expert, const float *v, uint64_t k,
                                float weight, const ditch_edit_options *opts);
/* The first n draws of Random.floatNorm(f32) from Zig's
 * std.Random.DefaultPrng.init(seed) (Xoshiro256++ seeded by SplitMix64, the
 * ziggurat normal): the full edit's test matrix, and, with seed ^
 * 0x5eedd1ec7105, the sketch's (directions.zig:65-67). Host only.         */
void ditch_hip_edit_gaussian(float *out, uint64_t n, uint64_t seed);

/* ------------------------------------------------------------------------ */
/* log-softmax of n rows (tensor.zig:1203-1210: f32 max, f64 sum, f32 x-lse). */
int32_t ditch_hip_logSoftmaxRows(ditch_hip *h, float *out, const float *x,
                                 uint64_t n, uint64_t len);
/* Per-row KL(base || trial) in f64 (scorers.zig:387-394): base_logprobs are
 * the baseline log-softmax rows, trial_logits raw logits.                 */
int32_t ditch_hip_klRows(ditch_hip *h, double *kl, const float *base_logprobs,
                         const float *trial_logits, uint64_t n, uint64_t vocab);
/* The same two on device memory, enqueued on `stream` (NULL = the context
 * stream) and not waited for: the scorer's inputs stay in HBM after
 * ditch_hip_forward_device. d_out may equal d_x (in place). These take no
 * buffer lengths: d_out and d_x hold n * len floats, d_base_logprobs and
 * d_trial_logits n * vocab floats, d_kl n doubles (a shorter buffer is
 * written or read past its end).                                          */
int32_t ditch_hip_logSoftmaxRows_device(ditch_hip *h, float *d_out,
                                        const float *d_x, uint64_t n,
                                        uint64_t len, void *stream);
int32_t ditch_hip_klRows_device(ditch_hip *h, double *d_kl,
                                const float *d_base_logprobs,
                                const float *d_trial_logits, uint64_t n,
                                uint64_t vocab, void *stream);

/* ------------------------------------------------------------------------ */
/* The step after residual capture, on device memory (enqueued on `stream`,
 * NULL = the context stream, not waited for). These take no buffer
 * lengths: every device buffer must hold the elements its shape below
 * names (d_first and d_take: prompts entries each; d_mean and d_sum: n;
 * d_dirs, d_good_means, d_bad_means, d_first (basis), d_center: entries *
 * hidden, d_dirs of the basis entries * k * hidden).                       */

/* Engine.forEachResidual's per-batch reduction (engine.zig:414-431): for
 * prompt b and layer entry l, v = mean of the prompt's take[b] captured rows
 * starting at capture index first[b] (the residuals of forward_device,
 * [entries][n_capture][hidden]), clamped to +-quantile(|v|, winsor_q) when
 * 0 <= winsor_q < 1 (torch.quantile interpolation, engine.zig:492-499);
 * written to d_vout [prompts][entries][hidden] and added, prompt after
 * prompt, to the f64 sums d_sum [entries][hidden] (getResidualMeanObserved,
 * engine.zig:314-337) and, when d_sq is not NULL, to the squares d_sq
 * (directions.Moments, directions.zig:196-205). Winsorising needs
 * hidden <= 16384.                                                          */
int32_t ditch_hip_residual_reduce_device(ditch_hip *h, const float *d_residuals,
                                         uint64_t entries, uint64_t n_capture,
                                         uint64_t hidden, const uint32_t *d_first,
                                         const uint32_t *d_take, uint64_t prompts,
                                         float winsor_q, float *d_vout,
                                         double *d_sum, double *d_sq, void *stream);
/* mean[i] = f32(sum[i] / max(count, 1))          (engine.zig:333-335)       */
int32_t ditch_hip_residual_mean_device(ditch_hip *h, float *d_mean, const double *d_sum,
                                       uint64_t count, uint64_t n, void *stream);
/* abliterate.computeDirections (abliterate.zig:88-109): unit bad - good per
 * entry, optionally orthogonal to the good mean.                           */
int32_t ditch_hip_directions_device(ditch_hip *h, float *d_dirs, const float *d_good_means,
                                    const float *d_bad_means, uint64_t entries,
                                    uint64_t hidden, int32_t orthogonalize, void *stream);
/* directions.Sketch.add (directions.zig:80-104) for a batch of per-prompt
 * residuals d_v [prompts][entries][hidden] (ditch_hip_residual_reduce's
 * d_vout): z = v - center, p = Omega^T z, Y += z p^T, W += p p^T in f64.
 * d_y [entries][m][hidden], d_w [entries][m][m], d_omega [m][hidden] (the
 * caller's Gaussian test matrix: the reference's is m = min(max(4k, 8),
 * hidden) rows of ditch_hip_edit_gaussian with seed ^ 0x5eedd1ec7105).     */
int32_t ditch_hip_sketch_add_device(ditch_hip *h, double *d_y, double *d_w,
                                    const float *d_omega, uint64_t m,
                                    const float *d_center, const float *d_v,
                                    uint64_t prompts, uint64_t entries,
                                    uint64_t hidden, void *stream);
/* directions.computeBasisFrom with Sketch.factor (directions.zig:108-134,
 * 371-455): the [entries][k][hidden] orthonormal bases from the first
 * directions, the good means and the sketch (any k and m; sketches of up
 * to 96 columns keep the eigen-solver in LDS, wider ones in global scratch). */
int32_t ditch_hip_basis_device(ditch_hip *h, float *d_dirs, const float *d_first,
                               const float *d_good_means, uint64_t entries,
                               uint64_t hidden, uint64_t k, int32_t orthogonalize,
                               const double *d_y, const double *d_w, uint64_t m,
                               void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DITCH_HIP_H */
