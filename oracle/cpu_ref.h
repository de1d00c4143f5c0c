/*
 * cpu_ref.h — CPU restatement of ditch's reference numerics (test
 * infrastructure only).
 *
 * This library is the ORACLE the HIP path is checked against. It is not part
 * of the product: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it, and nothing in ditch_amd/ links or calls it.
 *
 * Every function restates a reference function (file:line under the
 * reference's src/) in plain C: f32 arithmetic in the same order, fused
 * multiply-adds exactly where the reference writes @mulAdd (tensor.zig:
 * 676-687), no other contraction (built with -ffp-contract=off), f64 where
 * the reference uses f64. The lane width of the dot products is VL = 16, the
 * reference's AVX-512 build (tensor.zig:628-669).
 *
 * Parity unpinned: ref_zig_float64's extra draws when a draw's top 12 bits
 * are zero (Zig 0.16's Random.float, restated without a Zig toolchain to
 * run it); the rest of the Zig stream is pinned by Zig's own sequence tests
 * and the xoshiro256 jump polynomial.
 */
#ifndef DITCH_CPU_REF_H
#define DITCH_CPU_REF_H

#include <stddef.h>
#include <stdint.h>
#include "../include/ditch_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define REF_VL 16

/* conversions (tensor.zig:419-440) */
float ref_bf16_to_f32(uint16_t v);
uint16_t ref_f32_to_bf16(float v);
float ref_f16_to_f32(uint16_t v);
uint16_t ref_f32_to_f16(float v);
void ref_f32_to_bf16_array(const float *in, uint16_t *out, size_t n);
void ref_bf16_to_f32_array(const uint16_t *in, float *out, size_t n);

/* element tables (dequant.zig:259-310) */
float ref_fp8_value(uint8_t code, int e5m2);
float ref_e8m0_scale(uint8_t b);   /* e8m0Scale: 0 -> 2^-127 subnormal */
float ref_e8m0(uint8_t b);         /* e8m0: 255 -> NaN, else ldexp(1, b-127) */
uint32_t ref_unpack_field(const uint32_t *words, size_t i, int bits);

/* decoders */
size_t ref_row_bytes(int dtype, size_t cols);
/* GGUF block dequantisation of n elements (quant.zig:57-79). 0 on success. */
int ref_gguf_dequant(int dtype, const uint8_t *bytes, float *out, size_t n);
/* Q8_0 reference quantiser (quant.zig:245-255). */
void ref_quantize_q8_0(const float *x, size_t n, uint8_t *out);
/* Rows [row0, row0+nrows) of `w` as ditch_hip_dequant outputs them: bf16 for
 * DITCH_FP8/MXFP4/MXFP4_T/INT_PACKED, f32 otherwise. 0 on success. */
int ref_dequant_rows(const ditch_weight *w, size_t row0, size_t nrows, void *out);
/* One row of `w` widened to f32 (tensor.Weight.row, tensor.zig:523-526). */
int ref_weight_row(const ditch_weight *w, size_t r, float *out);

/* products (tensor.zig:545-558, 827-1122) */
float ref_dot(const float *a, const float *b, size_t n);
/* out[n][rows] = x @ W^T (+ x @ (B A)^T); rank 0 = no delta. */
int ref_matmulT(float *out, const float *x, size_t n, const ditch_weight *w,
                size_t rank, const float *a, const float *b, int threads);
int ref_matvecTMulti(float *out, const ditch_weight *w, const float *y, size_t q,
                     int threads);
int ref_rowNorms(float *out, const ditch_weight *w, int threads);

/* element-wise kernels (tensor.zig:1126-1381) */
void ref_attention_scores(float *scores, size_t n_keys, const float *q, size_t hd,
                          const float *k, size_t stride, float scale);
void ref_attention_values(float *out, size_t vd, const float *scores,
                          size_t n_keys, const float *v, size_t stride);
void ref_rmsnorm(float *out, const float *x, const float *w, size_t wlen,
                 size_t len, float eps, int gemma_style);
void ref_layernorm(float *out, const float *x, const float *w, size_t wlen,
                   const float *bias, size_t len, float eps, int one_plus);
void ref_softmax_inplace(float *x, size_t len);
void ref_log_softmax(float *out, const float *x, size_t len);
float ref_exp_cephes(float x);
float ref_act_scalar(uint32_t act, float x);
void ref_gated_activation(uint32_t act, float *out, const float *gate,
                          const float *up, size_t n, size_t len,
                          size_t in_stride, size_t out_stride);
void ref_rope_rows(float *x, size_t n, size_t dim, const float *cos_t,
                   const float *sin_t, size_t half, const uint32_t *pos,
                   uint32_t style);

/* RoPE tables (model.zig:2200-2282): cos/sin [len][rotary_dim/2]. */
int ref_fill_rope(const ditch_model_config *c, float *cos_t, float *sin_t);

/* KL of one row (scorers.zig:387-394) in f64. */
double ref_kl_row(const float *base_logprobs, const float *trial_logits,
                  size_t vocab);

/* edit, none mode (abliterate.zig:264-280) */
int ref_edit_delta(float *a, float *b, const ditch_weight *w, const float *v,
                   size_t k, float weight, int threads);

/* direction pipeline: engine.zig:414-431 (window mean, winsorising, f64
 * sums), directions.zig:196-205 (Moments), abliterate.zig:88-109, 409-423,
 * directions.zig:80-134, 371-500 (Sketch, computeBasisFrom)               */
int ref_residual_reduce(const float *res, size_t entries, size_t n_capture, size_t hidden, const uint32_t *first,
                        const uint32_t *take, size_t prompts, float q, float *vout, double *sum, double *sq);
void ref_directions(float *dirs, const float *good, const float *bad, size_t entries, size_t hidden,
                    int orthogonalize);
void ref_orthonormalize(float *vecs, size_t q, size_t n);
void ref_sketch_add(double *y, double *w, const float *omega, size_t m, const float *center, const float *v,
                    size_t prompts, size_t entries, size_t hidden);
void ref_symmetric_eigen(double *m, double *vecs, size_t n);
int ref_basis(float *dirs, const float *first, const float *good_means, size_t entries, size_t hidden, size_t k,
              int orthogonalize, const double *y, const double *w, size_t m);

/* the edit in every mode (abliterate.zig:223-538): mode 0 none, 1 pre,
 * 2 full (rank-r randomised SVD seeded by ref_edit_gaussian), optional
 * input-side ablation; a [rank][cols], b [rows][rank]                      */
void ref_edit_gaussian(float *out, size_t n, uint64_t seed);
/* Zig's std.Random stream (DefaultPrng, float(f64), floatNorm) and the
 * Sampler's pick over it                                                   */
void ref_zig_init(uint64_t st[4], uint64_t seed);
uint64_t ref_zig_next(uint64_t st[4]);
double ref_zig_float64(uint64_t st[4]);
double ref_zig_norm(uint64_t st[4]);
void ref_zig_norm_tables(double *x, double *f);
void ref_zig_draws(void *out, size_t n, uint64_t seed, int kind);
void ref_sampler_pick(uint32_t *out, const float *logits, size_t n, size_t vocab, uint64_t st[4],
                      float temperature, size_t top_k, float top_p);
void ref_jacobi_f32(float *m, float *vecs, size_t n);
int ref_edit_delta_ex(float *a_out, float *b_out, size_t *rank_out, const ditch_weight *w, const float *v, size_t k,
                      float weight, int mode, size_t lora_rank, uint64_t seed, int ablate, int threads);

/* model (model.zig:4619-4959, moe.zig:998-1228, model.zig:3292-3342) */
typedef struct ref_model ref_model;
ref_model *ref_model_create(const ditch_model_config *cfg);
void ref_model_free(ref_model *m);
int ref_model_set(ref_model *m, int layer, int slot, int expert,
                  const ditch_weight *w);
int ref_model_set_delta(ref_model *m, int layer, int slot, int expert,
                        size_t rank, const float *a, const float *b);
int ref_model_edit(ref_model *m, int layer, int slot, int expert,
                   const float *v, size_t k, float weight);
int ref_forward(ref_model *m, const uint32_t *tokens, const ditch_row *rows,
                size_t n, const uint64_t *capture_rows, size_t n_capture,
                float *residuals, const uint64_t *logit_rows, size_t n_logit,
                float *logits);
/* Layers run by the next ref_forward calls are [first, first+count) (for a
 * bounded CPU sample); count 0 = all layers. */
void ref_model_limit_layers(ref_model *m, size_t first, size_t count);
void ref_set_threads(ref_model *m, int threads);
void ref_model_keep_packed(ref_model *m, int on);
const char *ref_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
