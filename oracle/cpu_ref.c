/*
 * cpu_ref.c — CPU restatement of ditch's reference numerics. TEST
 * INFRASTRUCTURE ONLY (the oracle); see cpu_ref.h. Built with
 * -ffp-contract=off: every fused multiply-add below is an explicit fmaf()
 * where the reference calls @mulAdd (tensor.zig:676-687).
 */
#define _GNU_SOURCE
#include "cpu_ref.h"

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define VL REF_VL

static __thread char g_err[512];
const char *ref_last_error(void) { return g_err; }
static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* Conversions: tensor.zig:419-440                                          */

float ref_bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

uint16_t ref_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40); /* NaN */
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}

/* IEEE binary16 -> binary32, exact (the hardware cast of tensor.zig:432-435). */
float ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest even (tensor.zig:437-440). */
uint16_t ref_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (ax < 0x38800000u) {
        /* subnormal or zero in f16: value / 2^-24 rounded to nearest even */
        float a = u2f(ax);
        float q = a * 16777216.0f; /* exact scaling by 2^24 */
        float r = nearbyintf(q);   /* default rounding mode: nearest even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t man = ax & 0x7fffffu;
    uint32_t exp = (ax >> 23) - 112u;
    uint32_t h = (exp << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

void ref_f32_to_bf16_array(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = ref_f32_to_bf16(in[i]);
}
void ref_bf16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = ref_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Element tables: dequant.zig:259-321                                      */

static float pow2i(int e) { return u2f((uint32_t)(e + 127) << 23); }

/* fp8Table (dequant.zig:281-304) built value by value. */
float ref_fp8_value(uint8_t code, int e5m2) {
    int exp_bits = e5m2 ? 5 : 4;
    int man_bits = 7 - exp_bits;
    int bias = (1 << (exp_bits - 1)) - 1;
    int sign = code >> 7;
    int exp = (code >> man_bits) & ((1 << exp_bits) - 1);
    float man = (float)(code & ((1 << man_bits) - 1));
    float man_scale = 1.0f / (float)(1 << man_bits);
    float v;
    if (exp == 0) {
        v = man * man_scale * pow2i(1 - bias);
    } else if (exp_bits == 4 && exp == 15 && man == 7.0f) {
        v = u2f(0x7fc00000u); /* std.math.nan(f32) */
    } else if (exp_bits == 5 && exp == 31) {
        v = (man == 0.0f) ? u2f(0x7f800000u) : u2f(0x7fc00000u);
    } else {
        v = (1.0f + man * man_scale) * pow2i(exp - bias);
    }
    return sign ? -v : v;
}

float ref_e8m0_scale(uint8_t b) {
    return b == 0 ? u2f(0x00400000u) : u2f((uint32_t)b << 23);
}

float ref_e8m0(uint8_t b) {
    if (b == 255) return u2f(0x7fc00000u);
    return ldexpf(1.0f, (int)b - 127);
}

static const float e2m1_table[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                     -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

static inline uint32_t field_mask(int bits) { return bits >= 32 ? 0xffffffffu : ((1u << bits) - 1u); }

uint32_t ref_unpack_field(const uint32_t *words, size_t i, int bits) {
    size_t start = i * (size_t)bits;
    size_t w = start / 32;
    int off = (int)(start % 32);
    int lo = (32 - off) < bits ? (32 - off) : bits;
    uint32_t v = (words[w] >> off) & field_mask(lo);
    if (lo < bits) v |= (words[w + 1] & field_mask(bits - lo)) << lo;
    return v;
}

/* ------------------------------------------------------------------------ */
/* GGUF blocks: quant.zig:27-199                                            */

static size_t gguf_block_size(int dt) {
    switch (dt) {
    case DITCH_Q8_0: case DITCH_Q4_0: case DITCH_Q4_1: case DITCH_Q5_0: case DITCH_Q5_1: return 32;
    case DITCH_Q4_K: case DITCH_Q6_K: case DITCH_Q8_K: return 256;
    default: return 1;
    }
}
static size_t gguf_block_bytes(int dt) {
    switch (dt) {
    case DITCH_F32: return 4;
    case DITCH_F16: case DITCH_BF16: return 2;
    case DITCH_Q8_0: return 34;
    case DITCH_Q4_0: return 18;
    case DITCH_Q4_1: return 20;
    case DITCH_Q5_0: return 22;
    case DITCH_Q5_1: return 24;
    case DITCH_Q4_K: return 144;
    case DITCH_Q6_K: return 210;
    case DITCH_Q8_K: return 292;
    default: return 0;
    }
}

size_t ref_row_bytes(int dtype, size_t cols) {
    size_t bs = gguf_block_size(dtype), bb = gguf_block_bytes(dtype);
    if (bb == 0 || cols % bs) return 0;
    return cols / bs * bb;
}

static inline float rd_f16(const uint8_t *b) { return ref_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }
static inline uint32_t rd_u32(const uint8_t *b) { return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24); }

static void dq_q8_0(const uint8_t *b, float *y) {
    float d = rd_f16(b);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}
static void dq_q4_0(const uint8_t *b, float *y) {
    float d = rd_f16(b);
    for (int j = 0; j < 16; j++) {
        int x0 = (b[2 + j] & 0x0f) - 8, x1 = (b[2 + j] >> 4) - 8;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}
static void dq_q4_1(const uint8_t *b, float *y) {
    float d = rd_f16(b), m = rd_f16(b + 2);
    for (int j = 0; j < 16; j++) {
        y[j] = (float)(b[4 + j] & 0x0f) * d + m;
        y[j + 16] = (float)(b[4 + j] >> 4) * d + m;
    }
}
static void dq_q5_0(const uint8_t *b, float *y) {
    float d = rd_f16(b);
    uint32_t qh = rd_u32(b + 2);
    for (int j = 0; j < 16; j++) {
        uint32_t xh0 = ((qh >> j) << 4) & 0x10u;
        uint32_t xh1 = (qh >> (j + 12)) & 0x10u;
        int x0 = (int)((b[6 + j] & 0x0f) | xh0) - 16;
        int x1 = (int)((b[6 + j] >> 4) | xh1) - 16;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}
static void dq_q5_1(const uint8_t *b, float *y) {
    float d = rd_f16(b), m = rd_f16(b + 2);
    uint32_t qh = rd_u32(b + 4);
    for (int j = 0; j < 16; j++) {
        uint32_t xh0 = ((qh >> j) << 4) & 0x10u;
        uint32_t xh1 = (qh >> (j + 12)) & 0x10u;
        uint32_t x0 = (b[8 + j] & 0x0f) | xh0;
        uint32_t x1 = (b[8 + j] >> 4) | xh1;
        y[j] = (float)x0 * d + m;
        y[j + 16] = (float)x1 * d + m;
    }
}
static void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; return; }
    *d = (uint8_t)((q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
}
static void dq_q4_k(const uint8_t *b, float *y) {
    float d = rd_f16(b), mn = rd_f16(b + 2);
    const uint8_t *sc = b + 4, *q = b + 16;
    int is = 0, o = 0;
    for (int j = 0; j < 256; j += 64) {
        uint8_t s1, m1_, s2, m2_;
        scale_min_k4(is, sc, &s1, &m1_);
        scale_min_k4(is + 1, sc, &s2, &m2_);
        float d1 = d * (float)s1, m1 = mn * (float)m1_;
        float d2 = d * (float)s2, m2 = mn * (float)m2_;
        for (int l = 0; l < 32; l++) y[o + l] = d1 * (float)(q[l] & 0xf) - m1;
        for (int l = 0; l < 32; l++) y[o + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        o += 64; q += 32; is += 2;
    }
}
static void dq_q6_k(const uint8_t *b, float *y) {
    const uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
    float d = rd_f16(b + 208);
    int o = 0;
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xf) | (((qh[l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[o + l] = d * (float)(int8_t)sc[is] * (float)q1;
            y[o + l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
            y[o + l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
            y[o + l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
        }
        o += 128; ql += 64; qh += 32; sc += 8;
    }
}
static void dq_q8_k(const uint8_t *b, float *y) {
    float d = u2f(rd_u32(b));
    for (int j = 0; j < 256; j++) y[j] = d * (float)(int8_t)b[4 + j];
}

int ref_gguf_dequant(int dt, const uint8_t *bytes, float *out, size_t n) {
    size_t bs = gguf_block_size(dt), bb = gguf_block_bytes(dt);
    if (bs <= 1 || n % bs) return fail("gguf_dequant: bad dtype %d / n %zu", dt, n);
    for (size_t i = 0; i < n / bs; i++) {
        const uint8_t *b = bytes + i * bb;
        float *y = out + i * bs;
        switch (dt) {
        case DITCH_Q8_0: dq_q8_0(b, y); break;
        case DITCH_Q4_0: dq_q4_0(b, y); break;
        case DITCH_Q4_1: dq_q4_1(b, y); break;
        case DITCH_Q5_0: dq_q5_0(b, y); break;
        case DITCH_Q5_1: dq_q5_1(b, y); break;
        case DITCH_Q4_K: dq_q4_k(b, y); break;
        case DITCH_Q6_K: dq_q6_k(b, y); break;
        case DITCH_Q8_K: dq_q8_k(b, y); break;
        default: return fail("gguf_dequant: dtype %d", dt);
        }
    }
    return 0;
}

/* quantQ8_0 (quant.zig:245-255): amax/127 as f16, @round(x * id). */
void ref_quantize_q8_0(const float *x, size_t n, uint8_t *out) {
    for (size_t blk = 0; blk < n / 32; blk++) {
        const float *xb = x + blk * 32;
        uint8_t *b = out + blk * 34;
        float amax = 0;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        float d = amax / 127.0f;
        float id = d != 0 ? 1.0f / d : 0.0f;
        uint16_t h = ref_f32_to_f16(d);
        b[0] = (uint8_t)(h & 0xff);
        b[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
    }
}

/* ------------------------------------------------------------------------ */
/* Quantised-safetensors decoders -> bf16 (dequant.zig:471-673)             */

static float scale_to_f32(int sdt, const void *base, size_t idx) {
    switch (sdt) {
    case DITCH_F32: return ((const float *)base)[idx];
    case DITCH_BF16: return ref_bf16_to_f32(((const uint16_t *)base)[idx]);
    case DITCH_F16: return ref_f16_to_f32(((const uint16_t *)base)[idx]);
    case DITCH_E8M0: return ref_e8m0(((const uint8_t *)base)[idx]);
    default: return u2f(0x7fc00000u);
    }
}

/* dequant.zig:471-475 scaleRow */
static size_t fp8_scale_row(const ditch_weight *w, size_t r) {
    if (w->row_shard == 0) return r / w->block_rows;
    size_t per_shard = (w->row_shard + w->block_rows - 1) / w->block_rows;
    return r / w->row_shard * per_shard + (r % w->row_shard) / w->block_rows;
}

static void decode_fp8_row(const ditch_weight *w, size_t r, uint16_t *dst) {
    const uint8_t *codes = (const uint8_t *)w->data + r * w->cols;
    size_t srow = fp8_scale_row(w, r);
    for (size_t c = 0; c < w->cols; c++) {
        float s = scale_to_f32(w->scale_dtype, w->scale, srow * w->scale_cols + c / w->block_cols);
        dst[c] = ref_f32_to_bf16(ref_fp8_value(codes[c], w->fp8_e5m2) * s);
    }
}

static void decode_mxfp4_row(const ditch_weight *w, size_t r, uint16_t *dst) {
    size_t nblk = w->cols / 32;
    const uint8_t *prow = (const uint8_t *)w->data + r * (w->cols / 2);
    const uint8_t *srow = (const uint8_t *)w->scale + r * nblk;
    for (size_t k = 0; k < nblk; k++) {
        float sc = ref_e8m0_scale(srow[k]);
        for (int j = 0; j < 16; j++) {
            uint8_t b = prow[k * 16 + j];
            dst[k * 32 + 2 * j] = ref_f32_to_bf16(e2m1_table[b & 0x0f] * sc);
            dst[k * 32 + 2 * j + 1] = ref_f32_to_bf16(e2m1_table[b >> 4] * sc);
        }
    }
}

/* gpt-oss layout: view row h, column j = source row j, element h. */
static void decode_mxfp4_t_row(const ditch_weight *w, size_t h, uint16_t *dst) {
    size_t src_rows = w->cols, src_cols = w->rows;
    size_t nblk = src_cols / 32;
    size_t k = h / 32, i = h % 32;
    const uint8_t *blocks = (const uint8_t *)w->data;
    const uint8_t *scales = (const uint8_t *)w->scale;
    for (size_t j = 0; j < src_rows; j++) {
        const uint8_t *b = blocks + (j * nblk + k) * 16;
        float sc = ref_e8m0_scale(scales[j * nblk + k]);
        uint8_t byte = b[i / 2];
        float v = e2m1_table[(i & 1) ? (byte >> 4) : (byte & 0x0f)] * sc;
        dst[j] = ref_f32_to_bf16(v);
    }
}

static void decode_int_row(const ditch_weight *w, size_t r, uint16_t *dst) {
    int bits = w->bits;
    size_t wpr = (w->cols * (size_t)bits + 31) / 32;
    size_t groups = w->scale_cols;
    int offset = 1 << (bits - 1);
    const uint32_t *row_words = (const uint32_t *)w->data + r * wpr;
    const uint32_t *zw = (const uint32_t *)w->zero;
    for (size_t c = 0; c < w->cols; c++) {
        size_t g = w->g_idx ? (size_t)w->g_idx[c] : c / w->group;
        int zp = 0;
        if (zw) {
            size_t start = r * (size_t)bits;
            size_t wi = start / 32;
            int off = (int)(start % 32);
            int lo = (32 - off) < bits ? (32 - off) : bits;
            uint32_t v = (zw[wi * groups + g] >> off) & field_mask(lo);
            if (lo < bits) v |= (zw[(wi + 1) * groups + g] & field_mask(bits - lo)) << lo;
            zp = (int)v - offset;
        }
        int q = (int)ref_unpack_field(row_words, c, bits) - offset;
        float s = scale_to_f32(w->scale_dtype, w->scale, r * groups + g);
        dst[c] = ref_f32_to_bf16((float)(q - zp) * s);
    }
}

static int is_bf16_virtual(int dt) {
    return dt == DITCH_FP8 || dt == DITCH_MXFP4 || dt == DITCH_MXFP4_T || dt == DITCH_INT_PACKED;
}

static int decode_bf16_row(const ditch_weight *w, size_t r, uint16_t *dst) {
    switch (w->dtype) {
    case DITCH_FP8: decode_fp8_row(w, r, dst); return 0;
    case DITCH_MXFP4: decode_mxfp4_row(w, r, dst); return 0;
    case DITCH_MXFP4_T: decode_mxfp4_t_row(w, r, dst); return 0;
    case DITCH_INT_PACKED: decode_int_row(w, r, dst); return 0;
    default: return fail("decode_bf16_row: dtype %d", w->dtype);
    }
}

int ref_weight_row(const ditch_weight *w, size_t r, float *out) {
    size_t cols = w->cols;
    switch (w->dtype) {
    case DITCH_F32: memcpy(out, (const float *)w->data + r * cols, cols * 4); return 0;
    case DITCH_BF16: ref_bf16_to_f32_array((const uint16_t *)w->data + r * cols, out, cols); return 0;
    case DITCH_F16: {
        const uint16_t *s = (const uint16_t *)w->data + r * cols;
        for (size_t i = 0; i < cols; i++) out[i] = ref_f16_to_f32(s[i]);
        return 0;
    }
    case DITCH_Q8_0: case DITCH_Q4_0: case DITCH_Q4_1: case DITCH_Q5_0: case DITCH_Q5_1:
    case DITCH_Q4_K: case DITCH_Q6_K: case DITCH_Q8_K: {
        size_t rb = ref_row_bytes(w->dtype, cols);
        if (!rb) return fail("row bytes: cols %zu not a block multiple", cols);
        return ref_gguf_dequant(w->dtype, (const uint8_t *)w->data + r * rb, out, cols);
    }
    default:
        if (is_bf16_virtual(w->dtype)) {
            uint16_t *tmp = (uint16_t *)malloc(cols * 2);
            int rc = decode_bf16_row(w, r, tmp);
            ref_bf16_to_f32_array(tmp, out, cols);
            free(tmp);
            return rc;
        }
        return fail("weight_row: dtype %d", w->dtype);
    }
}

int ref_dequant_rows(const ditch_weight *w, size_t row0, size_t nrows, void *out) {
    if (row0 + nrows > w->rows) return fail("dequant_rows: range");
    for (size_t i = 0; i < nrows; i++) {
        int rc;
        if (is_bf16_virtual(w->dtype)) rc = decode_bf16_row(w, row0 + i, (uint16_t *)out + i * w->cols);
        else rc = ref_weight_row(w, row0 + i, (float *)out + i * w->cols);
        if (rc) return rc;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Thread pool: tensor.zig:1028-1044 row split (chunks = min(threads, n)).  */

typedef void (*range_fn)(void *ctx, size_t start, size_t end, size_t slot);
typedef struct { range_fn fn; void *ctx; size_t start, end, slot; } job_t;
static void *job_main(void *p) { job_t *j = (job_t *)p; j->fn(j->ctx, j->start, j->end, j->slot); return NULL; }

static size_t parallel_for(size_t n, int threads, range_fn fn, void *ctx) {
    if (n == 0) return 0;
    size_t chunks = (size_t)(threads < 1 ? 1 : threads);
    if (chunks > n) chunks = n;
    size_t per = (n + chunks - 1) / chunks;
    size_t slots = (n + per - 1) / per;
    if (slots == 1) { fn(ctx, 0, n, 0); return 1; }
    pthread_t *th = (pthread_t *)malloc(slots * sizeof *th);
    job_t *jobs = (job_t *)malloc(slots * sizeof *jobs);
    for (size_t s = 0; s < slots; s++) {
        jobs[s] = (job_t){fn, ctx, s * per, (s + 1) * per < n ? (s + 1) * per : n, s};
        pthread_create(&th[s], NULL, job_main, &jobs[s]);
    }
    for (size_t s = 0; s < slots; s++) pthread_join(th[s], NULL);
    free(th);
    free(jobs);
    return slots;
}

/* ------------------------------------------------------------------------ */
/* Dot products: tensor.zig:545-558 and dotTile 889-913. Lane-wise FMA over
 * VL-wide blocks, an in-order reduction, then a scalar FMA tail.           */

static inline float reduce_lanes(const float *acc) {
    float s = acc[0];
    for (int l = 1; l < VL; l++) s = s + acc[l];
    return s;
}

float ref_dot(const float *a, const float *b, size_t n) {
    float acc[VL] = {0};
    size_t i = 0;
    for (; i + VL <= n; i += VL)
        for (int l = 0; l < VL; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float s = reduce_lanes(acc);
    for (; i < n; i++) s = fmaf(a[i], b[i], s);
    return s;
}

/* 4 weight rows x 4 inputs register tile (tensor.zig:889-913); each output
 * is the same sequence of operations as ref_dot. */
static void dot_tile4x4(const float *w, const float *x, size_t cols, float out[4][4]) {
    float acc[4][4][VL];
    memset(acc, 0, sizeof acc);
    size_t i = 0;
    for (; i + VL <= cols; i += VL) {
        for (int ii = 0; ii < 4; ii++)
            for (int kk = 0; kk < 4; kk++)
                for (int l = 0; l < VL; l++)
                    acc[ii][kk][l] = fmaf(w[kk * cols + i + l], x[ii * cols + i + l], acc[ii][kk][l]);
    }
    for (int ii = 0; ii < 4; ii++)
        for (int kk = 0; kk < 4; kk++) {
            float s = reduce_lanes(acc[ii][kk]);
            for (size_t t = i; t < cols; t++) s = fmaf(w[kk * cols + t], x[ii * cols + t], s);
            out[ii][kk] = s;
        }
}

typedef struct {
    float *out;
    const float *x;
    size_t n;
    const ditch_weight *w;
    size_t rank;
    const float *a, *b, *xa;
    int err;
} mm_ctx;

static void matmul_worker(void *p, size_t start, size_t end, size_t slot) {
    (void)slot;
    mm_ctx *c = (mm_ctx *)p;
    size_t cols = c->w->cols, rows = c->w->rows, n = c->n;
    const size_t tile = 16;
    float *buf = (float *)malloc(tile * cols * sizeof(float));
    for (size_t r = start; r < end; r += tile) {
        size_t nr = end - r < tile ? end - r : tile;
        for (size_t k = 0; k < nr; k++)
            if (ref_weight_row(c->w, r + k, buf + k * cols)) c->err = 1;
        size_t i = 0;
        for (; i + 4 <= n; i += 4) {
            size_t k = 0;
            for (; k + 4 <= nr; k += 4) {
                float d[4][4];
                dot_tile4x4(buf + k * cols, c->x + i * cols, cols, d);
                for (int ii = 0; ii < 4; ii++)
                    for (int kk = 0; kk < 4; kk++) c->out[(i + ii) * rows + r + k + kk] = d[ii][kk];
            }
            for (; k < nr; k++)
                for (int ii = 0; ii < 4; ii++)
                    c->out[(i + ii) * rows + r + k] = ref_dot(buf + k * cols, c->x + (i + ii) * cols, cols);
        }
        for (; i < n; i++)
            for (size_t k = 0; k < nr; k++)
                c->out[i * rows + r + k] = ref_dot(buf + k * cols, c->x + i * cols, cols);
        if (c->rank) {
            /* delta epilogue, tensor.zig:871-880: v += b * xa (no fusion) */
            for (size_t ii = 0; ii < n; ii++) {
                const float *xa = c->xa + ii * c->rank;
                for (size_t kk = 0; kk < nr; kk++) {
                    float v = 0;
                    for (size_t j = 0; j < c->rank; j++) v = v + c->b[(r + kk) * c->rank + j] * xa[j];
                    c->out[ii * rows + r + kk] = c->out[ii * rows + r + kk] + v;
                }
            }
        }
    }
    free(buf);
}

int ref_matmulT(float *out, const float *x, size_t n, const ditch_weight *w, size_t rank,
                const float *a, const float *b, int threads) {
    if (w->rows == 0 || n == 0) return 0;
    float *xa = NULL;
    if (rank) {
        xa = (float *)malloc(n * rank * sizeof(float));
        for (size_t i = 0; i < n; i++)
            for (size_t j = 0; j < rank; j++) xa[i * rank + j] = ref_dot(a + j * w->cols, x + i * w->cols, w->cols);
    }
    mm_ctx c = {out, x, n, w, rank, a, b, xa, 0};
    parallel_for(w->rows, threads, matmul_worker, &c);
    free(xa);
    return c.err ? -1 : 0;
}

/* axpy: tensor.zig:563-572, `y + alpha * x` without fusion. */
static inline void axpy(float *y, float alpha, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = y[i] + alpha * x[i];
}

typedef struct {
    float *accs;
    const float *y;
    size_t q, per;
    const ditch_weight *w;
    int err;
} mvt_ctx;

static void matvecT_worker(void *p, size_t start, size_t end, size_t slot) {
    mvt_ctx *c = (mvt_ctx *)p;
    size_t cols = c->w->cols, rows = c->w->rows;
    float *acc = c->accs + slot * c->q * cols;
    float *buf = (float *)malloc(cols * sizeof(float));
    memset(acc, 0, c->q * cols * sizeof(float));
    for (size_t r = start; r < end; r++) {
        int any = 0;
        for (size_t j = 0; j < c->q; j++) any = any || c->y[j * rows + r] != 0;
        if (!any) continue;
        if (ref_weight_row(c->w, r, buf)) c->err = 1;
        for (size_t j = 0; j < c->q; j++) {
            float yr = c->y[j * rows + r];
            if (yr != 0) axpy(acc + j * cols, yr, buf, cols);
        }
    }
    free(buf);
}

/* tensor.zig:1056-1094: per-slot partial sums merged in slot order. */
int ref_matvecTMulti(float *out, const ditch_weight *w, const float *y, size_t q, int threads) {
    size_t rows = w->rows, cols = w->cols;
    size_t chunks = (size_t)(threads < 1 ? 1 : threads);
    if (chunks > rows) chunks = rows;
    if (chunks == 0) chunks = 1;
    size_t per = (rows + chunks - 1) / chunks;
    size_t slots = rows ? (rows + per - 1) / per : 1;
    float *accs = (float *)calloc(slots * q * cols, sizeof(float));
    mvt_ctx c = {accs, y, q, per, w, 0};
    parallel_for(rows, (int)chunks, matvecT_worker, &c);
    memset(out, 0, q * cols * sizeof(float));
    for (size_t s = 0; s < slots; s++) axpy(out, 1.0f, accs + s * q * cols, q * cols);
    free(accs);
    return c.err ? -1 : 0;
}

typedef struct { float *out; const ditch_weight *w; int err; } rn_ctx;
static void rownorm_worker(void *p, size_t start, size_t end, size_t slot) {
    (void)slot;
    rn_ctx *c = (rn_ctx *)p;
    float *buf = (float *)malloc(c->w->cols * sizeof(float));
    for (size_t r = start; r < end; r++) {
        if (ref_weight_row(c->w, r, buf)) c->err = 1;
        c->out[r] = sqrtf(ref_dot(buf, buf, c->w->cols));
    }
    free(buf);
}

int ref_rowNorms(float *out, const ditch_weight *w, int threads) {
    rn_ctx c = {out, w, 0};
    parallel_for(w->rows, threads, rownorm_worker, &c);
    return c.err ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* Element-wise kernels                                                     */

/* tensor.zig:1126-1144 (vector path, hd % VL == 0): per key a lane-wise FMA
 * over VL blocks, reduced, times scale. */
void ref_attention_scores(float *scores, size_t n_keys, const float *q, size_t hd,
                          const float *k, size_t stride, float scale) {
    for (size_t p = 0; p < n_keys; p++) {
        float acc[VL] = {0};
        for (size_t d = 0; d < hd; d += VL)
            for (int l = 0; l < VL; l++) acc[l] = fmaf(k[p * stride + d + l], q[d + l], acc[l]);
        scores[p] = reduce_lanes(acc) * scale;
    }
}

/* tensor.zig:1148-1160 (vector path, vd % VL == 0): four accumulators over
 * keys in groups of four, the tail into the first, combined pairwise. */
void ref_attention_values(float *out, size_t vd, const float *scores, size_t n_keys,
                          const float *v, size_t stride) {
    for (size_t j = 0; j < vd; j += VL) {
        float a[4][VL];
        memset(a, 0, sizeof a);
        size_t p = 0;
        for (; p + 4 <= n_keys; p += 4)
            for (int kk = 0; kk < 4; kk++)
                for (int l = 0; l < VL; l++) a[kk][l] = fmaf(v[(p + kk) * stride + j + l], scores[p + kk], a[kk][l]);
        for (; p < n_keys; p++)
            for (int l = 0; l < VL; l++) a[0][l] = fmaf(v[p * stride + j + l], scores[p], a[0][l]);
        for (int l = 0; l < VL; l++) out[j + l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    }
}

/* tensor.zig:1167-1179 */
void ref_rmsnorm(float *out, const float *x, const float *w, size_t wlen, size_t len, float eps, int gemma_style) {
    float ss = 0;
    for (size_t i = 0; i < len; i++) ss = ss + x[i] * x[i];
    float inv = 1.0f / sqrtf(ss / (float)len + eps);
    if (wlen == 0) {
        for (size_t i = 0; i < len; i++) out[i] = x[i] * inv;
    } else if (gemma_style) {
        for (size_t i = 0; i < len; i++) out[i] = x[i] * inv * (1.0f + w[i]);
    } else {
        for (size_t i = 0; i < len; i++) out[i] = x[i] * inv * w[i];
    }
}

/* tensor.zig:1343-1358 */
void ref_layernorm(float *out, const float *x, const float *w, size_t wlen, const float *bias, size_t len, float eps, int one_plus) {
    float n = (float)len, mean = 0, var = 0;
    for (size_t i = 0; i < len; i++) mean = mean + x[i];
    mean = mean / n;
    for (size_t i = 0; i < len; i++) var = var + (x[i] - mean) * (x[i] - mean);
    var = var / n;
    float inv = 1.0f / sqrtf(var + eps);
    for (size_t i = 0; i < len; i++) {
        float y = (x[i] - mean) * inv;
        if (wlen > 0) y = y * (one_plus ? 1.0f + w[i] : w[i]);
        if (bias) y = y + bias[i];
        out[i] = y;
    }
}

/* expVec (tensor.zig:1277-1294), one lane: Cephes expf. */
float ref_exp_cephes(float x_in) {
    float x = fminf(fmaxf(x_in, -87.3f), 88.0f);
    float fx = roundf(x * 1.44269504088896341f);
    float r = fmaf(fx, 2.12194440e-4f, fmaf(fx, -0.693359375f, x));
    float y = 1.9875691500e-4f;
    y = fmaf(y, r, 1.3981999507e-3f);
    y = fmaf(y, r, 8.3334519073e-3f);
    y = fmaf(y, r, 4.1665795894e-2f);
    y = fmaf(y, r, 1.6666665459e-1f);
    y = fmaf(y, r, 5.0000001201e-1f);
    y = fmaf(y, r * r, r + 1.0f);
    int e = (int)fx;
    return y * u2f((uint32_t)(e + 127) << 23);
}

/* tensor.zig:1181-1200: vector max, Cephes exp on whole VL blocks, libm exp
 * on the tail, multiply by 1/sum. */
void ref_softmax_inplace(float *x, size_t len) {
    float mv[VL];
    for (int l = 0; l < VL; l++) mv[l] = -INFINITY;
    size_t i = 0;
    for (; i + VL <= len; i += VL)
        for (int l = 0; l < VL; l++) mv[l] = fmaxf(mv[l], x[i + l]);
    float m = mv[0];
    for (int l = 1; l < VL; l++) m = fmaxf(m, mv[l]);
    for (; i < len; i++) m = fmaxf(m, x[i]);
    float sv[VL] = {0};
    i = 0;
    for (; i + VL <= len; i += VL)
        for (int l = 0; l < VL; l++) {
            float e = ref_exp_cephes(x[i + l] - m);
            x[i + l] = e;
            sv[l] = sv[l] + e;
        }
    float s = reduce_lanes(sv);
    for (; i < len; i++) {
        x[i] = expf(x[i] - m);
        s = s + x[i];
    }
    float inv = 1.0f / s;
    for (size_t t = 0; t < len; t++) x[t] = x[t] * inv;
}

/* tensor.zig:1203-1210 */
void ref_log_softmax(float *out, const float *x, size_t len) {
    float m = -INFINITY;
    for (size_t i = 0; i < len; i++) m = fmaxf(m, x[i]);
    double s = 0;
    for (size_t i = 0; i < len; i++) s += exp((double)(x[i] - m));
    float lse = m + (float)log(s);
    for (size_t i = 0; i < len; i++) out[i] = x[i] - lse;
}

static float erf_as(float x) {
    /* tensor.zig:1220-1225 (Abramowitz-Stegun 7.1.26) */
    float t = 1.0f / (1.0f + 0.3275911f * fabsf(x));
    float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t * expf(-x * x);
    return x >= 0 ? y : -y;
}

/* Activation.apply (tensor.zig:1239-1254) */
float ref_act_scalar(uint32_t act, float x) {
    switch (act) {
    case 0: return x / (1.0f + expf(-x));
    case 1: return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    case 2: return 0.5f * x * (1.0f + erf_as(x / 1.41421356237309504880f));
    case 3: return fmaxf(x, 0.0f);
    case 4: { float r = fmaxf(x, 0.0f); return r * r; }
    case 5: return x / (1.0f + expf(-1.702f * x));
    default: return x;
    }
}

/* Activation.applyVec (tensor.zig:1257-1274), one lane. */
static float act_vec_lane(uint32_t act, float x) {
    switch (act) {
    case 0: return x / (1.0f + ref_exp_cephes(-x));
    case 1: {
        float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
        float t = 1.0f - 2.0f / (ref_exp_cephes(u + u) + 1.0f);
        return 0.5f * x * (1.0f + t);
    }
    case 3: return fmaxf(x, 0.0f);
    case 4: { float r = fmaxf(x, 0.0f); return r * r; }
    case 5: return x / (1.0f + ref_exp_cephes(-1.702f * x));
    default: return ref_act_scalar(act, x);
    }
}

/* tensor.zig:1308-1337: VL blocks aligned to each row start use the vector
 * form, a partial block the scalar one; gelu (2) is always scalar. */
void ref_gated_activation(uint32_t act, float *out, const float *gate, const float *up, size_t n, size_t len,
                          size_t in_stride, size_t out_stride) {
    for (size_t r = 0; r < n; r++) {
        for (size_t j = 0; j < len; j += VL) {
            const float *g = gate + r * in_stride + j;
            const float *u = up ? up + r * in_stride + j : NULL;
            float *o = out + r * out_stride + j;
            float tmp[VL];
            if (j + VL <= len && act != 2) {
                for (int l = 0; l < VL; l++) tmp[l] = act_vec_lane(act, g[l]);
                if (u) for (int l = 0; l < VL; l++) tmp[l] = tmp[l] * u[l];
                memcpy(o, tmp, sizeof tmp);
            } else {
                size_t m = len - j < VL ? len - j : VL;
                for (size_t l = 0; l < m; l++) {
                    float v = ref_act_scalar(act, g[l]);
                    if (u) v = v * u[l];
                    o[l] = v;
                }
            }
        }
    }
}

static void rope_neox(float *x, size_t dim, const float *c, const float *s) {
    size_t half = dim / 2;
    for (size_t i = 0; i < half; i++) {
        float x1 = x[i], x2 = x[i + half];
        x[i] = x1 * c[i] - x2 * s[i];
        x[i + half] = x2 * c[i] + x1 * s[i];
    }
}
static void rope_gptj(float *x, size_t dim, const float *c, const float *s) {
    size_t half = dim / 2;
    for (size_t i = 0; i < half; i++) {
        float x1 = x[2 * i], x2 = x[2 * i + 1];
        x[2 * i] = x1 * c[i] - x2 * s[i];
        x[2 * i + 1] = x2 * c[i] + x1 * s[i];
    }
}

void ref_rope_rows(float *x, size_t n, size_t dim, const float *cos_t, const float *sin_t, size_t half,
                   const uint32_t *pos, uint32_t style) {
    for (size_t i = 0; i < n; i++) {
        const float *c = cos_t + (size_t)pos[i] * half, *s = sin_t + (size_t)pos[i] * half;
        if (style == DITCH_ROPE_GPTJ) rope_gptj(x + i * dim, dim, c, s);
        else rope_neox(x + i * dim, dim, c, s);
    }
}

/* model.zig:2200-2282 fillRope for the scalings in scope. */
int ref_fill_rope(const ditch_model_config *c, float *cos_t, float *sin_t) {
    size_t len = c->rope_len, dim = c->rotary_dim, half = dim / 2;
    if (half == 0) return 0;
    double *inv = (double *)malloc(half * sizeof(double));
    double theta = (double)c->rope_theta;
    for (size_t i = 0; i < half; i++) {
        double exponent = (double)(2 * i) / (double)dim;
        inv[i] = 1.0 / pow(theta, exponent);
    }
    double attention_factor = 1.0;
    switch (c->rope_scaling) {
    case DITCH_ROPE_SCALING_LINEAR:
        for (size_t i = 0; i < half; i++) inv[i] /= (double)c->rope_factor;
        break;
    case DITCH_ROPE_SCALING_LLAMA3: {
        /* The scaling fields are f32 (arch.zig:136): the wavelength bounds
         * divide in f32, everything meeting an f64 frequency widens. */
        double factor = c->rope_factor, lff = c->rope_low_freq_factor;
        double orig = c->rope_original_max_position;
        double low_wavelen = (double)(c->rope_original_max_position / c->rope_low_freq_factor);
        double high_wavelen = (double)(c->rope_original_max_position / c->rope_high_freq_factor);
        double band = (double)(c->rope_high_freq_factor - c->rope_low_freq_factor);
        for (size_t i = 0; i < half; i++) {
            double f = inv[i];
            double wavelen = 2.0 * 3.14159265358979323846 / f;
            if (wavelen < high_wavelen) {
            } else if (wavelen > low_wavelen) {
                f /= factor;
            } else {
                double smooth = (orig / wavelen - lff) / band;
                f = (1.0 - smooth) * f / factor + smooth * f;
            }
            inv[i] = f;
        }
        break;
    }
    case DITCH_ROPE_SCALING_YARN: {
        double base = theta, dimf = (double)dim;
        double maxp = c->rope_original_max_position;
        double low = (dimf * log(maxp / ((double)c->yarn_beta_fast * 2.0 * 3.14159265358979323846))) / (2.0 * log(base));
        double high = (dimf * log(maxp / ((double)c->yarn_beta_slow * 2.0 * 3.14159265358979323846))) / (2.0 * log(base));
        if (c->yarn_truncate) { low = floor(low); high = ceil(high); }
        if (low < 0) low = 0;
        if (high > dimf - 1) high = dimf - 1;
        if (low == high) high += 0.001;
        for (size_t i = 0; i < half; i++) {
            double ramp = ((double)i - low) / (high - low);
            if (ramp < 0) ramp = 0;
            if (ramp > 1) ramp = 1;
            double extrapolation_factor = 1.0 - ramp;
            double interp = inv[i] / (double)c->rope_factor;
            inv[i] = interp * (1.0 - extrapolation_factor) + inv[i] * extrapolation_factor;
        }
        attention_factor = (double)c->yarn_attention_factor;
        break;
    }
    case DITCH_ROPE_SCALING_FACTORS:
        for (size_t i = 0; i < half; i++)
            if (c->rope_factors) inv[i] /= (double)c->rope_factors[i];
        break;
    default: break;
    }
    for (size_t pos = 0; pos < len; pos++)
        for (size_t i = 0; i < half; i++) {
            double angle = (double)pos * inv[i];
            cos_t[pos * half + i] = (float)(cos(angle) * attention_factor);
            sin_t[pos * half + i] = (float)(sin(angle) * attention_factor);
        }
    free(inv);
    return 0;
}

/* scorers.zig:387-394 */
double ref_kl_row(const float *base, const float *trial, size_t vocab) {
    float *tmp = (float *)malloc(vocab * sizeof(float));
    ref_log_softmax(tmp, trial, vocab);
    double kl = 0;
    for (size_t j = 0; j < vocab; j++) {
        double p = exp((double)base[j]);
        kl += p * ((double)base[j] - (double)tmp[j]);
    }
    free(tmp);
    return kl;
}

/* abliterate.zig:270-279 */
int ref_edit_delta(float *a, float *b, const ditch_weight *w, const float *v, size_t k, float weight, int threads) {
    if (ref_matvecTMulti(a, w, v, k, threads)) return -1;
    for (size_t i = 0; i < w->rows; i++)
        for (size_t j = 0; j < k; j++) b[i * k + j] = -weight * v[j * w->rows + i];
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Model                                                                    */

typedef struct {
    ditch_weight w;  /* points into own; FP8/MXFP4/INT decoded to BF16     */
    void *own;
    float *vec;      /* norm / bias vectors as f32                          */
    size_t len;
    size_t rank;
    float *da, *db;
} rtensor;

typedef struct {
    rtensor attn_norm, q, k, v, o, q_bias, k_bias, v_bias, q_norm, k_norm, ffn_norm, gate, up, down;
    rtensor router, corr, sh_gate, sh_up, sh_down, q_a, q_a_norm, q_b, kv_a, kv_a_norm, kv_b;
    rtensor *eg, *eu, *ed;
} rlayer;

struct ref_model {
    ditch_model_config c;
    uint8_t *moe_layers;
    rtensor embed, final_norm, lm_head;
    rlayer *layers;
    float *rope_cos, *rope_sin;
    int threads;
    size_t first_layer, n_layers_run;
    int keep_packed;  /* quantised weights referenced as given, decoded per row at use */
};

ref_model *ref_model_create(const ditch_model_config *cfg) {
    ref_model *m = (ref_model *)calloc(1, sizeof *m);
    m->c = *cfg;
    m->moe_layers = (uint8_t *)calloc(cfg->layers ? cfg->layers : 1, 1);
    if (cfg->moe_layers) memcpy(m->moe_layers, cfg->moe_layers, cfg->layers);
    m->c.moe_layers = m->moe_layers;
    m->layers = (rlayer *)calloc(cfg->layers, sizeof(rlayer));
    for (size_t l = 0; l < cfg->layers; l++) {
        if (cfg->n_experts && m->moe_layers[l]) {
            m->layers[l].eg = (rtensor *)calloc(cfg->n_experts, sizeof(rtensor));
            m->layers[l].eu = (rtensor *)calloc(cfg->n_experts, sizeof(rtensor));
            m->layers[l].ed = (rtensor *)calloc(cfg->n_experts, sizeof(rtensor));
        }
    }
    size_t half = cfg->rotary_dim / 2;
    m->rope_cos = (float *)calloc(cfg->rope_len * half + 1, sizeof(float));
    m->rope_sin = (float *)calloc(cfg->rope_len * half + 1, sizeof(float));
    ref_fill_rope(&m->c, m->rope_cos, m->rope_sin);
    m->c.rope_factors = NULL;
    m->threads = 8;
    return m;
}

static void rt_free(rtensor *t) {
    free(t->own); free(t->vec); free(t->da); free(t->db);
    memset(t, 0, sizeof *t);
}

void ref_model_free(ref_model *m) {
    if (!m) return;
    rt_free(&m->embed); rt_free(&m->final_norm); rt_free(&m->lm_head);
    for (size_t l = 0; l < m->c.layers; l++) {
        rlayer *L = &m->layers[l];
        rtensor *all[] = {&L->attn_norm, &L->q, &L->k, &L->v, &L->o, &L->q_bias, &L->k_bias, &L->v_bias, &L->q_norm,
                          &L->k_norm, &L->ffn_norm, &L->gate, &L->up, &L->down, &L->router, &L->corr, &L->sh_gate,
                          &L->sh_up, &L->sh_down, &L->q_a, &L->q_a_norm, &L->q_b, &L->kv_a, &L->kv_a_norm, &L->kv_b};
        for (size_t i = 0; i < sizeof all / sizeof all[0]; i++) rt_free(all[i]);
        if (L->eg) {
            for (size_t e = 0; e < m->c.n_experts; e++) { rt_free(&L->eg[e]); rt_free(&L->eu[e]); rt_free(&L->ed[e]); }
            free(L->eg); free(L->eu); free(L->ed);
        }
    }
    free(m->layers); free(m->rope_cos); free(m->rope_sin); free(m->moe_layers);
    free(m);
}

void ref_set_threads(ref_model *m, int threads) { m->threads = threads < 1 ? 1 : threads; }
/* Streamed mode (WeightStore + Dequant.readRange, dequant.zig:427-456): the
 * virtual-bf16 formats (FP8, MXFP4, INT pack-quantized) set after this call
 * keep pointing at the caller's packed pieces, which must outlive the
 * model, and each product decodes the rows it multiplies (ref_weight_row:
 * the same bf16 value as the mapped mode's one-time decode). */
void ref_model_keep_packed(ref_model *m, int on) { m->keep_packed = on; }
void ref_model_limit_layers(ref_model *m, size_t first, size_t count) { m->first_layer = first; m->n_layers_run = count; }

static int is_vector_slot(int slot) {
    switch (slot) {
    case DITCH_SLOT_FINAL_NORM: case DITCH_SLOT_ATTN_NORM: case DITCH_SLOT_Q_BIAS: case DITCH_SLOT_K_BIAS:
    case DITCH_SLOT_V_BIAS: case DITCH_SLOT_Q_NORM: case DITCH_SLOT_K_NORM: case DITCH_SLOT_FFN_NORM:
    case DITCH_SLOT_ROUTER_CORRECTION: case DITCH_SLOT_MLA_Q_A_NORM: case DITCH_SLOT_MLA_KV_A_NORM:
        return 1;
    default: return 0;
    }
}

static rtensor *slot_ptr(ref_model *m, int layer, int slot, int expert) {
    if (slot == DITCH_SLOT_EMBED) return &m->embed;
    if (slot == DITCH_SLOT_FINAL_NORM) return &m->final_norm;
    if (slot == DITCH_SLOT_LM_HEAD) return &m->lm_head;
    if (layer < 0 || (size_t)layer >= m->c.layers) return NULL;
    rlayer *L = &m->layers[layer];
    switch (slot) {
    case DITCH_SLOT_ATTN_NORM: return &L->attn_norm;
    case DITCH_SLOT_Q: return &L->q;
    case DITCH_SLOT_K: return &L->k;
    case DITCH_SLOT_V: return &L->v;
    case DITCH_SLOT_O: return &L->o;
    case DITCH_SLOT_Q_BIAS: return &L->q_bias;
    case DITCH_SLOT_K_BIAS: return &L->k_bias;
    case DITCH_SLOT_V_BIAS: return &L->v_bias;
    case DITCH_SLOT_Q_NORM: return &L->q_norm;
    case DITCH_SLOT_K_NORM: return &L->k_norm;
    case DITCH_SLOT_FFN_NORM: return &L->ffn_norm;
    case DITCH_SLOT_GATE: return &L->gate;
    case DITCH_SLOT_UP: return &L->up;
    case DITCH_SLOT_DOWN: return &L->down;
    case DITCH_SLOT_ROUTER: return &L->router;
    case DITCH_SLOT_ROUTER_CORRECTION: return &L->corr;
    case DITCH_SLOT_SHARED_GATE: return &L->sh_gate;
    case DITCH_SLOT_SHARED_UP: return &L->sh_up;
    case DITCH_SLOT_SHARED_DOWN: return &L->sh_down;
    case DITCH_SLOT_MLA_Q_A: return &L->q_a;
    case DITCH_SLOT_MLA_Q_A_NORM: return &L->q_a_norm;
    case DITCH_SLOT_MLA_Q_B: return &L->q_b;
    case DITCH_SLOT_MLA_KV_A: return &L->kv_a;
    case DITCH_SLOT_MLA_KV_A_NORM: return &L->kv_a_norm;
    case DITCH_SLOT_MLA_KV_B: return &L->kv_b;
    case DITCH_SLOT_EXPERT_GATE: case DITCH_SLOT_EXPERT_UP: case DITCH_SLOT_EXPERT_DOWN:
        if (!L->eg || expert < 0 || (size_t)expert >= m->c.n_experts) return NULL;
        return slot == DITCH_SLOT_EXPERT_GATE ? &L->eg[expert] : slot == DITCH_SLOT_EXPERT_UP ? &L->eu[expert] : &L->ed[expert];
    default: return NULL;
    }
}

/* Rows of a virtual bf16 tensor decoded on the model's threads (each row on
 * its own: the decode has no cross-row state). */
typedef struct { const ditch_weight *w; uint16_t *out; int rc; } dq_ctx;
static void dq_range(void *c, size_t a, size_t b, size_t slot) {
    dq_ctx *x = (dq_ctx *)c;
    for (size_t r = a; r < b; r++)
        if (decode_bf16_row(x->w, r, x->out + r * x->w->cols)) x->rc = -1;
}

int ref_model_set(ref_model *m, int layer, int slot, int expert, const ditch_weight *w) {
    rtensor *t = slot_ptr(m, layer, slot, expert);
    if (!t) return fail("model_set: bad slot %d layer %d expert %d", slot, layer, expert);
    rt_free(t);
    if (is_vector_slot(slot)) {
        size_t len = w->rows * w->cols;
        t->vec = (float *)malloc(len * sizeof(float));
        t->len = len;
        ditch_weight flat = *w;
        flat.rows = 1;
        flat.cols = len;
        return ref_weight_row(&flat, 0, t->vec);
    }
    t->w = *w;
    if (is_bf16_virtual(w->dtype) && m->keep_packed) return 0;  /* borrowed, decoded per row */
    if (is_bf16_virtual(w->dtype)) {
        /* mapped mode: the virtual bf16 tensor decoded once (dequant.zig:841-845) */
        uint16_t *buf = (uint16_t *)malloc(w->rows * w->cols * 2);
        dq_ctx c = {w, buf, 0};
        parallel_for(w->rows, m->threads, dq_range, &c);
        if (c.rc) { free(buf); return -1; }
        memset(&t->w, 0, sizeof t->w);
        t->w.data = buf;
        t->w.dtype = DITCH_BF16;
        t->w.rows = w->rows;
        t->w.cols = w->cols;
        t->own = buf;
        return 0;
    }
    size_t bytes;
    if (w->dtype == DITCH_F32) bytes = w->rows * w->cols * 4;
    else if (w->dtype == DITCH_F16 || w->dtype == DITCH_BF16) bytes = w->rows * w->cols * 2;
    else bytes = w->rows * ref_row_bytes(w->dtype, w->cols);
    if (!bytes) return fail("model_set: dtype %d cols %zu", w->dtype, (size_t)w->cols);
    t->own = malloc(bytes);
    memcpy(t->own, w->data, bytes);
    t->w.data = t->own;
    return 0;
}

int ref_model_set_delta(ref_model *m, int layer, int slot, int expert, size_t rank, const float *a, const float *b) {
    rtensor *t = slot_ptr(m, layer, slot, expert);
    if (!t || !t->w.data) return fail("set_delta: bad slot");
    free(t->da); free(t->db);
    t->da = t->db = NULL;
    t->rank = rank;
    if (!rank) return 0;
    t->da = (float *)malloc(rank * t->w.cols * sizeof(float));
    t->db = (float *)malloc(t->w.rows * rank * sizeof(float));
    memcpy(t->da, a, rank * t->w.cols * sizeof(float));
    memcpy(t->db, b, t->w.rows * rank * sizeof(float));
    return 0;
}

int ref_model_edit(ref_model *m, int layer, int slot, int expert, const float *v, size_t k, float weight) {
    rtensor *t = slot_ptr(m, layer, slot, expert);
    if (!t || !t->w.data) return fail("edit: bad slot");
    float *a = (float *)malloc(k * t->w.cols * sizeof(float));
    float *b = (float *)malloc(t->w.rows * k * sizeof(float));
    int rc = ref_edit_delta(a, b, &t->w, v, k, weight, m->threads);
    if (!rc) rc = ref_model_set_delta(m, layer, slot, expert, k, a, b);
    free(a); free(b);
    return rc;
}

static int mm(ref_model *m, float *out, const float *x, size_t n, const rtensor *t) {
    if (!t->w.data) return fail("missing weight");
    return ref_matmulT(out, x, n, &t->w, t->rank, t->da, t->db, m->threads);
}

static void add_bias(float *buf, size_t n, size_t width, const float *bias) {
    for (size_t i = 0; i < n; i++) axpy(buf + i * width, 1.0f, bias, width);
}

/* runExpert (moe.zig:910-950) for a gated SiLU expert without biases. */
static int run_expert(ref_model *m, const rtensor *g, const rtensor *u, const rtensor *d, const float *x, size_t ne,
                      float *gate, float *up, float *out) {
    size_t inter = g->w.rows;
    if (mm(m, gate, x, ne, g) || mm(m, up, x, ne, u)) return -1;
    ref_gated_activation(0, gate, gate, up, ne, inter, inter, inter);
    return mm(m, out, gate, ne, d);
}

static inline float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

/* moe.forward (moe.zig:998-1228) for softmax / sigmoid routers, optional
 * correction bias and group-limited top-k, renormalisation, scaling, and
 * shared experts. */
static int moe_forward(ref_model *m, rlayer *L, float *out, const float *h, size_t n) {
    const ditch_model_config *c = &m->c;
    size_t hidden = c->hidden, ne_all = c->n_experts, k = c->top_k, inter = c->moe_inter;
    float *logits = (float *)malloc(n * ne_all * sizeof(float));
    if (mm(m, logits, h, n, &L->router)) { free(logits); return -1; }
    size_t *sel = (size_t *)malloc(n * k * sizeof(size_t));
    float *selw = (float *)malloc(n * k * sizeof(float));
    float *choice = (float *)malloc(ne_all * sizeof(float));
    size_t n_group = c->group_limited ? c->n_group : 1;
    float *gs = (float *)malloc((n_group ? n_group : 1) * sizeof(float));
    for (size_t t = 0; t < n; t++) {
        float *row = logits + t * ne_all;
        if (c->scoring == DITCH_SCORING_SOFTMAX) ref_softmax_inplace(row, ne_all);
        else for (size_t e = 0; e < ne_all; e++) row[e] = sigmoidf_(row[e]);
        for (size_t e = 0; e < ne_all; e++) choice[e] = row[e] + (L->corr.vec ? L->corr.vec[e] : 0.0f);
        if (c->group_limited && n_group > 1) {
            size_t per_group = ne_all / n_group;
            for (size_t g = 0; g < n_group; g++) {
                const float *s = choice + g * per_group;
                if (L->corr.vec) {
                    float b1 = -INFINITY, b2 = -INFINITY;
                    for (size_t i = 0; i < per_group; i++) {
                        if (s[i] > b1) { b2 = b1; b1 = s[i]; }
                        else if (s[i] > b2) b2 = s[i];
                    }
                    gs[g] = b1 + (per_group > 1 ? b2 : 0.0f);
                } else {
                    float best = -INFINITY;
                    for (size_t i = 0; i < per_group; i++) best = fmaxf(best, s[i]);
                    gs[g] = best;
                }
            }
            size_t keep = c->topk_group < n_group ? c->topk_group : n_group;
            for (size_t kept = 0; kept < keep; kept++) {
                size_t best = 0;
                float bv = -INFINITY;
                for (size_t g = 0; g < n_group; g++)
                    if (gs[g] > bv) { bv = gs[g]; best = g; }
                gs[best] = NAN;
            }
            for (size_t g = 0; g < n_group; g++)
                if (!isnan(gs[g]))
                    for (size_t i = 0; i < per_group; i++) choice[g * per_group + i] = -INFINITY;
        }
        /* topk (moe.zig:971-985): repeated argmax, strict '>' */
        for (size_t j = 0; j < k; j++) {
            size_t best = 0;
            float bv = -INFINITY;
            for (size_t e = 0; e < ne_all; e++)
                if (choice[e] > bv) { bv = choice[e]; best = e; }
            sel[t * k + j] = best;
            selw[t * k + j] = row[best];
            choice[best] = -INFINITY;
        }
        float sum = 0;
        for (size_t j = 0; j < k; j++) sum = sum + selw[t * k + j];
        if (c->norm_topk_prob && sum > 0)
            for (size_t j = 0; j < k; j++) selw[t * k + j] = selw[t * k + j] / sum;
        if (c->routed_scaling != 1.0f)
            for (size_t j = 0; j < k; j++) selw[t * k + j] = selw[t * k + j] * c->routed_scaling;
    }
    memset(out, 0, n * hidden * sizeof(float));
    /* an expert takes up to n * k pairs: a token selects expert 0 more than
     * once when fewer than k choices are above -inf (topk's argmax returns
     * index 0 then, moe.zig:971-985) */
    size_t np_ = n * k;
    size_t wi = inter > c->shared_inter ? inter : c->shared_inter;
    float *xg = (float *)malloc(np_ * hidden * sizeof(float));
    float *gate = (float *)malloc((np_ > n ? np_ : n) * wi * sizeof(float));
    float *up = (float *)malloc((np_ > n ? np_ : n) * wi * sizeof(float));
    float *eo = (float *)malloc((np_ > n ? np_ : n) * hidden * sizeof(float));
    size_t *tok = (size_t *)malloc(np_ * sizeof(size_t));
    float *wts = (float *)malloc(np_ * sizeof(float));
    uint8_t *used = (uint8_t *)calloc(ne_all, 1);
    for (size_t i = 0; i < n * k; i++) used[sel[i]] = 1;
    int rc = 0;
    for (size_t e = 0; e < ne_all && !rc; e++) {
        if (!used[e]) continue;
        size_t ne = 0;
        for (size_t t = 0; t < n; t++)
            for (size_t j = 0; j < k; j++)
                if (sel[t * k + j] == e) { tok[ne] = t; wts[ne] = selw[t * k + j]; ne++; }
        for (size_t j = 0; j < ne; j++) memcpy(xg + j * hidden, h + tok[j] * hidden, hidden * sizeof(float));
        rc = run_expert(m, &L->eg[e], &L->eu[e], &L->ed[e], xg, ne, gate, up, eo);
        for (size_t j = 0; j < ne && !rc; j++) axpy(out + tok[j] * hidden, wts[j], eo + j * hidden, hidden);
    }
    if (!rc && L->sh_gate.w.data) {
        rc = run_expert(m, &L->sh_gate, &L->sh_up, &L->sh_down, h, n, gate, up, eo);
        for (size_t t = 0; t < n && !rc; t++) axpy(out + t * hidden, 1.0f, eo + t * hidden, hidden);
    }
    free(logits); free(sel); free(selw); free(choice); free(gs); free(xg); free(gate); free(up); free(eo);
    free(tok); free(wts); free(used);
    return rc;
}

/* mlaProject (model.zig:3292-3342): fills q [n][heads][hd], k (rope part
 * shared), v [n][heads][hd] with v_head_dim valid. */
static int mla_project(ref_model *m, rlayer *L, float *q, float *k, float *v, const float *h, size_t n) {
    const ditch_model_config *c = &m->c;
    size_t nh = c->heads, hd = c->head_dim, nope = c->qk_nope_dim, rd = c->qk_rope_dim, vd = c->v_head_dim;
    float eps = c->mla_norm_eps;
    if (L->q_a.w.data) {
        size_t qlr = c->q_lora_rank;
        float *qa = (float *)malloc(n * qlr * sizeof(float));
        float *tmp = (float *)malloc(qlr * sizeof(float));
        if (mm(m, qa, h, n, &L->q_a)) return -1;
        for (size_t t = 0; t < n; t++) {
            ref_rmsnorm(tmp, qa + t * qlr, L->q_a_norm.vec, L->q_a_norm.len, qlr, eps, 0);
            memcpy(qa + t * qlr, tmp, qlr * sizeof(float));
        }
        int rc = mm(m, q, qa, n, &L->q_b);
        free(qa); free(tmp);
        if (rc) return rc;
    } else if (mm(m, q, h, n, &L->q_b)) return -1;
    size_t kvr = c->kv_lora_rank + rd;
    float *kva = (float *)malloc(n * kvr * sizeof(float));
    float *ckv = (float *)malloc(n * c->kv_lora_rank * sizeof(float));
    size_t kvb_rows = nh * (nope + vd);
    float *kvb = (float *)malloc(n * kvb_rows * sizeof(float));
    int rc = mm(m, kva, h, n, &L->kv_a);
    for (size_t t = 0; t < n && !rc; t++)
        ref_rmsnorm(ckv + t * c->kv_lora_rank, kva + t * kvr, L->kv_a_norm.vec, L->kv_a_norm.len, c->kv_lora_rank, eps, 0);
    if (!rc) rc = mm(m, kvb, ckv, n, &L->kv_b);
    for (size_t t = 0; t < n && !rc; t++) {
        const float *k_pe = kva + t * kvr + c->kv_lora_rank;
        for (size_t hh = 0; hh < nh; hh++) {
            const float *src = kvb + t * kvb_rows + hh * (nope + vd);
            float *kk = k + t * nh * hd + hh * hd;
            float *vv = v + t * nh * hd + hh * hd;
            memcpy(kk, src, nope * sizeof(float));
            memcpy(kk + nope, k_pe, rd * sizeof(float));
            memset(vv, 0, hd * sizeof(float));
            memcpy(vv, src + nope, vd * sizeof(float));
        }
    }
    free(kva); free(ckv); free(kvb);
    return rc;
}

typedef struct {
    ref_model *m;
    const ditch_row *rows;
    const float *q;
    float *out;
    const float *kc, *vc; /* cache [B][T][kvd] */
    size_t T, kvd, hd, vd, heads, groups, n;
    float scale;
} attn_ctx;

/* attentionWorker (model.zig:2935-2986) for one (row, head) task each. */
static void attn_worker(void *p, size_t start, size_t end, size_t slot) {
    (void)slot;
    attn_ctx *a = (attn_ctx *)p;
    size_t hd = a->hd, vd = a->vd;
    int vectorised = hd % VL == 0 && vd % VL == 0;
    float *scores = (float *)malloc((a->T + 1) * sizeof(float));
    for (size_t task = start; task < end; task++) {
        size_t r = task / a->heads, h = task % a->heads;
        ditch_row row = a->rows[r];
        size_t kvh = h / a->groups;
        const float *q = a->q + r * a->heads * hd + h * hd;
        float *out = a->out + r * a->heads * hd + h * hd;
        size_t n_keys = (size_t)row.pos + 1;
        const float *kb = a->kc + ((size_t)row.b * a->T) * a->kvd + kvh * hd;
        const float *vb = a->vc + ((size_t)row.b * a->T) * a->kvd + kvh * hd;
        if (vectorised) ref_attention_scores(scores, n_keys, q, hd, kb, a->kvd, a->scale);
        else for (size_t pp = 0; pp < n_keys; pp++) scores[pp] = ref_dot(q, kb + pp * a->kvd, hd) * a->scale;
        ref_softmax_inplace(scores, n_keys);
        if (vectorised) ref_attention_values(out, vd, scores, n_keys, vb, a->kvd);
        else {
            memset(out, 0, vd * sizeof(float));
            for (size_t pp = 0; pp < n_keys; pp++) axpy(out, scores[pp], vb + pp * a->kvd, vd);
        }
    }
    free(scores);
}

/* attention + attentionTail (model.zig:4147-4374) for the families in
 * scope; writes the o-projection into `o`. */
static int attention(ref_model *m, rlayer *L, const float *h, const ditch_row *rows, size_t n, float *o,
                     float *kc, float *vc, size_t T) {
    const ditch_model_config *c = &m->c;
    size_t nh = c->heads, nkv = c->mla ? c->heads : c->kv_heads, hd = c->head_dim;
    size_t vd = c->mla ? c->v_head_dim : hd;
    size_t qd = nh * hd, kvd = nkv * hd;
    float *q = (float *)calloc(n * qd, sizeof(float));
    float *k = (float *)calloc(n * kvd, sizeof(float));
    float *v = (float *)calloc(n * kvd, sizeof(float));
    float *att = (float *)calloc(n * qd, sizeof(float));
    int rc = 0;
    if (c->mla) {
        rc = mla_project(m, L, q, k, v, h, n);
    } else {
        rc = mm(m, q, h, n, &L->q);
        if (!rc && L->q_bias.vec) add_bias(q, n, qd, L->q_bias.vec);
        if (!rc) rc = mm(m, k, h, n, &L->k);
        if (!rc) rc = mm(m, v, h, n, &L->v);
        if (!rc && L->k_bias.vec) add_bias(k, n, kvd, L->k_bias.vec);
        if (!rc && L->v_bias.vec) add_bias(v, n, kvd, L->v_bias.vec);
    }
    if (rc) goto done;
    size_t rope_off = c->mla ? c->qk_nope_dim : 0;
    size_t half = c->rotary_dim / 2, d = 2 * half;
    for (size_t i = 0; i < n; i++) {
        size_t pos = rows[i].pos;
        size_t p = pos < c->rope_len - 1 ? pos : c->rope_len - 1;
        const float *cr = m->rope_cos + p * half, *sr = m->rope_sin + p * half;
        for (size_t hh = 0; hh < nh; hh++) {
            float *qh = q + i * qd + hh * hd;
            if (c->qk_norm && L->q_norm.vec) ref_rmsnorm(qh, qh, L->q_norm.vec, hd, hd, c->rms_eps, 0);
            if (d) {
                if (c->rope_style == DITCH_ROPE_GPTJ) rope_gptj(qh + rope_off, d, cr, sr);
                else rope_neox(qh + rope_off, d, cr, sr);
            }
        }
        for (size_t hh = 0; hh < nkv; hh++) {
            float *kh = k + i * kvd + hh * hd;
            if (c->qk_norm && L->k_norm.vec) ref_rmsnorm(kh, kh, L->k_norm.vec, hd, hd, c->rms_eps, 0);
            if (d) {
                if (c->rope_style == DITCH_ROPE_GPTJ) rope_gptj(kh + rope_off, d, cr, sr);
                else rope_neox(kh + rope_off, d, cr, sr);
            }
        }
        memcpy(kc + ((size_t)rows[i].b * T + pos) * kvd, k + i * kvd, kvd * sizeof(float));
        memcpy(vc + ((size_t)rows[i].b * T + pos) * kvd, v + i * kvd, kvd * sizeof(float));
    }
    attn_ctx ac = {m, rows, q, att, kc, vc, T, kvd, hd, vd, nh, nh / nkv, n, c->attn_scale};
    parallel_for(n * nh, m->threads, attn_worker, &ac);
    if (vd != hd) {
        size_t dst = 0;
        for (size_t hi = 0; hi < n * nh; hi++) {
            memmove(att + dst, att + hi * hd, vd * sizeof(float));
            dst += vd;
        }
    }
    rc = mm(m, o, att, n, &L->o);
done:
    free(q); free(k); free(v); free(att);
    return rc;
}

int ref_forward(ref_model *m, const uint32_t *tokens, const ditch_row *rows, size_t n, const uint64_t *capture_rows,
                size_t n_capture, float *residuals, const uint64_t *logit_rows, size_t n_logit, float *logits) {
    const ditch_model_config *c = &m->c;
    size_t hidden = c->hidden;
    if (!m->embed.w.data) return fail("forward: no embedding");
    size_t B = 0, T = 0;
    for (size_t i = 0; i < n; i++) {
        if (rows[i].b + 1 > B) B = rows[i].b + 1;
        if (rows[i].pos + 1 > T) T = rows[i].pos + 1;
    }
    size_t nkv = c->mla ? c->heads : c->kv_heads;
    size_t kvd = nkv * c->head_dim;
    float *x = (float *)malloc(n * hidden * sizeof(float));
    float *h = (float *)malloc(n * hidden * sizeof(float));
    float *o = (float *)malloc(n * hidden * sizeof(float));
    float *kc = (float *)calloc(B * T * kvd + 1, sizeof(float));
    float *vc = (float *)calloc(B * T * kvd + 1, sizeof(float));
    int rc = 0;
    for (size_t i = 0; i < n && !rc; i++) {
        if (tokens[i] >= m->embed.w.rows) { rc = fail("token %u outside the embedding table", tokens[i]); break; }
        rc = ref_weight_row(&m->embed.w, tokens[i], x + i * hidden);
    }
#define CAPTURE(entry)                                                                                     \
    if (residuals)                                                                                         \
        for (size_t ci = 0; ci < n_capture; ci++)                                                          \
            memcpy(residuals + ((size_t)(entry) * n_capture + ci) * hidden, x + capture_rows[ci] * hidden, \
                   hidden * sizeof(float));
    if (!rc) { CAPTURE(0) }
    size_t l0 = m->first_layer, l1 = m->n_layers_run ? m->first_layer + m->n_layers_run : c->layers;
    if (l1 > c->layers) l1 = c->layers;
    for (size_t li = l0; li < l1 && !rc; li++) {
        rlayer *L = &m->layers[li];
        for (size_t i = 0; i < n; i++)
            ref_rmsnorm(h + i * hidden, x + i * hidden, L->attn_norm.vec, L->attn_norm.len, hidden, c->rms_eps, 0);
        rc = attention(m, L, h, rows, n, o, kc, vc, T);
        if (rc) break;
        axpy(x, 1.0f, o, n * hidden);
        for (size_t i = 0; i < n; i++)
            ref_rmsnorm(h + i * hidden, x + i * hidden, L->ffn_norm.vec, L->ffn_norm.len, hidden, c->rms_eps, 0);
        if (c->n_experts && m->moe_layers[li]) {
            rc = moe_forward(m, L, o, h, n);
        } else {
            size_t inter = L->gate.w.rows;
            float *g = (float *)malloc(n * inter * sizeof(float));
            float *u = (float *)malloc(n * inter * sizeof(float));
            rc = mm(m, g, h, n, &L->gate);
            if (!rc) rc = mm(m, u, h, n, &L->up);
            if (!rc) {
                ref_gated_activation(0, g, g, u, n, inter, inter, inter);
                rc = mm(m, o, g, n, &L->down);
            }
            free(g); free(u);
        }
        if (rc) break;
        axpy(x, 1.0f, o, n * hidden);
        CAPTURE(li + 1)
    }
#undef CAPTURE
    if (!rc && n_logit) {
        float *hl = (float *)malloc(n_logit * hidden * sizeof(float));
        for (size_t i = 0; i < n_logit; i++)
            ref_rmsnorm(hl + i * hidden, x + logit_rows[i] * hidden, m->final_norm.vec, m->final_norm.len, hidden,
                        c->rms_eps, 0);
        const rtensor *lm = m->lm_head.w.data ? &m->lm_head : &m->embed;
        rc = mm(m, logits, hl, n_logit, lm);
        free(hl);
    }
    free(x); free(h); free(o); free(kc); free(vc);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* Direction pipeline (test oracle): the per-batch residual reduction of
 * Engine.forEachResidual, the difference-of-means directions, Moments and the
 * Nystrom sketch of multi-direction bases.                                 */

static int cmp_f32(const void *a, const void *b) {
    float x = *(const float *)a, y = *(const float *)b;
    return (x > y) - (x < y);
}

/* quantile, engine.zig:492-499 (torch.quantile's linear interpolation, f32) */
static float quantile_sorted(const float *s, size_t n, float q) {
    if (n == 0) return 0;
    float pos = q * (float)(n - 1);
    size_t lo = (size_t)floorf(pos);
    size_t hi = lo + 1 < n - 1 ? lo + 1 : n - 1;
    float frac = pos - floorf(pos);
    return s[lo] + frac * (s[hi] - s[lo]);
}

/* engine.zig:414-431 for one batch: per prompt b and entry l the mean of the
 * prompt's `take[b]` captured rows (from capture index first[b]) by axpy with
 * inv = 1/take, winsorised at quantile q of |v| (q outside [0,1): none),
 * written to vout[b][l] and added to the f64 sums (Acc.add, engine.zig:
 * 320-326) and, when sq is given, Moments.add (directions.zig:196-205).     */
int ref_residual_reduce(const float *res, size_t entries, size_t n_capture, size_t hidden, const uint32_t *first,
                        const uint32_t *take, size_t prompts, float q, float *vout, double *sum, double *sq) {
    float *sorted = (q >= 0 && q < 1) ? (float *)malloc(hidden * sizeof(float)) : NULL;
    for (size_t b = 0; b < prompts; b++) {
        size_t t_n = take[b];
        float inv = 1.0f / (float)(t_n > 1 ? t_n : 1);
        for (size_t l = 0; l < entries; l++) {
            float *v = vout + (b * entries + l) * hidden;
            memset(v, 0, hidden * sizeof(float));
            for (size_t t = 0; t < t_n; t++)
                axpy(v, inv, res + (l * n_capture + first[b] + t) * hidden, hidden);
            if (sorted) {
                for (size_t i = 0; i < hidden; i++) sorted[i] = fabsf(v[i]);
                qsort(sorted, hidden, sizeof(float), cmp_f32);
                float thr = quantile_sorted(sorted, hidden, q);
                for (size_t i = 0; i < hidden; i++) v[i] = fmaxf(-thr, fminf(v[i], thr));
            }
            if (sum)
                for (size_t i = 0; i < hidden; i++) sum[l * hidden + i] += v[i];
            if (sq)
                for (size_t i = 0; i < hidden; i++) sq[l * hidden + i] += (double)v[i] * (double)v[i];
        }
    }
    free(sorted);
    return 0;
}

/* tensor.normalize (tensor.zig:580-584) */
static void normalize_f32(float *x, size_t n) {
    float nrm = sqrtf(ref_dot(x, x, n));
    if (nrm > 1e-12f) {
        float s = 1.0f / nrm;
        for (size_t i = 0; i < n; i++) x[i] *= s;
    }
}

/* abliterate.computeDirections (abliterate.zig:88-109) */
void ref_directions(float *dirs, const float *good, const float *bad, size_t entries, size_t hidden,
                    int orthogonalize) {
    float *gd = (float *)malloc(hidden * sizeof(float));
    for (size_t e = 0; e < entries; e++) {
        float *d = dirs + e * hidden;
        const float *g = good + e * hidden, *b = bad + e * hidden;
        for (size_t i = 0; i < hidden; i++) d[i] = b[i] - g[i];
        normalize_f32(d, hidden);
        if (orthogonalize) {
            memcpy(gd, g, hidden * sizeof(float));
            normalize_f32(gd, hidden);
            float p = ref_dot(d, gd, hidden);
            axpy(d, -p, gd, hidden);
            normalize_f32(d, hidden);
        }
    }
    free(gd);
}

/* abliterate.orthonormalize (abliterate.zig:409-423): modified Gram-Schmidt,
 * two passes, rows normalised (or zeroed below 1e-20). */
void ref_orthonormalize(float *vecs, size_t q, size_t n) {
    for (size_t i = 0; i < q; i++) {
        float *vi = vecs + i * n;
        for (int pass = 0; pass < 2; pass++)
            for (size_t j = 0; j < i; j++) {
                const float *vj = vecs + j * n;
                float p = ref_dot(vi, vj, n);
                axpy(vi, -p, vj, n);
            }
        float nrm = sqrtf(ref_dot(vi, vi, n));
        if (nrm > 1e-20f) {
            float s = 1.0f / nrm;
            for (size_t k = 0; k < n; k++) vi[k] *= s;
        } else {
            memset(vi, 0, n * sizeof(float));
        }
    }
}

/* directions.Sketch.add (directions.zig:80-104) for prompts x entries
 * residuals v[b][e][hidden] in prompt order: z = r - center, p = Omega^T z,
 * Y[e] += z p^T ([m][hidden]), W[e] += p p^T ([m][m]), all f64.           */
void ref_sketch_add(double *y, double *w, const float *omega, size_t m, const float *center, const float *v,
                    size_t prompts, size_t entries, size_t hidden) {
    double *z = (double *)malloc(hidden * sizeof(double));
    double *p = (double *)malloc(m * sizeof(double));
    for (size_t b = 0; b < prompts; b++)
        for (size_t e = 0; e < entries; e++) {
            const float *r = v + (b * entries + e) * hidden;
            const float *c = center + e * hidden;
            for (size_t i = 0; i < hidden; i++) z[i] = (double)r[i] - (double)c[i];
            for (size_t j = 0; j < m; j++) {
                double acc = 0;
                for (size_t i = 0; i < hidden; i++) acc += z[i] * (double)omega[j * hidden + i];
                p[j] = acc;
            }
            double *ye = y + e * m * hidden, *we = w + e * m * m;
            for (size_t j = 0; j < m; j++)
                for (size_t i = 0; i < hidden; i++) ye[j * hidden + i] += z[i] * p[j];
            for (size_t j = 0; j < m; j++)
                for (size_t l = 0; l < m; l++) we[j * m + l] += p[j] * p[l];
        }
    free(z);
    free(p);
}

static double sign_f64(double x) { return x > 0 ? 1.0 : x < 0 ? -1.0 : 0.0; }

/* directions.symmetricEigen (directions.zig:463-500): cyclic Jacobi in f64,
 * m overwritten by its diagonalisation, eigenvectors in the columns of vecs. */
void ref_symmetric_eigen(double *m, double *vecs, size_t n) {
    memset(vecs, 0, n * n * sizeof(double));
    for (size_t i = 0; i < n; i++) vecs[i * n + i] = 1;
    for (int sweep = 0; sweep < 60; sweep++) {
        double off = 0, diag = 0;
        for (size_t i = 0; i < n; i++)
            for (size_t j = 0; j < n; j++) {
                if (i != j) off += m[i * n + j] * m[i * n + j];
                else diag += m[i * n + j] * m[i * n + j];
            }
        if (off <= 1e-24 * (diag > 1e-300 ? diag : 1e-300)) break;
        for (size_t p = 0; p < n; p++)
            for (size_t q = p + 1; q < n; q++) {
                double apq = m[p * n + q];
                if (fabs(apq) < 1e-300) continue;
                double theta = (m[q * n + q] - m[p * n + p]) / (2.0 * apq);
                double t = theta == 0 ? 1.0 : sign_f64(theta) / (fabs(theta) + sqrt(theta * theta + 1.0));
                double cs = 1.0 / sqrt(t * t + 1.0), sn = t * cs;
                for (size_t k = 0; k < n; k++) {
                    double akp = m[k * n + p], akq = m[k * n + q];
                    m[k * n + p] = cs * akp - sn * akq;
                    m[k * n + q] = sn * akp + cs * akq;
                }
                for (size_t k = 0; k < n; k++) {
                    double apk = m[p * n + k], aqk = m[q * n + k];
                    m[p * n + k] = cs * apk - sn * aqk;
                    m[q * n + k] = sn * apk + cs * aqk;
                }
                for (size_t k = 0; k < n; k++) {
                    double vkp = vecs[k * n + p], vkq = vecs[k * n + q];
                    vecs[k * n + p] = cs * vkp - sn * vkq;
                    vecs[k * n + q] = sn * vkp + cs * vkq;
                }
            }
    }
}

static void remove_f64(double *col, const float *unit, size_t n) {
    double p = 0;
    for (size_t i = 0; i < n; i++) p += col[i] * unit[i];
    for (size_t i = 0; i < n; i++) col[i] -= p * unit[i];
}

/* Sketch.factor (directions.zig:108-134) then directions.computeBasisFrom
 * (directions.zig:371-455): dirs [entries][k][hidden] from the first
 * directions, the good means and the sketch (y [entries][m][hidden], w
 * [entries][m][m]).                                                        */
int ref_basis(float *dirs, const float *first, const float *good_means, size_t entries, size_t hidden, size_t k,
              int orthogonalize, const double *y, const double *w, size_t m) {
    memset(dirs, 0, entries * k * hidden * sizeof(float));
    if (k == 1) {
        memcpy(dirs, first, entries * hidden * sizeof(float));
        return 0;
    }
    double *wm = (double *)malloc(m * m * sizeof(double)), *vecs = (double *)malloc(m * m * sizeof(double));
    double *bf = (double *)malloc(m * hidden * sizeof(double));
    double *gram = (double *)malloc(m * m * sizeof(double)), *gv = (double *)malloc(m * m * sizeof(double));
    float *gd = (float *)malloc(hidden * sizeof(float));
    size_t *order = (size_t *)malloc(m * sizeof(size_t));
    for (size_t e = 0; e < entries; e++) {
        float *basis = dirs + e * k * hidden;
        memcpy(basis, first + e * hidden, hidden * sizeof(float));
        memcpy(gd, good_means + e * hidden, hidden * sizeof(float));
        normalize_f32(gd, hidden);
        /* factor */
        memcpy(wm, w + e * m * m, m * m * sizeof(double));
        ref_symmetric_eigen(wm, vecs, m);
        double max_ev = 0;
        for (size_t j = 0; j < m; j++) max_ev = wm[j * m + j] > max_ev ? wm[j * m + j] : max_ev;
        const double *ye = y + e * m * hidden;
        size_t r = 0;
        for (size_t j = 0; j < m; j++) {
            double ev = wm[j * m + j];
            if (ev <= max_ev * 1e-9 || ev <= 0) continue;
            double s = 1.0 / sqrt(ev);
            double *col = bf + r * hidden;
            memset(col, 0, hidden * sizeof(double));
            for (size_t l = 0; l < m; l++) {
                double coef = vecs[l * m + j] * s;
                if (coef == 0) continue;
                for (size_t i = 0; i < hidden; i++) col[i] += coef * ye[l * hidden + i];
            }
            r++;
        }
        for (size_t c = 0; c < r; c++) {
            remove_f64(bf + c * hidden, basis, hidden);
            if (orthogonalize) remove_f64(bf + c * hidden, gd, hidden);
        }
        for (size_t i = 0; i < r; i++)
            for (size_t j = 0; j < r; j++) {
                double acc = 0;
                for (size_t t = 0; t < hidden; t++) acc += bf[i * hidden + t] * bf[j * hidden + t];
                gram[i * r + j] = acc;
            }
        ref_symmetric_eigen(gram, gv, r);
        /* order by descending eigenvalue, ties in index order (a stable sort) */
        for (size_t i = 0; i < r; i++) order[i] = i;
        for (size_t i = 1; i < r; i++) {
            size_t o = order[i], j = i;
            while (j > 0 && gram[order[j - 1] * r + order[j - 1]] < gram[o * r + o]) {
                order[j] = order[j - 1];
                j--;
            }
            order[j] = o;
        }
        for (size_t d = 1; d < k; d++) {
            float *dir = basis + d * hidden;
            memset(dir, 0, hidden * sizeof(float));
            if (d - 1 >= r) continue;
            size_t src = order[d - 1];
            double lambda = gram[src * r + src];
            if (lambda <= 0) continue;
            for (size_t c = 0; c < r; c++) {
                float coef = (float)(gv[c * r + src] / sqrt(lambda));
                const double *col = bf + c * hidden;
                for (size_t i = 0; i < hidden; i++) dir[i] = dir[i] + coef * (float)col[i];
            }
        }
        ref_orthonormalize(basis, k, hidden);
        if (e > 0) {
            const float *prev = dirs + (e - 1) * k * hidden;
            for (size_t d = 1; d < k; d++) {
                float *dir = basis + d * hidden;
                if (ref_dot(dir, prev + d * hidden, hidden) < 0)
                    for (size_t i = 0; i < hidden; i++) dir[i] *= -1.0f;
            }
        }
    }
    free(wm); free(vecs); free(bf); free(gram); free(gv); free(gd); free(order);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* The edit in every row-normalisation mode (test oracle):
 * abliterate.computeDelta / computeOutputDelta / ablateInputs /
 * DeltaOperator / randomizedSvd / jacobiEigen (abliterate.zig:223-538).    */

/* Zig's std.Random as the reference uses it (test oracle; Zig 0.16 std,
 * the reference's minimum_zig_version, build.zig.zon): DefaultPrng is
 * Xoshiro256++ whose state is four SplitMix64 outputs of the seed
 * (lib/std/Random/Xoshiro256.zig, SplitMix64.zig); Random.float(f64) takes
 * the exponent from a draw's leading zeros (lib/std/Random.zig); floatNorm
 * is the 256-layer ziggurat of lib/std/Random/ziggurat.zig with
 * r = 3.6541528853610088, v = 0.00492867323399. The reference draws from
 * it in randomizedSvd (abliterate.zig:473-479), Sketch.init
 * (directions.zig:65-67) and Sampler.pick (model.zig:5256).               */
static uint64_t zig_splitmix(uint64_t *x) {
    uint64_t z = (*x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void ref_zig_init(uint64_t st[4], uint64_t seed) {
    uint64_t x = seed;
    st[0] = zig_splitmix(&x);
    st[1] = zig_splitmix(&x);
    st[2] = zig_splitmix(&x);
    st[3] = zig_splitmix(&x);
}

static uint64_t zig_rotl(uint64_t x, unsigned k) { return (x << k) | (x >> (64 - k)); }

uint64_t ref_zig_next(uint64_t st[4]) {
    uint64_t out = zig_rotl(st[0] + st[3], 23) + st[0];
    uint64_t t = st[1] << 17;
    st[2] ^= st[0];
    st[3] ^= st[1];
    st[1] ^= st[2];
    st[0] ^= st[3];
    st[2] ^= t;
    st[3] = zig_rotl(st[3], 45);
    return out;
}

static unsigned zig_clz64(uint64_t x) { return x ? (unsigned)__builtin_clzll(x) : 64u; }

double ref_zig_float64(uint64_t st[4]) {
    uint64_t r = ref_zig_next(st);
    uint64_t lz = zig_clz64(r);
    if (lz >= 12) { /* the top 12 bits are zero: more draws extend the run */
        lz = 12;
        for (;;) {
            uint64_t more = zig_clz64(ref_zig_next(st));
            lz += more;
            if (more != 64) break;
            if (lz >= 1022) { lz = 1022; break; }
        }
    }
    uint64_t bits = ((1022 - lz) << 52) | (r & ((1ull << 52) - 1));
    double d;
    memcpy(&d, &bits, sizeof d);
    return d;
}

static double zig_norm_f(double x) { return exp(-x * x / 2.0); }

static double zig_tx[257], zig_tf[257];
static int zig_tables_ready;

void ref_zig_norm_tables(double *x, double *f) {
    if (!zig_tables_ready) {
        const double r = 3.6541528853610088, v = 0.00492867323399;
        zig_tx[0] = v / zig_norm_f(r);
        zig_tx[1] = r;
        for (int i = 2; i < 256; i++) {
            double prev = zig_tx[i - 1];
            zig_tx[i] = sqrt(-2.0 * log(v / prev + zig_norm_f(prev)));
        }
        zig_tx[256] = 0;
        for (int i = 0; i < 257; i++) zig_tf[i] = zig_norm_f(zig_tx[i]);
        zig_tables_ready = 1;
    }
    if (x) memcpy(x, zig_tx, sizeof zig_tx);
    if (f) memcpy(f, zig_tf, sizeof zig_tf);
}

double ref_zig_norm(uint64_t st[4]) {
    const double r = 3.6541528853610088;
    ref_zig_norm_tables(NULL, NULL);
    for (;;) {
        uint64_t bits = ref_zig_next(st);
        unsigned i = (unsigned)(bits & 255u);
        uint64_t repr = (0x400ull << 52) | (bits >> 12); /* [2, 4) */
        double u;
        memcpy(&u, &repr, sizeof u);
        u -= 3.0; /* [-1, 1) */
        double x = u * zig_tx[i];
        if (fabs(x) < zig_tx[i + 1]) return x;
        if (i == 0) { /* the tail beyond r */
            double tx = 1, ty = 0;
            while (-2.0 * ty < tx * tx) {
                tx = log(ref_zig_float64(st)) / r;
                ty = log(ref_zig_float64(st));
            }
            return u < 0 ? tx - r : r - tx;
        }
        if (zig_tf[i + 1] + (zig_tf[i] - zig_tf[i + 1]) * ref_zig_float64(st) < zig_norm_f(x)) return x;
    }
}

/* n draws of one kind (0 int(u64), 1 float(f64), 2 floatNorm(f64)) from
 * DefaultPrng.init(seed) */
void ref_zig_draws(void *out, size_t n, uint64_t seed, int kind) {
    uint64_t st[4];
    ref_zig_init(st, seed);
    for (size_t i = 0; i < n; i++) {
        if (kind == 0) ((uint64_t *)out)[i] = ref_zig_next(st);
        else if (kind == 1) ((double *)out)[i] = ref_zig_float64(st);
        else ((double *)out)[i] = ref_zig_norm(st);
    }
}

/* The full mode's test matrix: Random.floatNorm(f32) draws of
 * DefaultPrng.init(seed) in omega's order (abliterate.zig:474-479). */
void ref_edit_gaussian(float *out, size_t n, uint64_t seed) {
    uint64_t st[4];
    ref_zig_init(st, seed);
    for (size_t t = 0; t < n; t++) out[t] = (float)ref_zig_norm(st);
}

/* Sampler.pick (model.zig:5222-5263) for n rows in order, st the Sampler's
 * DefaultPrng state (Sampler.init, model.zig:5216-5218), advanced. */
void ref_sampler_pick(uint32_t *out, const float *logits, size_t n, size_t vocab, uint64_t st[4],
                      float temperature, size_t top_k, float top_p) {
    size_t kk = top_k < 1 ? 1 : top_k > 256 ? 256 : top_k;
    for (size_t row = 0; row < n; row++) {
        const float *x = logits + row * vocab;
        if (temperature <= 0) { /* argmax: the first maximum */
            size_t best = 0;
            for (size_t i = 1; i < vocab; i++)
                if (x[i] > x[best]) best = i;
            out[row] = (uint32_t)best;
            continue;
        }
        uint32_t ids[256];
        float vals[256];
        double probs[256];
        size_t k = kk < vocab ? kk : vocab, m = 0;
        for (size_t i = 0; i < vocab; i++) {
            if (m < k) {
                ids[m] = (uint32_t)i;
                vals[m] = x[i];
                m++;
            } else if (x[i] > vals[m - 1]) {
                ids[m - 1] = (uint32_t)i;
                vals[m - 1] = x[i];
            } else {
                continue;
            }
            for (size_t j = m - 1; j > 0 && vals[j] > vals[j - 1]; j--) {
                float tv = vals[j]; vals[j] = vals[j - 1]; vals[j - 1] = tv;
                uint32_t ti = ids[j]; ids[j] = ids[j - 1]; ids[j - 1] = ti;
            }
        }
        double total = 0;
        for (size_t i = 0; i < m; i++) {
            probs[i] = exp((double)(vals[i] - vals[0]) / (double)temperature);
            total += probs[i];
        }
        size_t kept = 0;
        double mass = 0;
        while (kept < m) {
            mass += probs[kept];
            kept++;
            if (mass >= (double)top_p * total) break;
        }
        double r = ref_zig_float64(st) * mass;
        uint32_t id = ids[kept - 1];
        for (size_t i = 0; i < kept; i++) {
            r -= probs[i];
            if (r <= 0) { id = ids[i]; break; }
        }
        out[row] = id;
    }
}

/* jacobiEigen (abliterate.zig:427-469): f32 cyclic Jacobi, f64 off-norm */
void ref_jacobi_f32(float *m, float *vecs, size_t n) {
    memset(vecs, 0, n * n * sizeof(float));
    for (size_t i = 0; i < n; i++) vecs[i * n + i] = 1;
    for (int sweep = 0; sweep < 50; sweep++) {
        double off = 0;
        for (size_t i = 0; i < n; i++)
            for (size_t j = 0; j < n; j++)
                if (i != j) off += (double)m[i * n + j] * m[i * n + j];
        if (off < 1e-18) break;
        for (size_t p = 0; p < n; p++)
            for (size_t q = p + 1; q < n; q++) {
                float apq = m[p * n + q];
                if (fabsf(apq) < 1e-20f) continue;
                float app = m[p * n + p], aqq = m[q * n + q];
                float theta = (aqq - app) / (2.0f * apq);
                float sg = theta > 0 ? 1.0f : theta < 0 ? -1.0f : 0.0f;
                float t = sg / (fabsf(theta) + sqrtf(theta * theta + 1.0f));
                float tf = theta == 0 ? 1.0f : t;
                float cs = 1.0f / sqrtf(tf * tf + 1.0f), sn = tf * cs;
                for (size_t k = 0; k < n; k++) {
                    float akp = m[k * n + p], akq = m[k * n + q];
                    m[k * n + p] = cs * akp - sn * akq;
                    m[k * n + q] = sn * akp + cs * akq;
                }
                for (size_t k = 0; k < n; k++) {
                    float apk = m[p * n + k], aqk = m[q * n + k];
                    m[p * n + k] = cs * apk - sn * aqk;
                    m[q * n + k] = sn * apk + cs * aqk;
                }
                for (size_t k = 0; k < n; k++) {
                    float vkp = vecs[k * n + p], vkq = vecs[k * n + q];
                    vecs[k * n + p] = cs * vkp - sn * vkq;
                    vecs[k * n + q] = sn * vkp + cs * vkq;
                }
            }
    }
}

typedef struct {
    const ditch_weight *w;
    const float *a, *c, *d;
    size_t k;
    int threads;
} dop;

/* DeltaOperator.applyMulti: out[q][rows] = (D X)^T (abliterate.zig:363-376) */
static int dop_apply(const dop *o, float *out, const float *x, size_t q) {
    size_t rows = o->w->rows, cols = o->w->cols;
    if (ref_matmulT(out, x, q, o->w, 0, NULL, NULL, o->threads)) return -1;
    for (size_t j = 0; j < q; j++) {
        float *oj = out + j * rows;
        for (size_t i = 0; i < rows; i++) oj[i] *= o->c[i];
        for (size_t l = 0; l < o->k; l++) {
            float ax = ref_dot(o->a + l * cols, x + j * cols, cols);
            axpy(oj, ax, o->d + l * rows, rows);
        }
    }
    return 0;
}

/* DeltaOperator.applyTMulti: out[q][cols] = (D^T Y)^T (abliterate.zig:379-393) */
static int dop_applyT(const dop *o, float *out, const float *y, size_t q) {
    size_t rows = o->w->rows, cols = o->w->cols;
    float *cy = (float *)calloc(q * rows, sizeof(float));
    for (size_t j = 0; j < q; j++)
        for (size_t i = 0; i < rows; i++) cy[j * rows + i] = o->c[i] * y[j * rows + i];
    int rc = ref_matvecTMulti(out, o->w, cy, q, o->threads);
    free(cy);
    if (rc) return -1;
    for (size_t j = 0; j < q; j++)
        for (size_t l = 0; l < o->k; l++) {
            float dy = ref_dot(o->d + l * rows, y + j * rows, rows);
            axpy(out + j * cols, dy, o->a + l * cols, cols);
        }
    return 0;
}

/* computeOutputDelta (abliterate.zig:264-350) then ablateInputs (234-261):
 * a [rank][cols], b [rows][rank]; *rank_out set. mode 0 none, 1 pre, 2 full. */
int ref_edit_delta_ex(float *a_out, float *b_out, size_t *rank_out, const ditch_weight *w, const float *v, size_t k,
                      float weight, int mode, size_t lora_rank, uint64_t seed, int ablate, int threads) {
    size_t rows = w->rows, cols = w->cols, r_out = k;
    size_t cap = lora_rank > k ? lora_rank : k; /* the output-side rank's bound */
    float *pa = (float *)malloc(cap * cols * sizeof(float)), *pb = (float *)malloc(rows * cap * sizeof(float));
    int rc = 0;
    if (mode == 0) {
        rc = ref_matvecTMulti(pa, w, v, k, threads);
        for (size_t i = 0; i < rows; i++)
            for (size_t j = 0; j < k; j++) pb[i * k + j] = -weight * v[j * rows + i];
    } else {
        float *norms = (float *)malloc(rows * sizeof(float)), *vn = (float *)malloc(k * rows * sizeof(float));
        rc |= ref_rowNorms(norms, w, threads);
        for (size_t j = 0; j < k; j++)
            for (size_t i = 0; i < rows; i++) vn[j * rows + i] = norms[i] > 0 ? v[j * rows + i] / norms[i] : 0;
        float *a = (float *)malloc(k * cols * sizeof(float));
        rc |= ref_matvecTMulti(a, w, vn, k, threads);
        if (mode == 1) {
            memcpy(pa, a, k * cols * sizeof(float));
            for (size_t i = 0; i < rows; i++)
                for (size_t j = 0; j < k; j++) pb[i * k + j] = -weight * v[j * rows + i] * norms[i];
        } else {
            float *wa = (float *)malloc(k * rows * sizeof(float)), *gram = (float *)malloc(k * k * sizeof(float));
            float *c = (float *)malloc(rows * sizeof(float)), *d = (float *)malloc(k * rows * sizeof(float));
            rc |= ref_matmulT(wa, a, k, w, 0, NULL, NULL, threads);
            for (size_t j = 0; j < k; j++)
                for (size_t l = 0; l < k; l++) gram[j * k + l] = ref_dot(a + j * cols, a + l * cols, cols);
            for (size_t i = 0; i < rows; i++) {
                float s2 = 1.0f;
                for (size_t j = 0; j < k; j++) {
                    float bij = -weight * v[j * rows + i];
                    float wnda = norms[i] > 0 ? wa[j * rows + i] / norms[i] : 0;
                    s2 += 2.0f * bij * wnda;
                    for (size_t l = 0; l < k; l++) s2 += bij * (-weight * v[l * rows + i]) * gram[j * k + l];
                }
                float s = sqrtf(s2 > 1e-12f ? s2 : 1e-12f);
                c[i] = 1.0f / s - 1.0f;
                for (size_t j = 0; j < k; j++) d[j * rows + i] = norms[i] * (-weight * v[j * rows + i]) / s;
            }
            size_t r = lora_rank > k ? lora_rank : k;
            size_t q = 2 * r + 4;
            if (q > rows) q = rows;
            if (q > cols) q = cols;
            dop o = {w, a, c, d, k, threads};
            float *omega = (float *)malloc(q * cols * sizeof(float)), *qy = (float *)malloc(q * rows * sizeof(float));
            float *qx = (float *)malloc(q * cols * sizeof(float));
            ref_edit_gaussian(omega, q * cols, seed);
            rc |= dop_apply(&o, qy, omega, q);
            ref_orthonormalize(qy, q, rows);
            for (int it = 0; it < 6; it++) {
                rc |= dop_applyT(&o, qx, qy, q);
                ref_orthonormalize(qx, q, cols);
                rc |= dop_apply(&o, qy, qx, q);
                ref_orthonormalize(qy, q, rows);
            }
            rc |= dop_applyT(&o, qx, qy, q); /* bt */
            float *bbt = (float *)malloc(q * q * sizeof(float)), *ev = (float *)malloc(q * q * sizeof(float));
            for (size_t i = 0; i < q; i++)
                for (size_t j = 0; j < q; j++) bbt[i * q + j] = ref_dot(qx + i * cols, qx + j * cols, cols);
            ref_jacobi_f32(bbt, ev, q);
            size_t *order = (size_t *)malloc(q * sizeof(size_t));
            for (size_t i = 0; i < q; i++) order[i] = i;
            for (size_t i = 1; i < q; i++) {
                size_t ov = order[i], j = i;
                while (j > 0 && bbt[order[j - 1] * q + order[j - 1]] < bbt[ov * q + ov]) {
                    order[j] = order[j - 1];
                    j--;
                }
                order[j] = ov;
            }
            r_out = r < q ? r : q;
            float *uk = (float *)malloc(rows * sizeof(float)), *vk = (float *)malloc(cols * sizeof(float));
            for (size_t t = 0; t < r_out; t++) {
                size_t src = order[t];
                float lambda = bbt[src * q + src] > 0 ? bbt[src * q + src] : 0;
                float sv = sqrtf(lambda);
                memset(uk, 0, rows * sizeof(float));
                memset(vk, 0, cols * sizeof(float));
                for (size_t i = 0; i < q; i++) axpy(uk, ev[i * q + src], qy + i * rows, rows);
                for (size_t i = 0; i < q; i++) axpy(vk, ev[i * q + src], qx + i * cols, cols);
                if (sv > 1e-12f) {
                    float inv = 1.0f / sv;
                    for (size_t j = 0; j < cols; j++) vk[j] *= inv;
                } else {
                    memset(vk, 0, cols * sizeof(float));
                }
                float sq = sqrtf(sv > 0 ? sv : 0);
                for (size_t j = 0; j < cols; j++) pa[t * cols + j] = sq * vk[j];
                for (size_t i = 0; i < rows; i++) pb[i * r_out + t] = uk[i] * sq;
            }
            free(uk); free(vk); free(bbt); free(ev); free(omega); free(qy); free(qx); free(order);
            free(wa); free(gram); free(c); free(d);
        }
        free(norms); free(vn); free(a);
    }
    size_t rank = r_out + (ablate ? k : 0);
    if (!ablate) {
        memcpy(a_out, pa, r_out * cols * sizeof(float));
        memcpy(b_out, pb, rows * r_out * sizeof(float));
    } else {
        float *u = (float *)malloc(k * cols * sizeof(float)), *wu = (float *)malloc(k * rows * sizeof(float));
        rc |= ref_matvecTMulti(u, w, v, k, threads);
        ref_orthonormalize(u, k, cols);
        rc |= ref_matmulT(wu, u, k, w, r_out, pa, pb, threads);
        memcpy(a_out, pa, r_out * cols * sizeof(float));
        memcpy(a_out + r_out * cols, u, k * cols * sizeof(float));
        for (size_t i = 0; i < rows; i++) {
            memcpy(b_out + i * rank, pb + i * r_out, r_out * sizeof(float));
            for (size_t j = 0; j < k; j++) b_out[i * rank + r_out + j] = -weight * wu[j * rows + i];
        }
        free(u); free(wu);
    }
    free(pa); free(pb);
    *rank_out = rank;
    return rc ? -1 : 0;
}
