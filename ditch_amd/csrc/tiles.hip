// tiles.hip — weight upload: raw checkpoint layouts -> HBM tiles, and the
// element decoders over both layouts.
//
// Raw layouts are the ones the reference reads (tensor.Weight rows, GGUF
// blocks quant.zig:27-42, the quantised-safetensors groups of dequant.zig:
// 477-673). Fused formats (TF_Q8/FP8/MX4/INT4/BF16/F16/F32) keep their codes
// and are re-tiled for the matmul kernels; the others are decoded once at
// upload to the reference's virtual dtype (bf16, or f32 for GGUF blocks).
#include <string.h>
#include "decode.h"
#include "internal.h"
#include "tiled.h"

namespace ditch {

bool is_bf16_virtual(int32_t dt) {
    return dt == DITCH_FP8 || dt == DITCH_MXFP4 || dt == DITCH_MXFP4_T || dt == DITCH_INT_PACKED;
}

__host__ __device__ static int gguf_block_size(int dt) {
    switch (dt) {
    case DITCH_Q8_0: case DITCH_Q4_0: case DITCH_Q4_1: case DITCH_Q5_0: case DITCH_Q5_1: return 32;
    case DITCH_Q4_K: case DITCH_Q6_K: case DITCH_Q8_K: return 256;
    default: return 0;
    }
}
__host__ __device__ static int gguf_block_bytes(int dt) {
    switch (dt) {
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

// ---------------------------------------------------------------------------
// Raw-layout element decode. One thread per output element.

struct RawView {
    const uint8_t *data;
    const uint8_t *scale;
    const uint8_t *zero;
    const int32_t *g_idx;
    int32_t dtype, scale_type;
    int64_t rows, cols;
    int64_t scale_cols, block_rows, block_cols, row_shard;
    int32_t e5m2, bits;
    int64_t group, groups;
};

__device__ __forceinline__ float rd_f16(const uint8_t *b) { return f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }
__device__ __forceinline__ uint32_t rd_u32(const uint8_t *b) {
    return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
}

// Element e of a GGUF block `b` (quant.zig:81-199), as f32.
__device__ float gguf_element(int dt, const uint8_t *b, int e) {
    switch (dt) {
    case DITCH_Q8_0: return __fmul_rn((float)(int8_t)b[2 + e], rd_f16(b));
    case DITCH_Q4_0: {
        int j = e & 15;
        int x = (e < 16 ? (b[2 + j] & 0x0f) : (b[2 + j] >> 4)) - 8;
        return __fmul_rn((float)x, rd_f16(b));
    }
    case DITCH_Q4_1: {
        int j = e & 15;
        int x = e < 16 ? (b[4 + j] & 0x0f) : (b[4 + j] >> 4);
        return __fadd_rn(__fmul_rn((float)x, rd_f16(b)), rd_f16(b + 2));
    }
    case DITCH_Q5_0: {
        uint32_t qh = rd_u32(b + 2);
        int j = e & 15;
        int x;
        if (e < 16) x = (int)((b[6 + j] & 0x0f) | (((qh >> j) << 4) & 0x10u)) - 16;
        else x = (int)((b[6 + j] >> 4) | ((qh >> (j + 12)) & 0x10u)) - 16;
        return __fmul_rn((float)x, rd_f16(b));
    }
    case DITCH_Q5_1: {
        uint32_t qh = rd_u32(b + 4);
        int j = e & 15;
        uint32_t x;
        if (e < 16) x = (b[8 + j] & 0x0f) | (((qh >> j) << 4) & 0x10u);
        else x = (b[8 + j] >> 4) | ((qh >> (j + 12)) & 0x10u);
        return __fadd_rn(__fmul_rn((float)x, rd_f16(b)), rd_f16(b + 2));
    }
    case DITCH_Q4_K: {
        float d = rd_f16(b), mn = rd_f16(b + 2);
        const uint8_t *sc = b + 4;
        int chunk = e / 64, within = e % 64;
        int is = 2 * chunk + (within >= 32 ? 1 : 0);
        uint32_t s, m;
        if (is < 4) { s = sc[is] & 63; m = sc[is + 4] & 63; }
        else { s = (sc[is + 4] & 0xf) | ((sc[is - 4] >> 6) << 4); m = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4); }
        uint8_t qb = b[16 + 32 * chunk + (within & 31)];
        uint32_t q = within < 32 ? (qb & 0xf) : (qb >> 4);
        float dd = __fmul_rn(d, (float)s), mm = __fmul_rn(mn, (float)m);
        return __fsub_rn(__fmul_rn(dd, (float)q), mm);
    }
    case DITCH_Q6_K: {
        int n128 = e / 128, rem = e % 128, l = rem % 32, quarter = rem / 32;
        const uint8_t *ql = b + 64 * n128, *qh = b + 128 + 32 * n128, *sc = b + 192 + 8 * n128;
        float d = rd_f16(b + 208);
        uint8_t lb = ql[l + 32 * (quarter & 1)];
        uint32_t nib = quarter >= 2 ? (lb >> 4) : (lb & 0xf);
        int q = (int)(nib | (((qh[l] >> (2 * quarter)) & 3u) << 4)) - 32;
        float s = (float)(int8_t)sc[l / 16 + 2 * quarter];
        return __fmul_rn(__fmul_rn(d, s), (float)q);
    }
    case DITCH_Q8_K: return __fmul_rn(u2f(rd_u32(b)), (float)(int8_t)b[4 + e]);
    default: return 0.0f;
    }
}

__device__ __forceinline__ uint32_t field_mask(int bits) { return bits >= 32 ? 0xffffffffu : ((1u << bits) - 1u); }

__device__ __forceinline__ uint32_t unpack_field(const uint32_t *words, int64_t i, int bits) {
    int64_t start = i * bits;
    int64_t w = start / 32;
    int off = (int)(start % 32);
    int lo = (32 - off) < bits ? (32 - off) : bits;
    uint32_t v = (words[w] >> off) & field_mask(lo);
    if (lo < bits) v |= (words[w + 1] & field_mask(bits - lo)) << lo;
    return v;
}


// Raw element (r, c): bf16 bits for the virtual-bf16 formats, f32 otherwise.
__device__ float raw_element_f32(const RawView &v, int64_t r, int64_t c) {
    switch (v.dtype) {
    case DITCH_F32: return ((const float *)v.data)[r * v.cols + c];
    case DITCH_F16: return f16_to_f32(((const uint16_t *)v.data)[r * v.cols + c]);
    case DITCH_BF16: return bf16_to_f32(((const uint16_t *)v.data)[r * v.cols + c]);
    default: {
        int bs = gguf_block_size(v.dtype), bb = gguf_block_bytes(v.dtype);
        const uint8_t *row = v.data + r * (v.cols / bs) * bb;
        return gguf_element(v.dtype, row + (c / bs) * bb, (int)(c % bs));
    }
    }
}

__device__ uint16_t raw_element_bf16(const RawView &v, int64_t r, int64_t c) {
    switch (v.dtype) {
    case DITCH_FP8: {
        uint32_t code = v.data[r * v.cols + c];
        int64_t sr = fp8_scale_row(r, v.block_rows, v.row_shard);
        float s = load_scale(v.scale, sr * v.scale_cols + c / v.block_cols, v.scale_type);
        return f32_to_bf16(mul_x86(fp8_value(code, v.e5m2), s));
    }
    case DITCH_MXFP4: {
        uint8_t byte = v.data[r * (v.cols / 2) + c / 2];
        uint32_t nib = (c & 1) ? (byte >> 4) : (byte & 0x0f);
        float sc = e8m0_scale(v.scale[r * (v.cols / 32) + c / 32]);
        return f32_to_bf16(mul_x86(e2m1_value(nib), sc));
    }
    case DITCH_MXFP4_T: {
        // view (h = r, j = c) is source row j, element h (dequant.zig:603-637)
        int64_t nblk = v.rows / 32;
        int64_t h = r, j = c;
        uint8_t byte = v.data[(j * nblk + h / 32) * 16 + (h % 32) / 2];
        uint32_t nib = (h & 1) ? (byte >> 4) : (byte & 0x0f);
        float sc = e8m0_scale(v.scale[j * nblk + h / 32]);
        return f32_to_bf16(mul_x86(e2m1_value(nib), sc));
    }
    case DITCH_INT_PACKED: {
        int bits = v.bits;
        int64_t wpr = (v.cols * bits + 31) / 32;
        int offset = 1 << (bits - 1);
        int64_t g = v.g_idx ? (int64_t)v.g_idx[c] : c / v.group;
        int zp = 0;
        if (v.zero) {
            const uint32_t *zw = (const uint32_t *)v.zero;
            int64_t start = r * bits;
            int64_t wi = start / 32;
            int off = (int)(start % 32);
            int lo = (32 - off) < bits ? (32 - off) : bits;
            uint32_t z = (zw[wi * v.groups + g] >> off) & field_mask(lo);
            if (lo < bits) z |= (zw[(wi + 1) * v.groups + g] & field_mask(bits - lo)) << lo;
            zp = (int)z - offset;
        }
        int q = (int)unpack_field((const uint32_t *)v.data + r * wpr, c, bits) - offset;
        float s = load_scale(v.scale, r * v.groups + g, v.scale_type);
        return f32_to_bf16(mul_x86((float)(q - zp), s));
    }
    default: return f32_to_bf16(raw_element_f32(v, r, c));
    }
}

__global__ void raw_dequant_kernel(RawView v, void *out, int64_t row0, int64_t nrows, int bf16_out) {
    int64_t total = nrows * v.cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = row0 + i / v.cols, c = i % v.cols;
        if (bf16_out) ((uint16_t *)out)[i] = raw_element_bf16(v, r, c);
        else ((float *)out)[i] = raw_element_f32(v, r, c);
    }
}

__global__ void tiled_dequant_kernel(TileView v, void *out, int64_t row0, int64_t nrows, int bf16_out) {
    int64_t total = nrows * v.cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = row0 + i / v.cols, c = i % v.cols;
        uint16_t b = 0;
        float f = tiled_element_f32(v, r, c, &b);
        if (bf16_out) ((uint16_t *)out)[i] = b;
        else ((float *)out)[i] = f;
    }
}

// ---------------------------------------------------------------------------
// Re-tiling kernels: one thread per (unit, lane) writes the lane's word(s).

struct RetileArgs {
    RawView src;        // raw codes on device
    uint8_t *codes;     // tiled output
    int32_t tf;
    int64_t rows, cols, units_k, groups_n;
    // decoded source (bf16 or f32 row-major) for TF_BF16/TF_F32 built by decode
    const void *dense;
    int32_t dense_f32;
};

__device__ __forceinline__ uint32_t src_code(const RetileArgs &a, int64_t n, int64_t k) {
    // raw code of element (n, k) for the fused formats; 0 outside the matrix
    if (n >= a.rows || k >= a.cols) return 0u;
    const RawView &s = a.src;
    switch (a.tf) {
    case TF_Q8: {
        const uint8_t *row = s.data + n * (s.cols / 32) * 34;
        return row[(k / 32) * 34 + 2 + (k % 32)];
    }
    case TF_FP8: return s.data[n * s.cols + k];
    case TF_MX4: {
        uint8_t byte = s.data[n * (s.cols / 2) + k / 2];
        return (k & 1) ? (byte >> 4) : (byte & 0x0f);
    }
    case TF_INT4: {
        int64_t wpr = (s.cols * 4 + 31) / 32;
        return unpack_field((const uint32_t *)s.data + n * wpr, k, 4);
    }
    case TF_BF16: case TF_F16: return ((const uint16_t *)(a.dense ? a.dense : s.data))[n * a.cols + k];
    case TF_F32: return ((const uint32_t *)(a.dense ? a.dense : s.data))[n * a.cols + k];
    default: return 0u;
    }
}

__global__ void retile_kernel(RetileArgs a) {
    int64_t total = a.groups_n * a.units_k * 64;
    int uk = unit_k_of(a.tf);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int lane = (int)(i % 64);
        int64_t unit = i / 64;
        int64_t g = unit / a.units_k, u = unit % a.units_k;
        int64_t n = g * 16 + lane % 16;
        int kq = lane / 16;
        uint8_t *base = a.codes + unit * unit_bytes_of(a.tf);
        switch (a.tf) {
        case TF_BF16: case TF_F16: {
            uint16_t w[8];
            for (int j = 0; j < 8; j++) w[j] = (uint16_t)src_code(a, n, u * uk + 8 * kq + j);
            uint4 o;
            o.x = w[0] | ((uint32_t)w[1] << 16); o.y = w[2] | ((uint32_t)w[3] << 16);
            o.z = w[4] | ((uint32_t)w[5] << 16); o.w = w[6] | ((uint32_t)w[7] << 16);
            *(uint4 *)(base + lane * 16) = o;
            break;
        }
        case TF_F32: {
            uint32_t w[8];
            for (int j = 0; j < 8; j++) w[j] = src_code(a, n, u * uk + 8 * kq + j);
            *(uint4 *)(base + lane * 16) = make_uint4(w[0], w[1], w[2], w[3]);
            *(uint4 *)(base + 1024 + lane * 16) = make_uint4(w[4], w[5], w[6], w[7]);
            break;
        }
        case TF_Q8: case TF_FP8: {
            uint32_t w[4] = {0, 0, 0, 0};
            for (int t = 0; t < 2; t++)
                for (int j = 0; j < 8; j++) {
                    uint32_t c = src_code(a, n, u * uk + 32 * t + 8 * kq + j) & 0xffu;
                    int s = t * 8 + j;
                    w[s / 4] |= c << (8 * (s % 4));
                }
            *(uint4 *)(base + lane * 16) = make_uint4(w[0], w[1], w[2], w[3]);
            break;
        }
        case TF_MX4: case TF_INT4: {
            uint32_t w[4] = {0, 0, 0, 0};
            for (int t = 0; t < 4; t++)
                for (int j = 0; j < 8; j++) {
                    uint32_t c = src_code(a, n, u * uk + 32 * t + 8 * kq + j) & 0xfu;
                    int s = t * 8 + j;  // nibble index in the 16 B word
                    w[s / 8] |= c << (4 * (s % 8));
                }
            *(uint4 *)(base + lane * 16) = make_uint4(w[0], w[1], w[2], w[3]);
            break;
        }
        }
    }
}

// Q8_0 scales: f16 of block (n, kt) -> [rows_pad][kt_pad]
__global__ void q8_scales_kernel(RawView s, uint16_t *out, int64_t rows, int64_t kt_src, int64_t kt_pad, int64_t rows_pad) {
    int64_t total = rows_pad * kt_pad;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t n = i / kt_pad, kt = i % kt_pad;
        uint16_t v = 0;
        if (n < rows && kt < kt_src) {
            const uint8_t *b = s.data + (n * kt_src + kt) * 34;
            v = (uint16_t)(b[0] | (b[1] << 8));
        }
        out[i] = v;
    }
}

// Copy of a [rows][cols] byte matrix into a zero-padded [rows_pad][cols_pad] one.
__global__ void pad_copy_kernel(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t cols_bytes, int64_t rows_pad,
                                int64_t cols_pad_bytes) {
    int64_t total = rows_pad * cols_pad_bytes;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r = i / cols_pad_bytes, c = i % cols_pad_bytes;
        dst[i] = (r < rows && c < cols_bytes) ? src[r * cols_bytes + c] : 0;
    }
}

// INT4 zero points: packed along rows (dequant.zig:548-561) -> field value [rows_pad][groups_pad]
__global__ void int_zero_kernel(const uint32_t *zw, uint8_t *out, int64_t rows, int64_t groups, int64_t rows_pad,
                                int64_t groups_pad) {
    int64_t total = rows_pad * groups_pad;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t n = i / groups_pad, g = i % groups_pad;
        uint8_t v = 8;  // field 8 = zero point 0
        if (n < rows && g < groups) {
            int64_t start = n * 4;
            v = (uint8_t)((zw[(start / 32) * groups + g] >> (start % 32)) & 0xfu);
        }
        out[i] = v;
    }
}

// MXFP4 codes in the B operand order of the scaled MFMA: unit (g, u), lane l
// = the 16 source bytes of row 16 g + l % 16, columns 128 u + 32 (l / 16) ..
// +32 (two codes a byte, the lower column in the low nibble: the order the
// MFMA reads e2m1 codes); zero past the matrix.
__global__ void mx_native_kernel(const uint8_t *src, int64_t rows, int64_t cols, uint8_t *out, int64_t groups,
                                 int64_t units) {
    const int64_t total = groups * units * 64;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % 64);
        const int64_t unit = i / 64, g = unit / units, u = unit % units;
        const int64_t n = g * 16 + lane % 16, k0 = u * 128 + 32 * (lane / 16);
        uint32_t w[4] = {0, 0, 0, 0};
        if (n < rows && k0 < cols) {
            const uint8_t *row = src + n * (cols / 2) + k0 / 2;  // MXFP4 columns come in whole 32-blocks
#pragma unroll
            for (int j = 0; j < 16; j++) w[j / 4] |= (uint32_t)row[j] << (8 * (j % 4));
        }
        *(uint4 *)(out + i * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Their E8M0 scales in the same order: (g, u) -> 64 bytes, byte l = the scale
// of row 16 g + l % 16, column block 4 u + l / 16 (zero past the matrix).
__global__ void mx_scales_kernel(const uint8_t *scale, int64_t rows, int64_t kt, uint8_t *out, int64_t groups,
                                 int64_t units) {
    const int64_t total = groups * units * 64;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % 64);
        const int64_t unit = i / 64, g = unit / units, u = unit % units;
        const int64_t n = g * 16 + lane % 16, b = u * 4 + lane / 16;
        out[i] = (n < rows && b < kt) ? scale[n * kt + b] : 0;
    }
}

// Side words of the tiled GEMM (TileView::side). FP8: the scale grid as f32
// (exact for f32, f16, bf16 and finite E8M0 scales).
__global__ void fp8_side_kernel(const void *scale, int32_t scale_type, uint32_t *out, int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f2u(load_scale(scale, i, scale_type));
}

// Q8_0 side words of the GEMV: per 16-row group and 64-column unit, the 16
// rows' two f16 block scales (low half the unit's first block) in one
// 64-byte run, [group][unit][row % 16], from the [rows_pad][kt_pad] scales.
__global__ void q8_side_kernel(const uint32_t *scale, uint32_t *out, int64_t groups, int64_t units) {
    const int64_t total = groups * units * 16;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r16 = i % 16, gu = i / 16, u = gu % units, g = gu / units;
        out[i] = scale[(g * 16 + r16) * units + u];
    }
}

// INT4: the 16-bit scale (f16 or bf16 bits) | zero field << 16 per (row, group).
__global__ void int4_side_kernel(const uint16_t *scale, const uint8_t *zero, uint32_t *out, int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint32_t)scale[i] | ((uint32_t)(zero ? zero[i] : 8u) << 16);
}

// ---------------------------------------------------------------------------
// Host side

static int grid_for(int64_t total) {
    int64_t g = (total + 255) / 256;
    if (g > 65536) g = 65536;
    if (g < 1) g = 1;
    return (int)g;
}

void *dev_alloc(size_t bytes) {
    void *p = nullptr;
    if (bytes == 0) bytes = 16;
    DITCH_TRY_HIP(hipMalloc(&p, bytes));
    return p;
}
void dev_free(void *p) {
    if (p) (void)hipFree(p);
}

static size_t scale_elem_bytes(int32_t st) {
    switch (st) {
    case DITCH_F32: return 4;
    case DITCH_F16: case DITCH_BF16: return 2;
    case DITCH_E8M0: return 1;
    default: return 0;
    }
}
static int32_t scale_type_code(int32_t st) {
    switch (st) {
    case DITCH_F16: return SC_F16;
    case DITCH_BF16: return SC_BF16;
    case DITCH_E8M0: return SC_E8M0;
    default: return SC_F32;
    }
}

// Validates `w` and fills the raw view plus the byte sizes of its pieces.
// a * b for sizes taken from a caller's description: refused when either is
// negative or the product does not fit
static int64_t mul_sz(int64_t a, int64_t b) {
    int64_t r;
    DITCH_CHECK(a >= 0 && b >= 0 && !__builtin_mul_overflow(a, b, &r), DITCH_INVALID_ARGUMENT,
                "weight size overflows");
    return r;
}

RawSizes raw_sizes(const ditch_weight *w) {
    RawSizes z{0, 0, 0, 0};
    DITCH_CHECK(w->rows < (1ull << 40) && w->cols < (1ull << 40), DITCH_INVALID_ARGUMENT, "weight shape too large");
    int64_t rows = (int64_t)w->rows, cols = (int64_t)w->cols;
    DITCH_CHECK(w->data != nullptr, DITCH_INVALID_ARGUMENT, "weight data is NULL");
    const int64_t rc = mul_sz(rows, cols);
    switch (w->dtype) {
    case DITCH_F32: z.data = mul_sz(rc, 4); break;
    case DITCH_F16: case DITCH_BF16: z.data = mul_sz(rc, 2); break;
    case DITCH_Q8_0: case DITCH_Q4_0: case DITCH_Q4_1: case DITCH_Q5_0: case DITCH_Q5_1:
    case DITCH_Q4_K: case DITCH_Q6_K: case DITCH_Q8_K: {
        int bs = gguf_block_size(w->dtype);
        DITCH_CHECK(cols % bs == 0, DITCH_INVALID_ARGUMENT, "GGUF row length is not a whole number of blocks");
        z.data = mul_sz(mul_sz(rows, cols / bs), gguf_block_bytes(w->dtype));
        break;
    }
    case DITCH_FP8:
        DITCH_CHECK(w->scale && w->block_rows > 0 && w->block_cols > 0 && w->scale_cols > 0 && w->scale_rows > 0,
                    DITCH_INVALID_ARGUMENT, "FP8 weight needs a scale grid and block sizes");
        DITCH_CHECK(scale_elem_bytes(w->scale_dtype) > 0, DITCH_INVALID_ARGUMENT, "FP8 scale dtype");
        DITCH_CHECK(w->scale_rows < (1ull << 40) && w->scale_cols < (1ull << 40), DITCH_INVALID_ARGUMENT,
                    "FP8 scale grid too large");
        z.data = rc;
        z.scale = mul_sz(mul_sz((int64_t)w->scale_rows, (int64_t)w->scale_cols), scale_elem_bytes(w->scale_dtype));
        {
            // the grid must cover every row (dequant.zig:471-475) and column block
            int64_t last = rows - 1, sr;
            if (w->row_shard == 0) sr = last / (int64_t)w->block_rows;
            else {
                int64_t per_shard = ((int64_t)w->row_shard + (int64_t)w->block_rows - 1) / (int64_t)w->block_rows;
                sr = last / (int64_t)w->row_shard * per_shard + (last % (int64_t)w->row_shard) / (int64_t)w->block_rows;
            }
            DITCH_CHECK(sr < (int64_t)w->scale_rows && (cols - 1) / (int64_t)w->block_cols < (int64_t)w->scale_cols,
                        DITCH_INVALID_ARGUMENT, "FP8 scale grid does not cover the matrix");
        }
        break;
    case DITCH_MXFP4:
        DITCH_CHECK(cols % 32 == 0 && w->scale, DITCH_INVALID_ARGUMENT, "MXFP4 needs cols % 32 == 0 and scales");
        z.data = rc / 2;
        z.scale = rc / 32;
        break;
    case DITCH_MXFP4_T:
        DITCH_CHECK(rows % 32 == 0 && w->scale, DITCH_INVALID_ARGUMENT, "transposed MXFP4 needs rows % 32 == 0 and scales");
        z.data = rc / 2;
        z.scale = rc / 32;
        break;
    case DITCH_INT_PACKED: {
        DITCH_CHECK(w->bits >= 1 && w->bits <= 8 && w->scale && w->scale_cols > 0, DITCH_INVALID_ARGUMENT,
                    "pack-quantized weight needs 1..8 bits and scales");
        DITCH_CHECK(w->g_idx || w->group > 0, DITCH_INVALID_ARGUMENT, "pack-quantized weight needs a group size");
        DITCH_CHECK(scale_elem_bytes(w->scale_dtype) > 1, DITCH_INVALID_ARGUMENT, "pack-quantized scale dtype");
        DITCH_CHECK(w->scale_cols < (1ull << 40), DITCH_INVALID_ARGUMENT, "pack-quantized scale grid too large");
        int64_t wpr = (cols * w->bits + 31) / 32;
        z.data = mul_sz(mul_sz(rows, wpr), 4);
        z.scale = mul_sz(mul_sz(rows, (int64_t)w->scale_cols), scale_elem_bytes(w->scale_dtype));
        if (w->zero) z.zero = mul_sz(mul_sz((rows * w->bits + 31) / 32, (int64_t)w->scale_cols), 4);
        if (w->g_idx) {
            z.gidx = mul_sz(cols, 4);
            for (int64_t c = 0; c < cols; c++)
                DITCH_CHECK(w->g_idx[c] >= 0 && (uint64_t)w->g_idx[c] < w->scale_cols, DITCH_INVALID_ARGUMENT,
                            "g_idx names a group beyond the scales");
        } else {
            DITCH_CHECK((uint64_t)((cols + (int64_t)w->group - 1) / (int64_t)w->group) <= w->scale_cols,
                        DITCH_INVALID_ARGUMENT, "fewer scale groups than columns need");
        }
        break;
    }
    default: throw Error{DITCH_UNSUPPORTED, "unsupported weight dtype " + std::to_string(w->dtype)};
    }
    return z;
}

// Whether the gfx950 conversion instructions decode every element of `w`
// (stored as tile format `tf`) exactly as the reference does; see
// TileView::fast. Scans the host copy of the codes and scales.
static bool has_byte(const uint8_t *p, size_t n, uint8_t mask, uint8_t value) {
    // any byte with (b & mask) == value, eight bytes at a time
    const uint64_t M = 0x0101010101010101ull * mask, V = 0x0101010101010101ull * value;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        uint64_t w;
        memcpy(&w, p + i, 8);
        uint64_t v = (w & M) ^ V;  // zero bytes where the pattern matches
        if ((v - 0x0101010101010101ull) & ~v & 0x8080808080808080ull) return true;
    }
    for (; i < n; i++)
        if ((p[i] & mask) == value) return true;
    return false;
}

static bool finite_scales(const void *p, size_t count, int32_t dtype) {
    for (size_t i = 0; i < count; i++) {
        switch (dtype) {
        case DITCH_F32: {
            uint32_t b;
            memcpy(&b, (const uint8_t *)p + 4 * i, 4);
            if ((b & 0x7f800000u) == 0x7f800000u) return false;
            break;
        }
        case DITCH_BF16: {
            uint16_t b;
            memcpy(&b, (const uint8_t *)p + 2 * i, 2);
            if ((b & 0x7f80u) == 0x7f80u) return false;
            break;
        }
        case DITCH_F16: {
            uint16_t b;
            memcpy(&b, (const uint8_t *)p + 2 * i, 2);
            if ((b & 0x7c00u) == 0x7c00u) return false;
            break;
        }
        case DITCH_E8M0:
            if (((const uint8_t *)p)[i] == 255u) return false;
            break;
        default: return false;
        }
    }
    return true;
}

static int fast_decode_ok(const ditch_weight *w, int tf) {
    switch (tf) {
    case TF_BF16: case TF_Q8: return 1;  // nothing decoded by conversion instructions
    case TF_MX4: return has_byte((const uint8_t *)w->scale, w->rows * w->cols / 32, 0xffu, 0xffu) ? 0 : 1;
    case TF_FP8: {
        if (w->block_cols % 64 != 0 || w->fp8_e5m2) return 0;  // E5M2 stays on the exact decoder
        bool special = w->fp8_e5m2 ? has_byte((const uint8_t *)w->data, w->rows * w->cols, 0x7cu, 0x7cu)
                                   : has_byte((const uint8_t *)w->data, w->rows * w->cols, 0x7fu, 0x7fu);
        return !special && finite_scales(w->scale, w->scale_rows * w->scale_cols, w->scale_dtype) ? 1 : 0;
    }
    case TF_INT4:
        // the tiled GEMM's side word holds a 16-bit scale; its decode forms
        // (q - z) s as q s - z s, which needs 15 s finite: bf16 scales below
        // 2^120 in magnitude (every f16 scale is)
        if (w->group % 64 != 0 || (w->scale_dtype != DITCH_F16 && w->scale_dtype != DITCH_BF16)) return 0;
        if (w->scale_dtype == DITCH_BF16) {
            const size_t count = w->rows * w->scale_cols;
            for (size_t i = 0; i < count; i++) {
                uint16_t b;
                memcpy(&b, (const uint8_t *)w->scale + 2 * i, 2);
                if (((b >> 7) & 0xffu) >= 127 + 120) return 0;
            }
            return 1;
        }
        return finite_scales(w->scale, w->rows * w->scale_cols, w->scale_dtype) ? 1 : 0;
    default: return 0;
    }
}

// Copies the raw pieces of `w` to one device staging buffer.
struct Staged {
    void *buf = nullptr;
    RawView v{};
    ~Staged() { dev_free(buf); }
};

static void stage_raw(const ditch_weight *w, hipStream_t s, Staged &st) {
    RawSizes z = raw_sizes(w);
    auto al = [](size_t b) { return (b + 255) / 256 * 256; };
    size_t total = al(z.data) + al(z.scale) + al(z.zero) + al(z.gidx);
    st.buf = dev_alloc(total);
    uint8_t *p = (uint8_t *)st.buf;
    RawView &v = st.v;
    v = RawView{};
    v.dtype = w->dtype;
    v.rows = (int64_t)w->rows;
    v.cols = (int64_t)w->cols;
    v.data = p;
    DITCH_TRY_HIP(hipMemcpyAsync(p, w->data, z.data, hipMemcpyHostToDevice, s));
    p += al(z.data);
    if (z.scale) {
        v.scale = p;
        DITCH_TRY_HIP(hipMemcpyAsync(p, w->scale, z.scale, hipMemcpyHostToDevice, s));
        p += al(z.scale);
    }
    if (z.zero) {
        v.zero = p;
        DITCH_TRY_HIP(hipMemcpyAsync(p, w->zero, z.zero, hipMemcpyHostToDevice, s));
        p += al(z.zero);
    }
    if (z.gidx) {
        v.g_idx = (const int32_t *)p;
        DITCH_TRY_HIP(hipMemcpyAsync(p, w->g_idx, z.gidx, hipMemcpyHostToDevice, s));
        p += al(z.gidx);
    }
    v.scale_type = scale_type_code(w->scale_dtype);
    v.scale_cols = (int64_t)w->scale_cols;
    v.block_rows = (int64_t)w->block_rows;
    v.block_cols = (int64_t)w->block_cols;
    v.row_shard = (int64_t)w->row_shard;
    v.e5m2 = w->fp8_e5m2;
    v.bits = w->bits;
    v.group = (int64_t)w->group;
    v.groups = (int64_t)w->scale_cols;
}

void launch_raw_dequant(const RawView &v, void *out, int64_t row0, int64_t nrows, int bf16_out, hipStream_t s) {
    int64_t total = nrows * v.cols;
    if (total <= 0) return;
    hipLaunchKernelGGL(raw_dequant_kernel, dim3(grid_for(total)), dim3(256), 0, s, v, out, row0, nrows, bf16_out);
    DITCH_TRY_HIP(hipGetLastError());
}

void launch_dequant(const TileView &v, void *out, int64_t row0, int64_t nrows, hipStream_t s) {
    int64_t total = nrows * v.cols;
    if (total <= 0) return;
    int bf16_out = is_bf16_virtual(v.orig_dtype) ? 1 : 0;
    hipLaunchKernelGGL(tiled_dequant_kernel, dim3(grid_for(total)), dim3(256), 0, s, v, out, row0, nrows, bf16_out);
    DITCH_TRY_HIP(hipGetLastError());
}

// Host-memory decode of rows (ditch_hip_dequant): raw-layout path.
void dequant_to_host(ditch_hip *h, void *out, const ditch_weight *w, uint64_t row0, uint64_t nrows) {
    hipStream_t s = h->stream;
    DITCH_CHECK(row0 + nrows <= w->rows, DITCH_INVALID_ARGUMENT, "row range outside the weight");
    Staged st;
    stage_raw(w, s, st);
    int bf16_out = is_bf16_virtual(w->dtype) ? 1 : 0;
    size_t bytes = nrows * w->cols * (bf16_out ? 2 : 4);
    void *d_out = dev_alloc(bytes);
    try {
        launch_raw_dequant(st.v, d_out, (int64_t)row0, (int64_t)nrows, bf16_out, s);
        DITCH_TRY_HIP(hipMemcpyAsync(out, d_out, bytes, hipMemcpyDeviceToHost, s));
        DITCH_TRY_HIP(hipStreamSynchronize(s));
    } catch (...) {
        dev_free(d_out);
        throw;
    }
    dev_free(d_out);
}

void free_tensor(ditch_hip_tensor *t) {
    if (!t) return;
    dev_free(t->codes);
    dev_free(t->scale);
    dev_free(t->zero);
    dev_free(t->side);
    dev_free(t->mx);
    dev_free(t->mx_scales);
    delete t;
}

ditch_hip_tensor *upload_weight(ditch_hip *h, const ditch_weight *w, hipStream_t s) {
    (void)h;
    DITCH_CHECK(w && w->rows > 0 && w->cols > 0, DITCH_INVALID_ARGUMENT, "empty weight");
    Staged st;
    stage_raw(w, s, st);
    auto *t = new ditch_hip_tensor();
    try {
        TileView &v = t->v;
        v = TileView{};
        v.rows = (int64_t)w->rows;
        v.cols = (int64_t)w->cols;
        v.orig_dtype = w->dtype;
        // choose the tile format
        int tf;
        void *dense = nullptr;
        int dense_f32 = 0;
        switch (w->dtype) {
        case DITCH_F32: tf = TF_F32; break;
        case DITCH_F16: tf = TF_F16; break;
        case DITCH_BF16: tf = TF_BF16; break;
        case DITCH_Q8_0: tf = TF_Q8; break;
        case DITCH_FP8:
            tf = (w->block_cols % 8 == 0) ? TF_FP8 : TF_BF16;
            break;
        case DITCH_MXFP4: tf = TF_MX4; break;
        case DITCH_INT_PACKED: tf = (w->bits == 4 && !w->g_idx) ? TF_INT4 : TF_BF16; break;
        case DITCH_MXFP4_T: tf = TF_BF16; break;
        default: tf = TF_F32; break;  // other GGUF blocks: decoded to f32 once
        }
        bool decode_first = (tf == TF_BF16 && w->dtype != DITCH_BF16) || (tf == TF_F32 && w->dtype != DITCH_F32);
        if (decode_first) {
            dense_f32 = (tf == TF_F32) ? 1 : 0;
            size_t bytes = (size_t)v.rows * v.cols * (dense_f32 ? 4 : 2);
            dense = dev_alloc(bytes);
            launch_raw_dequant(st.v, dense, 0, v.rows, dense_f32 ? 0 : 1, s);
        }
        v.tf = tf;
        v.fast = decode_first ? (tf == TF_BF16 ? 1 : 0) : fast_decode_ok(w, tf);
        int uk = unit_k_of(tf);
        int64_t rows_pad = pad_to(v.rows, 16), cols_pad = pad_to(v.cols, uk);
        v.units_k = cols_pad / uk;
        size_t code_bytes = (size_t)(rows_pad / 16) * v.units_k * unit_bytes_of(tf);
        t->codes = dev_alloc(code_bytes);
        t->part_bytes[0] = code_bytes;
        t->bytes = code_bytes;
        RetileArgs a{};
        a.src = st.v;
        a.codes = (uint8_t *)t->codes;
        a.tf = tf;
        a.rows = v.rows;
        a.cols = v.cols;
        a.units_k = v.units_k;
        a.groups_n = rows_pad / 16;
        a.dense = dense;
        a.dense_f32 = dense_f32;
        int64_t total = a.groups_n * a.units_k * 64;
        hipLaunchKernelGGL(retile_kernel, dim3(grid_for(total)), dim3(256), 0, s, a);
        DITCH_TRY_HIP(hipGetLastError());
        // scales
        switch (tf) {
        case TF_Q8: {
            int64_t kt_src = v.cols / 32, kt_pad = cols_pad / 32;
            size_t b = rows_pad * kt_pad * 2;
            t->scale = dev_alloc(b);
            t->part_bytes[1] = b;
            t->bytes += b;
            hipLaunchKernelGGL(q8_scales_kernel, dim3(grid_for(rows_pad * kt_pad)), dim3(256), 0, s, st.v,
                               (uint16_t *)t->scale, v.rows, kt_src, kt_pad, rows_pad);
            v.scale_cols = kt_pad;
            v.scale_type = SC_F16;
            break;
        }
        case TF_MX4: {
            int64_t kt_src = v.cols / 32, kt_pad = cols_pad / 32;
            size_t b = rows_pad * kt_pad;
            t->scale = dev_alloc(b);
            t->part_bytes[1] = b;
            t->bytes += b;
            hipLaunchKernelGGL(pad_copy_kernel, dim3(grid_for(rows_pad * kt_pad)), dim3(256), 0, s, st.v.scale,
                               (uint8_t *)t->scale, v.rows, kt_src, rows_pad, kt_pad);
            v.scale_cols = kt_pad;
            v.scale_type = SC_E8M0;
            break;
        }
        case TF_FP8: {
            // the grid as given; rows beyond the matrix clamp to the last grid row in the kernels
            size_t eb = scale_elem_bytes(w->scale_dtype);
            int64_t sr_pad = (int64_t)w->scale_rows + 1, sc_pad = pad_to(cols_pad, w->block_cols) / w->block_cols;
            if (sc_pad < (int64_t)w->scale_cols) sc_pad = (int64_t)w->scale_cols;
            size_t b = sr_pad * sc_pad * eb;
            t->scale = dev_alloc(b);
            t->part_bytes[1] = b;
            t->bytes += b;
            DITCH_TRY_HIP(hipMemsetAsync(t->scale, 0, b, s));
            hipLaunchKernelGGL(pad_copy_kernel, dim3(grid_for(sr_pad * sc_pad * eb)), dim3(256), 0, s, st.v.scale,
                               (uint8_t *)t->scale, (int64_t)w->scale_rows, (int64_t)(w->scale_cols * eb), sr_pad,
                               (int64_t)(sc_pad * eb));
            v.scale_cols = sc_pad;
            v.scale_type = scale_type_code(w->scale_dtype);
            v.block_rows = (int64_t)w->block_rows;
            v.block_cols = (int64_t)w->block_cols;
            v.row_shard = (int64_t)w->row_shard;
            v.e5m2 = w->fp8_e5m2;
            break;
        }
        case TF_INT4: {
            size_t eb = scale_elem_bytes(w->scale_dtype);
            int64_t groups = (int64_t)w->scale_cols;
            int64_t groups_pad = (cols_pad + (int64_t)w->group - 1) / (int64_t)w->group;
            if (groups_pad < groups) groups_pad = groups;
            size_t b = rows_pad * groups_pad * eb;
            t->scale = dev_alloc(b);
            t->part_bytes[1] = b;
            t->bytes += b;
            hipLaunchKernelGGL(pad_copy_kernel, dim3(grid_for(rows_pad * groups_pad * eb)), dim3(256), 0, s,
                               st.v.scale, (uint8_t *)t->scale, v.rows, (int64_t)(groups * eb), rows_pad,
                               (int64_t)(groups_pad * eb));
            if (w->zero) {
                size_t zb = rows_pad * groups_pad;
                t->zero = dev_alloc(zb);
                t->part_bytes[2] = zb;
                t->bytes += zb;
                hipLaunchKernelGGL(int_zero_kernel, dim3(grid_for(rows_pad * groups_pad)), dim3(256), 0, s,
                                   (const uint32_t *)st.v.zero, (uint8_t *)t->zero, v.rows, groups, rows_pad,
                                   groups_pad);
            }
            v.scale_cols = groups_pad;
            v.scale_type = scale_type_code(w->scale_dtype);
            v.group = (int64_t)w->group;
            break;
        }
        default: break;
        }
        DITCH_TRY_HIP(hipGetLastError());
        // side words of the tiled GEMM (the GEMV for Q8_0)
        if (tf == TF_Q8) {
            const int64_t total = a.groups_n * v.units_k * 16;
            t->side = dev_alloc(total * 4);
            t->part_bytes[3] = total * 4;
            t->bytes += total * 4;
            hipLaunchKernelGGL(q8_side_kernel, dim3(grid_for(total)), dim3(256), 0, s, (const uint32_t *)t->scale,
                               (uint32_t *)t->side, a.groups_n, v.units_k);
            v.side = (const uint32_t *)t->side;
            v.side_cols = v.units_k;
        } else if (v.fast && tf == TF_MX4) {
            v.side = (const uint32_t *)t->scale;
            v.side_cols = v.scale_cols / 4;
            t->mx = dev_alloc(code_bytes);
            t->part_bytes[4] = code_bytes;
            t->bytes += code_bytes;
            const int64_t total_mx = a.groups_n * v.units_k * 64;
            hipLaunchKernelGGL(mx_native_kernel, dim3(grid_for(total_mx)), dim3(256), 0, s, st.v.data, v.rows, v.cols,
                               (uint8_t *)t->mx, a.groups_n, v.units_k);
            t->mx_scales = dev_alloc(total_mx);
            t->part_bytes[5] = total_mx;
            t->bytes += total_mx;
            hipLaunchKernelGGL(mx_scales_kernel, dim3(grid_for(total_mx)), dim3(256), 0, s, (const uint8_t *)st.v.scale,
                               v.rows, v.cols / 32, (uint8_t *)t->mx_scales, a.groups_n, v.units_k);
            v.mx = (const uint8_t *)t->mx;
            v.mx_scales = (const uint8_t *)t->mx_scales;
        } else if (v.fast && tf == TF_FP8) {
            int64_t total = ((int64_t)w->scale_rows + 1) * v.scale_cols;
            t->side = dev_alloc(total * 4);
            t->part_bytes[3] = total * 4;
            t->bytes += total * 4;
            hipLaunchKernelGGL(fp8_side_kernel, dim3(grid_for(total)), dim3(256), 0, s, t->scale, v.scale_type,
                               (uint32_t *)t->side, total);
            v.side = (const uint32_t *)t->side;
            v.side_cols = v.scale_cols;
        } else if (v.fast && tf == TF_INT4) {
            int64_t total = pad_to(v.rows, 16) * v.scale_cols;
            t->side = dev_alloc(total * 4);
            t->part_bytes[3] = total * 4;
            t->bytes += total * 4;
            hipLaunchKernelGGL(int4_side_kernel, dim3(grid_for(total)), dim3(256), 0, s, (const uint16_t *)t->scale,
                               (const uint8_t *)t->zero, (uint32_t *)t->side, total);
            v.side = (const uint32_t *)t->side;
            v.side_cols = v.scale_cols;
        }
        DITCH_TRY_HIP(hipGetLastError());
        v.codes = (const uint8_t *)t->codes;
        v.scale = t->scale;
        v.zero = (const uint8_t *)t->zero;
        DITCH_TRY_HIP(hipStreamSynchronize(s));
        dev_free(dense);
    } catch (...) {
        free_tensor(t);
        throw;
    }
    return t;
}

// ---------------------------------------------------------------------------
// Residency of the per-call weights (compute.Residency, compute.zig:567-693):
// a byte-budgeted least-recently-used set of registered copies keyed by the
// host address and length of the weight's codes and the rest of its
// descriptor, each with a signature of sampled bytes so that new contents
// at a cached address are a miss, never a stale copy. Caching by address is
// sound only while the host buffers stay valid and unique (memory-mapped
// weights), so it is on only with `stable`; forget_weights clears it.

static uint64_t mix64(uint64_t h) {
    h ^= h >> 33;
    h *= 0xff51afd7ed558ccdull;
    h ^= h >> 33;
    h *= 0xc4ceb9fe1a85ec53ull;
    return h ^ (h >> 33);
}

// up to four 64-byte samples (start, two interior points, end), or the whole
// buffer when it is at most 256 bytes
static uint64_t sample_hash(uint64_t h, const void *p, size_t len) {
    if (!p || !len) return mix64(h ^ 0x9e3779b97f4a7c15ull);
    const uint8_t *b = (const uint8_t *)p;
    auto feed = [&](size_t at, size_t n) {
        for (size_t k = 0; k < n; k++) h = (h ^ b[at + k]) * 0x100000001b3ull;
    };
    h = mix64(h ^ len);
    if (len <= 256) feed(0, len);
    else
        for (size_t at : {(size_t)0, len / 3, 2 * (len / 3), len - 64}) feed(at, 64);
    return mix64(h);
}

static uint64_t weight_signature(const ditch_weight *w, const RawSizes &z) {
    uint64_t h = sample_hash(0x5151, w->data, z.data);
    h = sample_hash(h, w->scale, z.scale);
    h = sample_hash(h, w->zero, z.zero);
    return sample_hash(h, w->g_idx, z.gidx);
}

static uint64_t weight_desc(const ditch_weight *w) {
    const uint64_t f[] = {(uint64_t)w->dtype, (uint64_t)w->scale_dtype, w->rows, w->cols,
                          (uint64_t)(uintptr_t)w->scale, w->scale_rows, w->scale_cols, w->block_rows,
                          w->block_cols, w->row_shard, (uint64_t)w->fp8_e5m2, (uint64_t)w->bits, w->group,
                          (uint64_t)(uintptr_t)w->zero, (uint64_t)(uintptr_t)w->g_idx};
    uint64_t h = 0x1234;
    for (uint64_t v : f) h = mix64(h ^ v);
    return h;
}

static void residency_drop(ditch_hip *h, size_t i) {
    auto &r = h->res;
    free_tensor(r.entries[i].t);
    r.used -= r.entries[i].bytes < r.used ? r.entries[i].bytes : r.used;
    r.entries[i] = r.entries.back();
    r.entries.pop_back();
    r.evictions++;
}

// evicts least recently used entries until `bytes` more fit; false when they
// cannot (larger than the budget)
static bool residency_make_room(ditch_hip *h, uint64_t bytes) {
    auto &r = h->res;
    if (bytes > r.budget) return false;
    while (r.used + bytes > r.budget && !r.entries.empty()) {
        size_t oldest = 0;
        for (size_t k = 1; k < r.entries.size(); k++)
            if (r.entries[k].used_at < r.entries[oldest].used_at) oldest = k;
        residency_drop(h, oldest);
    }
    return r.used + bytes <= r.budget;
}

void residency_clear(ditch_hip *h) {
    auto &r = h->res;
    for (auto &e : r.entries) free_tensor(e.t);
    r.entries.clear();
    r.used = 0;
}

void residency_configure(ditch_hip *h, uint64_t budget, bool stable) {
    auto &r = h->res;
    r.budget = budget;
    r.stable = stable;
    if (!stable || budget == 0) residency_clear(h);
    else residency_make_room(h, 0);
}

void acquire_weight(ditch_hip *h, const ditch_weight *w, hipStream_t s, WeightRef &ref) {
    auto &r = h->res;
    DITCH_CHECK(w && w->rows > 0 && w->cols > 0, DITCH_INVALID_ARGUMENT, "empty weight");
    if (r.budget == 0 || !r.stable) {
        ref.t = upload_weight(h, w, s);
        ref.owned = true;
        return;
    }
    const RawSizes z = raw_sizes(w);
    const uint64_t desc = weight_desc(w), sig = weight_signature(w, z);
    for (size_t k = 0; k < r.entries.size(); k++) {
        auto &e = r.entries[k];
        if (e.data == w->data && e.len == z.data && e.desc == desc) {
            if (e.sig != sig) {  // new contents at a cached address
                residency_drop(h, k);
                break;
            }
            e.used_at = ++r.clock;
            r.hits++;
            ref.t = e.t;
            ref.owned = false;
            return;
        }
    }
    r.misses++;
    ref.t = upload_weight(h, w, s);
    ref.owned = true;
    if (residency_make_room(h, ref.t->bytes)) {
        r.entries.push_back(ditch_hip::ResidencyEntry{w->data, z.data, desc, sig, ref.t->bytes, ref.t, ++r.clock});
        r.used += ref.t->bytes;
        ref.owned = false;
    }
}

}  // namespace ditch
