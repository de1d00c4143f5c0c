// tiled.h — addressing and element decode of the HBM weight tiles
// (layout described in internal.h). Shared by the decode, norm and edit
// kernels; the matmul kernels decode whole 16-byte words instead.
#pragma once
#include "decode.h"
#include "internal.h"

namespace ditch {

__device__ __forceinline__ int64_t fp8_scale_row(int64_t r, int64_t block_rows, int64_t row_shard) {
    if (row_shard == 0) return r / block_rows;
    int64_t per_shard = (row_shard + block_rows - 1) / block_rows;
    return r / row_shard * per_shard + (r % row_shard) / block_rows;
}

// ---------------------------------------------------------------------------
// Tiled layout addressing (see internal.h).

__host__ __device__ inline int64_t pad_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Byte offset and position of element (n, k) in the tiled codes.
// Returns the byte offset of the lane's 16 B word and the element index
// inside it (`slot`: 0..7 for 16-bit, 0..15 for 8-bit, 0..31 for 4-bit).
__device__ __forceinline__ void tile_locate(int tf, int64_t units_k, int64_t n, int64_t k, int64_t *word, int *slot,
                                            int *half) {
    int uk = unit_k_of(tf);
    int64_t g = n / 16, u = k / uk;
    int kin = (int)(k % uk);
    int t = kin / 32, kq = (kin % 32) / 8, j = kin % 8;
    int lane = (int)(n % 16) + 16 * kq;
    int64_t base = (g * units_k + u) * unit_bytes_of(tf);
    *half = 0;
    switch (tf) {
    case TF_F32:
        *half = j / 4;
        *word = base + (*half) * 1024 + lane * 16;
        *slot = j % 4;
        break;
    case TF_Q8: case TF_FP8:
        *word = base + lane * 16;
        *slot = t * 8 + j;
        break;
    case TF_MX4: case TF_INT4:
        *word = base + lane * 16;
        *slot = t * 8 + j;
        break;
    default:
        *word = base + lane * 16;
        *slot = j;
        break;
    }
}

// Decode of element (n, k) from the tiled layout (same value as the raw path).
__device__ float tiled_element_f32(const TileView &v, int64_t n, int64_t k, uint16_t *bf16_bits) {
    int64_t word;
    int slot, half;
    tile_locate(v.tf, v.units_k, n, k, &word, &slot, &half);
    const uint8_t *p = v.codes + word;
    switch (v.tf) {
    case TF_BF16: {
        uint16_t b = ((const uint16_t *)p)[slot];
        *bf16_bits = b;
        return bf16_to_f32(b);
    }
    case TF_F16: return f16_to_f32(((const uint16_t *)p)[slot]);
    case TF_F32: return ((const float *)p)[slot];
    case TF_Q8: {
        float d = f16_to_f32(((const uint16_t *)v.scale)[n * v.scale_cols + k / 32]);
        return __fmul_rn((float)(int8_t)p[slot], d);
    }
    case TF_FP8: {
        int64_t sr = fp8_scale_row(n, v.block_rows, v.row_shard);
        float s = load_scale(v.scale, sr * v.scale_cols + k / v.block_cols, v.scale_type);
        uint16_t b = f32_to_bf16(mul_x86(fp8_value(p[slot], v.e5m2), s));
        *bf16_bits = b;
        return bf16_to_f32(b);
    }
    case TF_MX4: {
        uint8_t byte = p[slot / 2];
        uint32_t nib = (slot & 1) ? (byte >> 4) : (byte & 0x0f);
        float sc = e8m0_scale(((const uint8_t *)v.scale)[n * v.scale_cols + k / 32]);
        uint16_t b = f32_to_bf16(mul_x86(e2m1_value(nib), sc));
        *bf16_bits = b;
        return bf16_to_f32(b);
    }
    case TF_INT4: {
        uint8_t byte = p[slot / 2];
        int field = (slot & 1) ? (byte >> 4) : (byte & 0x0f);
        int64_t g = k / v.group;
        int zp = v.zero ? (int)v.zero[n * v.scale_cols + g] - 8 : 0;
        float s = load_scale(v.scale, n * v.scale_cols + g, v.scale_type);
        uint16_t b = f32_to_bf16(mul_x86((float)((field - 8) - zp), s));
        *bf16_bits = b;
        return bf16_to_f32(b);
    }
    default: return 0.0f;
    }
}

// One wave's part of x_row . a_j for the low-rank deltas' products
// (tensor.zig:1036-1042), directions j0 .. j0 + 3 below `rank` at once: the
// row is read once for the four, 16 bytes a lane with four such loads in
// flight (rows of whole, aligned float4s; else one float a lane). Lane sums
// in s, to be added over the wave.
__device__ __forceinline__ void delta_dot4(const float *xr, const float *a, int64_t cols, int64_t j0, int64_t rank,
                                           int lane, float (&s)[4]) {
    if ((cols & 3) == 0 && (((uintptr_t)xr | (uintptr_t)a) & 15) == 0) {
        constexpr int U = 4;
        for (int64_t c0 = 4 * lane; c0 < cols; c0 += 256 * U) {
            float4 xv[U];
#pragma unroll
            for (int u = 0; u < U; u++)
                xv[u] = c0 + 256 * u < cols ? *(const float4 *)(xr + c0 + 256 * u) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                if (j0 + jj >= rank) continue;
                const float *ar = a + (j0 + jj) * cols;
#pragma unroll
                for (int u = 0; u < U; u++) {
                    if (c0 + 256 * u >= cols) continue;
                    const float4 av = *(const float4 *)(ar + c0 + 256 * u);
                    s[jj] = __builtin_fmaf(av.x, xv[u].x, s[jj]);
                    s[jj] = __builtin_fmaf(av.y, xv[u].y, s[jj]);
                    s[jj] = __builtin_fmaf(av.z, xv[u].z, s[jj]);
                    s[jj] = __builtin_fmaf(av.w, xv[u].w, s[jj]);
                }
            }
        }
    } else {
        for (int64_t c = lane; c < cols; c += 64) {
            const float xv = xr[c];
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                if (j0 + jj < rank) s[jj] = __builtin_fmaf(a[(j0 + jj) * cols + c], xv, s[jj]);
        }
    }
}

}  // namespace ditch
