// decode.h — element decoders of the quantised weight formats, device side.
//
// Each function reproduces the reference's value bit for bit:
//   bf16 from f32 ........ tensor.zig:423-430 (RNE, NaN -> (bits>>16)|0x40)
//   f16 -> f32 ........... tensor.zig:432-435 (exact widening)
//   FP8 E4M3 / E5M2 ...... dequant.zig:281-307 (fp8Table, OCP "fn" E4M3)
//   E8M0 scales .......... dequant.zig:259-261 (e8m0Scale), :446 (e8m0)
//   E2M1 ................. dequant.zig:310 (e2m1_table)
//   GGUF blocks .......... quant.zig:81-199
// Products that can see a NaN or an infinity follow x86 SSE rules, the
// platform the CPU reference runs on: a NaN operand is returned quieted (the
// first one if both are NaN), an invalid product (0 * inf) is the negative
// default NaN 0xffc00000.
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ditch {

// A load from global memory (address space 1): the compiler then issues
// global_load rather than flat_load, whose completion it can only track
// together with LDS and scalar traffic.
template <typename T>
__device__ __forceinline__ T gload(const void *p) {
    if constexpr (sizeof(T) == 16) {
        typedef uint32_t v4_t __attribute__((ext_vector_type(4)));
        return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) v4_t *)p);
    } else if constexpr (sizeof(T) == 8) {
        typedef uint32_t v2_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) v2_t *)p);
    } else {
        return *(const __attribute__((address_space(1))) T *)p;
    }
}

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u);
    uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7fffu + lsb) >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

// f16 -> f32 by the hardware conversion: the same value for every finite
// f16 and infinity; a NaN stays a NaN, its payload not kept (for scales of
// products, where the payload does not matter).
__device__ __forceinline__ float f16_to_f32_hw(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        float v = (float)man * 5.9604644775390625e-08f;  // man * 2^-24, exact
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

__device__ __forceinline__ bool is_nan(float v) { return (f2u(v) & 0x7fffffffu) > 0x7f800000u; }

// a * b with x86 SSE NaN semantics (see the file comment).
__device__ __forceinline__ float mul_x86(float a, float b) {
    if (is_nan(a)) return u2f(f2u(a) | 0x00400000u);
    if (is_nan(b)) return u2f(f2u(b) | 0x00400000u);
    float r = __fmul_rn(a, b);
    if (is_nan(r)) return u2f(0xffc00000u);
    return r;
}

// fp8Table entry (dequant.zig:281-304).
__device__ __forceinline__ float fp8_value(uint32_t code, bool e5m2) {
    uint32_t sign = (code & 0x80u) << 24;
    if (!e5m2) {
        uint32_t e = (code >> 3) & 0xfu, m = code & 7u;
        if (e == 15u && m == 7u) return u2f(sign | 0x7fc00000u);
        if (e == 0u) {
            float v = (float)m * 0.001953125f;  // m/8 * 2^-6
            return sign ? -v : v;
        }
        return u2f(sign | ((e + 120u) << 23) | (m << 20));
    }
    uint32_t e = (code >> 2) & 0x1fu, m = code & 3u;
    if (e == 31u) return u2f(sign | (m == 0u ? 0x7f800000u : 0x7fc00000u));
    if (e == 0u) {
        float v = (float)m * 1.52587890625e-05f;  // m/4 * 2^-14
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 21));
}

// e8m0Scale (dequant.zig:259-261): byte 0 is the subnormal 2^-127.
__device__ __forceinline__ float e8m0_scale(uint32_t b) {
    return b == 0u ? u2f(0x00400000u) : u2f(b << 23);
}
// e8m0 (FP8 with exponent scales, dequant.zig:446): 255 is NaN.
__device__ __forceinline__ float e8m0_value(uint32_t b) {
    if (b == 255u) return u2f(0x7fc00000u);
    return b == 0u ? u2f(0x00400000u) : u2f(b << 23);
}

// e2m1_table (dequant.zig:310): sign in bit 3, values 0 .5 1 1.5 2 3 4 6.
__device__ __forceinline__ float e2m1_value(uint32_t nib) {
    uint32_t mag = nib & 7u;
    // magnitude bits: 0 -> 0; 1 -> 0.5; 2,3 -> 1,1.5; 4,5 -> 2,3; 6,7 -> 4,6
    uint32_t bits;
    if (mag == 0u) bits = 0u;
    else if (mag == 1u) bits = 0x3f000000u;
    else bits = ((126u + (mag >> 1)) << 23) | ((mag & 1u) << 22);
    return u2f(bits | ((nib & 8u) << 28));
}

// Scale dtypes of the FP8 / INT scale arrays.
enum ScaleType : int32_t { SC_F32 = 0, SC_F16 = 1, SC_BF16 = 2, SC_E8M0 = 40 };

__device__ __forceinline__ float load_scale(const void *base, size_t idx, int32_t st) {
    switch (st) {
    case SC_F16: return f16_to_f32(gload<uint16_t>((const uint16_t *)base + idx));
    case SC_BF16: return bf16_to_f32(gload<uint16_t>((const uint16_t *)base + idx));
    case SC_E8M0: return e8m0_value(gload<uint8_t>((const uint8_t *)base + idx));
    default: return gload<float>((const float *)base + idx);
    }
}

// expVec (tensor.zig:1277-1294): Cephes expf, restated lane for lane.
__device__ __forceinline__ float exp_cephes(float x_in) {
    float x = fminf(fmaxf(x_in, -87.3f), 88.0f);
    float fx = roundf(__fmul_rn(x, 1.44269504088896341f));
    float r = __builtin_fmaf(fx, 2.12194440e-4f, __builtin_fmaf(fx, -0.693359375f, x));
    float y = 1.9875691500e-4f;
    y = __builtin_fmaf(y, r, 1.3981999507e-3f);
    y = __builtin_fmaf(y, r, 8.3334519073e-3f);
    y = __builtin_fmaf(y, r, 4.1665795894e-2f);
    y = __builtin_fmaf(y, r, 1.6666665459e-1f);
    y = __builtin_fmaf(y, r, 5.0000001201e-1f);
    y = __builtin_fmaf(y, __fmul_rn(r, r), __fadd_rn(r, 1.0f));
    int e = (int)fx;
    return __fmul_rn(y, u2f((uint32_t)(e + 127) << 23));
}

// Activation.applyVec (tensor.zig:1257-1274); gelu (2) has no vector form
// and uses Abramowitz-Stegun erf (tensor.zig:1220-1225).
__device__ __forceinline__ float act_apply(uint32_t act, float x) {
    switch (act) {
    case 0: return __fdiv_rn(x, __fadd_rn(1.0f, exp_cephes(-x)));
    case 1: {
        float u = __fmul_rn(0.7978845608028654f, __fadd_rn(x, __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x)));
        float t = __fsub_rn(1.0f, __fdiv_rn(2.0f, __fadd_rn(exp_cephes(__fadd_rn(u, u)), 1.0f)));
        return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, t));
    }
    case 2: {
        float z = __fdiv_rn(x, 1.41421356237309504880f);
        float t = __fdiv_rn(1.0f, __fadd_rn(1.0f, __fmul_rn(0.3275911f, fabsf(z))));
        float p = __fsub_rn(__fmul_rn(1.061405429f, t), 1.453152027f);
        p = __fadd_rn(__fmul_rn(p, t), 1.421413741f);
        p = __fsub_rn(__fmul_rn(p, t), 0.284496736f);
        p = __fadd_rn(__fmul_rn(p, t), 0.254829592f);
        float y = __fsub_rn(1.0f, __fmul_rn(__fmul_rn(p, t), expf(-__fmul_rn(z, z))));
        float erf_v = z >= 0 ? y : -y;
        return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, erf_v));
    }
    case 3: return fmaxf(x, 0.0f);
    case 4: { float r = fmaxf(x, 0.0f); return __fmul_rn(r, r); }
    case 5: return __fdiv_rn(x, __fadd_rn(1.0f, exp_cephes(__fmul_rn(-1.702f, x))));
    default: return x;
    }
}

// The activation inside a fused gate/up epilogue whose output is split into
// fp6 or bf16 terms right away (so within 15^-4 of its block maximum, or
// 2^-18 of itself): SiLU as x * rcp(1 + 2^(-x log2 e)) on the hardware
// exp2 and reciprocal (about an ulp from x / (1 + expVec(-x))), the other
// activations exactly as act_apply. A is a compile-time activation code.
template <int A>
__device__ __forceinline__ float act_fused(float x) {
    if constexpr (A == 0) {
        const float e = __builtin_amdgcn_exp2f(__fmul_rn(x, -1.4426950408889634f));
        return __fmul_rn(x, __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e)));
    } else {
        return act_apply(A, x);
    }
}

// f(std::integral_constant<int, act>) with the run-time activation code made
// a compile-time one (one switch outside the loops that apply it).
template <typename F>
__device__ __forceinline__ void with_act(uint32_t act, F &&f) {
    switch (act) {
    case 0: f(std::integral_constant<int, 0>{}); break;
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 5: f(std::integral_constant<int, 5>{}); break;
    default: f(std::integral_constant<int, 6>{}); break;
    }
}

}  // namespace ditch
