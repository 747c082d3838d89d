// Device-side helpers shared by the MoE expert-path kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jx {

enum : int { T_F32 = 0, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

// Super-block formats (256 elements per K-unit, Q4_K-style header for Q4_K and Q5_K).
__host__ __device__ constexpr bool is_kquant(int t) { return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

constexpr int WAVE = 64;
constexpr int ROWS_PER_TILE = 32;   // weight rows per repacked tile (= one MFMA M/N edge)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ h2v as_h2(uint32_t v) { return __builtin_bit_cast(h2v, v); }

// 8 bytes (w0, w1) of small unsigned integers v (after mask/flip) -> 8 fp16
// c1 * (1024 + v) + c0, exact: the perm builds fp16 bit patterns 0x64vv =
// 1024 + vv and one fused fp16 fma removes the bias.
__device__ __forceinline__ h8 cvt8(uint32_t w0, uint32_t w1, uint32_t mask, uint32_t flip, h2v c1, h2v c0) {
    const uint32_t a = (w0 & mask) ^ flip, b = (w1 & mask) ^ flip;
    const h2v x0 = as_h2(__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u));
    const h2v x1 = as_h2(__builtin_amdgcn_perm(0x64646464u, a, 0x04030402u));
    const h2v x2 = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04010400u));
    const h2v x3 = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04030402u));
    const h2v y0 = __builtin_elementwise_fma(x0, c1, c0);
    const h2v y1 = __builtin_elementwise_fma(x1, c1, c0);
    const h2v y2 = __builtin_elementwise_fma(x2, c1, c0);
    const h2v y3 = __builtin_elementwise_fma(x3, c1, c0);
    return h8{y0.x, y0.y, y1.x, y1.y, y2.x, y2.y, y3.x, y3.y};
}

// Four bits -> bit 0 of four bytes (disjoint shifted copies, no carries).
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }

// ---------------------------------------------------------------- numerics

// fp32 -> fp16 bits, mantissa truncated (the store rule of the reference's
// Q8_0 activation scale, src/quant.cpp:909-925): subnormal results shift,
// results below 2^-24 become signed zero, |f| >= 2^16 (and inf/NaN) become
// signed infinity.
__device__ __forceinline__ uint32_t f32_to_f16_trunc(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 0xFFu) - 112;
    uint32_t m = b & 0x7FFFFFu;
    if (e <= 0) {
        if (e < -10) return sign;
        m |= 0x800000u;
        return sign | (m >> (uint32_t)(14 - e));
    }
    if (e >= 31) return sign | 0x7C00u;
    return sign | ((uint32_t)e << 10) | (m >> 13);
}

// fp16 -> fp32 (the low 16 bits of h): one v_cvt_f32_f16, exact for every
// finite input including subnormals (kernels run with fp16 denormals
// preserved: the default .amdhsa_float_denorm_mode_16_64 = 3).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Round half away from zero (C roundf), exact for every finite input.
__device__ __forceinline__ float round_away(float v) {
    const float t = __builtin_truncf(v);
    const float fr = v - t;  // exact
    return (__builtin_fabsf(fr) >= 0.5f) ? t + __builtin_copysignf(1.0f, v) : t;
}

enum : int { ACT_SILU = 0, ACT_GELU_TANH = 1 };

// The gated activation of matmul_swiglu_quant_f32 (src/quant.cpp:3999-4007):
// SiLU(g) * u, or with use_gelu (the gemma family, transformer.cpp:1995) the
// tanh form of GELU, 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) * u.
__device__ __forceinline__ float gated(float g, float u, int act) {
    if (act == ACT_GELU_TANH) {
        const float inner = 0.7978845608028654f * __builtin_fmaf(0.044715f * g * g, g, g);
        return 0.5f * g * (1.0f + tanhf(inner)) * u;
    }
    return (g / (1.0f + expf(-g))) * u;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// 6-bit (scale, min) j of a Q4_K super-block header (layout of
// include/quant.h:28-33, unpacking as get_scale_min_k4, quant.cpp:1107-1115).
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* s, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ float wave_max32(float v) {
    // max over the 32 lanes of each half-wave (order-independent)
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int wave_sum32i(int v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Non-temporal 16-byte load for weights streamed exactly once.
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

}  // namespace jx
