// Decode regime (few tokens per expert): bandwidth-bound dequant-GEMV.
//
// A block owns one 32-row tile of one active expert's matrix (or two: gate
// and up) and every token routed to that expert; its waves split K.  The
// block first stages its tokens' activations (Q8_0 quants and block scales,
// or fp32 rows) in LDS, so the only global loads in the K loop are weight
// streams: the activation loads are issued before the first weight loads, and
// inside the loop activations come over the LDS path with its own counter, so
// a wave never waits on an HBM prefetch it does not need yet.  Weights run
// through a three-deep register rotation (units u+1 and u+2 in flight while u
// is consumed).  Lane (m = lane % 32, h = lane / 32) reads 16-byte chunks of
// row m; the 32 lanes of a half-wave read one contiguous 512-byte run of the
// tile layout, a wave load is 1 KB contiguous.  Products use v_dot4_i32_i8;
// integer block sums are exact and each is scaled once in fp32 (weight scale
// x activation scale) as in the reference's vec_dot_*_q8_0 kernels
// (src/quant.cpp:3307-3573); only the fp32 summation order differs.
//
// K-units (four 1 KB wave loads each, more for the five- and six-bit formats):
//   Q4_K  one 256-element super-block: 4 pair chunks + the 16-byte header
//   Q5_K  half a super-block (sub-block pairs 2s, 2s + 1 of super-block u / 2, s = u % 2): 2 pair
//         chunks, the header and the 16-byte chunk of fifth bits of half h
//   Q6_K  half a super-block (128 elements, four 32-blocks): lanes of half h take elements
//         16h..16h+15 of each block (sub-block 2r + h of block r): ql chunks h and 2 + h and qh
//         chunk 4 + h of that half, its 8 scales and d
//   Q4_0  eight 32-blocks: lanes of half h take the four blocks of parity h
//   Q5_0  four 32-blocks: lanes of half h take the two blocks of parity h, with their 32 fifth
//         bits (fp32 activations only)
//   Q8_0  four 32-blocks: lanes of half h take half h of each
#include <algorithm>
#include <vector>

#include "jxmoe_device.h"
#include "jxmoe_dispatch.h"
#include "jxmoe_kernels.h"

namespace jx {

// ------------------------------------------------------------ weight chunks
struct RawB {
    uint4 q[4];
    uint32_t d[4];  // fp16 bits of the block scales
};
struct RawQ4K {
    uint4 q[4];
    uint4 hd;  // d | dmin << 16, then the 12 scale bytes
};
struct RawQ5K {
    uint4 q[2];  // pair chunks 2s, 2s + 1
    uint4 hd;
    uint4 qh;    // qh bytes 16h..16h+15 shifted right by 4s: bit j of each byte = fifth bit of sub-block 4s + j
    int s;       // which half of the super-block
};
struct RawQ6K {
    uint4 q[3];  // of the unit's 128-element half: ql chunks h, 2 + h, then qh chunk 4 + h
    uint2 sc;    // the half's 8 int8 sub-block scales
    uint32_t d;  // fp16 bits of d
};
struct RawB5 {
    uint4 q[2];
    uint32_t d[2];
    uint32_t qh[2];
};

template <int TYPE>
struct Fmt;

// load(c, W, e, rt, u, m, h, ok): every lane issues the same loads whatever
// `ok` and the unit's extent; a unit that is not wanted (ok false) or a block
// past the matrix's K reads the zeroed pad instead (its bytes are never used).
template <>
struct Fmt<T_Q4_0> {
    using Raw = RawB;
    static constexpr int BPU = 8;  // 32-blocks per unit
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        const size_t b0 = (size_t)rt * W.nkb + (size_t)u * BPU + h;
        const uint8_t* qb = W.qs + e * W.qs_es;
        const uint8_t* sb = W.sc + e * W.sc_es;
        const int left = W.nkb - u * BPU - h;  // blocks 2i with 2i < left exist
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool v = ok && 2 * i < left;
            const size_t qo = ((b0 + 2 * i) * 32 + m) * 16, so = ((b0 + 2 * i) * 32 + m) * 2;
            c.q[i] = ld_stream16(v ? qb + qo : W.pad_qs + m * 16);
            c.d[i] = *reinterpret_cast<const uint16_t*>(v ? sb + so : W.pad_sc + m * 2);
        }
    }
};

template <>
struct Fmt<T_Q8_0> {
    using Raw = RawB;
    static constexpr int BPU = 4;
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        const size_t b0 = (size_t)rt * W.nkb + (size_t)u * BPU;
        const uint8_t* qb = W.qs + e * W.qs_es;
        const uint8_t* sb = W.sc + e * W.sc_es;
        const int left = W.nkb - u * BPU;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool v = ok && i < left;
            const size_t qo = (((b0 + i) * 2 + h) * 32 + m) * 16, so = ((b0 + i) * 32 + m) * 2;
            c.q[i] = ld_stream16(v ? qb + qo : W.pad_qs + m * 16);
            c.d[i] = *reinterpret_cast<const uint16_t*>(v ? sb + so : W.pad_sc + m * 2);
        }
    }
};

template <>
struct Fmt<T_Q4_K> {
    using Raw = RawQ4K;
    static constexpr int BPU = 1;
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        const size_t t = (size_t)rt * W.nkb + u;
        const uint8_t* qb = ok ? W.qs + e * W.qs_es + (t * 8 + h) * 512 : W.pad_qs;
        const uint8_t* hb = ok ? W.sc + e * W.sc_es + t * 512 : W.pad_sc;
#pragma unroll
        for (int p = 0; p < 4; ++p) c.q[p] = ld_stream16(qb + p * 1024 + m * 16);
        c.hd = ld_stream16(hb + m * 16);
    }
};

template <>
struct Fmt<T_Q5_0> {
    using Raw = RawB5;
    static constexpr int BPU = 4;
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        const size_t b0 = (size_t)rt * W.nkb + (size_t)u * BPU + h;
        const uint8_t* qb = W.qs + e * W.qs_es;
        const uint8_t* sb = W.sc + e * W.sc_es;
        const uint8_t* xb = W.ex + e * W.ex_es;
        const int left = W.nkb - u * BPU - h;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const bool v = ok && 2 * i < left;
            const size_t t = (b0 + 2 * i) * 32 + m;
            c.q[i] = ld_stream16(v ? qb + t * 16 : W.pad_qs + m * 16);
            c.d[i] = *reinterpret_cast<const uint16_t*>(v ? sb + t * 2 : W.pad_sc + m * 2);
            c.qh[i] = *reinterpret_cast<const uint32_t*>(v ? xb + t * 4 : W.pad_ex + m * 4);
        }
    }
};

// Units are halves of super-blocks (unit u: super-block u / 2, sub-blocks 4 (u % 2) .. + 3).
template <>
struct Fmt<T_Q5_K> {
    using Raw = RawQ5K;
    static constexpr int BPU = 1;
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        const size_t t = (size_t)rt * W.nkb + (u >> 1);
        c.s = u & 1;
        const uint8_t* qb = ok ? W.qs + e * W.qs_es + (t * 8 + 4 * c.s + h) * 512 : W.pad_qs;
        const uint8_t* hb = ok ? W.sc + e * W.sc_es + t * 512 : W.pad_sc;
        const uint8_t* xb = ok ? W.ex + e * W.ex_es + (t * 2 + h) * 512 : W.pad_ex;
#pragma unroll
        for (int p = 0; p < 2; ++p) c.q[p] = ld_stream16(qb + p * 1024 + m * 16);
        c.hd = ld_stream16(hb + m * 16);
        const uint4 v = ld_stream16(xb + m * 16);
        const int sh = 4 * c.s;
        c.qh = make_uint4(v.x >> sh, v.y >> sh, v.z >> sh, v.w >> sh);
    }
};

// Units are 128-element halves of super-blocks (unit u: super-block u / 2, half u % 2).
template <>
struct Fmt<T_Q6_K> {
    using Raw = RawQ6K;
    static constexpr int BPU = 1;
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        const size_t t = (size_t)rt * W.nkb + (u >> 1);
        const int n = u & 1;
        const uint8_t* qb = ok ? W.qs + e * W.qs_es + t * 6144 + n * 3072 : W.pad_qs;  // 6 chunks of 512 B per half
#pragma unroll
        for (int k = 0; k < 3; ++k) c.q[k] = ld_stream16(qb + (2 * k + h) * 512 + m * 16);
        c.sc = *reinterpret_cast<const uint2*>((ok ? W.sc + e * W.sc_es + t * 512 + 8 * n : W.pad_sc) + m * 16);
        c.d = *reinterpret_cast<const uint16_t*>((ok ? W.ex + e * W.ex_es + t * 64 : W.pad_ex) + m * 2);
    }
};

// Activation elements one GEMV unit covers.
template <int TYPE>
__host__ __device__ constexpr int dp_unit_elems() {
    return (TYPE == T_Q5_K || TYPE == T_Q6_K) ? 128 : (TYPE == T_Q4_K ? 256 : 32 * Fmt<TYPE>::BPU);
}

template <int TYPE>
__host__ __device__ constexpr int n_units(int nkb) {
    return (TYPE == T_Q6_K || TYPE == T_Q5_K) ? 2 * nkb : (nkb + Fmt<TYPE>::BPU - 1) / Fmt<TYPE>::BPU;
}

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    const uint32_t w = i < 4 ? v.y : (i < 8 ? v.z : v.w);
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// (scale, min) of sub-block j from a Q4_K header held in registers
// (get_scale_min_k4, src/quant.cpp:1107-1115).
__device__ __forceinline__ void hd_scale_min(const uint4& hd, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = byte_of(hd, j) & 63;
        mn = byte_of(hd, j + 4) & 63;
    } else {
        sc = (byte_of(hd, j + 4) & 0x0F) | ((byte_of(hd, j - 4) >> 6) << 4);
        mn = (byte_of(hd, j + 4) >> 4) | ((byte_of(hd, j) >> 6) << 4);
    }
}

// Byte k (0..7) of 8 bytes, sign-extended (the Q6_K int8 scales).
__device__ __forceinline__ int sbyte(const uint2& v, int k) {
    return (int)(int8_t)(uint8_t)((k < 4 ? v.x : v.y) >> (8 * (k & 3)));
}

__device__ __forceinline__ uint32_t comp(const uint4& v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }

// Q6_K, 32-block r (0..3) of a unit, this lane's 16 elements as four words of 4 q6 bytes shifted
// left by 2 (4 q6, 0..252): the low nibble from ql chunk q[r & 1] (high nibble when r >= 2), the
// two high bits from bits 2r, 2r + 1 of qh chunk q[2] (block_q6_K layout, src/quant.cpp:1389-1428).
__device__ __forceinline__ void q6_words(const RawQ6K& c, int r, uint32_t (&w)[4]) {
    const uint4 lo = c.q[r & 1], hi = c.q[2];
    const int sh = (r >> 1) * 4;
#pragma unroll
    for (int z = 0; z < 4; ++z) {
        const uint32_t l4 = (comp(lo, z) >> sh) & 0x0F0F0F0Fu;
        const uint32_t h2 = (comp(hi, z) >> (2 * r)) & 0x03030303u;
        w[z] = (l4 << 2) | (h2 << 6);
    }
}

// Q5_K: the 5-bit quants of the unit's sub-block j (0..3; 2p: low nibbles of chunk p, 2p + 1:
// high) for this lane's 16 elements, fifth bit from bit j of the lane's shifted qh bytes
// (dequantize_row_q5_K, src/quant.cpp:1345-1387).
__device__ __forceinline__ void q5k_words(const RawQ5K& c, int j, uint32_t (&w)[4]) {
    const uint4 v = c.q[j >> 1];
    const int sh = (j & 1) * 4;
#pragma unroll
    for (int z = 0; z < 4; ++z) w[z] = ((comp(v, z) >> sh) & 0x0F0F0F0Fu) | (((comp(c.qh, z) >> j) & 0x01010101u) << 4);
}

// (scale, min) of sub-blocks 4s .. 4s + 3 of a Q5_K header (constant-index unpacking, then a select
// on the unit's half s).
__device__ __forceinline__ void q5k_unit_scales(const uint4& hd, int s, int (&sc)[4], int (&mn)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int a0, b0, a1, b1;
        hd_scale_min(hd, k, a0, b0);
        hd_scale_min(hd, 4 + k, a1, b1);
        sc[k] = s ? a1 : a0;
        mn[k] = s ? b1 : b0;
    }
}

// Activations of one token group in LDS: Q8_0 quants [TB][K] and (scale,
// sum) [TB][K/32], or fp32 rows [TB][K].
struct ActLds {
    const int8_t* q;
    const float2* s;
    const float* f;
    int K;
};

__device__ __forceinline__ uint4 lds16(const int8_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Accumulate one K-unit of one weight row against up to TB token rows.
template <int TYPE, int TB>
__device__ __forceinline__ void unit_accum(const typename Fmt<TYPE>::Raw& c, const ActLds& A, int u, int h, int nt,
                                           int nkb, float* acc) {
    const int KB = A.K / 32;
    if constexpr (TYPE == T_Q4_0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = u * 8 + 2 * i + h;
            if (b < nkb) {
                const float dw = f16_to_f32(c.d[i] & 0xFFFFu);
                const uint32_t q[4] = {c.q[i].x, c.q[i].y, c.q[i].z, c.q[i].w};
                int ql[4], qh[4];
#pragma unroll
                for (int z = 0; z < 4; ++z) {
                    ql[z] = (int)(q[z] & 0x0F0F0F0Fu);
                    qh[z] = (int)((q[z] >> 4) & 0x0F0F0F0Fu);
                }
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    if (j < nt) {
                        const uint4 a0 = lds16(A.q + j * A.K + b * 32);
                        const uint4 a1 = lds16(A.q + j * A.K + b * 32 + 16);
                        const float2 s = A.s[j * KB + b];
                        int isum = sdot4(ql[0], (int)a0.x, 0);
                        isum = sdot4(ql[1], (int)a0.y, isum);
                        isum = sdot4(ql[2], (int)a0.z, isum);
                        isum = sdot4(ql[3], (int)a0.w, isum);
                        isum = sdot4(qh[0], (int)a1.x, isum);
                        isum = sdot4(qh[1], (int)a1.y, isum);
                        isum = sdot4(qh[2], (int)a1.z, isum);
                        isum = sdot4(qh[3], (int)a1.w, isum);
                        isum -= 8 * (int)s.y;  // weights are nibble - 8
                        acc[j] = __builtin_fmaf(dw * s.x, (float)isum, acc[j]);
                    }
                }
            }
        }
    } else if constexpr (TYPE == T_Q8_0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = u * 4 + i;
            if (b < nkb) {
                const float dw = f16_to_f32(c.d[i] & 0xFFFFu);
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    if (j < nt) {
                        const uint4 a = lds16(A.q + j * A.K + b * 32 + 16 * h);
                        const float2 s = A.s[j * KB + b];
                        int isum = sdot4((int)c.q[i].x, (int)a.x, 0);
                        isum = sdot4((int)c.q[i].y, (int)a.y, isum);
                        isum = sdot4((int)c.q[i].z, (int)a.z, isum);
                        isum = sdot4((int)c.q[i].w, (int)a.w, isum);
                        acc[j] = __builtin_fmaf(dw * s.x, (float)isum, acc[j]);
                    }
                }
            }
        }
    } else if constexpr (TYPE == T_Q6_K) {
        // vec_dot_q6_K_q8_0 (src/quant.cpp:3723-3818): per 32-block the exact integer sum
        // sc * sum((q6 - 32) * y) of this lane's sub-block, scaled by d * dy
        const float d = f16_to_f32(c.d & 0xFFFFu);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w[4];
            q6_words(c, j, w);
            int wv[4];
#pragma unroll
            for (int z = 0; z < 4; ++z) wv[z] = (int)(w[z] ^ 0x80808080u);  // 4 (q6 - 32) as int8
            const int sc = sbyte(c.sc, 2 * j + h);
            const int b = u * 4 + j;
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                if (t < nt) {
                    const uint4 a = lds16(A.q + t * A.K + b * 32 + 16 * h);
                    int is = sdot4(wv[0], (int)a.x, 0);
                    is = sdot4(wv[1], (int)a.y, is);
                    is = sdot4(wv[2], (int)a.z, is);
                    is = sdot4(wv[3], (int)a.w, is);
                    acc[t] = __builtin_fmaf(d * A.s[t * KB + b].x, (float)(sc * (is >> 2)), acc[t]);
                }
            }
        }
    } else {  // Q4_K (whole super-block units) / Q5_K (half super-block units: pairs 2s, 2s + 1)
        constexpr int NP = TYPE == T_Q5_K ? 2 : 4;
        const int bb = TYPE == T_Q5_K ? u * 4 : u * 8;  // the unit's first 32-block in K
        int usc[4], umn[4];
        if constexpr (TYPE == T_Q5_K) q5k_unit_scales(c.hd, c.s, usc, umn);
        const float d = f16_to_f32(c.hd.x & 0xFFFFu), dmin = f16_to_f32(c.hd.x >> 16);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            int s0, m0, s1, m1;
            if constexpr (TYPE == T_Q5_K) {
                s0 = usc[2 * p], m0 = umn[2 * p], s1 = usc[2 * p + 1], m1 = umn[2 * p + 1];
            } else {
                hd_scale_min(c.hd, 2 * p, s0, m0);
                hd_scale_min(c.hd, 2 * p + 1, s1, m1);
            }
            const float fs0 = d * (float)s0, fm0 = dmin * (float)m0;
            const float fs1 = d * (float)s1, fm1 = dmin * (float)m1;
            int ql[4], qh[4];
            if constexpr (TYPE == T_Q5_K) {
                uint32_t wl[4], wh[4];
                q5k_words(c, 2 * p, wl);
                q5k_words(c, 2 * p + 1, wh);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ql[i] = (int)wl[i];
                    qh[i] = (int)wh[i];
                }
            } else {
                const uint32_t q[4] = {c.q[p].x, c.q[p].y, c.q[p].z, c.q[p].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ql[i] = (int)(q[i] & 0x0F0F0F0Fu);
                    qh[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
                }
            }
            const int b0 = bb + 2 * p;
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j < nt) {
                    const uint4 a = lds16(A.q + j * A.K + b0 * 32 + 16 * h);
                    const uint4 b = lds16(A.q + j * A.K + (b0 + 1) * 32 + 16 * h);
                    const float2 sa = A.s[j * KB + b0], sb = A.s[j * KB + b0 + 1];
                    int ia = sdot4(ql[0], (int)a.x, 0);
                    ia = sdot4(ql[1], (int)a.y, ia);
                    ia = sdot4(ql[2], (int)a.z, ia);
                    ia = sdot4(ql[3], (int)a.w, ia);
                    int ib = sdot4(qh[0], (int)b.x, 0);
                    ib = sdot4(qh[1], (int)b.y, ib);
                    ib = sdot4(qh[2], (int)b.z, ib);
                    ib = sdot4(qh[3], (int)b.w, ib);
                    float v = acc[j];
                    v = __builtin_fmaf(fs0 * sa.x, (float)ia, v);
                    v = __builtin_fmaf(fs1 * sb.x, (float)ib, v);
                    if (h == 0) {  // min term once per sub-block: sum(y) over all 32 elements
                        v = __builtin_fmaf(-(fm0 * sa.x), sa.y, v);
                        v = __builtin_fmaf(-(fm1 * sb.x), sb.y, v);
                    }
                    acc[j] = v;
                }
            }
        }
    }
}

// One row's 32 (or 16) quants against fp32 activations from LDS: sum_i w_i * y_i as an fp32 fma
// chain, w_i = (float)(byte i of the words) + off.
template <int NW>
__device__ __forceinline__ float dot_f32_words(const uint32_t (&w)[NW], const float* y, float off) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(y + 4 * i);
        s = __builtin_fmaf((float)(w[i] & 0xFFu) + off, v.x, s);
        s = __builtin_fmaf((float)((w[i] >> 8) & 0xFFu) + off, v.y, s);
        s = __builtin_fmaf((float)((w[i] >> 16) & 0xFFu) + off, v.z, s);
        s = __builtin_fmaf((float)(w[i] >> 24) + off, v.w, s);
    }
    return s;
}

// Accumulate one K-unit of one weight row against up to TB fp32 activation rows (the reference's
// vec_dot_quant_f32 dots, src/quant.cpp:3269-3305: vec_dot_q4_0_f32 2780-2827, vec_dot_q8_0_f32
// 2829-2862, vec_dot_q4_K_f32 2910-3013, vec_dot_q5_K_f32 3069-3085, vec_dot_q6_K_f32 3087-3165,
// vec_dot_q5_0_f32 3232-3234): each block or sub-block's weights times y as an fp32 chain, scaled
// once.  K-quant rows of y are zero-padded to whole super-blocks, so a partial last super-block
// needs no masking; only the fp32 summation order differs from the reference.
template <int TYPE, int TB>
__device__ __forceinline__ void unit_accum_f32(const typename Fmt<TYPE>::Raw& c, const ActLds& A, int u, int h,
                                               int nt, int nkb, float* acc) {
    if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
        constexpr int NP = TYPE == T_Q5_K ? 2 : 4;  // Q5_K: half super-block units (pairs 2s, 2s + 1)
        const int e0 = TYPE == T_Q5_K ? u * 128 : u * 256;  // the unit's first element
        int usc[4], umn[4];
        if constexpr (TYPE == T_Q5_K) q5k_unit_scales(c.hd, c.s, usc, umn);
        const float d = f16_to_f32(c.hd.x & 0xFFFFu), dmin = f16_to_f32(c.hd.x >> 16);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            int s0, m0, s1, m1;
            if constexpr (TYPE == T_Q5_K) {
                s0 = usc[2 * p], m0 = umn[2 * p], s1 = usc[2 * p + 1], m1 = umn[2 * p + 1];
            } else {
                hd_scale_min(c.hd, 2 * p, s0, m0);
                hd_scale_min(c.hd, 2 * p + 1, s1, m1);
            }
            const float fs0 = d * (float)s0, fm0 = dmin * (float)m0;
            const float fs1 = d * (float)s1, fm1 = dmin * (float)m1;
            uint32_t q[4];  // Q4_K: the chunk's bytes (low nibble: sub-block 2p, high: 2p + 1)
            uint32_t q5[4]; // Q5_K: the fifth bits of the lane's 16 elements
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                q[i] = comp(c.q[p], i);
                if constexpr (TYPE == T_Q5_K) q5[i] = comp(c.qh, i) >> (2 * p);
            }
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j < nt) {
                    const float* ya = A.f + j * A.K + e0 + 64 * p + 16 * h;
                    const float* yb = ya + 32;
                    float sa = 0.0f, sb = 0.0f, ta = 0.0f, tb = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float4 va = *reinterpret_cast<const float4*>(ya + 4 * i);
                        const float4 vb = *reinterpret_cast<const float4*>(yb + 4 * i);
                        const float fa[4] = {va.x, va.y, va.z, va.w};
                        const float fb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
                        for (int z = 0; z < 4; ++z) {
                            uint32_t lo = (q[i] >> (8 * z)) & 15u, hi = (q[i] >> (8 * z + 4)) & 15u;
                            if constexpr (TYPE == T_Q5_K) {
                                lo |= ((q5[i] >> (8 * z)) & 1u) << 4;
                                hi |= ((q5[i] >> (8 * z + 1)) & 1u) << 4;
                            }
                            sa = __builtin_fmaf((float)lo, fa[z], sa);
                            sb = __builtin_fmaf((float)hi, fb[z], sb);
                            ta = ta + fa[z];
                            tb = tb + fb[z];
                        }
                    }
                    float v = acc[j];
                    v = __builtin_fmaf(fs0, sa, v);
                    v = __builtin_fmaf(-fm0, ta, v);
                    v = __builtin_fmaf(fs1, sb, v);
                    v = __builtin_fmaf(-fm1, tb, v);
                    acc[j] = v;
                }
                // one token's activations at a time in registers
                if constexpr (TB > 1) __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else if constexpr (TYPE == T_Q6_K) {
        const float d = f16_to_f32(c.d & 0xFFFFu);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            uint32_t w[4];
            q6_words(c, jb, w);
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = (w[i] >> 2) & 0x3F3F3F3Fu;  // q6
            const float ds = d * (float)sbyte(c.sc, 2 * jb + h);
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j < nt) {
                    const float* y = A.f + j * A.K + u * 128 + 32 * jb + 16 * h;
                    acc[j] = __builtin_fmaf(ds, dot_f32_words<4>(w, y, -32.0f), acc[j]);
                }
                if constexpr (TB > 1) __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else if constexpr (TYPE == T_Q8_0) {  // half h of each of the unit's four blocks
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = u * 4 + i;
            if (b < nkb) {
                const float dw = f16_to_f32(c.d[i] & 0xFFFFu);
                uint32_t w[4];
#pragma unroll
                for (int z = 0; z < 4; ++z) w[z] = comp(c.q[i], z) ^ 0x80808080u;  // q + 128
#pragma unroll
                for (int j = 0; j < TB; ++j)
                    if (j < nt) acc[j] = __builtin_fmaf(dw, dot_f32_words<4>(w, A.f + j * A.K + b * 32 + 16 * h, -128.0f), acc[j]);
            }
        }
    } else {  // Q4_0 / Q5_0: whole blocks of parity h
        constexpr int NB = Fmt<TYPE>::BPU / 2;  // blocks per lane
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int b = u * Fmt<TYPE>::BPU + 2 * i + h;
            if (b < nkb) {
                const float dw = f16_to_f32(c.d[i] & 0xFFFFu);
                const float off = TYPE == T_Q5_0 ? -16.0f : -8.0f;
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    if (j < nt) {
                        // the low nibbles (elements 0..15), then the high ones (16..31), one half's
                        // activations in registers at a time
                        float s2[2];
#pragma unroll
                        for (int hb = 0; hb < 2; ++hb) {
                            uint32_t w[4];
#pragma unroll
                            for (int z = 0; z < 4; ++z) {
                                w[z] = (comp(c.q[i], z) >> (4 * hb)) & 0x0F0F0F0Fu;
                                if constexpr (TYPE == T_Q5_0)  // fifth bit e of element e (dequantize_row_q5_0)
                                    w[z] |= ((((c.qh[i] >> (16 * hb + 4 * z)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
                            }
                            s2[hb] = dot_f32_words<4>(w, A.f + j * A.K + b * 32 + 16 * hb, off);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        acc[j] = __builtin_fmaf(dw, s2[0] + s2[1], acc[j]);
                    }
                }
            }
        }
    }
}

// (expert, first pair, pair count, first token) of a slot: one 16-byte load
// of the dispatch record, so the weight streams start one L2 round trip after
// the kernel does.
// With router logits instead of tables (few-token decode), every wave derives
// the record itself.
__device__ __forceinline__ int4 group_of(const Groups& g, int slot) {
    if (g.identity) {
        if (!g.chunk) return make_int4(0, 0, slot == 0 ? g.n_tok : 0, 0);
        const int p = slot * g.chunk;
        return make_int4(0, p, max(0, min(g.chunk, g.n_tok - p)), p);
    }
    if (g.logits) return small_group(g, slot);
    return g.slots[slot];
}

// Token of sorted pair p0 + i of a group (the first one is in its record).
__device__ __forceinline__ int token_of(const Groups& g, const int4& rec, int i) {
    if (g.identity) return rec.y + i;
    if (g.logits) return rec.w + i;  // n <= 2: a group of two holds tokens 0 and 1
    return i == 0 ? rec.w : g.pair_tok[rec.y + i];
}

// On the few-token path one extra block of the routed gate/up GEMV writes the
// dispatch tables (ids, probs, shared-gate scale, counts, offsets, slots, pair
// lists) while the others stream weights; the kernels after it read them.
__device__ void small_tail(const SmallTail& t, int tid) {
    static_assert(SMALL_GROUP_MAX_E <= 128, "two expert chunks");
    if (tid < 64) topk_dispatch_wave<2>(t.a, t.o, t.a.logits, t.a.shgate ? t.a.shscale : nullptr);
}

// LDS bytes of one token group's staged activations.
__host__ __device__ inline size_t act_lds_bytes(int TB, int K, bool f32) {
    return f32 ? (size_t)TB * K * sizeof(float) : (size_t)TB * K + (size_t)TB * (K / 32) * sizeof(float2);
}

// Activation staging into LDS, split so the global loads can be issued
// before a wave's first weight loads and written to LDS after them: issue()
// loads MQ 16-byte quant chunks and MS 8-byte (scale, sum) chunks per thread
// into registers, write() stores them.  Indices past the group's last chunk
// are clamped to it (the duplicate store writes the same bytes), so neither
// half branches and the LDS stores wait only for the staging loads, not for
// the weight loads issued after them.  Launchers guarantee
// nt * K <= 16 * MQ * NTH and nt * K <= 32 * MS * NTH.
template <int NTH, int MQ, int MS>
struct StageQ8 {
    uint4 vq[MQ];
    float2 vs[MS];
    template <typename RowFn>
    __device__ __forceinline__ void issue(const ActQ8& g, int nt, RowFn src_row, int tid) {
        const int K = g.K, KB = K / 32, cq = K / 16;
#pragma unroll
        for (int r = 0; r < MQ; ++r) {
            const int i = min(tid + r * NTH, nt * cq - 1);
            const int j = i / cq, c = i - j * cq;
            vq[r] = ld16(g.q + src_row(j) * K + c * 16);
        }
#pragma unroll
        for (int r = 0; r < MS; ++r) {
            const int i = min(tid + r * NTH, nt * KB - 1);
            const int j = i / KB, c = i - j * KB;
            vs[r] = g.s[src_row(j) * KB + c];
        }
    }
    // LDS layout: quants [TB][K], then (scale, sum) [TB][K/32]
    __device__ __forceinline__ void write(int K, int TB, int nt, int8_t* lds, int tid) {
        const int KB = K / 32, cq = K / 16;
        float2* ls = reinterpret_cast<float2*>(lds + TB * K);
#pragma unroll
        for (int r = 0; r < MQ; ++r) {
            const int i = min(tid + r * NTH, nt * cq - 1);
            *reinterpret_cast<uint4*>(lds + i * 16) = vq[r];  // row j = i / cq at j * K + 16 (i % cq)
        }
#pragma unroll
        for (int r = 0; r < MS; ++r) {
            const int i = min(tid + r * NTH, nt * KB - 1);
            ls[i] = vs[r];
        }
    }
};

template <int NTH, int MF>
struct StageF32 {
    float4 v[MF];
    template <typename RowFn>
    __device__ __forceinline__ void issue(const float* src, int ld, int K, int nt, RowFn src_row, int tid) {
        const int cq = K / 4;
#pragma unroll
        for (int r = 0; r < MF; ++r) {
            const int i = min(tid + r * NTH, nt * cq - 1);
            const int j = i / cq, c = i - j * cq;
            v[r] = *reinterpret_cast<const float4*>(src + src_row(j) * (size_t)ld + c * 4);
        }
    }
    __device__ __forceinline__ void write(float* lds, int nt, int K, int tid) {
        const int cq = K / 4;
#pragma unroll
        for (int r = 0; r < MF; ++r) {
            const int i = min(tid + r * NTH, nt * cq - 1);
            *reinterpret_cast<float4*>(lds + i * 4) = v[r];
        }
    }
};

// Q8_0 of one 32-row block of h held by lanes 0..31 (quantize_row_q8_0).
__device__ __forceinline__ void store_q8_block(float hv, int m, bool writer, ActQ8& hq, size_t row, int blk) {
    float2 sv;
    const int q = q8_block_vals(hv, sv);
    if (writer) {
        hq.q[row * hq.K + blk * 32 + m] = (int8_t)q;
        if (m == 0) hq.s[row * (hq.K / 32) + blk] = sv;
    }
}

#ifndef JX_GEMV_DEPTH
#define JX_GEMV_DEPTH 2
#endif

// The K loop of one wave over units lo, lo + stride, ... < nu of one or two
// weight matrices: two register sets alternate, so unit u+stride is in flight
// while u is consumed (and u+2*stride is issued right after).  pre() runs
// after the first two units' loads are issued (it finishes the activation
// staging and synchronizes the block, so every wave calls it).
template <int TYPE, int NMAT, typename Pre, typename Acc>
__device__ __forceinline__ void kloop(const QMat& W0, const QMat& W1, int e, int rt, int lo, int nu, int stride, int m,
                                      int h, Pre&& pre, Acc&& accum) {
    using F = Fmt<TYPE>;
    typename F::Raw a0, a1, b0, b1;
    // loads are issued unconditionally (units past the end read the pad), so
    // every path through the loop has the same loads in flight and each wait
    // covers only the unit about to be consumed
    auto ld = [&](typename F::Raw& r0, typename F::Raw& r1, int u) {
        F::load(r0, W0, e, rt, u, m, h, u < nu);
        if constexpr (NMAT == 2) F::load(r1, W1, e, rt, u, m, h, u < nu);
    };
    int u = lo;
#if JX_GEMV_DEPTH == 1
    ld(a0, a1, u);
    pre();
    for (; u < nu; u += stride) {
        accum(a0, a1, u);
        ld(a0, a1, u + stride);
    }
    (void)b0;
    (void)b1;
#else
    ld(a0, a1, u);
    ld(b0, b1, u + stride);
    pre();
    for (; u < nu; u += 2 * stride) {
        accum(a0, a1, u);
        ld(a0, a1, u + 2 * stride);
        if (u + stride >= nu) break;
        accum(b0, b1, u + stride);
        ld(b0, b1, u + 3 * stride);
    }
#endif
}

// kloop with DEPTH units in flight per wave (a ring of register sets): the same units in the same
// order, so the same sums as kloop's.  pre() runs after the first DEPTH units' loads are issued.
template <int TYPE, int DEPTH, typename Pre, typename Acc>
__device__ __forceinline__ void kloop_d(const QMat& W, int e, int rt, int lo, int nu, int stride, int m, int h,
                                        Pre&& pre, Acc&& accum) {
    using F = Fmt<TYPE>;
    typename F::Raw r[DEPTH];
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) F::load(r[i], W, e, rt, lo + i * stride, m, h, lo + i * stride < nu);
    pre();
    for (int u = lo; u < nu; u += DEPTH * stride) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            const int ui = u + i * stride;
            if (ui >= nu) break;  // wave-uniform
            accum(r[i], ui);
            const int un = ui + DEPTH * stride;
            F::load(r[i], W, e, rt, un, m, h, un < nu);
        }
    }
}

// Resident waves per SIMD the GEMVs are compiled for (single-token groups:
// <= 128 VGPRs, every block of a decode step resident at once with enough
// 1 KB weight loads in flight per CU to cover HBM latency).  The single-token
// gate/up GEMV also comes compiled for 3 waves per SIMD (<= 168 VGPRs, no
// spills), taken when the whole grid is resident at that occupancy.
#ifndef JX_GEMV_TB4_WPS
#define JX_GEMV_TB4_WPS 2
#endif
#define GEMV_WAVES_PER_SIMD(TB) ((TB) == 1 ? 4 : JX_GEMV_TB4_WPS)
// The single-token down GEMV's fp32-activation dots of Q8_0 and Q6_K (matrices under 8 rows; Q6_K with
// K % 256 != 0) do not fit 128 VGPRs with two units in flight; they run at 2 waves per SIMD (one 8-wave
// block per CU).
template <int TYPE, int TB, bool F32ACT>
constexpr int down_wps() {
    return TB == 1 && F32ACT && (TYPE == T_Q8_0 || TYPE == T_Q6_K) ? 2 : GEMV_WAVES_PER_SIMD(TB);
}

// Gate + up + SwiGLU (matmul_swiglu_quant_f32, src/quant.cpp:3970-4009) and
// the Q8_0 quantization of the result for the down projection
// (matmul_quant_f32's quantize_row_q8_0, 3908-3914).  The first half of the
// waves streams the gate tile, the second half the up tile.  F32ACT: the
// fp32-activation dots (types without a Q8_0 form at this K) over xf rows of
// xf_ld floats, zero-padded to whole K-units, staged straight into LDS.
template <int TYPE, int TB, int WAVES, int WPS = GEMV_WAVES_PER_SIMD(TB), bool F32ACT = false>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WPS)))
k_gemv_gateup(QMat G, QMat U, ActQ8 xq, const float* xf, int xf_ld, Groups grp, ActQ8 hq, float* hf, int hf_ld,
              SmallTail tail) {
    constexpr int HW = WAVES / 2;  // waves per matrix
    extern __shared__ __align__(16) int8_t smem[];
    __shared__ float red[WAVES][TB][32];
    // grid: row tile fastest over the slots, then the one tail block
    if (tail.on && blockIdx.x == gridDim.x - 1) {  // the extra block: dispatch tables only
        small_tail(tail, threadIdx.x);
        return;
    }
    const int rt = blockIdx.x % G.nrt;
    const int4 rec = group_of(grp, blockIdx.x / G.nrt);
    const int e = rec.x, p0 = rec.y, cnt = rec.z;
    if (cnt == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    const int mat = wave / HW, kw = wave % HW;
    const QMat& W = mat ? U : G;
    const int K = F32ACT ? xf_ld : xq.K;
    const int nu = n_units<TYPE>(G.nkb);
    const ActLds A{smem, reinterpret_cast<const float2*>(smem + TB * K), reinterpret_cast<const float*>(smem), K};
    for (int tb0 = 0; tb0 < cnt; tb0 += TB) {
        const int nt = min(TB, cnt - tb0);
        if (tb0) __syncthreads();  // previous group's LDS reads are done
        auto src = [&](int j) { return (size_t)token_of(grp, rec, tb0 + j); };
        StageQ8<WAVES * 64, TB == 1 ? 4 : 8, TB == 1 ? 2 : 4> sg;
        if constexpr (!F32ACT) sg.issue(xq, nt, src, tid);
        float acc[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) acc[j] = 0.0f;
        kloop<TYPE, 1>(
            W, W, e, rt, kw, nu, HW, m, h,
            [&] {
                if constexpr (F32ACT) {
                    float* lf = reinterpret_cast<float*>(smem);
                    for (int i = tid; i < nt * (K / 4); i += WAVES * 64) {
                        const int j = i / (K / 4), c4 = i - j * (K / 4);
                        *reinterpret_cast<float4*>(lf + j * K + 4 * c4) =
                            *reinterpret_cast<const float4*>(xf + src(j) * (size_t)xf_ld + 4 * c4);
                    }
                } else {
                    sg.write(K, TB, nt, smem, tid);
                }
                __syncthreads();
            },
            [&](const typename Fmt<TYPE>::Raw& c, const typename Fmt<TYPE>::Raw&, int u) {
                if constexpr (F32ACT)
                    unit_accum_f32<TYPE, TB>(c, A, u, h, nt, G.nkb, acc);
                else
                    unit_accum<TYPE, TB>(c, A, u, h, nt, G.nkb, acc);
            });
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            acc[j] += __shfl_xor(acc[j], 32, 64);
            if (h == 0) red[wave][j][m] = acc[j];
        }
        __syncthreads();
        if (wave == 0) {
            for (int j = 0; j < nt; ++j) {
                float g = 0.0f, u = 0.0f;
#pragma unroll
                for (int w = 0; w < HW; ++w) {
                    g += red[w][j][m];
                    u += red[HW + w][j][m];
                }
                const float hv = gated(g, u, G.act);
                const size_t row = (size_t)(p0 + tb0 + j);
                store_q8_block(hv, m, h == 0 && hq.q != nullptr, hq, row, rt);
                if (hf && h == 0) hf[row * (size_t)hf_ld + rt * 32 + m] = hv;
            }
        }
    }
}

// Down projection into y[pair][rows].
template <int TYPE, int TB, int WAVES, bool F32ACT>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(down_wps<TYPE, TB, F32ACT>())))
k_gemv_down(QMat D, ActQ8 hq, const float* hf, int hf_ld, Groups grp, float* y, CombineOut comb) {
    extern __shared__ __align__(16) int8_t smem[];
    __shared__ float red[WAVES][TB][32];
    const int rt = blockIdx.x % D.nrt;  // grid: row tile fastest over the slots
    const int4 rec = group_of(grp, blockIdx.x / D.nrt);
    const int e = rec.x, p0 = rec.y, cnt = rec.z;
    if (cnt == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    const int K = F32ACT ? hf_ld : hq.K;
    const int nu = n_units<TYPE>(D.nkb);
    const ActLds A{smem, reinterpret_cast<const float2*>(smem + TB * K), reinterpret_cast<const float*>(smem), K};
    for (int tb0 = 0; tb0 < cnt; tb0 += TB) {
        const int nt = min(TB, cnt - tb0);
        if (tb0) __syncthreads();
        auto src = [&](int j) { return (size_t)(p0 + tb0 + j); };
        StageQ8<WAVES * 64, TB == 1 ? 4 : 8, TB == 1 ? 2 : 4> sq;
        StageF32<WAVES * 64, TB == 1 ? 2 : 4> sf;
        if constexpr (F32ACT)
            sf.issue(hf, hf_ld, K, nt, src, tid);
        else
            sq.issue(hq, nt, src, tid);
        float acc[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) acc[j] = 0.0f;
        kloop<TYPE, 1>(
            D, D, e, rt, wave, nu, WAVES, m, h,
            [&] {
                if constexpr (F32ACT)
                    sf.write(reinterpret_cast<float*>(smem), nt, K, tid);
                else
                    sq.write(K, TB, nt, smem, tid);
                __syncthreads();
            },
            [&](const typename Fmt<TYPE>::Raw& c, const typename Fmt<TYPE>::Raw&, int u) {
                if constexpr (F32ACT)
                    unit_accum_f32<TYPE, TB>(c, A, u, h, nt, D.nkb, acc);
                else
                    unit_accum<TYPE, TB>(c, A, u, h, nt, D.nkb, acc);
            });
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            acc[j] += __shfl_xor(acc[j], 32, 64);
            if (h == 0) red[wave][j][m] = acc[j];
        }
        __syncthreads();
        if (wave == 0 && h == 0) {
            for (int j = 0; j < nt; ++j) {
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) s += red[w][j][m];
                if (D.valid_rows && rt * 32 + m >= D.valid_rows) continue;  // padding rows of a single matrix
                if (comb.out) {  // folded combine: out[token] += p * y (CombineOut)
                    const int t = token_of(grp, rec, tb0 + j);
                    float p = 0.0f;
                    for (int q = 0; q < comb.k; ++q)
                        if (comb.ids[(size_t)t * comb.k + q] == e) p = comb.probs[(size_t)t * comb.k + q];
                    atomicAdd(comb.out + (size_t)t * D.rows + rt * 32 + m, p * s);
                } else {
                    y[(size_t)(p0 + tb0 + j) * D.rows + rt * 32 + m] = s;
                }
            }
        }
    }
}

// ---------------------------------------------------------------- several tokens per expert
// Multi-token GEMV on the matrix cores: one v_mfma_i32_32x32x32_i8 per 32-element block gives the
// exact integer block sums of up to MX_NT tokens against the 32 rows of a tile.  Operand B is the
// weight tile as the GEMV layout holds it (lane (m, h): 16 elements of row m, half h of the block;
// Q4_0 lanes load their block whole and take their nibble half); operand A holds the tokens' Q8_0
// quants (lane (t, g): token t, half g; tokens past the group give zeros).  Lane (m, g) receives
// D[token 8(r/4) + 4g + r%4][row m] in register r, r < 8.  Each sum is scaled in fp32 by its row's
// weight scale and its token's activation scale: the integer block sums and scale products of
// vec_dot_*_q8_0 (src/quant.cpp:3307-3573); Q4_0's -8 offset is in the weight operand (q - 8); only
// the fp32 summation order differs.  The weights are read once per MX_NT tokens instead of once per
// 4, and the scaling is a few instructions per (row, token, block) instead of the GEMV's per-token
// dot products.  The tokens' (scale, sum) pairs are staged in LDS per pass; quants and weights
// stream one unit ahead.
constexpr int MX_NT = 16;  // tokens per pass: D registers 0..7

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));

template <int TYPE>
struct Mx;

// Q4_K: one super-block per unit (the GEMV's unit); sub-block 2p = low nibbles of chunk p, 2p+1 = high.
template <>
struct Mx<T_Q4_K> {
    static constexpr int BPU = 8;
    using Raw = RawQ4K;
    __device__ static int units(const QMat& W) { return W.nkb; }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        Fmt<T_Q4_K>::load(c, W, e, rt, u, m, h, ok);
    }
    __device__ static uint4 bop(const Raw& c, int j, int) {
        const uint4 v = c.q[j >> 1];
        const int sh = (j & 1) * 4;
        return make_uint4((v.x >> sh) & 0x0F0F0F0Fu, (v.y >> sh) & 0x0F0F0F0Fu, (v.z >> sh) & 0x0F0F0F0Fu,
                          (v.w >> sh) & 0x0F0F0F0Fu);
    }
    // row scale and min scale of sub-block j (get_scale_min_k4, src/quant.cpp:1107-1115)
    __device__ static void scales(const Raw& c, int j, float& rs, float& rmin) {
        int sc, mn;
        hd_scale_min(c.hd, j, sc, mn);
        rs = f16_to_f32(c.hd.x) * (float)sc;
        rmin = -f16_to_f32(c.hd.x >> 16) * (float)mn;
    }
    // all eight at once, four bytes per operation: scales 0-3 and mins 0-3 are the low six bits of
    // scale bytes 0-3 and 4-7; scale (min) 4 + i takes the low (high) nibble of byte 8 + i and, as bits
    // 4-5, the top two bits of byte i (4 + i) -- the same values as scales(), in the same products
    struct Scl {
        float rs[8], rmin[8];
    };
    __device__ static Scl prep(const Raw& c) {
        const uint32_t y = c.hd.y, z = c.hd.z, w = c.hd.w;
        const uint32_t sc0 = y & 0x3F3F3F3Fu, mn0 = z & 0x3F3F3F3Fu;
        const uint32_t sc1 = (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
        const uint32_t mn1 = ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
        const float d = f16_to_f32(c.hd.x), dm = f16_to_f32(c.hd.x >> 16);
        Scl s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s.rs[i] = d * (float)((sc0 >> (8 * i)) & 0xFFu);
            s.rs[4 + i] = d * (float)((sc1 >> (8 * i)) & 0xFFu);
            s.rmin[i] = -dm * (float)((mn0 >> (8 * i)) & 0xFFu);
            s.rmin[4 + i] = -dm * (float)((mn1 >> (8 * i)) & 0xFFu);
        }
        return s;
    }
    __device__ static void scale(const Scl& s, const Raw&, int j, float& rs, float& rmin) {
        rs = s.rs[j];
        rmin = s.rmin[j];
    }
};

// Q5_K: as Q4_K with the fifth bits (values 0..31, exact in int8).
template <>
struct Mx<T_Q5_K> {
    static constexpr int BPU = 4;  // half super-block units
    using Raw = RawQ5K;
    __device__ static int units(const QMat& W) { return 2 * W.nkb; }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        Fmt<T_Q5_K>::load(c, W, e, rt, u, m, h, ok);
    }
    __device__ static uint4 bop(const Raw& c, int j, int) {
        uint32_t w[4];
        q5k_words(c, j, w);
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
    __device__ static void scales(const Raw& c, int j, float& rs, float& rmin) {
        int a0, b0, a1, b1;  // sub-block 4s + j (j is a constant after unrolling, s is not)
        hd_scale_min(c.hd, j, a0, b0);
        hd_scale_min(c.hd, 4 + j, a1, b1);
        rs = f16_to_f32(c.hd.x) * (float)(c.s ? a1 : a0);
        rmin = -f16_to_f32(c.hd.x >> 16) * (float)(c.s ? b1 : b0);
    }
    struct Scl {};
    __device__ static Scl prep(const Raw&) { return Scl{}; }
    __device__ static void scale(const Scl&, const Raw& c, int j, float& rs, float& rmin) { scales(c, j, rs, rmin); }
};

// Q6_K: lane (m, h) holds sub-block 2j + h of block j (the GEMV's split, half super-block units)
// as 4 (q6 - 32) in int8; the two sub-blocks of a block have their own scales, so each takes one
// MFMA with the other half's operand zeroed.
template <>
struct Mx<T_Q6_K> {
    static constexpr int BPU = 4;
    using Raw = RawQ6K;
    __device__ static int units(const QMat& W) { return 2 * W.nkb; }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        Fmt<T_Q6_K>::load(c, W, e, rt, u, m, h, ok);
    }
    __device__ static uint4 bop(const Raw& c, int j, int) {
        uint32_t w[4];
        q6_words(c, j, w);
        return make_uint4(w[0] ^ 0x80808080u, w[1] ^ 0x80808080u, w[2] ^ 0x80808080u, w[3] ^ 0x80808080u);
    }
    __device__ static void scales(const Raw& c, int, float& rs, float& rmin) {
        rs = f16_to_f32(c.d & 0xFFFFu);
        rmin = 0.0f;
    }
    struct Scl {};
    __device__ static Scl prep(const Raw&) { return Scl{}; }
    __device__ static void scale(const Scl&, const Raw& c, int j, float& rs, float& rmin) { scales(c, j, rs, rmin); }
};

// Q8_0: four blocks per unit, the GEMV layout (lane half h holds half h of each block).
template <>
struct Mx<T_Q8_0> {
    static constexpr int BPU = 4;
    using Raw = RawB;
    __device__ static int units(const QMat& W) { return (W.nkb + BPU - 1) / BPU; }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        Fmt<T_Q8_0>::load(c, W, e, rt, u, m, h, ok);
    }
    __device__ static uint4 bop(const Raw& c, int j, int) { return c.q[j]; }
    __device__ static void scales(const Raw& c, int j, float& rs, float& rmin) {
        rs = f16_to_f32(c.d[j] & 0xFFFFu);
        rmin = 0.0f;
    }
    struct Scl {};
    __device__ static Scl prep(const Raw&) { return Scl{}; }
    __device__ static void scale(const Scl&, const Raw& c, int j, float& rs, float& rmin) { scales(c, j, rs, rmin); }
};

// Q4_0: four blocks per unit; both lane halves load a row's whole block (16 bytes) and take the low
// (elements 0..15) or high (16..31) nibbles, as the signed bytes q - 8 (so the block sum is the
// reference's integer sum with no correction).
template <>
struct Mx<T_Q4_0> {
    static constexpr int BPU = 4;
    using Raw = RawB;
    __device__ static int units(const QMat& W) { return (W.nkb + BPU - 1) / BPU; }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int, bool ok) {
        const uint8_t* qb = W.qs + e * W.qs_es;
        const uint8_t* sb = W.sc + e * W.sc_es;
        const size_t b0 = (size_t)rt * W.nkb + (size_t)u * BPU;
        const int left = W.nkb - u * BPU;
#pragma unroll
        for (int i = 0; i < BPU; ++i) {
            const bool v = ok && i < left;
            c.q[i] = ld_stream16(v ? qb + ((b0 + i) * 32 + m) * 16 : W.pad_qs + m * 16);
            c.d[i] = *reinterpret_cast<const uint16_t*>(v ? sb + ((b0 + i) * 32 + m) * 2 : W.pad_sc + m * 2);
        }
    }
    // nibble n of half h -> the signed byte 16 (n - 8): the nibble moved to the byte's high half (h = 0
    // shifts the low nibbles up, h = 1 masks the high ones in place), and flipping bit 7 subtracts 128
    // without a borrow into the next byte: three operations per word instead of the four of n - 8.  The
    // block sums come out 16 times the exact ones (|16 sum| < 2^20, exact in fp32), and the scale below
    // carries the exact 1/16.
    __device__ static uint32_t s16(uint32_t v, int sh) { return ((v << sh) & 0xF0F0F0F0u) ^ 0x80808080u; }
    __device__ static uint4 bop(const Raw& c, int j, int h) {
        const uint4 v = c.q[j];
        const int sh = 4 - h * 4;
        return make_uint4(s16(v.x, sh), s16(v.y, sh), s16(v.z, sh), s16(v.w, sh));
    }
    __device__ static void scales(const Raw& c, int j, float& rs, float& rmin) {
        rs = f16_to_f32(c.d[j] & 0xFFFFu) * 0.0625f;
        rmin = 0.0f;
    }
    struct Scl {};
    __device__ static Scl prep(const Raw&) { return Scl{}; }
    __device__ static void scale(const Scl&, const Raw& c, int j, float& rs, float& rmin) { scales(c, j, rs, rmin); }
};

// Gate + up (+ SwiGLU + Q8_0 of h) or down for up to MX_NT tokens per pass of one expert's row tile.
// Gate/up: the first half of the waves streams the gate tile, the second half the up tile.
// Waves per SIMD the form is compiled for: 3 where it fits 168 VGPRs without spills (Q4_0, Q8_0,
// Q5_K), 2 for Q4_K and Q6_K (measured: Qwen3-shaped 32-token gate/up 66.7 -> 60.9 us; the
// Qwen1.5-shaped routed gate/up at 64 tokens 116 -> 100 us).
template <int TYPE>
constexpr int mx_wps() { return (TYPE == T_Q4_K || TYPE == T_Q6_K) ? 2 : 3; }

template <int TYPE, bool GATEUP, int WAVES>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(mx_wps<TYPE>())))
k_gemv_mx(QMat W0, QMat W1, ActQ8 act, Groups grp, ActQ8 hq, float* hf, int hf_ld, float* y, SmallTail tail) {
    using X = Mx<TYPE>;
    using Raw = typename X::Raw;
    constexpr int BPU = X::BPU;
    constexpr int HW = GATEUP ? WAVES / 2 : WAVES;  // waves per matrix
    extern __shared__ __align__(16) float2 msc[];   // [block][MX_NT]: (scale, sum) of each token
    __shared__ float red[WAVES][MX_NT / 2][64];
    // grid: row tile fastest over the slots, then (gate/up) the one tail block
    if (GATEUP && tail.on && blockIdx.x == gridDim.x - 1) {  // the extra block: dispatch tables only
        small_tail(tail, threadIdx.x);
        return;
    }
    const int rt = blockIdx.x % W0.nrt;
    const int4 rec = group_of(grp, blockIdx.x / W0.nrt);
    const int e = rec.x, p0 = rec.y, cnt = rec.z;
    if (cnt == 0 || (grp.cold_max > 0 && cnt >= grp.cold_max)) return;  // (the GEMMs take that expert)
    const int tid = threadIdx.x, lane = tid & 63, m = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar unit loop and branches
    const int kw = wave % HW;
    const QMat& W = (GATEUP && wave >= HW) ? W1 : W0;
    const int K = act.K, KB = K / 32;
    const int nu = X::units(W0);
    for (int tb0 = 0; tb0 < cnt; tb0 += MX_NT) {
        const int nt = min(MX_NT, cnt - tb0);
        if (tb0) __syncthreads();  // the previous pass is done with msc and red
        // the first two units' weights go out first: they need only the expert, while the activations wait
        // on the token list (the pair table) and the scales on both
        Raw wa, wb;
        uint4 aa[BPU], ab[BPU];
        X::load(wa, W, e, rt, kw, m, h, kw < nu);
        X::load(wb, W, e, rt, kw + HW, m, h, kw + HW < nu);
        auto src = [&](int i) -> size_t {
            return GATEUP ? (size_t)token_of(grp, rec, tb0 + i) : (size_t)(p0 + tb0 + i);
        };
        const bool hi8 = nt > 8;  // tokens 8.. present: D registers 4-7 carry results
        // A row of this lane: token m; lanes past the pass's tokens read token 0 (their D rows are dropped)
        const int8_t* arow = act.q + src(m < nt ? m : 0) * (size_t)K + 16 * h;
        float acc[MX_NT / 2];
#pragma unroll
        for (int r = 0; r < MX_NT / 2; ++r) acc[r] = 0.0f;
        auto lda = [&](uint4(&a)[BPU], int u) {
#pragma unroll
            for (int j = 0; j < BPU; ++j)  // in bounds past the end too (their results are never used)
                a[j] = ld16(arow + (size_t)min(u * BPU + j, KB - 1) * 32);
        };
        // two units in flight per wave, as the GEMV's K loop: their activations go out before the scales
        // are staged
        int u = kw;
        lda(aa, u);
        lda(ab, u + HW);
        // the tokens' (scale, sum) per block into LDS, MX_STAGE loads in flight per thread
        constexpr int MX_STAGE = 2;
        for (int i0 = tid; i0 < KB * MX_NT; i0 += MX_STAGE * WAVES * 64) {
            float2 v[MX_STAGE];
#pragma unroll
            for (int q = 0; q < MX_STAGE; ++q) {
                const int i = i0 + q * WAVES * 64, b = i / MX_NT, t = i - b * MX_NT;
                v[q] = (i < KB * MX_NT && t < nt) ? act.s[src(t) * KB + b] : make_float2(0.0f, 0.0f);
            }
#pragma unroll
            for (int q = 0; q < MX_STAGE; ++q) {
                const int i = i0 + q * WAVES * 64;
                // Q4_K / Q5_K: scale * sum (min term); the others do not read the sum
                if (i < KB * MX_NT)
                    msc[i] = make_float2(v[q].x, (TYPE == T_Q4_K || TYPE == T_Q5_K) ? v[q].x * v[q].y : v[q].y);
            }
        }
        auto ld = [&](Raw& w, uint4(&a)[BPU], int u) {
            X::load(w, W, e, rt, u, m, h, u < nu);
#pragma unroll
            for (int j = 0; j < BPU; ++j)  // in bounds past the end too (their results are never used)
                a[j] = ld16(arow + (size_t)min(u * BPU + j, KB - 1) * 32);
        };
        auto accum = [&](const Raw& w, const uint4(&a)[BPU], int u) {
            const auto scl = X::prep(w);
#pragma unroll
            for (int j = 0; j < BPU; ++j) {
                const int b = u * BPU + j;
                if (!is_kquant(TYPE) && b >= KB) break;  // wave-uniform; K-quant units are whole super-blocks
                const uint4 bw = X::bop(w, j, h);
                v16i_t D, D2;
                if constexpr (TYPE == T_Q6_K) {
                    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
                    D = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a[j]),
                                                              __builtin_bit_cast(v4i_t, h ? z : bw), v16i_t{}, 0, 0, 0);
                    D2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a[j]),
                                                               __builtin_bit_cast(v4i_t, h ? bw : z), v16i_t{}, 0, 0, 0);
                } else {
                    D = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a[j]),
                                                              __builtin_bit_cast(v4i_t, bw), v16i_t{}, 0, 0, 0);
                }
                float rs, rmin;
                X::scale(scl, w, j, rs, rmin);
                // tokens of registers 0-3: 4h..4h+3, of 4-7: 8+4h..11+4h (only when the pass has them)
                const float4* sp = reinterpret_cast<const float4*>(msc + b * MX_NT + 4 * h);
                const float4 s0 = sp[0], s1 = sp[1];
                const float4 s2 = hi8 ? sp[4] : s0, s3 = hi8 ? sp[5] : s1;
                const float sx[8] = {s0.x, s0.z, s1.x, s1.z, s2.x, s2.z, s3.x, s3.z};
                const float sy[8] = {s0.y, s0.w, s1.y, s1.w, s2.y, s2.w, s3.y, s3.w};
#pragma unroll
                for (int r = 0; r < MX_NT / 2; ++r) {
                    if (r >= 4 && !hi8) break;  // pass-uniform
                    if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
                        acc[r] = __builtin_fmaf(rs * sx[r], (float)D[r], acc[r]);
                        acc[r] = __builtin_fmaf(rmin, sy[r], acc[r]);
                    } else if constexpr (TYPE == T_Q6_K) {  // D = 4 sum((q6 - 32) y) per sub-block, exact
                        const int isum = sbyte(w.sc, 2 * j) * (D[r] >> 2) + sbyte(w.sc, 2 * j + 1) * (D2[r] >> 2);
                        acc[r] = __builtin_fmaf(rs * sx[r], (float)isum, acc[r]);
                    } else {
                        acc[r] = __builtin_fmaf(rs * sx[r], (float)D[r], acc[r]);
                    }
                }
            }
        };
        __syncthreads();  // msc staged
        for (; u < nu; u += 2 * HW) {
            accum(wa, aa, u);
            ld(wa, aa, u + 2 * HW);
            if (u + HW >= nu) break;
            accum(wb, ab, u + HW);
            ld(wb, ab, u + 3 * HW);
        }
#pragma unroll
        for (int r = 0; r < MX_NT / 2; ++r) red[wave][r][lane] = acc[r];
        __syncthreads();
        // result register r holds tokens 4h + r (r < 4) and 8 + 4h + r - 4 (r >= 4): only the registers whose
        // lane-half-0 token exists carry results; each is finished by one wave, the waves in turn
        const int nr = nt > 8 ? 4 + min(4, nt - 8) : min(4, nt);
        for (int r = wave; r < nr; r += WAVES) {  // wave-uniform
            const int t = (r < 4 ? 4 * h + r : 8 + 4 * h + (r - 4));
            float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
            for (int w = 0; w < HW; ++w) v0 += red[w][r][lane];
            const size_t row = (size_t)(p0 + tb0 + t);
            if constexpr (GATEUP) {
#pragma unroll
                for (int w = 0; w < HW; ++w) v1 += red[HW + w][r][lane];
                const float hv = gated(v0, v1, W0.act);
                store_q8_block(hv, m, t < nt && hq.q != nullptr, hq, row, rt);
                if (hf && t < nt) hf[row * (size_t)hf_ld + rt * 32 + m] = hv;
            } else {
                if (t < nt) y[row * W0.rows + rt * 32 + m] = v0;
            }
        }
    }
}

// Several row tiles per block (k_gemv_mxt): gate + up (+ SwiGLU + Q8_0 of h) or down for up to MX_NT
// tokens per pass of MR row tiles of one expert, as k_gemv_mx computes them.  A block stages its group's
// tokens once per pass for all its tiles; each wave walks its units (kw, kw + HW, ...) in order and, per
// unit, takes the unit's products for every tile against the same activation operands, reloading each
// tile's weight registers with that tile's next unit right after its products: MR units in flight per
// wave, and the activations read once per unit.  (One tile per block leaves a ~74 KB Q4_K gate/up tile
// behind a serial prologue of dependent loads -- slot record, token list, scales -- and an epilogue:
// blocks lived ~15 us for a few us of streaming.)  Launches with many (group, tile) items take it;
// launches with few (a dense shared expert) keep one tile per block, whose blocks fill more CUs.
// Measured at 32 tokens, weights from HBM: DeepSeek-V2-Lite-shaped routed Q4_K gate/up 89.5 -> 62.2 us
// (three tiles), Mixtral-shaped 184.6 -> 125.6 us; Qwen1.5-shaped Q4_0 at 64 tokens 85.8 -> 81.5 us and
// its down 43.5 -> 39.2 us (two tiles).  Q6_K and Q8_0 gate/up stay at one tile (Q8_0: 55.0 us against
// 59.3 at two tiles, Qwen3-shaped 32 tokens).
constexpr int MX_MR_MIN_ITEMS = 1024;
template <int TYPE, bool GATEUP>
constexpr int mx_mr_max() {
    return (TYPE == T_Q6_K || (TYPE == T_Q8_0 && GATEUP)) ? 1 : (TYPE == T_Q4_K || TYPE == T_Q5_K || (TYPE == T_Q4_0 && GATEUP)) ? 3 : 2;
}
// Static LDS of one k_gemv_mxt block: the MR tiles' per-wave partial sums.
template <int WAVES, int MR>
constexpr size_t mx_red_bytes() { return (size_t)MR * WAVES * (MX_NT / 2) * 64 * sizeof(float); }

template <int TYPE, bool GATEUP, int WAVES, int MR>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2)))
k_gemv_mxt(QMat W0r, QMat W1r, ActQ8 actr, Groups grpr, ActQ8 hqr, float* hfr, int hf_ldr, float* yr, SmallTail tail,
           SharedPart sh) {
    using X = Mx<TYPE>;
    using Raw = typename X::Raw;
    constexpr int BPU = X::BPU;
    constexpr int HW = GATEUP ? WAVES / 2 : WAVES;  // waves per matrix
    extern __shared__ __align__(16) float2 msc[];   // [block][MX_NT]: (scale, sum) of each token
    __shared__ float red[MR][WAVES][MX_NT / 2][64];
    static_assert(sizeof(red) == mx_red_bytes<WAVES, MR>(), "red");
    // grid: chunks of MR row tiles fastest over the slots, then the shared expert's blocks (chunks fastest
    // over its token groups, then its K parts), then (gate/up) the one tail block
    if (GATEUP && tail.on && blockIdx.x == gridDim.x - 1) {  // the extra block: dispatch tables only
        small_tail(tail, threadIdx.x);
        return;
    }
    const bool shb = sh.slots > 0 && (int)blockIdx.x >= sh.blocks0;  // block-uniform
    // the shared blocks' matrices: the routed ones with the shared bases (expert 0), rows and K (selecting
    // whole structs by reference made the Q4_K gate/up spill ~1900 VGPRs)
    QMat W0 = W0r, W1 = W1r;
    if (shb) {
        W0.qs = sh.g.qs;
        W0.sc = sh.g.sc;
        W0.ex = sh.g.ex;
        W0.nrt = sh.g.nrt;
        W0.rows = sh.g.rows;
        W0.nkb = sh.g.nkb;
        W0.act = sh.g.act;
        W1.qs = sh.u.qs;
        W1.sc = sh.u.sc;
        W1.ex = sh.u.ex;
    }
    const ActQ8& act = (shb && !GATEUP) ? sh.hq : actr;
    const Groups& grp = shb ? sh.grp : grpr;
    const int bi = shb ? (int)blockIdx.x - sh.blocks0 : (int)blockIdx.x;
    const int nch = (W0.nrt + MR - 1) / MR;
    const int rt0 = (bi % nch) * MR, nj = min(MR, W0.nrt - rt0);  // tiles rt0 .. rt0 + nj - 1
    const int gi = bi / nch, slot = shb ? gi % sh.slots : gi, kp = shb ? gi / sh.slots : 0;
    const int4 rec = group_of(grp, slot);
    const int e = rec.x, p0 = rec.y, cnt = rec.z;
    if (cnt == 0 || (grp.cold_max > 0 && cnt >= grp.cold_max)) return;  // (the GEMMs take that expert)
    const int tid = threadIdx.x, lane = tid & 63, m = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar unit loop and branches
    const int kw = wave % HW;
    const QMat& W = (GATEUP && wave >= HW) ? W1 : W0;
    const int K = act.K, KB = K / 32;
    // units ulo .. nu - 1 (a shared down's K part p: the p-th range of upp units), blocks kb0 .. kb1 - 1
    const int nua = X::units(W0), upp = (nua + sh.kparts - 1) / sh.kparts;
    const int ulo = (shb && !GATEUP) ? kp * upp : 0, nu = (shb && !GATEUP) ? min(nua, ulo + upp) : nua;
    const int kb0 = ulo * BPU, kb1 = min(KB, nu * BPU);
    ActQ8 hq = shb ? sh.hq : hqr;
    float* const hf = shb ? sh.hf : hfr;
    const int hf_ld = shb ? sh.hf_ld : hf_ldr;
    float* const y = shb ? sh.y + (size_t)kp * sh.grp.n_tok * W0.rows : yr;
    // one pass of up to MX_NT tokens.  R: result registers per lane, a compile-time switch (as a runtime
    // one it branched around single LDS reads and moves).  Token t of the pass sits in A row
    // 4 (t / R) + t % R for R <= 4 (8: rows t), so that lane-half h holds tokens hR .. hR + R - 1 in
    // D registers 0 .. R - 1: passes of at most 2 / 4 tokens scale 1 / 2 registers per block, not 4
    auto pass = [&](int tb0, int nt, auto rc) {
        constexpr int R = decltype(rc)::value;
        constexpr bool HI8 = R == 8;
        constexpr int NREG = R == 8 ? 8 : R;
        // every tile's first unit goes out first: the weights need only the expert, while the activations
        // wait on the token list (the pair table) and the scales on both (tiles past the matrix load the
        // last one; their results are dropped)
        Raw w[MR];
#pragma unroll
        for (int j = 0; j < MR; ++j) X::load(w[j], W, e, min(rt0 + j, W0.nrt - 1), ulo + kw, m, h, ulo + kw < nu);
        uint4 aa[BPU], ab[BPU];
        auto src = [&](int i) -> size_t {
            return GATEUP ? (size_t)token_of(grp, rec, tb0 + i) : (size_t)(p0 + tb0 + i);
        };
        // the token lookups of both the staging (below) and the A rows go out together
        static_assert((WAVES * 64) % MX_NT == 0, "one token per thread");
        const int tk = tid % MX_NT;
        const size_t srow = tk < nt ? src(tk) * (size_t)KB : 0;
        // A row m of this lane: its token (rows that hold none, and tokens past the pass, read token 0:
        // their D rows are dropped)
        const int ta = R >= 4 ? m : ((m & 3) < R && m < 8 ? (m >> 2) * R + (m & 3) : 0);
        const int8_t* arow = act.q + src(ta < nt ? ta : 0) * (size_t)K + 16 * h;
        float acc[MR][MX_NT / 2];
#pragma unroll
        for (int j = 0; j < MR; ++j)
#pragma unroll
            for (int r = 0; r < MX_NT / 2; ++r) acc[j][r] = 0.0f;
        auto lda = [&](uint4(&a)[BPU], int u) {
#pragma unroll
            for (int j = 0; j < BPU; ++j)  // in bounds past the end too (their results are never used)
                a[j] = ld16(arow + (size_t)min(u * BPU + j, KB - 1) * 32);
        };
        // the first two units' activations go out before the scales are staged
        int u = ulo + kw;
        lda(aa, u);
        lda(ab, u + HW);
        // the tokens' (scale, sum) of blocks kb0 .. kb1 - 1 into LDS, entry 16 (b - kb0) + t: a thread's
        // entries all belong to its token t = tid % 16 (the thread count is a multiple of 16), whose row was
        // looked up once above, and MX_STAGE scale loads are in flight per thread (one round at K <= 4096
        // for 4 waves: the token list and the scales are two dependent round trips, not one per entry group)
        constexpr int MX_STAGE = 4;
        const int nsc = (kb1 - kb0) * MX_NT;
        for (int i0 = tid; i0 < nsc; i0 += MX_STAGE * WAVES * 64) {
            float2 v[MX_STAGE];
#pragma unroll
            for (int q = 0; q < MX_STAGE; ++q) {
                const int i = i0 + q * WAVES * 64, b = kb0 + i / MX_NT;
                v[q] = (i < nsc && tk < nt) ? act.s[srow + b] : make_float2(0.0f, 0.0f);
            }
#pragma unroll
            for (int q = 0; q < MX_STAGE; ++q) {
                const int i = i0 + q * WAVES * 64;
                // Q4_K / Q5_K: scale * sum (min term); the others do not read the sum
                if (i < nsc)
                    msc[i] = make_float2(v[q].x, (TYPE == T_Q4_K || TYPE == T_Q5_K) ? v[q].x * v[q].y : v[q].y);
            }
        }
        // one unit of one tile: per 32-block, the integer block sums of the pass's tokens on the matrix core,
        // scaled into ac; block j + 1's products issue before block j's scaling, and nothing moves across a
        // block (unhindered, the scheduler hoists every product of the tiles' units ahead of the scaling,
        // 16 result registers each, and spills)
        auto mfma = [&](const Raw& wr, const uint4(&a)[BPU], int j, v16i_t& D, v16i_t& D2) {
            const uint4 bw = X::bop(wr, j, h);
            if constexpr (TYPE == T_Q6_K) {
                const uint4 z = make_uint4(0u, 0u, 0u, 0u);
                D = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a[j]),
                                                          __builtin_bit_cast(v4i_t, h ? z : bw), v16i_t{}, 0, 0, 0);
                D2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a[j]),
                                                           __builtin_bit_cast(v4i_t, h ? bw : z), v16i_t{}, 0, 0, 0);
            } else {
                D = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i_t, a[j]),
                                                          __builtin_bit_cast(v4i_t, bw), v16i_t{}, 0, 0, 0);
            }
        };
        // the tokens' (scale, sum) of block b for the pass's result registers: registers 0-3 hold tokens
        // 4h..4h+3, 4-7 hold 8+4h..11+4h (R = 8); hR..hR+R-1 (R <= 4)
        auto ldsx = [&](int b, float(&sx)[8], float(&sy)[8]) {
            if constexpr (R >= 4) {
                const float4* sp = reinterpret_cast<const float4*>(msc + (b - kb0) * MX_NT + 4 * h);
                const float4 s0 = sp[0], s1 = sp[1];
                const float4 s2 = HI8 ? sp[4] : s0, s3 = HI8 ? sp[5] : s1;
                const float ux[8] = {s0.x, s0.z, s1.x, s1.z, s2.x, s2.z, s3.x, s3.z};
                const float uy[8] = {s0.y, s0.w, s1.y, s1.w, s2.y, s2.w, s3.y, s3.w};
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    sx[r] = ux[r];
                    sy[r] = uy[r];
                }
            } else if constexpr (R == 2) {
                const float4 s0 = *reinterpret_cast<const float4*>(msc + (b - kb0) * MX_NT + 2 * h);
                sx[0] = s0.x;
                sy[0] = s0.y;
                sx[1] = s0.z;
                sy[1] = s0.w;
            } else {
                const float2 s0 = msc[(b - kb0) * MX_NT + h];
                sx[0] = s0.x;
                sy[0] = s0.y;
            }
        };
        auto accum = [&](const Raw& wr, const uint4(&a)[BPU], int u, float(&ac)[MX_NT / 2]) {
            const auto scl = X::prep(wr);
            // the unit's blocks in range: K-quant units are whole super-blocks; the others end at KB
            const int nbk = is_kquant(TYPE) ? BPU : min(BPU, KB - u * BPU);  // wave-uniform
            // PIPE: block j + 1's product and its tokens' scales go out before block j's scaling, so that
            // neither the matrix core's latency nor the LDS read sits between one block's scaling and the
            // next (left to itself, the scheduler issued the product after the scaling).  Not Q4_K, whose
            // gate/up then spilled.
            constexpr bool PIPE = TYPE != T_Q4_K;
            v16i_t D[2], D2[2];
            float sxb[2][8], syb[2][8];
            mfma(wr, a, 0, D[0], D2[0]);
            if constexpr (PIPE) ldsx(u * BPU, sxb[0], syb[0]);
#pragma unroll
            for (int j = 0; j < BPU; ++j) {
                if (j >= nbk) break;
                if (j + 1 < BPU && j + 1 < nbk) {
                    mfma(wr, a, j + 1, D[(j + 1) & 1], D2[(j + 1) & 1]);
                    if constexpr (PIPE) ldsx(u * BPU + j + 1, sxb[(j + 1) & 1], syb[(j + 1) & 1]);
                }
                if constexpr (PIPE) __builtin_amdgcn_sched_barrier(0);
                else ldsx(u * BPU + j, sxb[j & 1], syb[j & 1]);
                const v16i_t& Dj = D[j & 1];
                const v16i_t& D2j = D2[j & 1];
                const float(&sx)[8] = sxb[j & 1];
                const float(&sy)[8] = syb[j & 1];
                float rs, rmin;
                X::scale(scl, wr, j, rs, rmin);
#pragma unroll
                for (int r = 0; r < MX_NT / 2; ++r) {
                    if (r >= NREG) break;
                    if constexpr (TYPE == T_Q4_K || TYPE == T_Q5_K) {
                        ac[r] = __builtin_fmaf(rs * sx[r], (float)Dj[r], ac[r]);
                        ac[r] = __builtin_fmaf(rmin, sy[r], ac[r]);
                    } else if constexpr (TYPE == T_Q6_K) {  // D = 4 sum((q6 - 32) y) per sub-block, exact
                        const int isum = sbyte(wr.sc, 2 * j) * (Dj[r] >> 2) + sbyte(wr.sc, 2 * j + 1) * (D2j[r] >> 2);
                        ac[r] = __builtin_fmaf(rs * sx[r], (float)isum, ac[r]);
                    } else {
                        ac[r] = __builtin_fmaf(rs * sx[r], (float)Dj[r], ac[r]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // unit u's products for every tile, each tile's registers reloaded with its next unit right after
        // (past the last unit: the padding)
        auto unit = [&](const uint4(&a)[BPU], int u) {
#pragma unroll
            for (int j = 0; j < MR; ++j) {
                accum(w[j], a, u, acc[j]);
                X::load(w[j], W, e, min(rt0 + j, W0.nrt - 1), u + HW, m, h, u + HW < nu);
            }
        };
        __syncthreads();  // msc staged
        for (; u < nu; u += 2 * HW) {
            unit(aa, u);
            lda(aa, u + 2 * HW);
            if (u + HW >= nu) break;
            unit(ab, u + HW);
            lda(ab, u + 3 * HW);
        }
#pragma unroll
        for (int j = 0; j < MR; ++j)
#pragma unroll
            for (int r = 0; r < NREG; ++r) red[j][wave][r][lane] = acc[j][r];
        __syncthreads();
        // result register r holds tokens 4h + r (r < 4) and 8 + 4h + r - 4 (r >= 4) (R = 8), hR + r (R <= 4):
        // only the registers whose lane-half-0 token exists carry results; each (tile, register) is finished
        // by one wave, the waves in turn
        const int nr = R == 8 ? 4 + min(4, nt - 8) : min(R, nt);
        for (int q = wave; q < nj * nr; q += WAVES) {  // wave-uniform
            const int j = q / nr, r = q - j * nr, rt = rt0 + j;
            const int t = R == 8 ? (r < 4 ? 4 * h + r : 8 + 4 * h + (r - 4)) : h * R + r;
            float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
            for (int w = 0; w < HW; ++w) v0 += red[j][w][r][lane];
            const size_t row = (size_t)(p0 + tb0 + t);
            if constexpr (GATEUP) {
#pragma unroll
                for (int w = 0; w < HW; ++w) v1 += red[j][HW + w][r][lane];
                const float hv = gated(v0, v1, W0.act);
                store_q8_block(hv, m, t < nt && hq.q != nullptr, hq, row, rt);
                if (hf && t < nt) hf[row * (size_t)hf_ld + rt * 32 + m] = hv;
            } else {
                if (t < nt) y[row * W0.rows + rt * 32 + m] = v0;
            }
        }
    };
    for (int tb0 = 0; tb0 < cnt; tb0 += MX_NT) {
        const int nt = min(MX_NT, cnt - tb0);
        if (tb0) __syncthreads();  // the previous pass is done with msc and red
        if (nt > 8) {
            pass(tb0, nt, std::integral_constant<int, 8>{});
        } else if constexpr (TYPE == T_Q4_0) {
            // (Qwen1.5-shaped 16 / 64 tokens 106.4 / 137.2 -> 104.1 / 135.4 us; with the other formats'
            // passes the Q4_K gate/up spilled and ran slower, Q8_0 gained nothing)
            if (nt > 4) pass(tb0, nt, std::integral_constant<int, 4>{});
            else if (nt > 2) pass(tb0, nt, std::integral_constant<int, 2>{});
            else pass(tb0, nt, std::integral_constant<int, 1>{});
        } else {
            pass(tb0, nt, std::integral_constant<int, 4>{});
        }
    }
}

// ---------------------------------------------------------------- fp32-activation down, several tokens
// A down projection whose h has no Q8_0 form (Q5_0, or a K-quant whose d_ff is not a multiple of 256)
// takes the reference's fp32-activation dots (vec_dot_quant_f32, src/quant.cpp:3269-3305).  With a few
// tokens per expert (batched decode) it ran on the down GEMM's 64-pair tiles.  Here, as in k_gemv_mxt:
// MR row tiles of one expert per block, the pass's tokens staged once, each wave walking its units with
// one unit per tile in flight.  The tokens' operand is h's matrix-core hi form (fp16(h * 2^-E), E per
// token, k_f32_to_acth: relative error <= 2^-12 per value, as the down GEMM's), staged in LDS; the
// weights enter two v_mfma_f32_32x32x16_f16 per 32-block as exact small integers (Q4_K q, Q5_0 q - 16),
// and each block's fp32 sums are scaled by the row's block scale (Q4_K: plus the min term from the
// block's exact fp32 sum of h * 2^-E); 2^E at the end.
template <int TYPE>
struct Mh;

template <>
struct Mh<T_Q4_K> {  // super-block units, the GEMV layout of Mx<T_Q4_K>
    using X = Mx<T_Q4_K>;
    using Raw = X::Raw;
    using Scl = X::Scl;
    static constexpr int BPU = X::BPU;
    static constexpr bool MIN = true;
    static constexpr float C0 = -1024.0f;  // operand q
    __device__ static int units(const QMat& W) { return X::units(W); }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int h, bool ok) {
        X::load(c, W, e, rt, u, m, h, ok);
    }
    __device__ static uint4 bop(const Raw& c, int j, int h) { return X::bop(c, j, h); }
    __device__ static Scl prep(const Raw& c) { return X::prep(c); }
    __device__ static void scale(const Scl& s, const Raw& c, int j, float& rs, float& rmin) { X::scale(s, c, j, rs, rmin); }
};

template <>
struct Mh<T_Q5_0> {  // four blocks per unit; both lane halves load a row's whole block and take their half
    struct Raw {
        uint4 q[4];
        uint32_t d[4];
        uint32_t qh[4];
    };
    struct Scl {};
    static constexpr int BPU = 4;
    static constexpr bool MIN = false;
    static constexpr float C0 = -1040.0f;  // operand q5 - 16
    __device__ static int units(const QMat& W) { return (W.nkb + BPU - 1) / BPU; }
    __device__ static void load(Raw& c, const QMat& W, int e, int rt, int u, int m, int, bool ok) {
        const uint8_t* qb = W.qs + e * W.qs_es;
        const uint8_t* sb = W.sc + e * W.sc_es;
        const uint8_t* xb = W.ex + e * W.ex_es;
        const size_t b0 = (size_t)rt * W.nkb + (size_t)u * BPU;
        const int left = W.nkb - u * BPU;
#pragma unroll
        for (int i = 0; i < BPU; ++i) {
            const bool v = ok && i < left;
            const size_t t = (b0 + i) * 32 + m;
            c.q[i] = ld_stream16(v ? qb + t * 16 : W.pad_qs + m * 16);
            c.d[i] = *reinterpret_cast<const uint16_t*>(v ? sb + t * 2 : W.pad_sc + m * 2);
            c.qh[i] = *reinterpret_cast<const uint32_t*>(v ? xb + t * 4 : W.pad_ex + m * 4);
        }
    }
    // elements 16h .. 16h + 15: nibble half h of the 16 quant bytes, fifth bits 16h .. 16h + 15
    // (dequantize_row_q5_0, src/quant.cpp:1585-1600)
    __device__ static uint4 bop(const Raw& c, int j, int h) {
        const uint4 v = c.q[j];
        const uint32_t hb = c.qh[j] >> (16 * h);
        const int sh = 4 * h;
        return make_uint4(((v.x >> sh) & 0x0F0F0F0Fu) | (spread4(hb) << 4), ((v.y >> sh) & 0x0F0F0F0Fu) | (spread4(hb >> 4) << 4),
                          ((v.z >> sh) & 0x0F0F0F0Fu) | (spread4(hb >> 8) << 4),
                          ((v.w >> sh) & 0x0F0F0F0Fu) | (spread4(hb >> 12) << 4));
    }
    __device__ static Scl prep(const Raw&) { return Scl{}; }
    __device__ static void scale(const Scl&, const Raw& c, int j, float& rs, float& rmin) {
        rs = f16_to_f32(c.d[j] & 0xFFFFu);
        rmin = 0.0f;
    }
};

// Row tiles per block and waves per block of the fp32-activation multi-token down.
template <int TYPE>
constexpr int mxh_mr() { return TYPE == T_Q5_0 ? 2 : 3; }  // Q5_0: three units of 24 registers spill
constexpr int MXH_WAVES = 4;
// Dynamic LDS of one block: the staged tokens (fp16 rows of K + 8) and, for K-quants, the blocks' sums.
__host__ __device__ inline size_t mxh_lds(int K, bool kq, int ntp = MX_NT) {
    return (size_t)ntp * (K + 8) * 2 + (kq ? (size_t)(K / 32) * ntp * sizeof(float) : 0);
}

// NTP: tokens per pass, 16 or 8 (8: half the staged rows and no registers for tokens 8-15, so the build fits
// 3 waves per SIMD; groups of more tokens take more passes)
template <int TYPE, int WAVES, int MR, int NTP>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(2)))
k_gemv_mxh(QMat W, ActH hin, Groups grp, float* y) {
    using X = Mh<TYPE>;
    using Raw = typename X::Raw;
    constexpr int BPU = X::BPU;
    constexpr int NTH = WAVES * 64;
    extern __shared__ __align__(16) uint8_t mxh_lds_base[];
    __shared__ float red[MR][WAVES][MX_NT / 2][64];
    __shared__ float spe[MX_NT];
    const int nch = (W.nrt + MR - 1) / MR;
    const int rt0 = (int)(blockIdx.x % nch) * MR, nj = min(MR, W.nrt - rt0);  // tiles rt0 .. rt0 + nj - 1
    const int4 rec = group_of(grp, blockIdx.x / nch);
    const int e = rec.x, p0 = rec.y, cnt = rec.z;
    if (cnt == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, m = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = hin.K, KB = K / 32, KH = hin.KH, AS = K + 8;
    _Float16* As = reinterpret_cast<_Float16*>(mxh_lds_base);                  // [NTP][AS]: h * 2^-E
    float* Ss = reinterpret_cast<float*>(mxh_lds_base + (size_t)NTP * AS * 2);  // [KB][NTP]: sums
    const int nu = X::units(W);
    const h2v c1 = h2v{(_Float16)1.0f, (_Float16)1.0f}, c0 = h2v{(_Float16)X::C0, (_Float16)X::C0};
    auto pass = [&](int tb0, int nt, auto hi8c) {
        constexpr bool HI8 = decltype(hi8c)::value;
        // every tile's first unit goes out first
        Raw w[MR];
#pragma unroll
        for (int j = 0; j < MR; ++j) X::load(w[j], W, e, min(rt0 + j, W.nrt - 1), wave, m, h, wave < nu);
        // the tokens' rows of the hi form (zero rows past the pass), four 16-byte loads in flight per thread
        const size_t row0 = (size_t)(p0 + tb0);
        const int c8 = K / 8;
        for (int i0 = tid; i0 < NTP * c8; i0 += 4 * NTH) {
            uint4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = i0 + q * NTH, t = i / c8, k = 8 * (i - t * c8);
                v[q] = (i < NTP * c8 && t < nt)
                           ? *reinterpret_cast<const uint4*>(hin.hl + (row0 + t) * (size_t)KH * 256 + (k >> 7) * 256 + (k & 127))
                           : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int i = i0 + q * NTH, t = i / c8, k = 8 * (i - t * c8);
                if (i < NTP * c8) *reinterpret_cast<uint4*>(As + t * AS + k) = v[q];
            }
        }
        if (tid < MX_NT) spe[tid] = tid < nt ? hin.pe[(row0 + tid) * KH] : 0.0f;
        if constexpr (X::MIN) {
            // each block's fp32 sum of h * 2^-E from its three exact bf16 pieces
            for (int i = tid; i < KB * NTP; i += NTH) {
                const int b = i / NTP, t = i - b * NTP;
                float s = 0.0f;
                if (t < nt) {
                    const uint16_t* xp = hin.xm + (row0 + t) * (size_t)hin.KU * 24 + (b >> 3) * 24 + (b & 7);
                    s = (__uint_as_float((uint32_t)xp[0] << 16) + __uint_as_float((uint32_t)xp[8] << 16)) +
                        __uint_as_float((uint32_t)xp[16] << 16);
                }
                Ss[i] = s;
            }
        }
        __syncthreads();
        float acc[MR][MX_NT / 2];
#pragma unroll
        for (int j = 0; j < MR; ++j)
#pragma unroll
            for (int r = 0; r < MX_NT / 2; ++r) acc[j][r] = 0.0f;
        // A rows: token m % NTP (rows NTP-31 repeat 0..NTP-1; their D rows are not used)
        const _Float16* arow = As + (m & (NTP - 1)) * AS + 16 * h;
        for (int u = wave; u < nu; u += WAVES) {
#pragma unroll
            for (int j = 0; j < MR; ++j) {
                const auto scl = X::prep(w[j]);
#pragma unroll
                for (int jb = 0; jb < BPU; ++jb) {
                    const int b = u * BPU + jb;
                    if (!is_kquant(TYPE) && b >= KB) break;  // wave-uniform
                    const uint4 bw = X::bop(w[j], jb, h);
                    const h8 b0 = cvt8(bw.x, bw.y, 0xFFFFFFFFu, 0u, c1, c0), b1 = cvt8(bw.z, bw.w, 0xFFFFFFFFu, 0u, c1, c0);
                    const h8 a0 = *reinterpret_cast<const h8*>(arow + b * 32), a1 = *reinterpret_cast<const h8*>(arow + b * 32 + 8);
                    v16f D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, v16f{}, 0, 0, 0);
                    D = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, D, 0, 0, 0);
                    float rs, rmin;
                    X::scale(scl, w[j], jb, rs, rmin);
                    // tokens of registers 0-3: 4h..4h+3, of 4-7: 8+4h..11+4h
                    float sy[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    if constexpr (X::MIN) {
                        const float4 s0 = *reinterpret_cast<const float4*>(Ss + b * NTP + 4 * h);
                        const float4 s1 = HI8 ? *reinterpret_cast<const float4*>(Ss + b * NTP + 8 + 4 * h) : s0;
                        sy[0] = s0.x; sy[1] = s0.y; sy[2] = s0.z; sy[3] = s0.w;
                        sy[4] = s1.x; sy[5] = s1.y; sy[6] = s1.z; sy[7] = s1.w;
                    }
#pragma unroll
                    for (int r = 0; r < MX_NT / 2; ++r) {
                        if (r >= 4 && !HI8) break;
                        acc[j][r] = __builtin_fmaf(rs, D[r], acc[j][r]);
                        if constexpr (X::MIN) acc[j][r] = __builtin_fmaf(rmin, sy[r], acc[j][r]);
                    }
                    __builtin_amdgcn_sched_barrier(0);  // one block's products at a time (16 result registers)
                }
                X::load(w[j], W, e, min(rt0 + j, W.nrt - 1), u + WAVES, m, h, u + WAVES < nu);
            }
        }
#pragma unroll
        for (int j = 0; j < MR; ++j)
#pragma unroll
            for (int r = 0; r < MX_NT / 2; ++r) red[j][wave][r][lane] = acc[j][r];
        __syncthreads();
        const int nr = nt > 8 ? 4 + min(4, nt - 8) : min(4, nt);
        for (int q = wave; q < nj * nr; q += WAVES) {  // wave-uniform
            const int j = q / nr, r = q - j * nr, rt = rt0 + j;
            const int t = (r < 4 ? 4 * h + r : 8 + 4 * h + (r - 4));
            float v0 = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < WAVES; ++w2) v0 += red[j][w2][r][lane];
            if (t < nt) y[(row0 + t) * W.rows + rt * 32 + m] = v0 * spe[t];
        }
    };
    for (int tb0 = 0; tb0 < cnt; tb0 += NTP) {
        const int nt = min(NTP, cnt - tb0);
        if (tb0) __syncthreads();  // the previous pass is done with the staged tokens, spe and red
        if constexpr (NTP > 8) {
            if (nt > 8) pass(tb0, nt, std::integral_constant<bool, true>{});
            else pass(tb0, nt, std::integral_constant<bool, false>{});
        } else {
            pass(tb0, nt, std::integral_constant<bool, false>{});
        }
    }
}

#ifndef JX_GEMV_GATEUP_WAVES
#define JX_GEMV_GATEUP_WAVES 4
#endif
#ifndef JX_GEMV_DOWN_WAVES
#define JX_GEMV_DOWN_WAVES 8
#endif
constexpr int GATEUP_WAVES = JX_GEMV_GATEUP_WAVES;
constexpr int DOWN_WAVES = JX_GEMV_DOWN_WAVES;

// Largest K one token group of TB rows stages (the StageQ8 / StageF32
// register slots: 16 * MQ * NTH quant bytes, 32 * MS * NTH block scales,
// 4 * MF * NTH floats).
int gemv_max_k(bool gateup, int tb, bool f32) {
    const int nth = 64 * (gateup ? GATEUP_WAVES : DOWN_WAVES);
    if (f32 && gateup) return (144 * 1024 / 4) / (tb <= 1 ? 1 : 4) / 256 * 256;  // staged straight into LDS
    if (f32) return (tb <= 1 ? 2 : 4) * 4 * nth / (tb <= 1 ? 1 : 4);
    const int mq = tb <= 1 ? 4 : 8, ms = tb <= 1 ? 2 : 4, rows = tb <= 1 ? 1 : 4;
    return std::min(16 * mq * nth, 32 * ms * nth) / rows;
}

// Dynamic LDS above the default 64 KB needs the kernel's opt-in (a refusal
// surfaces as the launch's error).
template <typename Kern>
static void lds_optin(Kern k, size_t bytes) {
    if (bytes > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)bytes);
}

// Compute units of the current device (cached per device).
static int num_cus() {
    static int cached[64] = {0};
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

template <int TYPE>
static bool gateup_q8(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots, int tb, ActQ8 hq,
                      float* hf, int hf_ld, dim3 grid, hipStream_t st, const SmallTail& tail, SharedPart* sh);

template <int TYPE>
static bool gateup_t(const QMat& g, const QMat& u, const ActQ8& xq, const float* xf, int xf_ld, const Groups& grp,
                     int slots, int tb, ActQ8 hq, float* hf, hipStream_t st, const SmallTail& tail, SharedPart* sh) {
    dim3 grid(g.nrt * slots + (tail.on ? 1 : 0));
    const int hf_ld = ((g.rows + 255) / 256) * 256;
    if (xf) {  // fp32 activations: one token, or groups of 4
        const int rows = tb <= 1 ? 1 : 4;
        const size_t lds = act_lds_bytes(rows, xf_ld, true);
        auto go = [&](auto kern) {
            lds_optin(kern, lds);
            hipLaunchKernelGGL(kern, grid, dim3(GATEUP_WAVES * 64), lds, st, g, u, xq, xf, xf_ld, grp, hq, hf, hf_ld,
                               tail);
        };
        if (rows == 1) go(k_gemv_gateup<TYPE, 1, GATEUP_WAVES, 2, true>);
        else go(k_gemv_gateup<TYPE, 4, GATEUP_WAVES, 2, true>);
        return false;
    }
    if constexpr (TYPE != T_Q5_0) return gateup_q8<TYPE>(g, u, xq, grp, slots, tb, hq, hf, hf_ld, grid, st, tail, sh);
    return false;
}

// The Q8_0-activation forms (not for Q5_0).
template <int TYPE>
static bool gateup_q8(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots, int tb, ActQ8 hq,
                      float* hf, int hf_ld, dim3 grid, hipStream_t st, const SmallTail& tail, SharedPart* sh) {
    if (tb <= 1) {
        const size_t lds = act_lds_bytes(1, xq.K, false);
        // every block resident at 3 waves per SIMD: the spill-free build (measured: Qwen3-shaped 32.6 -> 31.0 us,
        // Qwen1.5-shaped 43.6 -> 40 us per token; Mixtral-shaped, 896 blocks, keeps 4 waves per SIMD)
        const bool w3 = (size_t)grid.x * GATEUP_WAVES <= (size_t)3 * 4 * num_cus();
        auto go = [&](auto kern) {
            lds_optin(kern, lds);
            hipLaunchKernelGGL(kern, grid, dim3(GATEUP_WAVES * 64), lds, st, g, u, xq, nullptr, 0, grp, hq, hf, hf_ld,
                               tail);
        };
        if (w3) go(k_gemv_gateup<TYPE, 1, GATEUP_WAVES, 3>);
        else go(k_gemv_gateup<TYPE, 1, GATEUP_WAVES, 4>);
    } else if (tb <= 4) {
        const size_t lds = act_lds_bytes(4, xq.K, false);
        lds_optin(k_gemv_gateup<TYPE, 4, GATEUP_WAVES>, lds);
        hipLaunchKernelGGL((k_gemv_gateup<TYPE, 4, GATEUP_WAVES>), grid, dim3(GATEUP_WAVES * 64), lds, st, g, u, xq,
                           nullptr, 0, grp, hq, hf, hf_ld, tail);
    } else {  // several tokens per expert: the matrix-core form
        const size_t lds = (size_t)(xq.K / 32) * MX_NT * sizeof(float2);
        constexpr int MR = mx_mr_max<TYPE, true>();
        if constexpr (MR > 1) {
            if (g.nrt * slots >= MX_MR_MIN_ITEMS) {
                // the shared expert's blocks join where it has this launch's weight format and every block
                // stays in one resident round
                const bool shm = sh && sh->slots > 0 && sh->g.type == TYPE && sh->u.type == TYPE && sh->g.nkb == g.nkb &&
                                 sh->u.nkb == g.nkb && sh->g.nrt == sh->u.nrt &&
                                 gemv_gateup_joins(TYPE, g.nrt, slots, tb, sh->g.nrt, sh->slots);
                SharedPart sp = shm ? *sh : SharedPart{};
                const int rb = (g.nrt + MR - 1) / MR * slots;
                sp.blocks0 = rb;
                sp.kparts = 1;
                const int nb = rb + (shm ? (sp.g.nrt + MR - 1) / MR * sp.slots : 0);
                auto go = [&](auto kern, int waves) {
                    lds_optin(kern, lds);
                    hipLaunchKernelGGL(kern, dim3(nb + (tail.on ? 1 : 0)), dim3(waves * 64), lds, st, g, u, xq, grp, hq,
                                       hf, hf_ld, nullptr, tail, sp);
                };
                // 2-wave blocks (a gate and an up wave, twice the units each, four blocks per CU) where
                // that puts every block in one resident round: no second round of block prologues and
                // no tail (measured from HBM: DeepSeek-V2-Lite-shaped 32 tokens 140 -> 130 us,
                // Qwen1.5-shaped 64 tokens 152 -> 146 us; Mixtral-shaped 32 tokens, 1200 blocks, 213 us
                // at 4 waves against 236 at 2)
                if (nb <= 4 * num_cus())
                    go(k_gemv_mxt<TYPE, true, 2, MR>, 2);
                else
                    go(k_gemv_mxt<TYPE, true, GATEUP_WAVES, MR>, GATEUP_WAVES);
                return shm;
            }
        }
        lds_optin(k_gemv_mx<TYPE, true, GATEUP_WAVES>, lds);
        hipLaunchKernelGGL((k_gemv_mx<TYPE, true, GATEUP_WAVES>), dim3(g.nrt * slots + (tail.on ? 1 : 0)),
                           dim3(GATEUP_WAVES * 64), lds, st, g, u, xq, grp, hq, hf, hf_ld, nullptr, tail);
    }
    return false;
}

bool launch_gemv_gateup(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots, int tb,
                        ActQ8 hq, float* hf, hipStream_t st, const SmallTail* tail, const float* xf, int xf_ld,
                        SharedPart* sh) {
    const SmallTail t = tail ? *tail : SmallTail{};
    switch (g.type) {
        case T_Q4_0: return gateup_t<T_Q4_0>(g, u, xq, xf, xf_ld, grp, slots, tb, hq, hf, st, t, sh);
        case T_Q8_0: return gateup_t<T_Q8_0>(g, u, xq, xf, xf_ld, grp, slots, tb, hq, hf, st, t, sh);
        case T_Q4_K: return gateup_t<T_Q4_K>(g, u, xq, xf, xf_ld, grp, slots, tb, hq, hf, st, t, sh);
        case T_Q5_K: return gateup_t<T_Q5_K>(g, u, xq, xf, xf_ld, grp, slots, tb, hq, hf, st, t, sh);
        case T_Q6_K: return gateup_t<T_Q6_K>(g, u, xq, xf, xf_ld, grp, slots, tb, hq, hf, st, t, sh);
        case T_Q5_0:  // fp32 activations only
            if (xf) return gateup_t<T_Q5_0>(g, u, xq, xf, xf_ld, grp, slots, tb, hq, hf, st, t, sh);
            return false;
        default: return false;
    }
}

template <int TYPE, bool F32ACT>
static bool down_t(const QMat& dn, const ActQ8& hq, const float* hf, int hf_ld, const Groups& grp, int slots,
                   int tb, float* y, hipStream_t st, const CombineOut& comb, SharedPart* sh) {
    dim3 grid(dn.nrt * slots);
    const int K = F32ACT ? hf_ld : hq.K;
    if (tb <= 1) {
        const size_t lds = act_lds_bytes(1, K, F32ACT);
        lds_optin(k_gemv_down<TYPE, 1, DOWN_WAVES, F32ACT>, lds);
        hipLaunchKernelGGL((k_gemv_down<TYPE, 1, DOWN_WAVES, F32ACT>), grid, dim3(DOWN_WAVES * 64), lds, st, dn, hq,
                           hf, hf_ld, grp, y, comb);
    } else if (tb > 4 && !F32ACT) {  // several tokens per expert: the matrix-core form
        if constexpr (!F32ACT) {
            // 4-wave blocks (more of them resident per CU) unless the grid is too small to fill half
            // the CUs (one dense matrix, few tokens); measured: Qwen1.5-shaped 64 tokens routed down
            // 75 -> 44 us, Qwen3-shaped 32 tokens 62 -> 33 us
            size_t lds = (size_t)(K / 32) * MX_NT * sizeof(float2);
            // and 8-wave blocks where two 4-wave blocks' LDS would not fit one CU (long K: the staged scales
            // plus the tiles' partial sums)
            constexpr int MR = mx_mr_max<TYPE, false>();
            if constexpr (MR > 1) {
                // (slots 0 with sh: the shared down alone, its K in parts)
                if (dn.nrt * slots >= MX_MR_MIN_ITEMS || (sh && slots == 0)) {
                    // the shared down's blocks join (its K in parts of at most a routed block's units) where it
                    // has this launch's weight format and Q8_0 h
                    const bool shm = sh && sh->slots > 0 && sh->g.type == TYPE && sh->hq.q != nullptr &&
                                     sh->g.rows == dn.rows && sh->hq.K == sh->g.cols;
                    SharedPart sp = shm ? *sh : SharedPart{};
                    const int rb = (dn.nrt + MR - 1) / MR * slots;
                    sp.blocks0 = rb;
                    if (!shm) sp.kparts = 1;
                    if (shm) {
                        constexpr int BPU = Mx<TYPE>::BPU;
                        const int ub = (sp.hq.K / 32 + BPU - 1) / BPU, upp = (ub + sp.kparts - 1) / sp.kparts;
                        // a K part stages only its own blocks' token scales; with no routed blocks that is all
                        const size_t lp = (size_t)upp * BPU * MX_NT * sizeof(float2);
                        lds = rb == 0 ? lp : std::max(lds, lp);
                    }
                    const int nb = rb + (shm ? (sp.g.nrt + MR - 1) / MR * sp.slots * sp.kparts : 0);
                    auto go = [&](auto kern, int waves) {
                        lds_optin(kern, lds);
                        hipLaunchKernelGGL(kern, dim3(nb), dim3(waves * 64), lds, st, dn, dn, hq, grp, ActQ8{}, nullptr, 0,
                                           y, SmallTail{}, sp);
                    };
                    const bool lds2 = 2 * (lds + mx_red_bytes<4, MR>()) <= (size_t)160 * 1024;
                    // Fewer waves per block where the CU's LDS holds the extra blocks: the same waves per CU, each
                    // with more of its block's units behind one round trip for the first (Q4_0: one wave,
                    // Qwen1.5-shaped 48 / 64 tokens 125.1 / 133.8 -> 119.2 / 129.1 us per step; Q8_0: two,
                    // Qwen3-shaped 32 tokens 100.0 -> 98.0 us, one wave measured 104.6)
                    const bool lds_w1 = 8 * (lds + mx_red_bytes<1, MR>()) <= (size_t)160 * 1024;
                    const bool lds_w2 = 4 * (lds + mx_red_bytes<2, MR>()) <= (size_t)160 * 1024;
                    if (2 * nb < num_cus() || !lds2) {
                        go(k_gemv_mxt<TYPE, false, 8, MR>, 8);
                    } else if constexpr (TYPE == T_Q4_0) {
                        if (lds_w1) go(k_gemv_mxt<TYPE, false, 1, MR>, 1);
                        else if (lds_w2) go(k_gemv_mxt<TYPE, false, 2, MR>, 2);
                        else go(k_gemv_mxt<TYPE, false, 4, MR>, 4);
                    } else if constexpr (TYPE == T_Q8_0) {
                        if (lds_w2) go(k_gemv_mxt<TYPE, false, 2, MR>, 2);
                        else go(k_gemv_mxt<TYPE, false, 4, MR>, 4);
                    } else {
                        go(k_gemv_mxt<TYPE, false, 4, MR>, 4);
                    }
                    return shm;
                }
            }
            auto go = [&](auto kern, int waves) {
                lds_optin(kern, lds);
                hipLaunchKernelGGL(kern, grid, dim3(waves * 64), lds, st, dn, dn, hq, grp, ActQ8{}, nullptr, 0, y,
                                   SmallTail{});
            };
            if (2 * (int)grid.x < num_cus()) go(k_gemv_mx<TYPE, false, 8>, 8);
            else go(k_gemv_mx<TYPE, false, 4>, 4);
        }
    } else {
        const size_t lds = act_lds_bytes(4, K, F32ACT);
        lds_optin(k_gemv_down<TYPE, 4, DOWN_WAVES, F32ACT>, lds);
        hipLaunchKernelGGL((k_gemv_down<TYPE, 4, DOWN_WAVES, F32ACT>), grid, dim3(DOWN_WAVES * 64), lds, st, dn, hq,
                           hf, hf_ld, grp, y, comb);
    }
    return false;
}

// ---------------------------------------------------------------- one-token step in one launch
// A one-token decode step (even top-k, Q8_0 activations on both sides, a shared expert of the routed
// formats or none) as one grid of 512-thread blocks, in index order:
//   router     one block per router row (and the shared-expert gate row): the row and the token staged
//              chain-major in LDS, the vec_dot_f32 chain (as k_route_small), the logit published as
//              one device-coherent 64-bit word (epoch << 32 | bits).  Block 0 first zeroes the folded
//              combine's output.
//   tables     once every logit of this launch is out: the dispatch tables (topk_dispatch_wave,
//              with the shared-expert gate) and the Q8_0 of x, for the caller.
//   shared g/u two row tiles of the shared expert's gate/up per block (waves 0-3 and 4-7, each the
//              4-wave single-token GEMV); they need no routing and stream from the start.
//   gate/up    row tile rt of slots 2s and 2s + 1 likewise, each slot's expert from the published
//              logits (small_group).  Every gate/up block forms the Q8_0 of x in LDS itself and
//              stores its Q8_0 block of h device-coherently: the quants, then the scale word carrying
//              the launch's tag.
//   down       row tile rt of one routed slot, then of the shared expert: the 8-wave single-token down
//              GEMV, its first weight units in flight before it waits for every scale word of its h to
//              carry the tag; the quants are then read device-coherently.  Top-2 without a shared
//              expert adds p * y into the output (the folded combine); otherwise y and ysh are
//              written for launch_combine.
// The arithmetic is that of the separate launches (same chains, quantization, unit order and
// reductions), so the results are bit-identical to them.  A block waits only on blocks with smaller
// indices, which the dispatcher starts first, so every wait ends; each is bounded anyway (giving up
// sets sync->err, and the block goes on with in-bounds reads).  The launch number tags the logits
// (32 bits) and h's scales (htag, 13 bits: an fp16 scale widened to fp32 has its low 13 mantissa
// bits zero), so nothing is reset between launches and no two blocks update one word (atomic
// read-modify-writes on one line serialize at the memory side).  Blocks hand over through
// device-scope atomic loads and stores only (a device-scope fence writes back the whole L2 on this
// part).  Calls on one layer must be stream-ordered.
constexpr int DEC_THREADS = 512;

// A wait that gave up: the device word, and the host-visible one the runtime checks on the layer's next
// call whatever its flags (so an asynchronous caller learns of it too).
__device__ __forceinline__ void dec_fail(const Decode1Args& a) {
    __hip_atomic_store(&a.sync->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.herr) __hip_atomic_store(a.herr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Wave 0: wait until the first n logit words carry this launch's tag, then put the logits in lg
// (LDS); the caller synchronizes the block.
__device__ void dec_wait_logits(const Decode1Args& a, int n, float* lg) {
    const int lane = threadIdx.x & 63;
    for (int it = 0;; ++it) {
        uint64_t w0 = 0, w1 = 0;
        bool ok = true;
        if (lane < n) {
            w0 = __hip_atomic_load(a.sync->tag + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = (uint32_t)(w0 >> 32) == a.epoch;
        }
        if (64 + lane < n) {
            w1 = __hip_atomic_load(a.sync->tag + 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = ok && (uint32_t)(w1 >> 32) == a.epoch;
        }
        const bool all = __all(ok && !a.giveup_test);
        if (all || it >= (int)a.spin_limit) {
            if (!all && lane == 0) dec_fail(a);
            if (lane < n) lg[lane] = __uint_as_float((uint32_t)w0);
            if (64 + lane < n) lg[64 + lane] = __uint_as_float((uint32_t)w1);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

constexpr uint32_t DEC_HTAG_MASK = 0x1FFFu;  // low mantissa bits of h's stored scale

// TSD: the shared down's format; DF32: the routed down takes fp32 h (no Q8_0 form at d_ff: its gate/up
// blocks publish h as tagged 64-bit words (epoch << 32 | fp32 bits), and its down blocks read them
// until every word carries this launch's number, as k_gemv_gateup / k_gemv_down<..., true> hand fp32 h
// over in the separate launches).
template <int TG, int TD, int TSD, bool DF32>
__global__ void __launch_bounds__(DEC_THREADS) __attribute__((amdgpu_waves_per_eu(GEMV_WAVES_PER_SIMD(1))))
k_decode1(Decode1Args a) {
    extern __shared__ __align__(16) int8_t smem[];
    __shared__ float lg[SMALL_GROUP_MAX_E];
    __shared__ float red[DEC_THREADS / 64][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    const int E = a.E, d = a.d;
    const int R = E + (a.shgate ? 1 : 0);                       // router rows
    const int ngs = a.sh ? (a.SG.nrt + 1) / 2 : 0;              // shared gate/up blocks
    const int ng = a.G.nrt * (a.k / 2);                         // routed gate/up blocks
    const int nd = a.D.nrt * a.k;                               // routed down blocks
    const int b_sg = R + 1, b_gu = b_sg + ngs, b_dn = b_gu + ng, b_sd = b_dn + nd;
    const int blk = blockIdx.x;
    Groups grp;  // the slot records follow from the logits (small_group)
    grp.logits = lg;
    grp.n_experts = E;
    grp.top_k = a.k;
    grp.n_tok = 1;

    // One gate/up row tile per half (waves 0-3, 4-7): expert e's rows 32 rt.. of Wg / Wu against the
    // Q8_0 of x in LDS; SwiGLU and h's Q8_0 block into row p0 of hout, device-coherently, the tagged
    // scale last.  An inactive half loads the pad and stores nothing (both halves meet every barrier).
    auto gateup_tile = [&](const QMat& Wg, const QMat& Wu, int e, int rt, int p0, const ActQ8& hout, bool active,
                           uint64_t* hfw) {
        const int half = wave >> 2, lw = wave & 3, mat = lw >> 1, kw = lw & 1;
        const ActLds A{smem, reinterpret_cast<const float2*>(smem + d), nullptr, d};
        const QMat& W = mat ? Wu : Wg;
        const int nu = active ? n_units<TG>(Wg.nkb) : 0;
        float acc[1] = {0.0f};
        kloop<TG, 1>(
            W, W, e, rt, kw, nu, 2, m, h, [] {},
            [&](const typename Fmt<TG>::Raw& c, const typename Fmt<TG>::Raw&, int u) {
                unit_accum<TG, 1>(c, A, u, h, 1, Wg.nkb, acc);
            });
        acc[0] += __shfl_xor(acc[0], 32, 64);
        if (h == 0) red[wave][m] = acc[0];
        __syncthreads();
        if (lw == 0 && active) {  // waves 0 and 4: SwiGLU and the Q8_0 block of h (as k_gemv_gateup)
            float gv = 0.0f, uv = 0.0f;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                gv += red[4 * half + w][m];
                uv += red[4 * half + 2 + w][m];
            }
            if (DF32 && hfw) {  // fp32 h as tagged words, row p0 of d_ff values
                if (h == 0)
                    __hip_atomic_store(hfw + (size_t)p0 * hout.K + rt * 32 + m,
                                       ((uint64_t)a.epoch << 32) | __float_as_uint(gated(gv, uv, Wg.act)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
            float2 sv;
            const int q = q8_block_vals(gated(gv, uv, Wg.act), sv);
            const uint32_t q1 = (uint32_t)__shfl_down(q, 1, 64), q2 = (uint32_t)__shfl_down(q, 2, 64),
                           q3 = (uint32_t)__shfl_down(q, 3, 64);
            const uint32_t word = ((uint32_t)q & 0xFFu) | ((q1 & 0xFFu) << 8) | ((q2 & 0xFFu) << 16) | (q3 << 24);
            if (h == 0 && (m & 3) == 0)
                __hip_atomic_store(reinterpret_cast<uint32_t*>(hout.q + (size_t)p0 * hout.K + rt * 32 + m), word,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the quants are out before the tagged scale
            if (lane == 0)
                __hip_atomic_store(reinterpret_cast<uint64_t*>(hout.s + (size_t)p0 * (hout.K / 32) + rt),
                                   ((uint64_t)__float_as_uint(sv.y) << 32) | __float_as_uint(sv.x) | a.htag,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };

    // A down tile's lanes' partial sums: the 8 waves' sums in wave order, into y_out[row] or p * s added
    // into the output (folded combine)
    auto down_out = [&](const QMat& Wd, int rt, float* y_out, float p, float acc) {
        acc += __shfl_xor(acc, 32, 64);
        if (h == 0) red[wave][m] = acc;
        __syncthreads();
        if (wave == 0 && h == 0) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < DEC_THREADS / 64; ++w) s += red[w][m];
            const int row = rt * 32 + m;
            if (!(Wd.valid_rows && row >= Wd.valid_rows)) {
                if (y_out) y_out[row] = s;
                else atomicAdd(a.out + row, p * s);
            }
        }
    };

    // Down row tile rt of expert e of Wd against row p0 of hin (once every scale word of that row
    // carries this launch's tag): y_out[row] = s, or p * s added into the output (folded combine).
    auto down_tile = [&](auto tdc, const QMat& Wd, int e, int rt, int p0, const ActQ8& hin, float* y_out, float p) {
        constexpr int T = decltype(tdc)::value;
        const int K = hin.K, KB = K / 32;
        const ActLds A{smem, reinterpret_cast<const float2*>(smem + K), nullptr, K};
        const int nu = n_units<T>(Wd.nkb);
        float acc[1] = {0.0f};
        kloop<T, 1>(
            Wd, Wd, e, rt, wave, nu, DEC_THREADS / 64, m, h,
            [&] {  // after the first two units' loads: wait for the tags, then stage h
                const uint64_t* ss = reinterpret_cast<const uint64_t*>(hin.s + (size_t)p0 * KB);
                uint64_t sv = 0;
                for (int it = 0;; ++it) {
                    if (tid < KB) sv = __hip_atomic_load(ss + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const bool ok = (tid >= KB || ((uint32_t)sv & DEC_HTAG_MASK) == a.htag) && !a.giveup_test;
                    if (__syncthreads_and(ok)) break;  // block-uniform
                    if (it >= (int)a.spin_limit) {
                        if (tid == 0) dec_fail(a);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                constexpr int QPER = 16384 / 4 / DEC_THREADS;  // d_ff <= 16384
                const uint32_t* qs = reinterpret_cast<const uint32_t*>(hin.q + (size_t)p0 * K);
                uint32_t qv[QPER];
#pragma unroll
                for (int q = 0; q < QPER; ++q) {
                    const int i = tid + q * DEC_THREADS;
                    qv[q] = i < K / 4 ? __hip_atomic_load(qs + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
                }
#pragma unroll
                for (int q = 0; q < QPER; ++q) {
                    const int i = tid + q * DEC_THREADS;
                    if (i < K / 4) reinterpret_cast<uint32_t*>(smem)[i] = qv[q];
                }
                if (tid < KB) reinterpret_cast<uint64_t*>(smem + K)[tid] = sv & ~(uint64_t)DEC_HTAG_MASK;
                __syncthreads();
            },
            [&](const typename Fmt<T>::Raw& c, const typename Fmt<T>::Raw&, int u) {
                unit_accum<T, 1>(c, A, u, h, 1, Wd.nkb, acc);
            });
        down_out(Wd, rt, y_out, p, acc[0]);
    };

    // The same over fp32 h: row p0's tagged words, staged in LDS as floats zero-padded to a.hf_ld (whole
    // K-units), against the fp32-activation dots of k_gemv_down<..., true>.
    auto down_tile_f32 = [&](const QMat& Wd, int e, int rt, int p0, float* y_out, float p) {
        const int F = a.hq.K, KP = a.hf_ld;
        float* hl = reinterpret_cast<float*>(smem);
        const ActLds A{nullptr, nullptr, hl, KP};
        const int nu = n_units<TD>(Wd.nkb);
        float acc[1] = {0.0f};
        kloop<TD, 1>(
            Wd, Wd, e, rt, wave, nu, DEC_THREADS / 64, m, h,
            [&] {  // after the first two units' loads: every word of the row, once it carries the launch number
                const uint64_t* hw = a.hfw + (size_t)p0 * F;
                for (int it = 0;; ++it) {
                    bool ok = true;
                    for (int i = tid; i < F; i += DEC_THREADS) {
                        const uint64_t w = __hip_atomic_load(hw + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const bool t = (uint32_t)(w >> 32) == a.epoch;
                        if (t) hl[i] = __uint_as_float((uint32_t)w);
                        ok = ok && t;
                    }
                    if (__syncthreads_and(ok && !a.giveup_test)) break;  // block-uniform
                    if (it >= (int)a.spin_limit) {
                        if (tid == 0) dec_fail(a);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                for (int i = F + tid; i < KP; i += DEC_THREADS) hl[i] = 0.0f;
                __syncthreads();
            },
            [&](const typename Fmt<TD>::Raw& c, const typename Fmt<TD>::Raw&, int u) {
                unit_accum_f32<TD, 1>(c, A, u, h, 1, Wd.nkb, acc);
            });
        down_out(Wd, rt, y_out, p, acc[0]);
    };

    // Q8_0 of x into LDS (the gate/up blocks' activations), one 32-block per half-wave and step, as
    // the router kernels form it
    auto quantize_x = [&] {
        int8_t* xq = smem;
        float2* xs = reinterpret_cast<float2*>(smem + d);
        constexpr int XPER = 8192 / 32 / (2 * DEC_THREADS / 64);  // d <= 8192
        const int KB = d / 32, hw = 2 * wave + h;
        float xv[XPER];
#pragma unroll
        for (int q = 0; q < XPER; ++q) {
            const int bb = hw + q * (2 * DEC_THREADS / 64);
            xv[q] = bb < KB ? a.x[bb * 32 + m] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < XPER; ++q) {
            const int bb = hw + q * (2 * DEC_THREADS / 64);
            if (bb < KB) {  // half-wave uniform
                float2 sv;
                xq[bb * 32 + m] = (int8_t)q8_block_vals(xv[q], sv);
                if (m == 0) xs[bb] = sv;
            }
        }
    };

    if (blk < R) {  // ---- router row blk (row E: the shared-expert gate, fp32 order)
        float* lds = reinterpret_cast<float*>(smem);
        const int S = rs_stride(d), RS = 16 * S;
        if (blk == 0 && a.out) {  // the folded combine's output starts at zero
            for (int i = tid; i < d; i += DEC_THREADS)
                __hip_atomic_store(reinterpret_cast<uint32_t*>(a.out) + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // complete before the logit is out
        }
        const float* wrow = blk < E ? a.router + (size_t)blk * d : a.shgate;
        {  // row + token -> LDS, chain-major, every load in flight before the first store
            constexpr int PER = 2 * 8192 / 4 / DEC_THREADS;  // d <= 8192
            const int c4 = d / 4, tot = 2 * c4;
            float4 v[PER];
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int i = tid + q * DEC_THREADS;
                if (i >= tot) break;
                const int row = i / c4, c = i - row * c4;
                v[q] = *reinterpret_cast<const float4*>((row == 0 ? wrow : a.x) + 4 * c);
            }
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int i = tid + q * DEC_THREADS;
                if (i >= tot) break;
                const int row = i / c4, c = i - row * c4;
                float* dst = lds + row * RS + 4 * (c & 3) * S + (c >> 2);
                dst[0] = v[q].x;
                dst[S] = v[q].y;
                dst[2 * S] = v[q].z;
                dst[3 * S] = v[q].w;
            }
        }
        __syncthreads();
        if (wave == 0 && lane < 16) {
            const bool c8 = a.chain8 != 0 && blk < E;
            const float s = chain_sum(chain_dot_lds(lds, lds + RS, S, d, lane, c8), c8);
            if (lane == 0) {
                const float l = (blk < E && a.bias) ? s + a.bias[blk] : s;
                if (blk < E) a.ra.logits[blk] = l;
                __hip_atomic_store(a.sync->tag + blk, ((uint64_t)a.epoch << 32) | __float_as_uint(l), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        return;
    }

    if (blk == R) {  // ---- the caller's dispatch tables and Q8_0 of x
        if (wave == 0) dec_wait_logits(a, R, lg);
        __syncthreads();
        if (wave == 0) {
            topk_dispatch_wave<SMALL_GROUP_MAX_E / 64>(a.ra, a.o, lg, a.shgate ? lg + E : nullptr);
        } else {
            const int nb = d / 32, hw = 2 * (wave - 1) + h;
            for (int b = hw; b < nb; b += 2 * (DEC_THREADS / 64 - 1)) {  // half-wave uniform
                float2 sv;
                a.xq.q[b * 32 + m] = (int8_t)q8_block_vals(a.x[b * 32 + m], sv);
                if (m == 0) a.xq.s[b] = sv;
            }
        }
        return;
    }

    if (blk < b_gu) {  // ---- shared gate/up: row tiles 2 b, 2 b + 1
        const int rt = 2 * (blk - b_sg) + (wave >> 2);
        quantize_x();
        __syncthreads();
        gateup_tile(a.SG, a.SU, 0, rt < a.SG.nrt ? rt : 0, 0, a.hqs, rt < a.SG.nrt, nullptr);
        return;
    }

    if (blk < b_dn) {  // ---- routed gate/up: row tile rt of slots 2 sp, 2 sp + 1
        const int b = blk - b_gu, rt = b % a.G.nrt, sp = b / a.G.nrt;
        quantize_x();  // while the router runs
        if (wave == 0) dec_wait_logits(a, E, lg);
        __syncthreads();  // the logits and the Q8_0 of x
        const int4 rec = small_group(grp, 2 * sp + (wave >> 2));
        gateup_tile(a.G, a.U, rec.x, rt, rec.y, a.hq, true, DF32 ? a.hfw : nullptr);
        return;
    }

    if (blk < b_sd) {  // ---- routed down: row tile rt of one slot
        const int b = blk - b_dn, rt = b % a.D.nrt, slot = b / a.D.nrt;
        if (wave == 0) dec_wait_logits(a, E, lg);
        __syncthreads();
        const int4 rec = small_group(grp, slot);
        float p = 0.0f;
        if (a.out) {  // this slot's weight: the softmax of topk_token_wave, as in the tables
            RouteArgs r = a.ra;
            r.ids = nullptr;
            r.probs = nullptr;
            r.shscale = nullptr;
            uint64_t msk[SMALL_GROUP_MAX_E / 64];
            float myp = 0.0f;
            const int myid = topk_token_wave<SMALL_GROUP_MAX_E / 64>(r, lg, 0, nullptr, msk, &myp);
            for (int q = 0; q < a.k; ++q) {
                const int id = __shfl(myid, q, 64);
                const float pq = __shfl(myp, q, 64);
                if (id == rec.x) p = pq;
            }
        }
        float* const yo = a.out ? nullptr : a.y + (size_t)rec.y * a.D.rows;
        if constexpr (DF32)
            down_tile_f32(a.D, rec.x, rt, rec.y, yo, p);
        else
            down_tile(std::integral_constant<int, TD>{}, a.D, rec.x, rt, rec.y, a.hq, yo, p);
        return;
    }

    // ---- shared down: row tile rt
    down_tile(std::integral_constant<int, TSD>{}, a.SD, 0, blk - b_sd, 0, a.hqs, a.ysh, 0.0f);
}

static bool fmt_q8(int t) { return t == T_Q4_0 || t == T_Q8_0 || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K; }

bool decode1_fits(int gtype, int dtype, int d, int f, int E, int k, int fs, bool shgate, int sdtype, bool df32) {
    // built: one format on both sides, or a K-quant gate/up with a Q6_K down (the _M mixes); with fp32 h at
    // d_ff, a Q4_K gate/up with a Q4_K or Q5_0 down and a shared down of Q4_K or Q6_K (DeepSeek-V2-Lite-shaped
    // Q4_K and Q4_K_M)
    const bool q8 = !df32 && fmt_q8(gtype) && (gtype == dtype || ((gtype == T_Q4_K || gtype == T_Q5_K) && dtype == T_Q6_K)) &&
                    (fs == 0 || sdtype == dtype);
    const bool hf = df32 && gtype == T_Q4_K &&
                    ((dtype == T_Q4_K && (fs == 0 || sdtype == T_Q4_K)) || (dtype == T_Q5_0 && (fs == 0 || sdtype == T_Q6_K)));
    const bool built = q8 || hf;
    return built && E >= 1 && E + (shgate ? 1 : 0) <= SMALL_GROUP_MAX_E && k >= 2 && k % 2 == 0 && k <= MAX_SLOTS_DEC && k <= E &&
           d % 32 == 0 && d <= 8192 && f % 32 == 0 && f <= 16384 && fs % 32 == 0 && fs <= 16384;
}

// The fused launch pays where its gate/up blocks fit one per CU.  Larger gate/up phases leave the
// down blocks to the slots the gate/up blocks free, unevenly (measured, Mixtral-shaped: 64 CUs run two
// down blocks while 64 run none).  Measured per step: toy 15.9 -> 11.2 us, Qwen3-shaped 26.1 -> 24.9
// us, Mixtral-shaped 46.1 -> 48.6 us (not taken).
// (Measured and dropped: a cooperative launch whose first gate/up blocks, one per CU, go on with the
// down tiles, so that the down work is spread evenly: Mixtral-shaped 64 us per step.)
bool decode1_pays(int gate_nrt, int k, int sgate_nrt) {
    return gate_nrt * (k / 2) + (sgate_nrt + 1) / 2 <= num_cus();
}

void launch_decode1(const Decode1Args& a, int gtype, int dtype, hipStream_t st, int sdtype, bool df32) {
    const dim3 grid(a.E + (a.shgate ? 1 : 0) + 1 + (a.sh ? (a.SG.nrt + 1) / 2 + a.SD.nrt : 0) +
                    a.G.nrt * (a.k / 2) + a.D.nrt * a.k);
    // LDS: router row + token chain-major, or a gate/up's Q8_0 of x, or a down's Q8_0 (or fp32) h
    const size_t lds = std::max({(size_t)2 * 16 * rs_stride(a.d) * sizeof(float), act_lds_bytes(1, a.d, false),
                                 act_lds_bytes(1, a.hq.K, false), act_lds_bytes(1, a.sh ? a.hqs.K : 0, false),
                                 df32 ? (size_t)a.hf_ld * sizeof(float) : (size_t)0});
    auto go = [&](auto kern) {
        lds_optin(kern, lds);
        hipLaunchKernelGGL(kern, grid, dim3(DEC_THREADS), lds, st, a);
    };
    if (!a.sh) sdtype = dtype == T_Q5_0 ? T_Q6_K : dtype;  // no shared blocks: any built instance
#define JX_DEC1(G, D, SD, F32) \
    if (gtype == G && dtype == D && sdtype == SD && df32 == F32) return go(k_decode1<G, D, SD, F32>);
    JX_DEC1(T_Q4_0, T_Q4_0, T_Q4_0, false)
    JX_DEC1(T_Q8_0, T_Q8_0, T_Q8_0, false)
    JX_DEC1(T_Q4_K, T_Q4_K, T_Q4_K, false)
    JX_DEC1(T_Q5_K, T_Q5_K, T_Q5_K, false)
    JX_DEC1(T_Q6_K, T_Q6_K, T_Q6_K, false)
    JX_DEC1(T_Q4_K, T_Q6_K, T_Q6_K, false)
    JX_DEC1(T_Q5_K, T_Q6_K, T_Q6_K, false)
    JX_DEC1(T_Q4_K, T_Q4_K, T_Q4_K, true)
    JX_DEC1(T_Q4_K, T_Q5_0, T_Q6_K, true)
#undef JX_DEC1
}

// ---------------------------------------------------------------- one-token step, one block per CU
// Layers whose gate/up row tiles outnumber the CUs several times (Mixtral-shaped: 896 tiles on 256
// CUs; k_decode1 leaves its down blocks to the CUs its gate/up blocks free, unevenly) as one grid of
// one 1024-thread block per CU:
//   route    the first E blocks run one router row each (the row and the token chain-major in LDS, the
//            vec_dot_f32 chains of k_route_small) and publish the logit as a tagged word; every block
//            forms the Q8_0 of x in LDS meanwhile, then selects the experts from the logits (the same
//            selection in every block).  Block 0 writes the logits, the Q8_0 of x and the dispatch
//            tables for the caller; each block first zeroes the output rows of its first-slot down
//            tile (the folded combine adds into them).
//   gate/up  (slot, row tile) tiles G-1-b, 2G-1-b, 3G-1-b, 4G-1-b of the G blocks, one per group of four
//            waves (the 4-wave single-token GEMV), so every CU streams about the same bytes.  h's
//            Q8_0 quants go out as 64-bit words carrying the launch number, its scales with the
//            launch's tag in their low mantissa bits, so no store waits for another.
//   down     the block's down tiles b, b + G on waves 0 .. DOWN_WAVES - 1 (the single-token down
//            GEMV's unit split and wave-order sum): the first weight units in flight, then h read
//            until every word of the slot carries this launch's number or tag, and p * y added into
//            the output (two adds onto an exact zero per element).
// The step is bit-identical to the separate launches.  Every down tile waits on h from blocks across
// the grid, so the grid must be resident at once: one block per CU (its LDS leaves no room for a
// second) and a grid of one block per CU.  A kernel of another stream or process holding CUs delays
// the step; every wait is bounded, and giving up sets sync->err and the host-visible herr, which the
// runtime reports on the synchronous call, on jx_moe_layer_status and on the layer's next forward.  The zeroing of a row is ordered before the block's own slot-1 h stores, which the other
// down tile of that row waits for (decodep_fits checks the tile layout gives every zeroing block one).
// Measured Mixtral-shaped, host clock over 300 queued steps: 42.2 us per step against 46.3 us for the
// separate launches (route, gate/up GEMV, down GEMV).
constexpr int DP_THREADS = 1024, DP_WAVES = DP_THREADS / 64, DP_GROUPS = DP_WAVES / 4;
// Units in flight per wave (kloop_d).  Measured Mixtral-shaped: 2 -> 42.2 us per step, 3 -> 45, 4 -> 54
// (more requests in flight slow the stream); likewise four gate/up groups streaming at once against two
// (42.2 / 42.2 us) or one (51 us), and 16 down waves against 8 (42.4 / 42.2 us).
constexpr int DP_DEPTH = 2;
constexpr int DP_HDEPTH = 3;         // units of h words in flight per poller wave
constexpr int DP_MAX_UNITS = 16384 / 128;  // down units of a d_ff <= 16384 (128-element units at most)
constexpr size_t DP_LDS_MAX = 156 * 1024;

__host__ __device__ inline size_t decodep_route_bytes(int d, int E) {
    (void)E;
    return (size_t)2 * 16 * rs_stride(d) * sizeof(float);  // a router row and the token, chain-major
}
// LDS offset of the Q8_0 of x, above the router staging and the down projection's staged h
__host__ __device__ inline size_t decodep_xoff(int d, int f, int E) {
    const size_t r = decodep_route_bytes(d, E), hb = act_lds_bytes(1, f, false);
    return r > hb ? r : hb;
}

// Gate/up tile (slot * nrt + row tile) of group g of block b among nb, or -1: top-2, so 2 nrt tiles,
// q = 2 nrt / nb per block and one more on the last r = 2 nrt % nb blocks.  The tiles form a list in
// row-tile order (both slots of a row tile side by side); its first positions go to the blocks with q
// tiles, which are done first, round-robin over them, so the low row tiles -- the low K of h, which every
// down wave consumes first -- are ready first.  The router rows sit on the first blocks, among those with
// fewer tiles.  Within a position pair (both slots of a row tile) the slots alternate with the group, so
// each block streams both slots (decodep_fits relies on it).  -1 where the layout does not hold
// (decodep_fits then refuses the shape).
__host__ __device__ inline int decodep_gu_tile(int b, int g, int nb, int nrt) {
    const int T = 2 * nrt, q = T / nb, r = T % nb, n0 = nb - r;
    int p, pl, C;
    if (b < n0) {
        if (g >= q) return -1;
        C = n0;
        pl = g * n0 + b;
        p = pl;
    } else {
        if (g > q) return -1;
        C = r;
        pl = g * r + (b - n0);
        p = n0 * q + pl;
    }
    if ((n0 * q) % 2) return -1;  // a position pair would straddle the two classes
    const int rt = p / 2, sl = (p + (C % 2 == 0 ? pl / C : 0)) % 2;
    return sl * nrt + rt;
}

// Dynamic LDS of k_decode_p: the router staging or the down projection's h, then the Q8_0 of x, and at
// least 96 KB so that no CU holds two of the blocks (each waits on the others).
static size_t decodep_lds(int d, int f, int E) {
    return std::max<size_t>(decodep_xoff(d, f, E) + act_lds_bytes(1, d, false), 96 * 1024);
}

template <int TG, int TD>
__global__ void __launch_bounds__(DP_THREADS) __attribute__((amdgpu_waves_per_eu(DP_WAVES / 4)))
k_decode_p(Decode1Args a) {
    extern __shared__ __align__(16) int8_t smem[];
    __shared__ float lg[SMALL_GROUP_MAX_E];
    __shared__ float red[DP_WAVES][32];
    __shared__ int s_e[MAX_SLOTS_DEC];
    __shared__ float s_p[MAX_SLOTS_DEC];
    __shared__ int hflag[DP_MAX_UNITS];  // per down unit: h staged in LDS (the tile's value, 0 before)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    const int E = a.E, d = a.d, k = a.k, NB = gridDim.x, b = blockIdx.x;
    if (tid < DP_MAX_UNITS) hflag[tid] = 0;  // before the block's first barrier
    const int ng = a.G.nrt * k, nd = a.D.nrt * k;
    int8_t* xq = smem + decodep_xoff(d, a.hq.K, E);  // Q8_0 of x: quants [d], then (scale, sum) [d / 32]
    float2* xs = reinterpret_cast<float2*>(xq + d);

    // ---- route
    for (int j = 0; j < 2; ++j) {  // the output rows of this block's first-slot down tiles start at zero
        const int t = b + j * NB;
        if (t < a.D.nrt && tid < 32)
            __hip_atomic_store(reinterpret_cast<uint32_t*>(a.out) + t * 32 + tid, 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // complete before the block's h stores (the barriers below)
    // router row of this block: the first E blocks, which the dispatcher starts first, so the routing
    // never waits on a block that has not started; they are among those with fewer gate/up tiles
    const int rr = b;
    if (rr < E) {  // router row rr against the token, chain-major in LDS (as k_decode1's router blocks)
        float* lds = reinterpret_cast<float*>(smem);
        const int S = rs_stride(d), RS = 16 * S;
        {
            constexpr int PER = 2 * 8192 / 4 / DP_THREADS;  // d <= 8192
            const int c4 = d / 4, tot = 2 * c4;
            float4 v[PER];
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int i = tid + q * DP_THREADS;
                if (i >= tot) break;
                const int row = i / c4, c = i - row * c4;
                v[q] = *reinterpret_cast<const float4*>((row == 0 ? a.router + (size_t)rr * d : a.x) + 4 * c);
            }
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int i = tid + q * DP_THREADS;
                if (i >= tot) break;
                const int row = i / c4, c = i - row * c4;
                float* dst = lds + row * RS + 4 * (c & 3) * S + (c >> 2);
                dst[0] = v[q].x;
                dst[S] = v[q].y;
                dst[2 * S] = v[q].z;
                dst[3 * S] = v[q].w;
            }
        }
        __syncthreads();
        if (wave == 0 && lane < 16) {
            const bool c8 = a.chain8 != 0;
            const float s = chain_sum(chain_dot_lds(lds, lds + RS, S, d, lane, c8), c8);
            if (lane == 0)
                __hip_atomic_store(a.sync->tag + rr, ((uint64_t)a.epoch << 32) | __float_as_uint(a.bias ? s + a.bias[rr] : s),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    {  // Q8_0 of x from the token row, one 32-block per half-wave and step, as the router kernels form it
        constexpr int XPER = 8192 / 32 / (2 * DP_WAVES);  // d <= 8192
        const int nb = d / 32, hw = 2 * wave + h;
        float xv[XPER];
#pragma unroll
        for (int q = 0; q < XPER; ++q) {
            const int bb = hw + q * (2 * DP_WAVES);
            xv[q] = bb < nb ? a.x[bb * 32 + m] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < XPER; ++q) {
            const int bb = hw + q * (2 * DP_WAVES);
            if (bb < nb) {  // half-wave uniform
                float2 sv;
                const int v = q8_block_vals(xv[q], sv);
                xq[bb * 32 + m] = (int8_t)v;
                if (m == 0) xs[bb] = sv;
                if (b == 0) {
                    a.xq.q[bb * 32 + m] = (int8_t)v;
                    if (m == 0) a.xq.s[bb] = sv;
                }
            }
        }
    }
    if (wave == 0) dec_wait_logits(a, E, lg);
    __syncthreads();
    if (wave == 0) {  // this launch's experts and weights in selection order (every block alike)
        RouteArgs r = a.ra;
        r.ids = nullptr;
        r.probs = nullptr;
        r.shscale = nullptr;
        uint64_t msk[SMALL_GROUP_MAX_E / 64];
        float myp = 0.0f;
        const int myid = topk_token_wave<SMALL_GROUP_MAX_E / 64>(r, lg, 0, nullptr, msk, &myp);
        if (lane < k) {
            s_e[lane] = myid;
            s_p[lane] = myp;
        }
    } else if (wave == 1 && b == 0) {  // the caller's logits and dispatch tables
        if (lane < E) a.ra.logits[lane] = lg[lane];
        if (64 + lane < E) a.ra.logits[64 + lane] = lg[64 + lane];
        topk_dispatch_wave<SMALL_GROUP_MAX_E / 64>(a.ra, a.o, lg, nullptr);
    }
    __syncthreads();

    // ---- gate/up: tile decodep_gu_tile(b, grp) of the (slot, row tile) list on waves 4 grp .. 4 grp + 3
    {
        const int grp = wave >> 2, lw = wave & 3, mat = lw >> 1, kw = lw & 1;
        const int t = decodep_gu_tile(b, grp, NB, a.G.nrt);
        const bool active = t >= 0 && t < ng;
        const int slot = active ? t / a.G.nrt : 0, rt = active ? t - slot * a.G.nrt : 0;
        const int e = s_e[slot];
        const ActLds A{xq, xs, nullptr, d};
        const QMat& W = mat ? a.U : a.G;
        const int nu = active ? n_units<TG>(a.G.nkb) : 0;
        float acc[1] = {0.0f};
        kloop_d<TG, DP_DEPTH>(
            W, e, rt, kw, nu, 2, m, h, [] {},
            [&](const typename Fmt<TG>::Raw& c, int u) { unit_accum<TG, 1>(c, A, u, h, 1, a.G.nkb, acc); });
        acc[0] += __shfl_xor(acc[0], 32, 64);
        if (h == 0) red[wave][m] = acc[0];
        __syncthreads();
        if (lw == 0 && active) {  // SwiGLU and h's Q8_0 block (as k_gemv_gateup), device-coherent
            const float gv = red[wave][m] + red[wave + 1][m], uv = red[wave + 2][m] + red[wave + 3][m];
            float2 sv;
            const int q = q8_block_vals(gated(gv, uv, a.G.act), sv);
            const uint32_t q1 = (uint32_t)__shfl_down(q, 1, 64), q2 = (uint32_t)__shfl_down(q, 2, 64),
                           q3 = (uint32_t)__shfl_down(q, 3, 64);
            const uint32_t word = ((uint32_t)q & 0xFFu) | ((q1 & 0xFFu) << 8) | ((q2 & 0xFFu) << 16) | (q3 << 24);
            // every word carries the launch number, so neither store waits for the other
            if (h == 0 && (m & 3) == 0)
                __hip_atomic_store(a.hw + (size_t)slot * (a.hq.K / 4) + rt * 8 + (m >> 2),
                                   ((uint64_t)a.epoch << 32) | word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0)
                __hip_atomic_store(reinterpret_cast<uint64_t*>(a.hq.s + (size_t)slot * (a.hq.K / 32) + rt),
                                   ((uint64_t)__float_as_uint(sv.y) << 32) | __float_as_uint(sv.x) | a.htag,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // ---- down: tiles b, b + G of the (slot, row tile) list on waves 0 .. DOWN_WAVES - 1 (the single-token
    // down GEMV's unit split and wave-order sum, so the step is bit-identical to the separate launches).
    // h is taken unit by unit as it is published: waves DOWN_WAVES .. 2 DOWN_WAVES - 1 each serve one down
    // wave, reading the h words of its units' K ranges (DP_HDEPTH units ahead) until every word carries
    // this launch's number (quants) or tag (scales), staging them into the LDS copy of h and raising the
    // unit's LDS flag; the down wave streams its weight units (DP_DEPTH ahead) and consumes each once its
    // flag is up, in ascending order as before.  The low K of h is published first (decodep_gu_tile), so
    // the down streams start while the last gate/up tiles are still running.
    static_assert(2 * DOWN_WAVES <= DP_WAVES, "a poller wave per down wave");
    constexpr int UE = dp_unit_elems<TD>();  // h elements per down unit
    static_assert(UE / 4 <= 64 && UE % 32 == 0, "one h word per lane");
    for (int j = 0; j < 2; ++j) {
        const int t = b + j * NB;
        if (t >= nd) break;  // block-uniform
        const int slot = t / a.D.nrt, rt = t - slot * a.D.nrt;
        const int e = s_e[slot];
        const float p = s_p[slot];
        const int K = a.hq.K, KB = K / 32;
        const ActLds A{smem, reinterpret_cast<const float2*>(smem + K), nullptr, K};
        const int nu = n_units<TD>(a.D.nkb);
        const int flag = j + 1;  // this tile's value of a unit's LDS flag
        if (j) __syncthreads();  // the previous tile's reduction has read red and its h
        float acc[1] = {0.0f};
        if (wave < DOWN_WAVES) {
            // the down wave: weight units wave, wave + DOWN_WAVES, ... with DP_DEPTH in flight
            typename Fmt<TD>::Raw r[DP_DEPTH];
#pragma unroll
            for (int i = 0; i < DP_DEPTH; ++i) {
                const int u = wave + i * DOWN_WAVES;
                Fmt<TD>::load(r[i], a.D, e, rt, u, m, h, u < nu);
            }
            for (int u = wave; u < nu; u += DP_DEPTH * DOWN_WAVES) {
#pragma unroll
                for (int i = 0; i < DP_DEPTH; ++i) {
                    const int ui = u + i * DOWN_WAVES;
                    if (ui >= nu) break;  // wave-uniform
                    // its h is staged once the flag is up (the poller raises it on giving up too)
                    for (int it = 0; __hip_atomic_load(hflag + ui, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != flag;
                         ++it) {
                        if (it >= 64 * (int)a.spin_limit) {  // a backstop: the poller bounds the wait
                            if (lane == 0) dec_fail(a);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                    }
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
                    unit_accum<TD, 1>(r[i], A, ui, h, 1, a.D.nkb, acc);
                    const int un = ui + DP_DEPTH * DOWN_WAVES;
                    Fmt<TD>::load(r[i], a.D, e, rt, un, m, h, un < nu);
                }
            }
        } else if (wave < 2 * DOWN_WAVES) {
            // the poller of down wave pw: its units' h words, DP_HDEPTH units ahead
            const int pw = wave - DOWN_WAVES;
            const uint64_t* qw = a.hw + (size_t)slot * (K / 4);
            const uint64_t* ss = reinterpret_cast<const uint64_t*>(a.hq.s + (size_t)slot * KB);
            // this lane's words of unit u: quant word u * UE / 4 + lane, scale word u * UE / 32 + lane
            // (words outside the unit or past K read as published)
            auto hload = [&](int u, uint64_t& hv, uint64_t& sv) {
                const int w = u * (UE / 4) + lane, sw = u * (UE / 32) + lane;
                const bool in = u < nu;
                hv = (in && lane < UE / 4 && w < K / 4) ? __hip_atomic_load(qw + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                                        : (uint64_t)a.epoch << 32;
                sv = (in && lane < UE / 32 && sw < KB) ? __hip_atomic_load(ss + sw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                                       : (uint64_t)a.htag;
            };
            uint64_t hv[DP_HDEPTH], sv[DP_HDEPTH];
#pragma unroll
            for (int i = 0; i < DP_HDEPTH; ++i) hload(pw + i * DOWN_WAVES, hv[i], sv[i]);
            for (int u = pw; u < nu; u += DP_HDEPTH * DOWN_WAVES) {
#pragma unroll
                for (int i = 0; i < DP_HDEPTH; ++i) {
                    const int ui = u + i * DOWN_WAVES;
                    if (ui >= nu) break;  // wave-uniform
                    for (int it = 0;; ++it) {
                        const bool ok = (uint32_t)(hv[i] >> 32) == a.epoch && ((uint32_t)sv[i] & DEC_HTAG_MASK) == a.htag;
                        if (__all(ok && !a.giveup_test)) break;
                        if (it >= (int)a.spin_limit) {
                            if (lane == 0) dec_fail(a);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(1);
                        hload(ui, hv[i], sv[i]);
                    }
                    const int w = ui * (UE / 4) + lane, sw = ui * (UE / 32) + lane;
                    if (lane < UE / 4 && w < K / 4) reinterpret_cast<uint32_t*>(smem)[w] = (uint32_t)hv[i];
                    if (lane < UE / 32 && sw < KB) reinterpret_cast<uint64_t*>(smem + K)[sw] = sv[i] & ~(uint64_t)DEC_HTAG_MASK;
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // h of the unit is in LDS before its flag
                    if (lane == 0) __hip_atomic_store(hflag + ui, flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    hload(ui + DP_HDEPTH * DOWN_WAVES, hv[i], sv[i]);
                }
            }
        }
        acc[0] += __shfl_xor(acc[0], 32, 64);
        if (h == 0 && wave < DOWN_WAVES) red[wave][m] = acc[0];
        __syncthreads();
        if (wave == 0 && h == 0) {
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < DOWN_WAVES; ++w) s += red[w][m];
            const int row = rt * 32 + m;
            if (!(a.D.valid_rows && row >= a.D.valid_rows)) atomicAdd(a.out + row, p * s);
        }
    }
}

bool decodep_fits(int gtype, int dtype, int d, int f, int E, int k, bool shared, bool fold, int gate_nrt,
                  int down_nrt) {
    const int nb = num_cus();
    if (shared || !fold || k != 2 || !decode1_fits(gtype, dtype, d, f, E, k, 0, false, dtype, false) || E > nb ||
        decodep_lds(d, f, E) > DP_LDS_MAX || down_nrt * k > 2 * nb)
        return false;
    // gate/up: at most DP_GROUPS tiles per block; a block zeroing output rows (its down tile of slot 0)
    // also stores h of slot 1 afterwards, which the slot-1 down tile of those rows waits for
    const int ng = gate_nrt * k;
    if (ng > DP_GROUPS * nb) return false;
    // every tile on exactly one (block, group)
    std::vector<int> seen(ng, 0);
    for (int b = 0; b < nb; ++b)
        for (int j = 0; j < DP_GROUPS; ++j) {
            const int t = decodep_gu_tile(b, j, nb, gate_nrt);
            if (t >= ng) return false;
            if (t >= 0) ++seen[t];
        }
    for (int c : seen)
        if (c != 1) return false;
    for (int b = 0; b < nb && b < down_nrt; ++b) {
        bool s1 = false;
        for (int j = 0; j < DP_GROUPS; ++j) {
            const int t = decodep_gu_tile(b, j, nb, gate_nrt);
            s1 = s1 || (t >= gate_nrt && t < ng);
        }
        if (!s1) return false;
    }
    return true;
}

// One block per CU, every block resident at once (its LDS leaves room for no second one): a plain
// launch.  (A cooperative launch, which checks the co-residency itself, measured ~15 us more per step.)
int launch_decode_p(const Decode1Args& a, int gtype, int dtype, hipStream_t st) {
    const size_t lds = decodep_lds(a.d, a.hq.K, a.E);
    hipError_t err = hipErrorInvalidValue;
    auto go = [&](auto kern) {
        lds_optin(kern, lds);
        hipLaunchKernelGGL(kern, dim3(num_cus()), dim3(DP_THREADS), lds, st, a);
        err = hipGetLastError();
    };
#define JX_DECP(G, D) \
    if (gtype == G && dtype == D) { go(k_decode_p<G, D>); return err == hipSuccess ? 0 : -1; }
    JX_DECP(T_Q4_0, T_Q4_0)
    JX_DECP(T_Q8_0, T_Q8_0)
    JX_DECP(T_Q4_K, T_Q4_K)
    JX_DECP(T_Q5_K, T_Q5_K)
    JX_DECP(T_Q6_K, T_Q6_K)
    JX_DECP(T_Q4_K, T_Q6_K)
    JX_DECP(T_Q5_K, T_Q6_K)
#undef JX_DECP
    return -1;
}

bool launch_gemv_down(const QMat& dn, const ActQ8& hq, const float* hf, int hf_ld, const Groups& grp, int slots,
                      int tb, float* y, hipStream_t st, const CombineOut& comb, SharedPart* sh) {
    // the folded combine is written for the single-token and four-token GEMVs (the few-token path)
    const CombineOut c = tb <= 4 ? comb : CombineOut{};
    if (hf) {  // fp32 activations
        switch (dn.type) {
            case T_Q4_0: return down_t<T_Q4_0, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, nullptr);
            case T_Q5_0: return down_t<T_Q5_0, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, nullptr);
            case T_Q8_0: return down_t<T_Q8_0, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, nullptr);
            case T_Q4_K: return down_t<T_Q4_K, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, nullptr);
            case T_Q5_K: return down_t<T_Q5_K, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, nullptr);
            case T_Q6_K: return down_t<T_Q6_K, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, nullptr);
            default: return false;
        }
    }
    switch (dn.type) {
        case T_Q4_0: return down_t<T_Q4_0, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, sh);
        case T_Q8_0: return down_t<T_Q8_0, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, sh);
        case T_Q4_K: return down_t<T_Q4_K, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, sh);
        case T_Q5_K: return down_t<T_Q5_K, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, sh);
        case T_Q6_K: return down_t<T_Q6_K, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st, c, sh);
        default: return false;
    }
}

bool gemv_gateup_joins(int type, int nrt, int slots, int tb, int snrt, int sslots) {
    if (!gemv_mxt_takes(type, true, nrt, slots, tb)) return false;
    int mr = 1;
    switch (type) {
        case T_Q4_0: mr = mx_mr_max<T_Q4_0, true>(); break;
        case T_Q8_0: mr = mx_mr_max<T_Q8_0, true>(); break;
        case T_Q4_K: mr = mx_mr_max<T_Q4_K, true>(); break;
        case T_Q5_K: mr = mx_mr_max<T_Q5_K, true>(); break;
        case T_Q6_K: mr = mx_mr_max<T_Q6_K, true>(); break;
        default: return false;
    }
    return (nrt + mr - 1) / mr * slots + (snrt + mr - 1) / mr * sslots <= 4 * num_cus();
}

bool gemv_mxt_takes(int type, bool gateup, int nrt, int slots, int tb) {
    if (tb <= 4 || nrt * slots < MX_MR_MIN_ITEMS) return false;
    switch (type) {
        case T_Q4_0: return (gateup ? mx_mr_max<T_Q4_0, true>() : mx_mr_max<T_Q4_0, false>()) > 1;
        case T_Q8_0: return (gateup ? mx_mr_max<T_Q8_0, true>() : mx_mr_max<T_Q8_0, false>()) > 1;
        case T_Q4_K: return (gateup ? mx_mr_max<T_Q4_K, true>() : mx_mr_max<T_Q4_K, false>()) > 1;
        case T_Q5_K: return (gateup ? mx_mr_max<T_Q5_K, true>() : mx_mr_max<T_Q5_K, false>()) > 1;
        case T_Q6_K: return (gateup ? mx_mr_max<T_Q6_K, true>() : mx_mr_max<T_Q6_K, false>()) > 1;
        default: return false;
    }
}

int shared_down_kparts(int type, int K, int Ks) {
    int bpu = 0;
    switch (type) {
        case T_Q4_0: bpu = Mx<T_Q4_0>::BPU; break;
        case T_Q8_0: bpu = Mx<T_Q8_0>::BPU; break;
        case T_Q4_K: bpu = Mx<T_Q4_K>::BPU; break;
        case T_Q5_K: bpu = Mx<T_Q5_K>::BPU; break;
        case T_Q6_K: bpu = Mx<T_Q6_K>::BPU; break;
        default: return 1;
    }
    const int u = (K / 32 + bpu - 1) / bpu, us = (Ks / 32 + bpu - 1) / bpu;
    return std::max(1, std::min(SHARED_KPARTS_MAX, (us + u - 1) / std::max(1, u)));
}

template <int TYPE>
static size_t mxh_lds_total(int K) {
    constexpr int MR = mxh_mr<TYPE>();
    return mxh_lds(K, is_kquant(TYPE)) + (size_t)MR * MXH_WAVES * (MX_NT / 2) * 64 * sizeof(float) + MX_NT * sizeof(float);
}

bool gemv_down_f16_fits(int type, int K) {
    if (K % 128 != 0) return false;
    switch (type) {
        case T_Q4_K: return mxh_lds_total<T_Q4_K>(K) <= (size_t)160 * 1024;
        case T_Q5_0: return mxh_lds_total<T_Q5_0>(K) <= (size_t)160 * 1024;
        default: return false;
    }
}

void launch_gemv_down_f16(const QMat& dn, const ActH& hh, const Groups& grp, int slots, float* y, hipStream_t st) {
    const int K = hh.K;
    // 8-token passes up to 4 pairs per expert slot on average (DeepSeek-V2-Lite-shaped 16 / 32 tokens
    // 112.9 / 131.4 -> 109.1 / 123.8 us per step, Q4_K_M mix at 32 tokens 132.6 -> 124.5 us); beyond, the
    // groups' second passes cost more (64 / 96 tokens 149.8 / 193.4 -> 151.5 / 203.6 us)
    const int ntp = (size_t)grp.n_tok * grp.top_k <= (size_t)4 * slots ? 8 : MX_NT;
    auto go = [&](auto k8, auto k16, int mr, bool kq) {
        const size_t lds = mxh_lds(K, kq, ntp);
        const dim3 grid((dn.nrt + mr - 1) / mr * slots), blk(MXH_WAVES * 64);
        if (ntp == 8) {
            lds_optin(k8, lds);
            hipLaunchKernelGGL(k8, grid, blk, lds, st, dn, hh, grp, y);
        } else {
            lds_optin(k16, lds);
            hipLaunchKernelGGL(k16, grid, blk, lds, st, dn, hh, grp, y);
        }
    };
    switch (dn.type) {
        case T_Q4_K:
            go(k_gemv_mxh<T_Q4_K, MXH_WAVES, mxh_mr<T_Q4_K>(), 8>, k_gemv_mxh<T_Q4_K, MXH_WAVES, mxh_mr<T_Q4_K>(), MX_NT>,
               mxh_mr<T_Q4_K>(), true);
            break;
        case T_Q5_0:
            go(k_gemv_mxh<T_Q5_0, MXH_WAVES, mxh_mr<T_Q5_0>(), 8>, k_gemv_mxh<T_Q5_0, MXH_WAVES, mxh_mr<T_Q5_0>(), MX_NT>,
               mxh_mr<T_Q5_0>(), false);
            break;
        default: break;
    }
}

}  // namespace jx
